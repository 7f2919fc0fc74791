#!/usr/bin/env python3
"""Per-wave timeline of the decode ring kernel at the Llama-3-8B MLP decode shapes (BASELINE
gate/up N=14336 K=4096 and down N=4096 K=14336, M = 1, 4, 8, 16, G = 128).

Loads libw4a16_hip_stamps.so (built by build.py: the library rebuilt with -DW4A16_WAVE_STAMPS, in
which lane 0 of every decode-ring wave records the chip-wide 100 MHz clock at kernel entry, after
the prologue's loads are issued, after its first chunk pair is consumed, when its stream is done
and after its output is written and acknowledged, plus its CU (HW_ID) and XCD (XCC_ID)) through
the C ABI, and for each shape:

  1. plans the call (auto planner) and uploads enough weight copies to exceed 2x the 256 MB
     Infinity Cache, so that the timed call reads its weights from HBM;
  2. warms the clock by replaying a graph of calls over the copies for --warm-ms;
  3. clears the stamps, replays the graph once more and reads the stamps, which are those of the
     graph's last call: a call that ran right behind others on the same stream, as the calls of
     bench.py do; repeated --reps times (each statistic below is the median over the repetitions).

Per shape it reports p10 / p50 / p90 over the waves of each point (microseconds from the
earliest wave's entry) and the last wave's `stored`, and, split by how many workgroups a CU ran,
the median `stream done` and the last `stored` of those CUs' waves.  The instrumented kernel
runs a few percent slower than the product kernel (the stamps wait for their own clock reads).

    python w4a16-gemm_amd/wave_timeline.py --md gpurun_out/timeline.md --json gpurun_out/timeline.json
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
STAMPS_LIB = os.path.join(HERE, "libw4a16_hip_stamps.so")
WORDS = 8                      # per wave: entry, issued, first, done, stored, HW_ID, XCC_ID, block
TICK_US = 0.01                 # s_memrealtime runs at 100 MHz
POINTS = ("entry", "issued", "first", "done", "stored")

SHAPES = [("gate_up", m, 14336, 4096) for m in (1, 4, 8, 16)] + [("down", m, 4096, 14336) for m in (1, 4, 8, 16)]


class Problem(ctypes.Structure):
    _fields_ = [("M", ctypes.c_int64), ("K", ctypes.c_int64), ("N", ctypes.c_int64),
                ("groups", ctypes.c_int64), ("wp_words", ctypes.c_int64),
                ("Wp", ctypes.c_void_p), ("x", ctypes.c_void_p), ("scales", ctypes.c_void_p)]


class Limits(ctypes.Structure):
    _fields_ = [("cu_count", ctypes.c_int32), ("lds_bytes_per_block", ctypes.c_int32),
                ("max_threads_per_block", ctypes.c_int32), ("gcn_arch", ctypes.c_int32)]


class Plan(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("M", "N", "K", "G", "kernel", "splits", "slab_chunks", "tile_n",
                                              "grid", "block", "counter_slots", "decode_variant")] + \
               [("workspace_bytes", ctypes.c_uint64)]


def load_lib(path: str = STAMPS_LIB) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise SystemExit(f"{path} is missing: run python w4a16-gemm_amd/build.py first")
    L = ctypes.CDLL(path)
    L.w4a16_plan_create.argtypes = [ctypes.POINTER(Problem), ctypes.c_int, ctypes.POINTER(Limits),
                                    ctypes.POINTER(Plan), ctypes.c_char_p, ctypes.c_size_t]
    L.w4a16_launch.argtypes = [ctypes.POINTER(Plan)] + [ctypes.c_void_p] * 7
    L.w4a16_query_device.argtypes = [ctypes.c_int, ctypes.POINTER(Limits)]
    L.w4a16_debug_wave_stamps.argtypes = [ctypes.c_void_p, ctypes.c_int32]
    L.w4a16_debug_wave_stamps_clear.argtypes = []
    L.w4a16_max_counter_slots.restype = ctypes.c_int32
    return L


def pct(v, q):
    """q-th percentile (0..100) of a list, nearest rank."""
    s = sorted(v)
    return s[min(len(s) - 1, max(0, round(q / 100 * (len(s) - 1))))]


def analyse(raw, nwaves):
    """Per-launch statistics from the raw stamp words of `nwaves` waves."""
    waves = [raw[i * WORDS:(i + 1) * WORDS] for i in range(nwaves)]
    missing = sum(1 for w in waves if w[0] == 0)
    if missing:
        raise RuntimeError(f"{missing} of {nwaves} waves recorded no stamps")
    t0 = min(w[0] for w in waves)
    rel = {p: [((w[k] - t0) & 0xFFFFFFFF) * TICK_US for w in waves] for k, p in enumerate(POINTS)}
    out = {p: (pct(rel[p], 10), pct(rel[p], 50), pct(rel[p], 90)) for p in POINTS}
    out["stored_max"] = max(rel["stored"])
    # CU of each wave: XCD and the CU/SH/SE fields of HW_ID; workgroups per CU from the block index.
    cu_of = [(w[6] & 0xF, (w[5] >> 8) & 0xFF) for w in waves]
    blocks = {}
    for cu, w in zip(cu_of, waves):
        blocks.setdefault(cu, set()).add(w[7])
    by_load = {}
    for i, cu in enumerate(cu_of):
        by_load.setdefault(len(blocks[cu]), []).append(i)
    out["by_load"] = {n: {"cus": sum(1 for b in blocks.values() if len(b) == n),
                          "done_p50": statistics.median(rel["done"][i] for i in idx),
                          "stored_max": max(rel["stored"][i] for i in idx)}
                      for n, idx in sorted(by_load.items())}
    out["cus"] = len(blocks)
    return out


def run(args):
    import torch

    L = load_lib(args.lib)
    dev = torch.device("cuda:0")
    lim = Limits()
    assert L.w4a16_query_device(0, ctypes.byref(lim)) == 0
    cnt = torch.zeros(L.w4a16_max_counter_slots() + 64, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    results = []
    for layer, M, N, K in SHAPES:
        G = 128
        wbytes = N * K // 2
        copies = max(2, int(args.target_mb * 2**20 // wbytes) + 1)
        g = torch.Generator(device=dev).manual_seed(M * 7 + N)
        Wp = [torch.randint(-2**31, 2**31 - 1, (N, K // 8), dtype=torch.int32, device=dev, generator=g)
              for _ in range(copies)]
        sc = [(torch.rand(K // G, N, device=dev, generator=g) * 0.02 + 0.001).half() for _ in range(copies)]
        x = (torch.randn(M, K, device=dev, generator=g) * 0.5).half()
        y = torch.empty(M, N, dtype=torch.half, device=dev)
        pr = Problem(M, K, N, K // G, N * K // 8, Wp[0].data_ptr(), x.data_ptr(), sc[0].data_ptr())
        pl = Plan()
        err = ctypes.create_string_buffer(512)
        assert L.w4a16_plan_create(ctypes.byref(pr), -1, ctypes.byref(lim), ctypes.byref(pl), err, 512) == 0, err.value
        assert pl.counter_slots <= cnt.numel() - 64
        ws = torch.empty(max(1, pl.workspace_bytes) // 4 + 64, dtype=torch.float32, device=dev)
        nwaves = pl.grid * (pl.block // 64)
        if nwaves > 8192:
            raise SystemExit(f"{layer} M={M}: {nwaves} waves exceed the stamp buffer")

        def launch(c):
            return L.w4a16_launch(ctypes.byref(pl), Wp[c].data_ptr(), x.data_ptr(), sc[c].data_ptr(), y.data_ptr(),
                                  ws.data_ptr(), cnt.data_ptr(), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))

        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            for c in range(copies):
                assert launch(c) == 0
        s.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            for c in range(copies - 1):
                launch(c)
        reps = []
        for r in range(args.reps):
            t0 = time.perf_counter()
            while (time.perf_counter() - t0) * 1e3 < args.warm_ms:
                graph.replay()
            torch.cuda.synchronize()
            assert L.w4a16_debug_wave_stamps_clear() == 0
            graph.replay()             # every call overwrites the stamps: the last call's remain
            torch.cuda.synchronize()
            raw = (ctypes.c_uint32 * (nwaves * WORDS))()
            assert L.w4a16_debug_wave_stamps(raw, nwaves) == 0
            reps.append(analyse(list(raw), nwaves))
        med = {p: tuple(statistics.median(rp[p][i] for rp in reps) for i in range(3)) for p in POINTS}
        med["stored_max"] = statistics.median(rp["stored_max"] for rp in reps)
        loads = sorted({n for rp in reps for n in rp["by_load"]})
        med["by_load"] = {n: {k: statistics.median(rp["by_load"][n][k] for rp in reps if n in rp["by_load"])
                              for k in ("cus", "done_p50", "stored_max")} for n in loads}
        row = {"layer": layer, "M": M, "N": N, "K": K, "G": G, "decode_variant": pl.decode_variant,
               "splits": pl.splits, "grid": pl.grid, "block": pl.block, "waves": nwaves, "reps": args.reps,
               "cus": statistics.median(rp["cus"] for rp in reps), **med}
        results.append(row)
        print(f"{layer} M={M}: d{pl.decode_variant}/{pl.splits} grid {pl.grid} x {pl.block}: "
              + ", ".join(f"{p} {med[p][1]:.2f}" for p in POINTS) + f", stored max {med['stored_max']:.2f} us",
              flush=True)
        del Wp, sc, graph
        torch.cuda.empty_cache()
    return results


def markdown(results) -> str:
    lines = ["| call | config (split) | workgroups x threads | entry | prologue issued | first pair done | stream done | stored (max) |",
             "|---|---|---|---|---|---|---|---|"]
    for r in results:
        cells = [" / ".join(f"{v:.2f}" for v in r[p]) for p in POINTS[:4]]
        lines.append(f"| {r['layer']} M={r['M']} | d{r['decode_variant']} ({r['splits']}) | {r['grid']} x {r['block']} | "
                     + " | ".join(cells) + f" | {r['stored_max']:.2f} |")
    lines += ["", "| call | CUs by workgroups run | stream done p50 | stored max |", "|---|---|---|---|"]
    for r in results:
        for n, b in r["by_load"].items():
            lines.append(f"| {r['layer']} M={r['M']} | {b['cus']:.0f} CUs x {n} | {b['done_p50']:.2f} | {b['stored_max']:.2f} |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--lib", default=STAMPS_LIB)
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--warm-ms", type=float, default=30.0)
    ap.add_argument("--target-mb", type=float, default=512.0, help="weight copies per shape (MiB in total)")
    ap.add_argument("--md", default=None)
    ap.add_argument("--json", default=None)
    a = ap.parse_args(argv)
    res = run(a)
    md = markdown(res)
    print(md)
    if a.md:
        with open(a.md, "w") as f:
            f.write(md)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(res, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
