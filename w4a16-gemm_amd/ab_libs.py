#!/usr/bin/env python3
"""Alternating A/B timing of builds of libw4a16_hip.so, or of forced plans of one build, in one
process through the C ABI (include/w4a16.h).

    python w4a16-gemm_amd/ab_libs.py SPEC [SPEC ...] [--cases decode;c1;M,N,K,G ...] [--reps 7]
    SPEC = path/to/libw4a16_hip.so[@VAR=VALUE[+VAR=VALUE...]]

The environment after `@` (e.g. W4A16_DECODE=18,1 to force a decode shape) is set while that
spec's calls are planned and captured.  Giving a spec several times (A B A B ...) alternates it.

Per case (M, N, K, G): random packed weights and scales in enough copies that one pass over them
exceeds 600 MB (over twice the 256 MB Infinity Cache, so every call reads its weights from HBM),
one eager pass and one HIP graph per spec over all copies (each spec writes its own outputs),
--warm-ms of untimed replays of all graphs, then --reps rounds in which each graph in turn is
replayed --replays times between two HIP events, the order rotating by one spec per round (the
graph timed first after a round's synchronisation reads slightly slower; give --reps as a
multiple of the number of specs).  Prints the median microseconds per call of each
spec, the mean per distinct spec over its repetitions, the plans (kernel, decode shape, splits,
grid), and whether every spec's outputs equal the first spec's bit for bit (else the largest
difference relative to the largest output).

The same plan given twice reads within a few hundredths of a microsecond per decode call this way
on one box; the decode and planner changes in the design notes were measured with it.
"""
from __future__ import annotations

import argparse
import ctypes
import os
import statistics
import time


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


# Named case sets: BASELINE configs[1] (the Llama-3-8B MLP decode calls), configs[0], configs[2]
# and configs[3].
CASE_SETS = {
    "decode": [(m, 14336, 4096, 128) for m in (1, 4, 8, 16)] + [(m, 4096, 14336, 128) for m in (1, 4, 8, 16)],
    "c1": [(1, 4096, 4096, 128)],
    "moderate": [(128, 14336, 4096, 64)],
    "prefill": [(2048, 28672, 8192, 128)],
}
WORKING_SET_BYTES = 600 * 2**20


def parse_cases(text: str):
    cases = []
    for tok in filter(None, (t.strip() for t in text.split(";"))):
        if tok in CASE_SETS:
            cases += CASE_SETS[tok]
        else:
            M, N, K, G = (int(v) for v in tok.split(","))
            cases.append((M, N, K, G))
    return cases


def parse_spec(spec: str):
    """'path[@A=1+B=2]' -> (path, {A: 1, B: 2})."""
    path, _, env = spec.partition("@")
    pairs = {}
    for kv in filter(None, env.split("+")):
        k, _, v = kv.partition("=")
        pairs[k] = v
    return path, pairs


def load(path: str) -> ctypes.CDLL:
    L = ctypes.CDLL(os.path.abspath(path))
    L.w4a16_plan_create.argtypes = [ctypes.POINTER(Problem), ctypes.c_int, ctypes.POINTER(Limits),
                                    ctypes.POINTER(Plan), ctypes.c_char_p, ctypes.c_size_t]
    L.w4a16_launch.argtypes = [ctypes.POINTER(Plan)] + [ctypes.c_void_p] * 7
    L.w4a16_query_device.argtypes = [ctypes.c_int, ctypes.POINTER(Limits)]
    return L


class with_env:
    def __init__(self, env):
        self.env, self.saved = env, {}

    def __enter__(self):
        for k, v in self.env.items():
            self.saved[k] = os.environ.get(k)
            os.environ[k] = v

    def __exit__(self, *exc):
        for k, v in self.saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def run_case(torch, libs, specs, case, lim, args):
    M, N, K, G = case
    wbytes = N * K // 2 + (K // G) * N * 2
    copies = max(2, min(64, -(-WORKING_SET_BYTES // wbytes)))
    gen = torch.Generator(device="cuda").manual_seed(1234)
    Wps = [torch.randint(-2**31, 2**31 - 1, (N * K // 8,), dtype=torch.int32, device="cuda", generator=gen)
           for _ in range(copies)]
    scs = [(torch.rand(K // G, N, device="cuda", generator=gen) * 0.018 + 0.002).half() for _ in range(copies)]
    x = torch.randn(M, K, device="cuda", generator=gen).half()
    stream = torch.cuda.Stream()
    graphs, outs, keep, plans = [], [], [], []
    for (path, env), L in zip(specs, libs):
        with with_env(env):
            ps = []
            for c in range(copies):
                prob = Problem(M, K, N, K // G, N * K // 8, Wps[c].data_ptr(), x.data_ptr(), scs[c].data_ptr())
                plan, err = Plan(), ctypes.create_string_buffer(512)
                rc = L.w4a16_plan_create(ctypes.byref(prob), args.variant, ctypes.byref(lim), ctypes.byref(plan), err, 512)
                if rc != 0:
                    raise SystemExit(f"{path}: plan of M={M} N={N} K={K} G={G} refused: {err.value.decode()}")
                ps.append(plan)
            plans.append((ps[0].kernel, ps[0].decode_variant, ps[0].splits, ps[0].grid))
            y = torch.empty(copies, M, N, dtype=torch.half, device="cuda")
            ws = torch.empty(max(1, max(p.workspace_bytes for p in ps)) // 4 + 64, dtype=torch.float32, device="cuda")
            cnt = torch.zeros(max(1 << 18, max(p.counter_slots for p in ps)) + 64, dtype=torch.int32, device="cuda")
            keep.append((ps, ws, cnt))
            torch.cuda.synchronize()                    # the zero fill ran on the default stream

            def launch_all(s):
                for c in range(copies):
                    rc = L.w4a16_launch(ctypes.byref(ps[c]), Wps[c].data_ptr(), x.data_ptr(), scs[c].data_ptr(),
                                        y[c].data_ptr(), ws.data_ptr(), cnt.data_ptr(), s)
                    if rc != 0:
                        raise SystemExit(f"{path}: launch failed ({rc})")
            with torch.cuda.stream(stream):
                launch_all(stream.cuda_stream)
            stream.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                launch_all(torch.cuda.current_stream().cuda_stream)
        graphs.append(g)
        outs.append(y)
    for g in graphs:
        for _ in range(3):
            g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < args.warm_ms:
        for g in graphs:
            g.replay()
        torch.cuda.synchronize()
    # Each round starts after a synchronisation, and the graph replayed first in a round reads
    # ~0.05 us per call slower (same plan in two positions); the order rotates by one per round,
    # so with --reps a multiple of the spec count every spec goes first equally often.
    times = [[] for _ in graphs]
    for rep in range(args.reps):
        for j in range(len(graphs)):
            i = (rep + j) % len(graphs)
            g = graphs[i]
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.replays):
                g.replay()
            e1.record()
            e1.synchronize()
            times[i].append(e0.elapsed_time(e1) * 1e3 / (args.replays * copies))
    if all(torch.equal(outs[0], o) for o in outs[1:]):
        same = "equal"
    else:
        ref = outs[0].float()
        scale = ref.abs().max().item() or 1.0
        same = "maxrel=" + ",".join(f"{(o.float() - ref).abs().max().item() / scale:.1e}" for o in outs[1:])
    med = [statistics.median(t) for t in times]
    b = wbytes + M * K * 2 + M * N * 2
    cols = " ".join(f"{us:8.3f}us({b / us / 1e3:5.0f}GB/s,{2 * M * N * K / us / 1e6:6.1f}TF)" for us in med)
    print(f"M={M:5d} N={N:6d} K={K:6d} G={G}: {cols}  plans={plans} outputs={same}", flush=True)
    by_spec = {}
    for (path, env), us in zip(specs, med):
        key = path + ("@" + "+".join(f"{k}={v}" for k, v in env.items()) if env else "")
        by_spec.setdefault(key, []).append(us)
    if len(by_spec) < len(specs):
        print("    mean per spec: " + "; ".join(f"{k}: {statistics.mean(v):.3f}us" for k, v in by_spec.items()),
              flush=True)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("specs", nargs="+", help="library path, optionally @VAR=VALUE[+VAR=VALUE]")
    ap.add_argument("--cases", default="decode", help="named sets (decode, c1, moderate, prefill) or M,N,K,G; ';'-separated")
    ap.add_argument("--reps", type=int, default=7)
    ap.add_argument("--replays", type=int, default=4)
    ap.add_argument("--variant", type=int, default=-1, help="variant passed to w4a16_plan_create")
    ap.add_argument("--warm-ms", type=float, default=30.0)
    args = ap.parse_args(argv)
    cases = parse_cases(args.cases)
    specs = [parse_spec(s) for s in args.specs]
    import torch
    if not torch.cuda.is_available():
        raise SystemExit("ab_libs.py times GPU launches: no GPU visible")
    cache = {}
    libs = [cache.setdefault(path, load(path)) for path, _ in specs]
    lim = Limits()
    if libs[0].w4a16_query_device(torch.cuda.current_device(), ctypes.byref(lim)) != 0:
        raise SystemExit("w4a16_query_device failed")
    for case in cases:
        run_case(torch, libs, specs, case, lim, args)
        torch.cuda.empty_cache()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
