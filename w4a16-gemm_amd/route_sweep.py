#!/usr/bin/env python3
"""Auto-route quality: the planner's choice against every forced config, per shape and batch size.

For each (N, K, G) shape and M, times `w4a16_gemm(Wp, x, scales)` with the auto planner and with
each prefill tile config forced through W4A16_PREFILL (M > 16) or each decode kernel shape and
split count forced through W4A16_DECODE (M <= 16), and reports the auto config, the fastest
forced config and their ratio.  Timing is bench_gemm's: a HIP graph of calls over distinct weight
copies (working set --target-mb), replayed untimed for --warm-ms first, median per call over
--reps replays, the faster of two rounds (auto first in one, last in the other).  A forced
setting the planner ignores (the config does not fit the shape) is skipped.

    python w4a16-gemm_amd/route_sweep.py --md out.md
"""
from __future__ import annotations

import argparse
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

from bench_gemm import LLAMA3_8B, GraphTimer, load_weights  # noqa: E402

# Llama-3-8B projections (bench_gemm), plus BASELINE configs[2] and configs[3].
SHAPES = [(name, n, k, 128) for name, (n, k) in LLAMA3_8B.items()] + [
    ("configs[2] gate", 14336, 4096, 64), ("configs[3] 70B gate_up", 28672, 8192, 128)]
PREFILL_CONFIGS = range(1, 25)
DECODE_VARIANTS = range(0, 32)
DECODE_SPLITS = (1, 2, 4)


def settled_timer(torch, calls, warm_ms: float):
    """bench_gemm's GraphTimer, replayed untimed for at least warm_ms of wall time first: the
    shader clock of a power-bound launch takes tens of milliseconds to settle after the GPU idles
    (graph capture, a switch of shapes), and a few warm replays leave a setting timed early in that
    ramp reading several percent high."""
    timer = GraphTimer(torch, calls)
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(4):
            timer.graph.replay()
        torch.cuda.synchronize()
    return timer


def forced_plans(w4a16_opt, M, N, K, G):
    """(label, env name, env value, kernel name) of every forced setting the planner accepts."""
    out = []
    if M <= 16:
        for v in DECODE_VARIANTS:
            for sp in DECODE_SPLITS:
                os.environ["W4A16_DECODE"] = f"{v},{sp}"
                info = w4a16_opt.plan_info(M, N, K, G)
                del os.environ["W4A16_DECODE"]
                if info["kernel"] == 0 and info["decode_variant"] == v and info["splits"] == sp:
                    out.append((f"d{v}/{sp}", "W4A16_DECODE", f"{v},{sp}", info["kernel_name"]))
    else:
        for cfg in PREFILL_CONFIGS:
            os.environ["W4A16_PREFILL"] = str(cfg)
            info = w4a16_opt.plan_info(M, N, K, G)
            del os.environ["W4A16_PREFILL"]
            if info["kernel"] == cfg:
                out.append((f"p{cfg}", "W4A16_PREFILL", str(cfg), info["kernel_name"]))
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--M", default="1,4,8,16,17,32,64,128,256,512,1024,2048")
    ap.add_argument("--shape", action="append", help="name,N,K,G (repeatable); default: Llama-3-8B + configs[2..3]")
    ap.add_argument("--target-mb", type=float, default=512)
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--warm-ms", type=float, default=30.0, help="untimed replays before each timing (ms of wall time)")
    ap.add_argument("--md", default=None, help="write the summary table (Markdown) here")
    ap.add_argument("--json", default=None, help="write every timing (auto and each forced setting) here")
    args = ap.parse_args(argv)
    Ms = [int(v) for v in args.M.split(",")]
    shapes = SHAPES if not args.shape else [
        (f[0], int(f[1]), int(f[2]), int(f[3])) for f in (s.split(",") for s in args.shape)]

    import torch
    import w4a16_opt
    from w4a16_opt import w4a16_gemm
    for var in ("W4A16_PREFILL", "W4A16_DECODE"):
        os.environ.pop(var, None)

    rows, dump = [], []
    for index, (name, N, K, G) in enumerate(shapes):
        weights, _ = load_weights(torch, N, K, G, args.target_mb, seed=index)
        for M in Ms:
            x = torch.randn((M, K), device="cuda", dtype=torch.float16)
            calls = [lambda w=w, s=s: w4a16_gemm(w, x, s) for w, s in weights]
            auto = w4a16_opt.plan_info(M, N, K, G)
            # Every setting is timed in each of two rounds (auto first in one, last in the
            # other) and keeps its faster median: a graph timed right after a switch of shapes
            # or clocks reads high.
            forced = forced_plans(w4a16_opt, M, N, K, G)
            times = {}
            for order in (["auto"] + forced, forced + ["auto"]):
                for item in order:
                    if item == "auto":
                        us = settled_timer(torch, calls, args.warm_ms).per_call_us(args.reps)[0]
                        times["auto"] = min(times.get("auto", us), us)
                        continue
                    label, var, value, kname = item
                    os.environ[var] = value
                    try:
                        us = settled_timer(torch, calls, args.warm_ms).per_call_us(args.reps)[0]
                    finally:
                        del os.environ[var]
                    times[label] = min(times.get(label, us), us)
            auto_us = times["auto"]
            best = min(((label, times[label], kname) for label, _, _, kname in forced), key=lambda b: b[1])
            rows.append((name, N, K, G, M, auto["kernel_name"], auto_us, best))
            dump.append({"shape": name, "N": N, "K": K, "G": G, "M": M, "auto": auto["kernel_name"],
                         "times_us": times, "kernels": {label: kname for label, _, _, kname in forced}})
            print(f"{name} N={N} K={K} G={G} M={M}: auto {auto['kernel_name']} {auto_us:.2f} us; "
                  f"best forced {best[0]} {best[2]} {best[1]:.2f} us; auto/best {auto_us / best[1]:.3f}", flush=True)
            del x, calls
        del weights
        torch.cuda.empty_cache()

    lines = ["| shape | N | K | G | M | auto kernel | auto us | best forced | best us | auto / best |",
             "|---|---|---|---|---|---|---|---|---|---|"]
    for name, N, K, G, M, akern, aus, (blabel, bus, bkern) in rows:
        flag = " **(>5%)**" if aus > 1.05 * bus else ""
        lines.append(f"| {name} | {N} | {K} | {G} | {M} | `{akern}` | {aus:.2f} | {blabel} `{bkern}` | {bus:.2f} | "
                     f"{aus / bus:.3f}{flag} |")
    table = "\n".join(lines)
    print(table)
    if args.md:
        with open(args.md, "w", encoding="utf-8") as f:
            f.write(table + "\n")
    if args.json:
        import json
        with open(args.json, "w", encoding="utf-8") as f:
            json.dump(dump, f, indent=1)
    worst = max(aus / bus for *_, aus, (_, bus, _) in rows)
    print(f"worst auto/best ratio: {worst:.3f}; rows over 1.05: {sum(aus > 1.05 * bus for *_, aus, (_, bus, _) in rows)}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
