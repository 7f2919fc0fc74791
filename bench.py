#!/usr/bin/env python3
"""Benchmark of the MI355X W4A16 GEMM on BASELINE.json's metric.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload decode|prefill|moderate|c1|quantize|gemv|copy]
                    [--no-cpu] [--no-prefill] [--json PATH]

Headline (default): decode GB/s on the Llama-3-8B MLP shapes,
gate/up (K=4096, N=14336) and down (K=14336, N=4096) at M = 1, 4, 8, 16, G = 128.  One
"step" is one call of the op for each of those 8 (shape, M) cases.  Weights rotate through
enough copies that the working set (>= 720 MB) exceeds twice the 256 MB Infinity Cache, so
every call streams its weights from HBM; x, scales and weights are resident in HBM before the
timed region.  The calls are captured in HIP graphs (as the reference benchmark does with CUDA
graphs, benchmarks/bench_gemm.py:36-56) and timed with HIP events on the launch stream.

Second leg: prefill TFLOP/s at M=2048, K=8192, N=28672, G=128.
Third leg: prefill at moderate batch, M=128, K=4096, N=14336, G=64,
reported against both rooflines (its arithmetic intensity sits just above the ridge point).
Eager leg (`eager` in the line): the op called as the reference's callers call it, without graphs:
microseconds per call for the 8 configs[1] calls and for configs[0] back to back, and the host
cost per call alone (measured while the GPU is held busy).
Fourth leg: the baseline GEMV of the reference's second extension (w4a16_ext.w4a16_gemv, its own
row-major [N, K/8] format) on the configs[0] shape K = N = 4096 and the gate/up shape K = 4096,
N = 14336; bytes = N*K/2 + 2*K + 6*N per call (W, A, sW, zW, C).  `--workload gemv` prints it
as the JSON line.

Algorithmic work (the roofline numerator): bytes = N*K/2 + (K/G)*N*2 + M*K*2 + M*N*2 per call,
flops = 2*M*N*K per call.  Peaks: HBM 8000 GB/s, fp16 dense MFMA 2500 TFLOP/s (MI355X spec).

The CPU baseline times the reference CPU path (unpack + fp16 (q-8)*s dequant, then the fp32
torch matmul and the fp16 cast: tests/quant.py:51-59, 77-85, restated in oracle/torch_ref.py) on
torch-CPU with every host thread, median of 5 reps per case (2 for configs[3], on a column slice),
with the dequant / matmul split and the CPU model in the JSON.  The baseline GEMV leg times the
oracle's C reference-order GEMV.  Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "w4a16-gemm_amd")
sys.path.insert(0, ROOT)
sys.path.insert(0, PKG)

HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFS = 2500.0
MALL_BYTES = 256 * 2**20

DECODE_CASES = [("gate_up", 14336, 4096, m) for m in (1, 4, 8, 16)] + \
               [("down", 4096, 14336, m) for m in (1, 4, 8, 16)]
PREFILL_CASE = ("mlp70b", 28672, 8192, 2048)
MODERATE_CASE = ("gate_up", 14336, 4096, 128, 64)          # M=128, G=64
GRAPH_STEPS = 400                                            # longest timed region captured as one graph
SIDE_STEPS, SIDE_WARMUP = 200, 20                            # timed and warm-up steps of the side legs
GEMV_CASES = [("c1_shape", 4096, 4096), ("gate_up", 14336, 4096)]    # (name, N, K) of w4a16_ext.w4a16_gemv
C1_CASE = ("c1", 4096, 4096, 1)                              # M=1, K=N=4096, G=128
G = 128


def alg_bytes(M, N, K, G=G):
    return N * K // 2 + (K // G) * N * 2 + M * K * 2 + M * N * 2


def alg_flops(M, N, K):
    return 2 * M * N * K


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_weights(torch, N, K, seed, copies, G=G):
    """BASELINE distributions: q ~ U{0..15} packed in the reference layout, scales ~ U[0.002, 0.02].
    The packing runs once on the host (oracle.quant.pack_int4 is only data preparation here); the
    copies are device clones."""
    from oracle import quant
    q, scales = quant.gen_codes_scales(N, K, G, seed)
    Wp = torch.from_numpy(quant.pack_int4(q)).cuda()
    s = torch.from_numpy(scales).cuda()
    return [(Wp, s)] + [(Wp.clone(), s.clone()) for _ in range(copies - 1)]


def graph_of(torch, fn_list):
    for f in fn_list:
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fn_list:
            f()
    torch.cuda.synchronize()
    return g


def time_graph(torch, graphs, steps, warmup):
    """Replay graphs[i % len] for warmup then exactly `steps` timed steps; HIP events on the
    current stream (where the op launches).  Returns elapsed ms of the timed region."""
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    end.record()
    end.synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def time_steps(torch, big, per_big, singles, steps, warmup):
    """Exactly `steps` timed steps: `big` (a graph of `per_big` steps) replayed steps // per_big
    times, then the remaining steps from the single-step graphs; `warmup` untimed single steps
    first.  HIP events on the current stream.  Returns elapsed ms of the timed region."""
    for i in range(warmup):
        singles[i % len(singles)].replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n_big, rem = divmod(steps, per_big)
    start.record()
    for _ in range(n_big):
        big.replay()
    for i in range(rem):
        singles[i % len(singles)].replay()
    end.record()
    end.synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def bench_decode(torch, gemm, steps, warmup):
    copies = 12                                    # per shape: 2 x 12 x ~30 MB = 720 MB > 2 x MALL
    w = {"gate_up": make_weights(torch, 14336, 4096, 101, copies),
         "down": make_weights(torch, 4096, 14336, 102, copies)}
    xs = {(name, M): torch.randn(M, K, device="cuda").half() for name, N, K, M in DECODE_CASES}
    per_shape = 4                                  # calls per shape per step
    phases = copies // per_shape                   # distinct copy rotations
    ys = []

    def step_calls(ph):
        calls = []
        for name, N, K, M in DECODE_CASES:
            idx = ph * per_shape + [c[3] for c in DECODE_CASES if c[0] == name].index(M)
            Wp, s = w[name][idx]
            x = xs[(name, M)]
            calls.append(lambda Wp=Wp, s=s, x=x: ys.append(gemm(Wp, x, s)))
        return calls
    # Every graph launch pays a bubble (~8 us on this box, a tenth of a step); like the reference
    # benchmark (one graph over many calls), the timed steps are captured as one graph of exactly
    # `steps` steps (GRAPH_STEPS at a time beyond that), cycling through the copy phases, so the
    # bubble is paid once per timed region whatever --steps is.  Single-step graphs serve the
    # untimed warm-up steps.
    per_big = min(steps, GRAPH_STEPS)
    singles = [graph_of(torch, step_calls(ph)) for ph in range(phases)]
    big = graph_of(torch, [c for i in range(per_big) for c in step_calls(i % phases)])
    # per-case timing (each case alone, rotating over all its copies)
    cases = []
    for name, N, K, M in DECODE_CASES:
        x = xs[(name, M)]
        g = graph_of(torch, [lambda Wp=Wp, s=s: gemm(Wp, x, s) for Wp, s in w[name]])
        reps = []
        for _ in range(5):
            reps.append(time_graph(torch, [g], 4, 1) / (4 * copies))
        us = statistics.median(reps) * 1e3
        b = alg_bytes(M, N, K)
        import w4a16_opt
        cases.append({"layer": name, "M": M, "N": N, "K": K, "us": round(us, 3),
                      "GBps": round(b / us / 1e3, 1), "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                      "kernel": w4a16_opt.plan_info(M, N, K, G)["kernel_name"]})
        log(f"decode {name} M={M}: {us:.2f} us  {b / us / 1e3:.0f} GB/s")
    ms = time_steps(torch, big, per_big, singles, steps, warmup)
    step_bytes = sum(alg_bytes(M, N, K) for _, N, K, M in DECODE_CASES)
    ms_per_step = ms / steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    avg_launch_us = ms_per_step * 1e3 / len(DECODE_CASES)
    return {"value": value, "ms_per_step": ms_per_step, "step_bytes": step_bytes,
            "avg_launch_us": avg_launch_us, "bytes_per_launch": step_bytes / len(DECODE_CASES),
            "cases": cases, "copies": copies, "steps_per_graph": per_big}


def bench_c1(torch, gemm, steps, warmup):
    """BASELINE configs[0] through w4a16_gemm (M=1, K=N=4096, G=128): the reference's published
    decode row "o, M=1" (benchmarks/results/latest.json:368-384).  Weights rotate over copies whose
    working set exceeds twice the Infinity Cache, in one graph; HIP events on the launch stream."""
    import w4a16_opt
    name, N, K, M = C1_CASE
    copies = max(2, -(-2 * MALL_BYTES // (N * K // 2 + (K // G) * N * 2)))
    w = make_weights(torch, N, K, 105, copies)
    x = torch.randn(M, K, device="cuda").half()
    g = graph_of(torch, [lambda Wp=Wp, s=s: gemm(Wp, x, s) for Wp, s in w])
    reps = [time_graph(torch, [g], max(1, steps // 10), 1) / (max(1, steps // 10) * copies) for _ in range(5)]
    us = statistics.median(reps) * 1e3
    gbs = alg_bytes(M, N, K) / (us * 1e-6) / 1e9
    log(f"decode c1 M={M} N={N} K={K}: {us:.2f} us  {gbs:.0f} GB/s")
    return {"us": us, "GBs": gbs, "copies": copies, "kernel": w4a16_opt.plan_info(M, N, K, G)["kernel_name"]}


def bench_prefill(torch, gemm, steps, warmup):
    name, N, K, M = PREFILL_CASE
    copies = 5                                     # 5 x 121 MB of weights + scales > 2 x MALL
    w = make_weights(torch, N, K, 103, copies)
    x = torch.randn(M, K, device="cuda").half()
    # One graph over the copies (one step = one call), replayed, plus single-call graphs for the
    # remainder, so a graph launch is paid per `copies` calls, as in the decode leg.
    calls = [lambda Wp=Wp, s=s: gemm(Wp, x, s) for Wp, s in w]
    singles = [graph_of(torch, [c]) for c in calls]
    big = graph_of(torch, calls)
    ms = time_steps(torch, big, len(calls), singles, steps, warmup)
    us = ms * 1e3 / steps
    tfs = alg_flops(M, N, K) / (us * 1e-6) / 1e12
    log(f"prefill {name} M={M}: {us:.1f} us  {tfs:.1f} TFLOP/s")
    import w4a16_opt
    return {"us": us, "TFLOPs": tfs, "steps": steps, "warmup": warmup,
            "kernel": w4a16_opt.plan_info(M, N, K, G)["kernel_name"]}


def bench_moderate(torch, gemm, steps, warmup):
    """BASELINE configs[2] (prefill at moderate batch: M=128, K=4096, N=14336, G=64): arithmetic
    intensity ~419 flop/B, just above the MI355X ridge (~315 flop/B), so both rooflines apply."""
    name, N, K, M, Gm = MODERATE_CASE
    copies = max(2, -(-2 * MALL_BYTES // (N * K // 2 + (K // Gm) * N * 2)))
    w = make_weights(torch, N, K, 104, copies, G=Gm)
    x = torch.randn(M, K, device="cuda").half()
    graphs = [graph_of(torch, [lambda Wp=Wp, s=s: gemm(Wp, x, s) for Wp, s in w])]
    ms = time_graph(torch, graphs, steps, warmup)
    us = ms * 1e3 / (steps * len(w))
    tfs = alg_flops(M, N, K) / (us * 1e-6) / 1e12
    gbs = alg_bytes(M, N, K, Gm) / (us * 1e-6) / 1e9
    log(f"moderate {name} M={M} G={Gm}: {us:.1f} us  {tfs:.1f} TFLOP/s  {gbs:.0f} GB/s")
    import w4a16_opt
    return {"us": us, "TFLOPs": tfs, "GBs": gbs, "copies": len(w),
            "kernel": w4a16_opt.plan_info(M, N, K, Gm)["kernel_name"]}


def bench_eager(torch, gemm, calls=240):
    """The op as the reference's callers use it: eager calls of w4a16_gemm, no graphs
    (tests/test_w4a16.py:25-27, kernel.cu:36-53, 174-201).
      * per call: `calls` calls back to back on one stream (configs[1]: the 8 decode calls in
        turn; configs[0]: the one call), weights rotating over copies that exceed twice the
        Infinity Cache, HIP events around the loop after a warm-up;
      * host: the same loop issued while the GPU is held busy by torch.cuda._sleep, so the wall
        time of the Python loop is the host cost alone (pybind, tensor checks, plan, y allocation,
        launch), per call."""
    from oracle import quant  # noqa: F401  (make_weights packs on the host)
    copies = 10                                    # per shape: 2 x 10 x ~30 MB = 600 MB > 2 x MALL
    w = {"gate_up": make_weights(torch, 14336, 4096, 111, copies),
         "down": make_weights(torch, 4096, 14336, 112, copies)}
    xs = {(name, M): torch.randn(M, K, device="cuda").half() for name, N, K, M in DECODE_CASES}
    seq = [(w[name][i % copies], xs[(name, M)]) for i in range(calls) for name, N, K, M in [DECODE_CASES[i % 8]]]
    c1n, c1N, c1K, c1M = C1_CASE
    c1copies = max(2, -(-2 * MALL_BYTES // (c1N * c1K // 2 + (c1K // G) * c1N * 2)))
    wc1 = make_weights(torch, c1N, c1K, 113, c1copies)
    xc1 = torch.randn(c1M, c1K, device="cuda").half()
    seq_c1 = [(wc1[i % c1copies], xc1) for i in range(calls)]

    def run(sq):
        for (Wp, s), x in sq:
            gemm(Wp, x, s)

    def device_us(sq):
        run(sq[:48])
        torch.cuda.synchronize()
        reps = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            run(sq)
            e1.record()
            e1.synchronize()
            reps.append(e0.elapsed_time(e1) * 1e3 / len(sq))
        return statistics.median(reps)

    def host_us(sq):
        reps = []
        for _ in range(3):
            torch.cuda.synchronize()
            torch.cuda._sleep(int(60e6))           # holds the GPU (tens of ms) while the loop issues
            t0 = time.perf_counter()
            run(sq)
            reps.append((time.perf_counter() - t0) * 1e6 / len(sq))
            torch.cuda.synchronize()
        return statistics.median(reps)

    dec_us, c1_us = device_us(seq), device_us(seq_c1)
    dec_host, c1_host = host_us(seq), host_us(seq_c1)
    # where the host time of one call goes (C++ steady-clock timing inside the binding, configs[0])
    import w4a16_opt
    torch.cuda.synchronize()
    torch.cuda._sleep(int(60e6))
    parts = w4a16_opt._debug_host_breakdown(wc1[0][0], xc1, wc1[0][1], 200)
    torch.cuda.synchronize()
    parts = {k: round(v, 3) for k, v in parts.items()}
    log(f"eager host breakdown (us per call): {parts}")
    log(f"eager: configs[1] {dec_us:.2f} us/call (host {dec_host:.2f}), configs[0] {c1_us:.2f} us/call "
        f"(host {c1_host:.2f})")
    step_bytes = sum(alg_bytes(M, N, K) for _, N, K, M in DECODE_CASES)
    return {"decode_us_per_call": round(dec_us, 3), "decode_GBps": round(step_bytes / 8 / dec_us / 1e3, 1),
            "decode_host_us_per_call": round(dec_host, 3),
            "c1_us_per_call": round(c1_us, 3), "c1_GBps": round(alg_bytes(c1M, c1N, c1K) / c1_us / 1e3, 1),
            "c1_host_us_per_call": round(c1_host, 3), "host_breakdown_us": parts,
            "method": f"{calls} eager w4a16_gemm calls back to back on the current stream (configs[1]: the 8 calls "
                      "in turn; configs[0]: one shape), weight copies > 2x Infinity Cache, HIP events; host = wall "
                      "time of the same Python loop while torch.cuda._sleep holds the GPU"}


def gemv_bytes(N, K):
    """Algorithmic bytes of one baseline GEMV call: W int4, A, and sW, zW, C fp16."""
    return N * K // 2 + 2 * K + 6 * N


def bench_gemv(torch, steps, warmup):
    """Baseline GEMV (w4a16_ext.w4a16_gemv) on GEMV_CASES.  One step = one call per case; weights
    rotate through copies whose working set exceeds twice the Infinity Cache, in HIP graphs."""
    import w4a16_ext
    cases, graphs, per_graph = [], [], []
    for name, N, K in GEMV_CASES:
        copies = max(2, -(-2 * MALL_BYTES // (N * K // 2)))
        Ws = [torch.randint(-2**31, 2**31 - 1, (N, K // 8), dtype=torch.int32, device="cuda") for _ in range(copies)]
        A = torch.randn(K, device="cuda").half()
        sW = (torch.rand(N, device="cuda") * 0.018 + 0.002).half()
        zW = torch.randn(N, device="cuda").half()
        g = graph_of(torch, [lambda W=W: w4a16_ext.w4a16_gemv(W, A, sW, zW) for W in Ws])
        ms = time_graph(torch, [g], steps, warmup)
        us = ms * 1e3 / (steps * copies)
        gbs = gemv_bytes(N, K) / (us * 1e-6) / 1e9
        log(f"gemv {name} N={N} K={K}: {us:.2f} us  {gbs:.0f} GB/s")
        rt = 2 if -(-N // 32) >= torch.cuda.get_device_properties(0).multi_processor_count else 1
        cases.append({"layer": name, "N": N, "K": K, "us": round(us, 3), "GBps": round(gbs, 1),
                      "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "copies": copies,
                      "kernel": f"w4a16::(anonymous namespace)::gemv_kernel<true, true, {rt}>"})
        del Ws, g
    total_b = sum(gemv_bytes(c["N"], c["K"]) for c in cases)
    total_us = sum(c["us"] for c in cases)
    return {"value": total_b / (total_us * 1e-6) / 1e9, "us_per_step": total_us, "bytes_per_step": total_b,
            "bytes_per_launch": total_b / len(cases), "avg_launch_us": total_us / len(cases), "cases": cases}


def cpu_baseline_gemv(max_seconds=12.0):
    """The oracle's reference-order loop (fp32 sum in k order, src/baseline/kernel.cu:22-33),
    repeated on a 256-row slice of the first GEMV case until max_seconds (the rate does not
    depend on the number of rows)."""
    import numpy as np
    from oracle import c_oracle
    nthreads = c_oracle.max_threads()
    rng = np.random.default_rng(13)
    total_b, total_t, rows = 0, 0.0, 0
    name, N, K = GEMV_CASES[0]
    R = 256
    W = rng.integers(-2**31, 2**31, (R, K // 8), dtype=np.int64).astype(np.int32)
    A = rng.standard_normal(K).astype(np.float16)
    s = rng.uniform(0.002, 0.02, R).astype(np.float16)
    z = rng.standard_normal(R).astype(np.float16)
    c_oracle.gemv(W, A, s, z, exact=False)                 # warm-up
    while total_t < max_seconds:
        t0 = time.perf_counter()
        c_oracle.gemv(W, A, s, z, exact=False)
        total_t += time.perf_counter() - t0
        total_b += gemv_bytes(R, K)
        rows += R
    return {"value": round(total_b / total_t / 1e9, 3), "unit": "GB/s", "cores": nthreads, "kind": "port",
            "sample": f"oracle C reference-order GEMV, {rows // R} calls on a {R}-row slice of the {name} shape "
                      f"(K={K}; {total_t:.2f} s, {nthreads} OpenMP threads, host {os.cpu_count()} cpus)"}


def bench_copy(torch, steps):
    """Calibration workload for HBM-traffic counters: an elementwise copy (torch.mul by 1) of a
    64 MiB fp16 tensor reads and writes exactly 64 MiB per launch."""
    n = 32 * 2**20
    a = torch.randn(n, device="cuda").half()
    b = torch.empty_like(a)
    for _ in range(steps):
        torch.mul(a, 1.0, out=b)
    torch.cuda.synchronize()
    return {"workload": "copy", "bytes_read_per_launch": 2 * n, "bytes_written_per_launch": 2 * n,
            "launches": steps}


QUANT_CASE = ("mlp70b", 28672, 8192)


def quant_bytes(N, K, G=G):
    """Algorithmic bytes of one quantise+pack of an fp16 [N, K] weight: read W, write Wp and scales."""
    return N * K * 2 + N * K // 2 + (K // G) * N * 2


def bench_quantize(torch, steps, warmup):
    """Device quantise + pack (w4a16_opt.quantize_pack) of the BASELINE prefill weight, fp16 input.
    W (470 MB) exceeds the Infinity Cache, so every launch streams it from HBM."""
    import w4a16_opt
    name, N, K = QUANT_CASE
    W = (torch.randn(N, K, device="cuda") * 0.02).half()
    for _ in range(max(1, warmup)):
        w4a16_opt.quantize_pack(W, G)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        w4a16_opt.quantize_pack(W, G)
    end.record()
    end.synchronize()
    us = start.elapsed_time(end) * 1e3 / steps
    gbs = quant_bytes(N, K) / (us * 1e-6) / 1e9
    log(f"quantize_pack {name} N={N} K={K}: {us:.1f} us  {gbs:.1f} GB/s")
    return {"us": us, "GBs": gbs}


def cpu_baseline_quantize(max_seconds=12.0):
    """The oracle's numpy quantize_w4 + pack_int4 (restatement of the reference's torch CPU path)
    on 1024-row slices of the quantise workload until max_seconds (rate is size-independent)."""
    import numpy as np
    from oracle import quant
    _, N, K = QUANT_CASE
    R = 1024
    W = (np.random.default_rng(12).standard_normal((R, K), dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    done, dt = 0, 0.0
    while dt < max_seconds and done < N // R:
        t0 = time.perf_counter()
        q, _ = quant.quantize_w4(W.astype(np.float32), G)
        quant.pack_int4(q)
        dt += time.perf_counter() - t0
        done += 1
    return {"value": round(quant_bytes(done * R, K) / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle numpy quantize_w4 + pack_int4 on {done} slices of 1024 x {K} fp16 ({dt:.2f} s)"}


def cpu_threads():
    """Threads for the CPU baseline: the host's CPUs available to this process, capped by
    OMP_NUM_THREADS when that is set (the GPU box gives each GPU job a share of its cores)."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except AttributeError:
        pass
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _median_s(fn, reps):
    fn()                                                     # warm-up
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _cpu_path_times(torch, N, K, Ms, G, seed, reps):
    """Median seconds of the reference CPU path (oracle/torch_ref.py: unpack + fp16 dequant, then
    the fp32 matmul and the fp16 cast) on torch-CPU: (dequant_s, {M: matmul_s})."""
    import numpy as np
    from oracle import quant, torch_ref
    q, scales = quant.gen_codes_scales(N, K, G, seed)
    Wp = torch.from_numpy(quant.pack_int4(q))
    s = torch.from_numpy(scales)
    del q
    box = {}

    def dequant():
        box["W"] = torch_ref.dequantize_w4(torch, torch_ref.unpack_int4(torch, Wp, N, K), s, G)
    t_deq = _median_s(dequant, reps)
    W = box.pop("W")
    t_mm = {}
    for M in Ms:
        x = torch.from_numpy(np.random.default_rng([seed, M]).standard_normal((M, K)).astype(np.float16))
        t_mm[M] = _median_s(lambda: torch_ref.ref_gemm(torch, x, W).half(), reps)
    return t_deq, t_mm


def cpu_baseline(cases, reps=5):
    """The reference CPU path (unpack, fp16 dequant, fp32 matmul: tests/quant.py:51-59, 77-85)
    timed on torch-CPU on the host, per decode case: one call = dequant + matmul."""
    import torch
    nthreads = cpu_threads()
    torch.set_num_threads(nthreads)
    shapes = {}
    for name, N, K, M in cases:
        shapes.setdefault((name, N, K), []).append(M)
    total_b, t_deq_all, t_mm_all, per = 0, 0.0, 0.0, []
    t0 = time.perf_counter()
    for i, ((name, N, K), Ms) in enumerate(shapes.items()):
        t_deq, t_mm = _cpu_path_times(torch, N, K, Ms, G, 7 + i, reps)
        for M in Ms:
            total_b += alg_bytes(M, N, K)
            t_deq_all += t_deq
            t_mm_all += t_mm[M]
            per.append(f"{name} M={M}: {1e3 * (t_deq + t_mm[M]):.1f} ms")
    wall = time.perf_counter() - t0
    tot = t_deq_all + t_mm_all
    return {"value": round(total_b / tot / 1e9, 3), "unit": "GB/s", "cores": nthreads, "kind": "port",
            "dequant_s": round(t_deq_all, 4), "matmul_s": round(t_mm_all, 4), "total_s": round(tot, 4),
            "cpu": cpu_model(), "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "sample": f"reference CPU path on torch-CPU (oracle/torch_ref.py: unpack + fp16 (q-8)*s, then "
                      f"x.float() @ W.float().t() and fp16 cast), each of the {len(cases)} decode calls once "
                      f"(median of {reps} reps after a warm-up; dequant timed once per weight shape and charged "
                      f"to every call of that shape): " + "; ".join(per) + f"; {wall:.1f} s wall"}


def cpu_baseline_prefill(ns=4096, reps=2):
    """The reference CPU path on torch-CPU for configs[3] (M=2048, K=8192) on an N-column slice of
    the weight (the rate does not depend on N): dequant + matmul, median of reps."""
    import torch
    nthreads = cpu_threads()
    torch.set_num_threads(nthreads)
    _, N, K, M = PREFILL_CASE
    t0 = time.perf_counter()
    t_deq, t_mm = _cpu_path_times(torch, ns, K, [M], G, 9, reps)
    tot = t_deq + t_mm[M]
    return {"value": round(alg_flops(M, ns, K) / tot / 1e12, 4), "unit": "TFLOP/s", "cores": nthreads,
            "kind": "port", "dequant_s": round(t_deq, 4), "matmul_s": round(t_mm[M], 4), "total_s": round(tot, 4),
            "cpu": cpu_model(), "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "sample": f"reference CPU path on torch-CPU (oracle/torch_ref.py) for M={M}, K={K} on an N={ns} "
                      f"column slice of the N={N} weight, median of {reps} reps after a warm-up "
                      f"({time.perf_counter() - t0:.1f} s wall)"}


def load_counters(kind, kernels):
    """Counter-derived figures for one workload from the committed rocprofv3 PMC summary
    (profiles/traffic.json): {field: value, "source": ..., "measured_on": [...]}, or None when that
    file has no entry or its entry was measured on other kernels than `kernels` (the ones this run
    launched) -- such figures would describe other code."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            ent = json.load(f).get(kind)
    except (OSError, ValueError):
        return None
    if not isinstance(ent, dict) or sorted(ent.get("kernels", [])) != sorted(set(kernels)):
        return None
    return ent


def tag_counters(roof, kind, kernels, fields):
    """Set roof[f] for f in fields from load_counters (None when not measured on these kernels)
    and name the source of the figures."""
    ent = load_counters(kind, kernels)
    for f in fields:
        roof[f] = ent.get(f) if ent else None
    roof["counters_source"] = (f"{ent['source']} (rocprofv3 --pmc, measured on the kernels named in kernel)"
                               if ent else "not measured on these kernels (profiles/traffic.json)")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--prefill-steps", type=int, default=60)
    ap.add_argument("--prefill-warmup", type=int, default=60,
                    help="untimed prefill calls before the prefill leg of the decode run: the clock settles "
                         "after ~50 calls of this power-bound shape")
    ap.add_argument("--workload", choices=("decode", "prefill", "moderate", "c1", "quantize", "gemv", "copy"),
                    default="decode",
                    help="prefill: configs[3] alone; moderate: configs[2] alone; c1: configs[0] alone (w4a16_gemm, "
                         "M=1, K=N=4096); quantize: device quantise+pack of "
                         "the prefill weight; gemv: the baseline GEMV (w4a16_ext); copy: HBM-counter calibration "
                         "kernel (64 MiB elementwise copy), no benchmark line")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill leg")
    ap.add_argument("--no-c1", action="store_true",
                    help="skip the configs[0] decode leg (for counter runs of the headline calls: its kernel has "
                         "the name of the down M=1 kernel)")
    ap.add_argument("--json", default=None, help="also write the JSON line to this file")
    a = ap.parse_args(argv)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the op runs on one GPU; several GPUs would shard "
              "N column-parallel or K row-parallel); use --gpus 1", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU available", file=sys.stderr)
        return 2
    from w4a16_opt import w4a16_gemm as gemm          # in-tree HIP build; no fallback
    torch.manual_seed(0)
    dev = torch.cuda.get_device_properties(0)
    log(f"device: {dev.name} ({getattr(dev, 'gcnArchName', '?')}), CUs={dev.multi_processor_count}")

    if a.workload == "copy":
        print(json.dumps(bench_copy(torch, a.steps)), flush=True)
        return 0
    if a.workload == "quantize":
        qr = bench_quantize(torch, a.steps, a.warmup)
        _, N, K = QUANT_CASE
        out = {"metric": "quantize+pack GB/s (algorithmic bytes: fp16 W read, Wp + scales written)",
               "value": round(qr["GBs"], 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
               "ms_per_step": round(qr["us"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
               "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
               "config": {"workload": f"quantize_pack of an fp16 [{N}, {K}] weight (BASELINE configs[3] weight), G={G}"},
               "roofline": {"bound": "hbm", "achieved": round(qr["GBs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(qr["GBs"] / HBM_PEAK_GBS, 4),
                            "kernel": "w4a16::quantize_pack_kernel<_Float16, 128>", "bytes_per_launch": quant_bytes(N, K)}}
        tag_counters(out["roofline"], "quantize", [out["roofline"]["kernel"]], ["traffic"])
        if not a.no_cpu:
            out["cpu_baseline"] = cpu_baseline_quantize()
        line = json.dumps(out)
        print(line, flush=True)
        if a.json:
            with open(a.json, "w") as f:
                f.write(line + "\n")
        return 0
    if a.workload == "gemv":
        gv = bench_gemv(torch, a.steps, a.warmup)
        out = {"metric": "baseline GEMV GB/s & %HBM peak (w4a16_ext.w4a16_gemv)",
               "value": round(gv["value"], 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
               "ms_per_step": round(gv["us_per_step"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
               "vs_baseline": None, "dtype": "int8 MFMA (exact), fp32 epilogue", "data": "synthetic",
               "config": {"workload": "baseline GEMV, W int32 [N, K/8]; one step = one call each of " +
                                      ", ".join(f"{n} N={N} K={K}" for n, N, K in GEMV_CASES),
                          "timing": "HIP graph replay over rotating weight copies, HIP events"},
               "roofline": {"bound": "hbm", "achieved": round(gv["value"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(gv["value"] / HBM_PEAK_GBS, 4),
                            "kernel": " + ".join(sorted({c["kernel"] for c in gv["cases"]})),
                            "bytes_per_launch": gv["bytes_per_launch"],
                            "avg_launch_us": round(gv["avg_launch_us"], 3)},
               "cases": gv["cases"]}
        tag_counters(out["roofline"], "gemv", [c["kernel"] for c in gv["cases"]], ["traffic"])
        if not a.no_cpu:
            out["cpu_baseline"] = cpu_baseline_gemv()
        line = json.dumps(out)
        print(line, flush=True)
        if a.json:
            with open(a.json, "w") as f:
                f.write(line + "\n")
        return 0
    if a.workload == "moderate":
        mod = bench_moderate(torch, gemm, a.steps, a.warmup)
        _, N, K, M, Gm = MODERATE_CASE
        out = {"metric": "prefill TFLOP/s & %MFMA peak at moderate batch (BASELINE configs[2])",
               "value": round(mod["TFLOPs"], 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
               "ms_per_step": round(mod["us"] * mod["copies"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
               "vs_baseline": None, "dtype": "fp16 (fp32 accumulate)", "data": "synthetic",
               "config": {"workload": f"BASELINE configs[2]: prefill M={M} K={K} N={N} G={Gm}; one step = one call "
                                      f"on each of {mod['copies']} weight copies"},
               "roofline": {"bound": "mfma", "achieved": round(mod["TFLOPs"], 1), "peak": FP16_MFMA_PEAK_TFS,
                            "unit": "TFLOP/s", "frac": round(mod["TFLOPs"] / FP16_MFMA_PEAK_TFS, 4),
                            "frac_hbm": round(mod["GBs"] / HBM_PEAK_GBS, 4), "kernel": mod["kernel"],
                            "flops_per_launch": alg_flops(M, N, K), "bytes_per_launch": alg_bytes(M, N, K, Gm)}}
        tag_counters(out["roofline"], "moderate", [mod["kernel"]], ["traffic"])
        out["roofline"].update({"mfma_busy_frac": None, "clock_ghz": None})
        line = json.dumps(out)
        print(line, flush=True)
        if a.json:
            with open(a.json, "w") as f:
                f.write(line + "\n")
        return 0
    if a.workload == "c1":
        c1 = bench_c1(torch, gemm, a.steps, a.warmup)
        name, N, K, M = C1_CASE
        out = {"metric": "decode GB/s & %HBM peak at BASELINE configs[0] (w4a16_gemm, M=1, K=N=4096, G=128)",
               "value": round(c1["GBs"], 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
               "ms_per_step": round(c1["us"] / 1e3, 6), "higher_is_better": True, "scaling": "weak",
               "vs_baseline": None, "dtype": "fp16 (fp32 accumulate)", "data": "synthetic",
               "config": {"workload": "BASELINE configs[0]: w4a16_gemm decode M=1 K=4096 N=4096 G=128; one step = "
                                      "one call", "weight_copies": c1["copies"],
                          "reference_published": "58.94 us median on an RTX 3050 Laptop GPU "
                                                 "(benchmarks/results/latest.json:368-384)"},
               "roofline": {"bound": "hbm", "achieved": round(c1["GBs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(c1["GBs"] / HBM_PEAK_GBS, 4), "kernel": c1["kernel"],
                            "bytes_per_launch": alg_bytes(M, N, K), "avg_launch_us": round(c1["us"], 3)}}
        tag_counters(out["roofline"], "c1", [c1["kernel"]], ["traffic"])
        if not a.no_cpu:
            out["cpu_baseline"] = cpu_baseline([C1_CASE])
        line = json.dumps(out)
        print(line, flush=True)
        if a.json:
            with open(a.json, "w") as f:
                f.write(line + "\n")
        return 0
    pre = None
    dec = bench_decode(torch, gemm, a.steps, a.warmup) if a.workload == "decode" else None
    if a.workload == "prefill" or not a.no_prefill:
        pre = bench_prefill(torch, gemm, a.prefill_steps if a.workload == "decode" else a.steps,
                            a.warmup if a.workload == "prefill" else a.prefill_warmup)
    # The side legs (configs[2], configs[0], the baseline GEMV) take SIDE_STEPS after SIDE_WARMUP
    # whatever --steps is (like the prefill leg's own counts): after the HBM-bound legs the time per
    # call of configs[2] falls over the first few hundred calls (30 timed steps after 3 warm-up
    # steps read 29.0 us, 20 after 5 26.5 us, 200 after 20 25.0 us; one box).  ~150 ms in all.
    mod = bench_moderate(torch, gemm, SIDE_STEPS, SIDE_WARMUP) if (dec is not None and not a.no_prefill) else None
    c1 = bench_c1(torch, gemm, SIDE_STEPS, SIDE_WARMUP) if (dec is not None and not a.no_c1) else None
    gv = bench_gemv(torch, SIDE_STEPS, SIDE_WARMUP) if (dec is not None and not a.no_prefill) else None
    eager = bench_eager(torch, gemm) if (dec is not None and not a.no_c1) else None

    out = {"metric": "decode GB/s & %HBM peak (M=1..16); prefill TFLOP/s & %MFMA peak (M=2048)"}
    if dec is not None:
        ach = dec["bytes_per_launch"] / (dec["avg_launch_us"] * 1e-6) / 1e9
        out.update({
            "value": round(dec["value"], 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
            "ms_per_step": round(dec["ms_per_step"], 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp16 (fp32 accumulate)", "data": "synthetic",
            "config": {"workload": "BASELINE configs[1]: decode, Llama-3-8B MLP gate/up K=4096 N=14336 and down "
                                   "K=14336 N=4096, M in {1,4,8,16}, G=128; one step = the 8 calls",
                       "G": G, "weight_copies_per_shape": dec["copies"], "timing": f"HIP graph replay ({dec['steps_per_graph']} steps per graph), HIP events"},
            "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4),
                         "kernel": " + ".join(sorted({c["kernel"] for c in dec["cases"]})),
                         "bytes_per_launch": dec["bytes_per_launch"],
                         "avg_launch_us": round(dec["avg_launch_us"], 3)},
            "cases": dec["cases"],
        })
        tag_counters(out["roofline"], "decode", [c["kernel"] for c in dec["cases"]], ["traffic"])
    if pre is not None:
        _, N, K, M = PREFILL_CASE
        pre_obj = {"value": round(pre["TFLOPs"], 1), "unit": "TFLOP/s", "us_per_call": round(pre["us"], 1),
                   "steps": pre["steps"], "warmup": pre["warmup"],
                   "config": {"workload": "BASELINE configs[3]: prefill M=2048 K=8192 N=28672 G=128"},
                   "roofline": {"bound": "mfma", "achieved": round(pre["TFLOPs"], 1), "peak": FP16_MFMA_PEAK_TFS,
                                "unit": "TFLOP/s", "frac": round(pre["TFLOPs"] / FP16_MFMA_PEAK_TFS, 4),
                                "kernel": pre["kernel"], "flops_per_launch": alg_flops(M, N, K)}}
        # rocprofv3 counters of the same kernel: HBM traffic, and the MFMA-busy fraction
        # SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x 1024 SIMDs) at the measured clock
        tag_counters(pre_obj["roofline"], "prefill", [pre["kernel"]], ["traffic", "mfma_busy_frac", "clock_ghz"])
        if dec is None:
            out.update({"value": pre_obj["value"], "unit": "TFLOP/s", "n_gpus": 1, "steps": a.steps,
                        "warmup": a.warmup, "ms_per_step": round(pre["us"] / 1e3, 5), "higher_is_better": True,
                        "scaling": "weak", "vs_baseline": None, "dtype": "fp16 (fp32 accumulate)",
                        "data": "synthetic", "config": pre_obj["config"], "roofline": pre_obj["roofline"]})
        else:
            out["prefill"] = pre_obj
    if mod is not None:
        _, N, K, M, Gm = MODERATE_CASE
        out["moderate"] = {
            "value": round(mod["TFLOPs"], 1), "unit": "TFLOP/s", "us_per_call": round(mod["us"], 2),
            "GB_per_s": round(mod["GBs"], 1),
            "config": {"workload": "BASELINE configs[2]: prefill M=128 K=4096 N=14336 G=64",
                       "weight_copies": mod["copies"]},
            "roofline": {"bound": "both (intensity ~419 flop/B, ridge ~315)", "kernel": mod["kernel"],
                         "frac_mfma": round(mod["TFLOPs"] / FP16_MFMA_PEAK_TFS, 4),
                         "frac_hbm": round(mod["GBs"] / HBM_PEAK_GBS, 4),
                         "flops_per_launch": alg_flops(M, N, K), "bytes_per_launch": alg_bytes(M, N, K, Gm)}}
        tag_counters(out["moderate"]["roofline"], "moderate", [mod["kernel"]], ["traffic"])
        # GRBM_GUI_ACTIVE over-counts for a ~30 us dispatch, so the busy fraction and clock derived
        # from it are not reported for this leg
        out["moderate"]["roofline"].update({"mfma_busy_frac": None, "clock_ghz": None})
    if c1 is not None:
        _, N, K, M = C1_CASE
        out["decode_c1"] = {
            "value": round(c1["GBs"], 1), "unit": "GB/s", "us_per_call": round(c1["us"], 3),
            "config": {"workload": "BASELINE configs[0]: w4a16_gemm decode M=1 K=4096 N=4096 G=128",
                       "weight_copies": c1["copies"],
                       "reference_published": "58.94 us median on an RTX 3050 Laptop GPU "
                                              "(benchmarks/results/latest.json:368-384)"},
            "roofline": {"bound": "hbm", "achieved": round(c1["GBs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(c1["GBs"] / HBM_PEAK_GBS, 4), "kernel": c1["kernel"],
                         "bytes_per_launch": alg_bytes(M, N, K)}}
        tag_counters(out["decode_c1"]["roofline"], "c1", [c1["kernel"]], ["traffic"])
    if eager is not None:
        out["eager"] = eager
    if gv is not None:
        out["baseline_gemv"] = {"value": round(gv["value"], 1), "unit": "GB/s",
                                "frac_hbm": round(gv["value"] / HBM_PEAK_GBS, 4),
                                "us_per_step": round(gv["us_per_step"], 2), "cases": gv["cases"],
                                "kernel": " + ".join(sorted({c["kernel"] for c in gv["cases"]}))}
    if not a.no_cpu:
        if dec is not None:
            out["cpu_baseline"] = cpu_baseline(DECODE_CASES)
            if gv is not None:
                out["baseline_gemv"]["cpu_baseline"] = cpu_baseline_gemv(5.0)
            if pre is not None:
                out["prefill"]["cpu_baseline"] = cpu_baseline_prefill()
        else:
            out["cpu_baseline"] = cpu_baseline_prefill()
    line = json.dumps(out)
    print(line, flush=True)
    if a.json:
        with open(a.json, "w") as f:
            f.write(line + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
