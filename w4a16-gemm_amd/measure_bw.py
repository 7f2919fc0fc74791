#!/usr/bin/env python3
"""Achievable HBM bandwidth on this GPU (the practical roofline next to the 8 TB/s spec).

Counterpart of the reference's benchmarks/measure_bw.py (same method: best of 30 timed runs of a
device copy and of a read-only pass, bandwidth = bytes moved / time), sized for MI355X: the
default buffer is 1 GiB, four times the 256 MB Infinity Cache (the reference's 256 MiB default
would be cache-resident here).  The copy is measured twice, with torch's copy_ (the reference's
method) and with a one-shot copy kernel; the read-only pass is a one-shot streaming-read kernel
(both in csrc/bw_probe.hip, built into libw4a16_bwprobe.so by build.py): torch's reductions on
this GPU run far below the memory rate, so they would measure the reduction kernel, not the
memory.  It also measures the per-launch rate at the size of one
decode call (30 MiB) the way bench.py times the op: a HIP graph of launches over buffer copies
whose working set exceeds the Infinity Cache, so every launch streams from HBM and pays its
launch cost.

    python w4a16-gemm_amd/measure_bw.py [--mb 1024] [--call-mb 30] [--json out.json]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def load_probe():
    path = os.path.join(HERE, "libw4a16_bwprobe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (python w4a16-gemm_amd/build.py)")
    lib = ctypes.CDLL(path)
    lib.w4a16_bw_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    lib.w4a16_bw_read.restype = ctypes.c_int
    lib.w4a16_bw_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.w4a16_bw_copy.restype = ctypes.c_int
    return lib


def best_ms(torch, fn, iters: int = 30) -> float:
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(iters):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        best = min(best, a.elapsed_time(b))
    return best


def per_launch_us(torch, fns, reps: int = 30):
    """Median and minimum microseconds per launch of a graph of `fns` (one launch each)."""
    for f in fns:
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    samples = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        samples.append(a.elapsed_time(b) * 1e3 / len(fns))
    return statistics.median(samples), min(samples)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--mb", type=int, default=1024, help="buffer size in MiB (must be >> the 256 MB Infinity Cache)")
    ap.add_argument("--call-mb", type=float, default=30, help="bytes read per launch for the per-launch rate (MiB)")
    ap.add_argument("--json", default=None, help="also write the results to this file")
    a = ap.parse_args(argv)
    import torch
    if not torch.cuda.is_available():
        print("measure_bw.py: no GPU available", file=sys.stderr)
        return 2
    probe = load_probe()
    n = a.mb * 2**20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_()
    dst = torch.empty_like(src)
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")

    def read(buf, nbytes):
        rc = probe.w4a16_bw_read(buf.data_ptr(), nbytes, sink.data_ptr(), torch.cuda.current_stream().cuda_stream)
        if rc:
            raise RuntimeError(f"w4a16_bw_read failed ({rc})")

    def copy(s, d, nbytes):
        rc = probe.w4a16_bw_copy(s.data_ptr(), d.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream)
        if rc:
            raise RuntimeError(f"w4a16_bw_copy failed ({rc})")

    out = {"gpu": torch.cuda.get_device_name(), "buffer_mib": a.mb}
    out["copy_torch_gbs"] = 2 * n / best_ms(torch, lambda: dst.copy_(src)) / 1e6
    out["copy_gbs"] = 2 * n / best_ms(torch, lambda: copy(src, dst, n)) / 1e6
    if not torch.equal(src, dst):
        raise RuntimeError("w4a16_bw_copy produced a wrong copy")
    out["read_gbs"] = n / best_ms(torch, lambda: read(src, n)) / 1e6
    del dst
    # Per-launch read rate at one call's size: distinct slices of the big buffer (>= 2x the MALL).
    m = int(a.call_mb * 2**20) // 16 * 16
    copies = max(2, min(n // m, math.ceil(2 * 256 * 2**20 / m)))
    views = [src[i * m:(i + 1) * m] for i in range(copies)]
    med, mn = per_launch_us(torch, [lambda v=v: read(v, m) for v in views])
    out.update({"call_mib": a.call_mb, "call_copies": copies, "call_median_us": med, "call_min_us": mn,
                "call_read_gbs": m / (med * 1e-6) / 1e9})
    print(out["gpu"])
    print(f"copy (read+write) : {out['copy_gbs']:8.1f} GB/s   ({a.mb} MiB buffers; torch copy_: "
          f"{out['copy_torch_gbs']:.1f} GB/s)")
    print(f"read (read only)  : {out['read_gbs']:8.1f} GB/s")
    print(f"per-launch read   : {out['call_read_gbs']:8.1f} GB/s   ({a.call_mb:g} MiB per launch, {copies} buffers "
          f"in a graph: median {med:.2f} us, min {mn:.2f} us per launch)")
    if a.json:
        with open(a.json, "w") as f:
            json.dump(out, f, indent=1)
            f.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
