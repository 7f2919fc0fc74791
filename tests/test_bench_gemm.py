"""The shape-sweep harness w4a16-gemm_amd/bench_gemm.py: reference schema and options on the CPU,
one small sweep on the GPU."""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest

from oracle import quant

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "w4a16-gemm_amd"))
import bench_gemm  # noqa: E402

# Row and document keys of the reference's result JSON (benchmarks/bench_gemm.py:302-307, 317-340).
REF_ROW_KEYS = {"mode", "layer", "N", "K", "M", "G"}
REF_PARAM_KEYS = {"group_size", "target_weight_mib", "repetitions", "shapes", "phase_M", "backends", "timing"}


def _args(argv):
    import argparse
    ns = argparse.Namespace(shape=None, phase="both", prefill_M="128,512,1024,2048,4096,8192",
                            decode_M="1,2,4,8,16,32", M=None, G=128, target_mb=1024, reps=30)
    for k, v in argv.items():
        setattr(ns, k, v)
    return ns


def test_defaults_mirror_the_reference_sweep():
    shapes, phase_m = bench_gemm.sweep_cases(_args({}))
    assert [n for n, _ in shapes] == ["qkv", "o", "gate_up", "down"]
    assert dict(shapes)["gate_up"] == (28672, 4096)
    assert phase_m == {"prefill": [128, 512, 1024, 2048, 4096, 8192], "decode": [1, 2, 4, 8, 16, 32]}
    assert bench_gemm.sweep_cases(_args({"phase": "decode", "M": "3,3,5"}))[1] == {"decode": [3, 5]}
    assert bench_gemm.sweep_cases(_args({"shape": ["256,1024"]}))[0] == [("256x1024", (256, 1024))]
    with pytest.raises(ValueError):
        bench_gemm.sweep_cases(_args({"M": "0"}))


def test_row_and_document_schema():
    row = bench_gemm.make_row("decode", "o", 4096, 4096, 1, 128, {"hip": (10.0, 9.0), "hipblaslt": (20.0, 19.0)})
    assert REF_ROW_KEYS <= set(row)
    for key in ("hip", "hipblaslt"):
        assert {f"{key}_us", f"{key}_min_us", f"{key}_tflops"} <= set(row)
    assert row["hip_tflops"] == pytest.approx(2 * 4096 * 4096 / 10e6)
    bytes_ = 4096 * 4096 // 2 + 32 * 4096 * 2 + 4096 * 2 + 4096 * 2
    assert row["hip_gbps"] == pytest.approx(bytes_ / 10e-6 / 1e9)
    doc = bench_gemm.make_result([row], [("o", (4096, 4096))], {"decode": [1]}, _args({}), "gpu", "t", "h", None)
    assert REF_PARAM_KEYS <= set(doc["parameters"])
    assert doc["parameters"]["backends"] == ["HIP W4A16", "hipBLASLt fp16"]
    json.dumps(doc)
    assert "hip us" in bench_gemm.format_table([row], markdown=True)


@pytest.mark.parametrize("N,K,G", [(32, 128, 64), (48, 256, 128)])
def test_dense_comparator_weights_are_the_reference_dequantisation(N, K, G):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(N)
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = rng.uniform(0.002, 0.02, (K // G, N)).astype(np.float16)
    d = bench_gemm.dequantize_device(torch, torch.from_numpy(quant.pack_int4(q)), torch.from_numpy(s), N, K, G)
    assert np.array_equal(d.numpy().view(np.uint16), quant.dequantize_w4(q, s, G).view(np.uint16))


@pytest.mark.gpu
def test_small_sweep_on_gpu(tmp_path):
    from tests._helpers import torch_cuda
    torch = torch_cuda()
    out = tmp_path / "sweep.json"
    assert bench_gemm.main(["--shape", "256,1024", "--M", "1,40", "--reps", "3", "--target-mb", "4",
                            "--json", str(out)]) == 0
    doc = json.loads(out.read_text())
    assert len(doc["rows"]) == 4 and REF_PARAM_KEYS <= set(doc["parameters"])
    for row in doc["rows"]:
        assert row["hip_us"] > 0 and row["hipblaslt_us"] > 0 and row["hip_min_us"] <= row["hip_us"]
    # the comparator multiplies the same weights
    hip, dense = bench_gemm.load_weights(torch, 256, 1024, 128, 1, seed=0)
    import w4a16_opt
    x = torch.randn(40, 1024, device="cuda", dtype=torch.float16)
    y = w4a16_opt.w4a16_gemm(hip[0][0], x, hip[0][1]).float()
    ref = x.float() @ dense[0].float().t()
    assert (y - ref).abs().max().item() / ref.abs().max().item() < 2e-3
