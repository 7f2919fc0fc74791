"""w4a16-gemm_amd/ab_libs.py, the alternating A/B timer of library builds and forced plans:
argument parsing on the CPU, one small alternating run through the in-tree library on the GPU."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "w4a16-gemm_amd"))
import ab_libs  # noqa: E402

LIB = os.path.join(ROOT, "w4a16-gemm_amd", "libw4a16_hip.so")


def test_case_sets_are_the_baseline_configs():
    assert ab_libs.parse_cases("decode") == [(1, 14336, 4096, 128), (4, 14336, 4096, 128), (8, 14336, 4096, 128),
                                             (16, 14336, 4096, 128), (1, 4096, 14336, 128), (4, 4096, 14336, 128),
                                             (8, 4096, 14336, 128), (16, 4096, 14336, 128)]
    assert ab_libs.parse_cases("c1;moderate;prefill") == [(1, 4096, 4096, 128), (128, 14336, 4096, 64),
                                                        (2048, 28672, 8192, 128)]
    assert ab_libs.parse_cases("8,6144,4096,128;c1") == [(8, 6144, 4096, 128), (1, 4096, 4096, 128)]


def test_spec_environment():
    assert ab_libs.parse_spec("a/lib.so") == ("a/lib.so", {})
    assert ab_libs.parse_spec("lib.so@W4A16_DECODE=18,1") == ("lib.so", {"W4A16_DECODE": "18,1"})
    assert ab_libs.parse_spec("lib.so@A=1+B=x,y") == ("lib.so", {"A": "1", "B": "x,y"})


def test_with_env_restores_the_environment(monkeypatch):
    monkeypatch.setenv("W4A16_TEST_KEEP", "1")
    monkeypatch.delenv("W4A16_TEST_NEW", raising=False)
    with ab_libs.with_env({"W4A16_TEST_KEEP": "2", "W4A16_TEST_NEW": "3"}):
        assert os.environ["W4A16_TEST_KEEP"] == "2" and os.environ["W4A16_TEST_NEW"] == "3"
    assert os.environ["W4A16_TEST_KEEP"] == "1" and "W4A16_TEST_NEW" not in os.environ


@pytest.mark.gpu
def test_alternating_run_on_gpu(capsys):
    """The in-tree library against itself with a decode shape forced: two small cases, outputs
    equal between the auto plans and different only within tolerance for the forced shape."""
    from tests._helpers import torch_cuda
    torch_cuda()
    rc = ab_libs.main([LIB, f"{LIB}@W4A16_DECODE=19,1", LIB, "--cases", "4,256,4096,64;40,512,1024,128",
                       "--reps", "2", "--replays", "1", "--warm-ms", "1"])
    assert rc == 0
    out = capsys.readouterr().out
    lines = [l for l in out.splitlines() if l.startswith("M=")]
    assert len(lines) == 2, out
    assert "mean per spec" in out
    # M = 4 (decode): the forced ring shape (19) runs; it sums K in another order than the auto
    # plan, so its output may differ, within tolerance; the two auto runs are equal
    assert "(0, 19, 1, " in lines[0] and "(0, 0, 1, " in lines[0], lines[0]
    if "maxrel=" in lines[0]:
        rels = [float(v) for v in lines[0].split("maxrel=")[1].split()[0].split(",")]
        assert max(rels) < 2e-3 and rels[1] == 0.0, lines[0]
    # M = 40 (prefill): the decode override does not apply, every spec gives the same bits
    assert "outputs=equal" in lines[1], lines[1]
