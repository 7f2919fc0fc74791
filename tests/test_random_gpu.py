"""Seeded random-shape sweeps on the GPU, beside the fixed parametrisations of the other files.

* w4a16_gemm: random (M, N, K, G) within the shape contract (N % 16 == 0, K % 64 == 0,
  K % G == 0), auto routing; a second sampler puts half of its small-M shapes on the decode
  route and every sixth shape at a long K.  Each result is checked against the oracle within the reference
  tolerance (max |y - ref| / max |ref| < 2e-3, tests/test_w4a16.py:41-44); shapes that route to
  prefill must also be bitwise equal to forced variant 4, since every prefill config accumulates
  the same k-slot groups in the same order.
* w4a16_gemv: random (N, K) with K % 8 == 0, random misalignment of W and A; bit-exact against
  the oracle's exact mode.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests._helpers import assert_close, gemm, make_problem, ref_gemm, torch_cuda


def _gemm_shapes(n=24, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        G = int(rng.choice([64, 128]))
        M = int(rng.choice([int(rng.integers(1, 17)), int(rng.integers(17, 640))]))
        N = 16 * int(rng.integers(1, 320))
        K = G * int(rng.integers(1, 6400 // G + 1))
        if K % 64 == 0:
            out.append((M, N, K, G))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,G", _gemm_shapes())
def test_random_shapes_vs_oracle(M, N, K, G):
    print(f"random gemm M={M} N={N} K={K} G={G}", flush=True)
    x, q, scales, Wp, key = make_problem(M, N, K, G, seed=M + N + K)
    y = gemm(Wp, x, scales)
    assert_close(y, ref_gemm(x, q, scales, G, key))
    decode = M <= 16 and N % 64 == 0 and K % 512 == 0
    if not decode:
        torch = torch_cuda()
        assert torch.equal(y, gemm(Wp, x, scales, variant=4)), "prefill configs must be bit-identical"



def _gemm_shapes_decode_and_long_k(n=32, seed=20261203):
    """A second sampler: M log-uniform in 1..700; half of the M <= 16 shapes rounded onto the
    decode route's grid (N % 64 == 0, K % 512 == 0, kernel.cu:242-249), which the sampler above
    rarely meets; every sixth shape a long K (8256..16384: the canonical segmented order)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        G = int(rng.choice([64, 128]))
        M = int(np.exp(rng.uniform(0.0, np.log(700.0))))
        if i % 6 == 5:
            K = G * int(rng.integers(8256 // G + 1, 16384 // G + 1))
            N = 16 * int(rng.integers(1, 65))
        else:
            K = G * int(rng.integers(1, 41))
            N = 16 * int(rng.integers(1, 201))
        if M <= 16 and i % 2 == 0:
            N, K = -(-N // 64) * 64, max(1, K // 512) * 512
        out.append((M, N, K, G))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,G", _gemm_shapes_decode_and_long_k())
def test_random_decode_and_long_k_shapes_vs_oracle(M, N, K, G):
    torch = torch_cuda()
    import w4a16_opt
    info = w4a16_opt.plan_info(M, N, K, G)
    print(f"random gemm M={M} N={N} K={K} G={G}: {info['kernel_name']} splits {info['splits']}", flush=True)
    x, q, scales, Wp, key = make_problem(M, N, K, G, seed=M)
    y = gemm(Wp, x, scales)
    assert_close(y, ref_gemm(x, q, scales, G, key))
    if not (M <= 16 and N % 64 == 0 and K % 512 == 0):
        assert torch.equal(y, gemm(Wp, x, scales, variant=4)), "prefill configs must be bit-identical"

def _gemv_shapes(n=24, seed=77):
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 2500)), 8 * int(rng.integers(1, 2600)), int(rng.integers(0, 4)),
             int(rng.integers(0, 8))) for _ in range(n)]


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,w_off,a_off", _gemv_shapes())
def test_random_gemv_vs_oracle(N, K, w_off, a_off):
    print(f"random gemv N={N} K={K} w_off={w_off} a_off={a_off}", flush=True)
    from oracle import c_oracle
    from tests.test_gemv import _run, bits, make_gemv
    W, A, sW, zW = make_gemv(N, K, 5, special=True)
    C = _run(W, A, sW, zW, w_offset=w_off, a_offset=a_off).cpu().numpy()
    assert np.array_equal(bits(C), bits(c_oracle.gemv(W, A, sW, zW, exact=True)))
