"""GPU parity tests of the device quantiser ``w4a16_opt.quantize_pack`` (C ABI
``w4a16_quantize_pack``) against the oracle's quantize_w4 + pack_int4 (restatement of the
reference's tests/quant.py:62-74, 34-48).  Integer outputs: the packed words and the fp16
scale bits must be identical.

    python -u -m pytest tests/test_quantize_gpu.py -m gpu -x -v --timeout 120 --timeout-method thread
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import quant
from tests._helpers import assert_close, gemm, ref_gemm, torch_cuda

pytestmark = pytest.mark.gpu

SHAPES = [(16, 64), (16, 128), (32, 256), (48, 384), (272, 1152), (4096, 4096), (1024, 14336)]


def _oracle(Wh: np.ndarray, G: int):
    q, s = quant.quantize_w4(Wh.astype(np.float32), G)
    return quant.pack_int4(q), s


def _device(W, G):
    import w4a16_opt
    Wp, s = w4a16_opt.quantize_pack(W, G)
    return Wp.cpu().numpy(), s.cpu().numpy()


def _check(Wh: np.ndarray, G: int):
    torch = torch_cuda()
    Wp, s = _device(torch.from_numpy(Wh).cuda(), G)
    Wp_ref, s_ref = _oracle(Wh, G)
    assert s.shape == s_ref.shape and s.dtype == np.float16
    assert np.array_equal(s.view(np.uint16), s_ref.view(np.uint16)), \
        f"{int((s.view(np.uint16) != s_ref.view(np.uint16)).sum())} scales differ"
    bad = np.flatnonzero(Wp != Wp_ref)
    assert bad.size == 0, f"{bad.size} words differ, first at {bad[:4]}"


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
@pytest.mark.parametrize("G", [64, 128])
@pytest.mark.parametrize("N,K", SHAPES)
def test_quantize_pack_matches_oracle(N, K, G, dtype):
    if K % G:
        pytest.skip("K must be a multiple of the group size")
    print(f"quantize_pack N={N} K={K} G={G} {dtype}", flush=True)
    rng = np.random.default_rng([N, K, G])
    W = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    # per-row magnitudes spread over 2^-12 .. 2^6, so scales cover much of the fp16 range
    W *= np.exp2(rng.integers(-12, 7, (N, 1))).astype(np.float32)
    _check(W.astype(np.float16) if dtype == "fp16" else W, G)


@pytest.mark.parametrize("G", [64, 128])
def test_quantize_pack_ties_zero_groups_and_exact_codes(G):
    """Half-to-even ties, all-zero groups (scale clamped to fp16(1e-4), codes 8), negative
    absmax, and exactly representable (q - 8) * s inputs that must come back unchanged."""
    N, K = 32, 256
    rng = np.random.default_rng(G)
    q = rng.integers(1, 16, (N, K), dtype=np.uint8)
    q[:, ::G] = 15
    q[1::2, G::G] = 1                                       # absmax from a negative value too
    s = (rng.integers(64, 256, (K // G, N)) * 2.0 ** rng.integers(-16, -8, (K // G, N))).astype(np.float16)
    W = quant.dequantize_w4(q, s, G).astype(np.float32)
    W[3, :] = 0.0                                           # all-zero groups
    W[5, :G] = 0.0
    W[5, 0] = 7.0                                           # s = 1: ties at x.5
    W[5, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -6.5]
    _check(W, G)
    _check(W.astype(np.float16), G)
    torch = torch_cuda()
    Wp, s_dev = _device(torch.from_numpy(W).cuda(), G)
    qd = quant.unpack_int4(Wp, N, K)
    assert qd[5, 1:9].tolist() == [8, 10, 10, 8, 6, 6, 12, 2]
    assert np.all(qd[3] == 8) and float(s_dev[0, 3]) == float(np.float16(1e-4))
    rows = [r for r in range(N) if r not in (3, 5)]
    assert np.array_equal(qd[rows], q[rows])
    assert np.array_equal(s_dev[:, rows].view(np.uint16), s[:, rows].view(np.uint16))


@pytest.mark.parametrize("G", [64, 128])
def test_quantize_pack_fp32_near_ties(G):
    """fp32 inputs 0..3 ulps either side of (n + 1/2) * s for an fp16-exact s: exact ties go to
    even, and values a few ulps off a tie must round as the correctly rounded quotient does."""
    rng = np.random.default_rng(G + 1)
    s = np.float32(np.float16(0.0123))
    base = ((rng.integers(-7, 7, (64, 512)) + 0.5) * s).astype(np.float32)
    W = base.copy()
    for d in range(-3, 4):
        x = base[:, d + 3::7]
        for _ in range(abs(d)):
            x = np.nextafter(x, np.float32(np.inf) if d > 0 else np.float32(-np.inf)).astype(np.float32)
        W[:, d + 3::7] = x
    W[:, ::G] = np.float32(7) * s
    _check(W, G)


def test_quantize_pack_overflowing_scale():
    """fp32 groups whose absmax/7 exceeds fp16's range: the scale is +inf and every code is 8,
    as with the reference's torch arithmetic (half() overflows to inf, W / inf = 0)."""
    W = np.zeros((16, 128), np.float32)
    W[0, :64] = 1e6
    W[1, 64:] = -5e5
    W[2, :] = np.linspace(-3, 3, 128, dtype=np.float32)
    with np.errstate(over="ignore"):
        _check(W, 64)


def test_quantize_pack_feeds_the_gemm():
    """Device-quantised weights drive w4a16_gemm exactly as the oracle-quantised ones do."""
    torch = torch_cuda()
    N, K, G, M = 4096, 4096, 128, 4
    rng = np.random.default_rng(11)
    Wh = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    Wp, s = __import__("w4a16_opt").quantize_pack(torch.from_numpy(Wh).cuda(), G)
    x = torch.from_numpy(rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)).cuda()
    y = gemm(Wp, x, s)
    q, s_ref = quant.quantize_w4(Wh.astype(np.float32), G)
    assert_close(y, ref_gemm(x, q, s_ref, G))
    y2 = gemm(torch.from_numpy(quant.pack_int4(q)).cuda(), x, torch.from_numpy(s_ref).cuda())
    assert torch.equal(y, y2)


def test_quantize_pack_full_size():
    """BASELINE prefill weight (N=28672, K=8192, G=128, fp16), checked whole against the oracle
    in blocks of 1024 rows (a block of n16 blocks owns a contiguous range of Wp)."""
    torch = torch_cuda()
    import w4a16_opt
    N, K, G, R = 28672, 8192, 128, 1024
    g = torch.Generator(device="cuda").manual_seed(5)
    W = (torch.randn(N, K, device="cuda", generator=g) * 0.02).half()
    Wp, s = w4a16_opt.quantize_pack(W, G)
    Wp, s = Wp.cpu().numpy(), s.cpu().numpy()
    for r0 in range(0, N, R):
        words, st = _oracle(W[r0:r0 + R].cpu().numpy(), G)
        assert np.array_equal(Wp[r0 * K // 8:(r0 + R) * K // 8], words), r0
        assert np.array_equal(s[:, r0:r0 + R].view(np.uint16), st.view(np.uint16)), r0


def test_quantize_pack_rejects_bad_shapes():
    torch = torch_cuda()
    import w4a16_opt
    with pytest.raises(RuntimeError, match="multiple of 16"):
        w4a16_opt.quantize_pack(torch.zeros(24, 128, device="cuda", dtype=torch.float16), 64)
    with pytest.raises(RuntimeError, match="group size"):
        w4a16_opt.quantize_pack(torch.zeros(16, 96, device="cuda", dtype=torch.float16), 64)
    with pytest.raises(RuntimeError, match="unsupported group size"):
        w4a16_opt.quantize_pack(torch.zeros(16, 256, device="cuda", dtype=torch.float16), 32)
    with pytest.raises(RuntimeError, match="fp16 or fp32"):
        w4a16_opt.quantize_pack(torch.zeros(16, 128, device="cuda", dtype=torch.bfloat16), 64)
    Wp, s = w4a16_opt.quantize_pack(torch.zeros(0, 128, device="cuda", dtype=torch.float16), 64)
    assert Wp.numel() == 0 and tuple(s.shape) == (2, 0)
