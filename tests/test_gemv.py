"""Baseline W4A16 GEMV (reference src/baseline/: w4a16_ext.w4a16_gemv, kernel.cu:8-72).

The reference ships no test or golden data for this extension, so the oracle
(oracle/w4a16_oracle.c: w4a16_oracle_gemv) is pinned here on the CPU by:
  * an integer brute force of the exact sum (Python ints, explicit round-to-nearest-even), which
    fixes the exact mode bit for bit;
  * the reference's own loop order (kernel.cu:22-30) restated with numpy float32 scalars, which
    fixes the sequential mode bit for bit;
  * closed forms: one-hot A against every nibble value at every nibble position (sign extension
    kernel.cu:26-27 and nibble order kernel.cu:25-28), zero A gives fp16(-z * s);
  * the fp32 rounding-error bound between the two modes (they differ only by summation order);
  * IEEE classes of non-finite inputs, which both modes must agree on.
The kernel's index math (digit table, operand bytes, load addresses) is emulated with numpy.
GPU tests (marked gpu) compare the HIP kernel with the exact mode bit for bit, and with the
reference order within the op's tolerance (max |C - ref| / max |ref| < 2e-3, the bound of the
reference suite's assert_close, tests/test_w4a16.py:41-44).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from oracle import c_oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "w4a16-gemm_amd", "libw4a16_hip.so")


# ----------------------------------------------------------------------------- problem makers

def make_gemv(N, K, seed=0, a_scale=1.0, special=False):
    rng = np.random.default_rng([seed, N, K])
    W = rng.integers(-2**31, 2**31, (N, K // 8), dtype=np.int64).astype(np.int32)
    A = (rng.standard_normal(K) * a_scale).astype(np.float16)
    if special and K >= 16:
        # subnormals, the largest finite values and signed zeros at random positions
        idx = rng.choice(K, size=min(K, 12), replace=False)
        A[idx] = np.array([6e-8, -6e-8, 3e-5, -1e-7, 65504, -65504, 0.0, -0.0, 2.0**-14, 1e4, -3e4, 5e-6],
                          dtype=np.float16)[:len(idx)]
    sW = rng.uniform(0.002, 0.02, N).astype(np.float16)
    zW = rng.standard_normal(N).astype(np.float16)
    return W, A, sW, zW


def signed_nibbles(W, K):
    """wv[n, k]: nibble k % 8 of word k // 8 of row n as a signed 4-bit value."""
    u = W.view(np.uint32)
    nib = np.stack([(u >> (4 * j)) & 15 for j in range(8)], axis=-1).reshape(W.shape[0], K).astype(np.int64)
    return np.where(nib >= 8, nib - 16, nib)


def round_int_to_f32(v: int) -> np.float32:
    """Nearest-even fp32 of an integer (exact integer arithmetic, no double rounding)."""
    a, neg = abs(v), v < 0
    if a.bit_length() > 24:
        shift = a.bit_length() - 24
        q, rem = divmod(a, 1 << shift)
        half = 1 << (shift - 1)
        if rem > half or (rem == half and q & 1):
            q += 1
        a = q << shift
    f = np.float32(float(a))
    return -f if neg else f


def brute_force_exact(W, A, sW, zW):
    K = A.shape[0]
    wv = signed_nibbles(W, K)
    X = [int(float(a) * 2**24) for a in A.astype(np.float64)]     # exact: fp16 values are k * 2^-24
    out = np.empty(W.shape[0], dtype=np.float16)
    for n in range(W.shape[0]):
        total = sum(int(w) * x for w, x in zip(wv[n], X))
        acc = round_int_to_f32(total) * np.float32(2.0**-24)
        out[n] = np.float16(np.float32(np.float32(acc - np.float32(zW[n])) * np.float32(sW[n])))
    return out


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


# ----------------------------------------------------------------------------- oracle pins (CPU)

@pytest.mark.parametrize("N,K,seed,special", [(5, 8, 0, False), (7, 64, 1, True), (3, 200, 2, True),
                                              (4, 512, 3, False)])
def test_oracle_exact_mode_matches_integer_brute_force(N, K, seed, special):
    W, A, sW, zW = make_gemv(N, K, seed, special=special)
    assert np.array_equal(bits(c_oracle.gemv(W, A, sW, zW, exact=True)), bits(brute_force_exact(W, A, sW, zW)))


def test_oracle_exact_rounding_of_wide_sums():
    # K = 4096 with large A: the int64 sums need ~45 bits, so the single rounding to fp32 matters
    W, A, sW, zW = make_gemv(6, 4096, 7, a_scale=3000.0, special=True)
    assert np.array_equal(bits(c_oracle.gemv(W, A, sW, zW, exact=True)), bits(brute_force_exact(W, A, sW, zW)))


@pytest.mark.parametrize("N,K,seed", [(4, 64, 0), (3, 256, 5)])
def test_oracle_sequential_mode_is_the_reference_loop(N, K, seed):
    W, A, sW, zW = make_gemv(N, K, seed, special=True)
    wv = signed_nibbles(W, K)
    ref = np.empty(N, dtype=np.float16)
    for n in range(N):
        acc = np.float32(0.0)
        for k in range(K):                                   # kernel.cu:22-30, k order
            acc = np.float32(acc + np.float32(wv[n, k]) * np.float32(A[k]))
        ref[n] = np.float16(np.float32(np.float32(acc - np.float32(zW[n])) * np.float32(sW[n])))
    assert np.array_equal(bits(c_oracle.gemv(W, A, sW, zW, exact=False)), bits(ref))


@pytest.mark.parametrize("exact", [True, False])
def test_oracle_one_hot_every_nibble_value_and_position(exact):
    # row n = 16 * j + v holds nibble value v at nibble position j of word 1 (k = 8 + j)
    K, N = 32, 128
    W = np.zeros((N, K // 8), dtype=np.uint32)
    for j in range(8):
        for v in range(16):
            W[16 * j + v, 1] = np.uint32(v << (4 * j))
    W = W.view(np.int32)
    rng = np.random.default_rng(3)
    sW = rng.uniform(0.5, 2.0, N).astype(np.float16)
    zW = rng.standard_normal(N).astype(np.float16)
    for j in range(8):
        A = np.zeros(K, dtype=np.float16)
        A[8 + j] = np.float16(1.375)
        got = c_oracle.gemv(W, A, sW, zW, exact=exact)
        for v in range(16):
            n = 16 * j + v
            wv = v - 16 if v >= 8 else v
            want = np.float16(np.float32(np.float32(np.float32(wv) * np.float32(1.375) - np.float32(zW[n]))
                                         * np.float32(sW[n])))
            assert bits(got[n:n + 1])[0] == bits(np.array([want]))[0], (j, v)
        # rows whose nibble sits at another position see zero
        other = [16 * jj + v for jj in range(8) if jj != j for v in range(16)]
        want0 = (np.float32(-zW[other].astype(np.float32)) * sW[other].astype(np.float32)).astype(np.float16)
        assert np.array_equal(bits(got[other]), bits(want0)), j


def test_oracle_modes_differ_only_by_fp32_rounding():
    N, K = 96, 4096
    W, A, sW, zW = make_gemv(N, K, 11, special=True)
    ce = c_oracle.gemv(W, A, sW, zW, exact=True).astype(np.float64)
    cs = c_oracle.gemv(W, A, sW, zW, exact=False).astype(np.float64)
    wv = signed_nibbles(W, K).astype(np.float64)
    mass = np.abs(wv) @ np.abs(A.astype(np.float64))              # sum_k |wv * a|
    # sequential fp32 summation error <= (K-1) u mass (u = 2^-24), scaled by s, plus one fp16
    # rounding of each result (2^-11 relative, or half the smallest subnormal)
    bound = np.abs(sW.astype(np.float64)) * (K * 2.0**-24 * mass) + 2.0**-10 * np.maximum(np.abs(ce), np.abs(cs)) \
        + 2.0**-24
    assert (np.abs(ce - cs) <= bound).all()
    assert np.abs(ce - cs).max() / np.abs(ce).max() < 2e-3
    assert (ce == cs).mean() > 0.5


def test_oracle_zero_input_and_empty_k():
    W, A, sW, zW = make_gemv(32, 64, 4)
    want = (np.float32(0.0) - zW.astype(np.float32)) * sW.astype(np.float32)
    for exact in (True, False):
        got = c_oracle.gemv(W, np.zeros(64, np.float16), sW, zW, exact=exact)
        assert np.array_equal(bits(got), bits(want.astype(np.float16)))
        got0 = c_oracle.gemv(W[:, :0], np.zeros(0, np.float16), sW, zW, exact=exact)
        assert np.array_equal(bits(got0), bits(want.astype(np.float16)))


def test_oracle_nonfinite_classes_agree_with_reference_order():
    rng = np.random.default_rng(9)
    N, K = 200, 64
    for trial in range(20):
        W, A, sW, zW = make_gemv(N, K, 100 + trial)
        W[rng.random((N, K // 8)) < 0.3] = 0                     # zero weights meet the infinities
        idx = rng.choice(K, size=int(rng.integers(1, 4)), replace=False)
        A[idx] = rng.choice(np.array([np.inf, -np.inf, np.nan], dtype=np.float16), size=len(idx))
        ce = c_oracle.gemv(W, A, sW, zW, exact=True)
        cs = c_oracle.gemv(W, A, sW, zW, exact=False)
        assert np.array_equal(np.isnan(ce), np.isnan(cs)), trial
        fin = ~np.isnan(ce)
        assert np.array_equal(bits(ce[fin]), bits(cs[fin])), trial


# ----------------------------------------------------------------------------- kernel emulation (CPU)

SEG, SUPER, WAVES, DIGITS = 4096, 128, 8, 6
THREADS, PER_WAVE = 64 * WAVES, SEG // SUPER // WAVES
BIAS = 0x808080808080


def biased_fixed(h):
    """Vectorised biased_fixed() of the kernel: a * 2^24 + BIAS (X = 0 for inf / NaN)."""
    h = h.astype(np.int64)
    e, m = (h >> 10) & 31, h & 1023
    mag = np.where(e == 0, m, (1024 | m) << np.maximum(e - 1, 0))
    v = np.where(h & 0x8000, BIAS - mag, BIAS + mag)
    return np.where(e == 31, BIAS, v)


def test_digit_decomposition_of_every_fp16():
    h = np.arange(65536, dtype=np.uint16)
    finite = ((h >> 10) & 31) != 31
    v = biased_fixed(h)
    digits = np.stack([((v >> (8 * j)) & 0xFF) - 128 for j in range(DIGITS)])
    assert digits.min() >= -128 and digits.max() <= 127
    X = sum(digits[j] * (256 ** j) for j in range(DIGITS))
    a = h.view(np.float16).astype(np.float64)
    assert np.array_equal(X[finite], (a[finite] * 2.0**24).astype(np.int64))
    assert (X[~finite] == 0).all()


def test_signed_nibble_bytes():
    w = np.arange(16, dtype=np.uint32)
    words = (w[:, None] << (4 * np.arange(8, dtype=np.uint32))).astype(np.uint32)   # nibble v at position j
    for shift in (0, 4):
        u = ((words ^ np.uint32(0x88888888)) >> np.uint32(shift)) & np.uint32(0x0F0F0F0F)
        s = (u + np.uint32(0x78787878)) ^ np.uint32(0x80808080)
        sb = s.view(np.uint8).reshape(16, 8, 4).view(np.int8)
        for j in range(8):
            if (j & 1) * 4 != shift:
                continue
            for v in range(16):
                want = np.zeros(4, np.int8)
                want[j // 2] = v - 16 if v >= 8 else v
                assert np.array_equal(sb[v, j], want), (shift, j, v)


def emulate_gemv_kernel(W, A, N, K, wvec, rt=1):
    """Digit sums P[n, j] of one launch, following gemv_kernel's indexing exactly: the A loads of
    the table build, each lane's weight-load word indices (checked in bounds), the digit table,
    the operand bytes and a 16x16x64 MFMA (A and B use the same k position for the same lane
    group and byte, so any consistent hardware k order gives the same integer sums)."""
    kw = K // 8
    Wu = W.view(np.uint32)
    h_all = A.view(np.uint16)
    P = np.zeros((N, DIGITS), dtype=object)
    for row0 in range(0, N, 16 * rt):
        rows = [min(row0 + 16 * t + r, N - 1) for t in range(rt) for r in range(16)]
        acc = np.zeros((WAVES, 16 * rt, 16), dtype=np.int64)   # per wave: [row, column]
        for seg in range(0, K, SEG):
            seglen = min(SEG, K - seg)
            nsc = (seglen + SUPER - 1) // SUPER
            per = (nsc + WAVES - 1) // WAVES
            table = np.full(SEG // SUPER * 768, 0xEE, dtype=np.uint8)   # poison: unwritten bytes
            for tid in range(THREADS):
                for u in (tid,):
                    k0 = seg + 8 * u
                    src = k0 if k0 < K else 0
                    assert 0 <= src and (K == 0 or src + 8 <= K)
                    if u >= nsc * 16:
                        continue
                    inside = k0 < K
                    v = biased_fixed(h_all[src:src + 8]) if inside else np.full(8, BIAS, np.int64)
                    p, rr = u >> 4, (u & 15) * 8
                    gg, m, hh = rr >> 5, (rr >> 4) & 1, (rr >> 3) & 1
                    base = p * 768 + ((m * 4 + gg) * DIGITS) * 16 + 8 * hh
                    for j in range(DIGITS):
                        for par in range(2):
                            for i in range(4):
                                byte = ((int(v[par + 2 * i]) >> (8 * j)) & 0xFF) ^ 0x80
                                table[base + 16 * j + 4 * par + i] = byte
            for wave in range(WAVES):
                for i in range(PER_WAVE):
                    p = wave * per + i
                    p_load = wave * per + min(i, per - 1)          # loads past the share repeat
                    lanes_words = {}
                    for g in range(4):
                        for r in range(16 * rt):                   # row tile r // 16, lane row r % 16
                            wi = ((seg + p_load * SUPER) >> 3) + 4 * g
                            if wvec:
                                idx = [wi + e for e in range(4)] if wi + 4 <= kw else [e for e in range(4)]
                            else:
                                idx = [wi + e if wi + e < kw else 0 for e in range(4)]
                            assert all(0 <= x < kw for x in idx), (seg, p, g, idx)
                            lanes_words[(r, g)] = [int(Wu[rows[r], x]) for x in idx]
                    if i >= per or p >= nsc:
                        break
                    for m in range(2):
                        Abytes = np.zeros((16 * rt, 4, 16), dtype=np.int64)  # [row r, group g, byte]
                        Bbytes = np.zeros((16, 4, 16), dtype=np.int64)       # [column r, group g, byte]
                        for g in range(4):
                            for r in range(16 * rt):
                                w = lanes_words[(r, g)]
                                w0, w1 = (w[2], w[3]) if m else (w[0], w[1])
                                dws = []
                                for ww in (w0, w1):
                                    for shift in (0, 4):
                                        uu = ((ww ^ 0x88888888) >> shift) & 0x0F0F0F0F
                                        dws.append(((uu + 0x78787878) ^ 0x80808080) & 0xFFFFFFFF)
                                Abytes[r, g] = np.array(dws, dtype=np.uint32).view(np.int8)
                                if r < DIGITS and r < 16:
                                    off = p * 768 + ((m * 4 + g) * DIGITS + r) * 16
                                    tb = table[off:off + 16]
                                    assert not (tb == 0xEE).all(), "read of an unwritten table entry"
                                    Bbytes[r, g] = tb.view(np.int8)
                        acc[wave] += np.einsum("rgb,cgb->rc", Abytes, Bbytes)
        for r in range(16 * rt):
            if row0 + r < N:
                for j in range(DIGITS):
                    P[row0 + r, j] = int(acc[:, r, j].sum())
    return P


@pytest.mark.parametrize("N,K,wvec,rt", [(16, 512, True, 1), (13, 4096 + 384, True, 1), (5, 1032, False, 1),
                                         (3, 8, False, 1), (17, 160, True, 1), (40, 640, True, 2),
                                         (29, 1032, False, 2), (32, 4096 + 128, True, 2)])
def test_gemv_kernel_index_math_emulated(N, K, wvec, rt):
    W, A, _, _ = make_gemv(N, K, 21, special=True)
    P = emulate_gemv_kernel(W, A, N, K, wvec, rt)
    wv = signed_nibbles(W, K)
    X = [int(float(a) * 2**24) for a in A.astype(np.float64)]
    for n in range(N):
        total = sum(P[n, j] * 256 ** j for j in range(DIGITS))
        assert total == sum(int(w) * x for w, x in zip(wv[n], X)), n
        assert all(abs(P[n, j]) < 2**31 for j in range(DIGITS))


# ----------------------------------------------------------------------------- C ABI and binding (CPU)

@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.skip("libw4a16_hip.so not built")
    L = ctypes.CDLL(LIB)
    L.w4a16_gemv.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
    L.w4a16_gemv.restype = ctypes.c_int
    L.w4a16_last_error.restype = ctypes.c_char_p
    return L


@pytest.mark.parametrize("N,K,ptrs,msg", [
    (16, 12, (16, 16, 16, 16, 16), "K must be a multiple of 8"),
    (16, (1 << 20) + 8, (16, 16, 16, 16, 16), "K must be at most 1048576"),
    (-1, 64, (16, 16, 16, 16, 16), "dimensions out of range"),
    (16, 64, (0, 16, 16, 16, 16), "null pointer"),
    (16, 64, (18, 16, 16, 16, 16), "W must be 4-byte aligned"),
    (16, 64, (16, 17, 16, 16, 16), "2-byte aligned"),
])
def test_gemv_abi_validation(lib, N, K, ptrs, msg):
    # every case is rejected before any launch (the pointers are never dereferenced)
    rc = lib.w4a16_gemv(*[ctypes.c_void_p(p) for p in ptrs], N, K, None)
    assert rc == 1
    assert msg in lib.w4a16_last_error().decode()


def test_gemv_abi_empty_n_is_a_no_op(lib):
    assert lib.w4a16_gemv(None, None, None, None, None, 0, 64, None) == 0


def test_w4a16_ext_binding_rejects_host_tensors():
    import torch
    import w4a16_ext
    W, A, sW, zW = (torch.from_numpy(t) for t in make_gemv(16, 64))
    with pytest.raises(RuntimeError, match="all tensors must be CUDA"):
        w4a16_ext.w4a16_gemv(W, A, sW, zW)


# ----------------------------------------------------------------------------- GPU parity

def _cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")
    return torch


def _run(W, A, sW, zW, w_offset=0, a_offset=0):
    """The op under test on device copies; offsets (in elements) misalign W or A on purpose."""
    torch = _cuda()
    import w4a16_ext
    N, kw = W.shape
    wbuf = torch.zeros(W.size + 4, dtype=torch.int32, device="cuda")
    wbuf[w_offset:w_offset + W.size] = torch.from_numpy(W.reshape(-1)).cuda()
    Wd = wbuf[w_offset:w_offset + W.size].view(N, kw)
    abuf = torch.zeros(A.size + 8, dtype=torch.float16, device="cuda")
    abuf[a_offset:a_offset + A.size] = torch.from_numpy(A).cuda()
    Ad = abuf[a_offset:a_offset + A.size]
    return w4a16_ext.w4a16_gemv(Wd, Ad, torch.from_numpy(sW).cuda(), torch.from_numpy(zW).cuda())


GPU_SHAPES = [
    (1, 8), (16, 64), (17, 136), (100, 4096), (257, 4104), (64, 8192 + 160), (48, 12288),
    (4096, 4096), (14336, 4096), (4096, 14336), (7, 20000),
]


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", GPU_SHAPES)
def test_gemv_bit_exact_vs_oracle(N, K):
    print(f"gemv N={N} K={K}", flush=True)
    W, A, sW, zW = make_gemv(N, K, 1, special=True)
    C = _run(W, A, sW, zW).cpu().numpy()
    assert np.array_equal(bits(C), bits(c_oracle.gemv(W, A, sW, zW, exact=True)))


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,w_off,a_off", [(64, 4096, 1, 0), (64, 4096, 0, 1), (33, 1024, 2, 3), (40, 520, 1, 1),
                                             (8200, 1032, 1, 0), (8224, 136, 0, 1), (8208, 4104, 0, 0)])
def test_gemv_misaligned_operands(N, K, w_off, a_off):
    print(f"gemv misaligned N={N} K={K} w_off={w_off} a_off={a_off}", flush=True)
    W, A, sW, zW = make_gemv(N, K, 2, special=True)
    C = _run(W, A, sW, zW, w_offset=w_off, a_offset=a_off).cpu().numpy()
    assert np.array_equal(bits(C), bits(c_oracle.gemv(W, A, sW, zW, exact=True)))


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(4096, 4096), (512, 14336)])
def test_gemv_within_tolerance_of_reference_order(N, K):
    W, A, sW, zW = make_gemv(N, K, 3)
    C = _run(W, A, sW, zW).float().cpu().numpy().astype(np.float64)
    ref = c_oracle.gemv(W, A, sW, zW, exact=False).astype(np.float64)
    assert np.isfinite(C).all()
    assert np.abs(C - ref).max() / np.abs(ref).max() < 2e-3


@pytest.mark.gpu
def test_gemv_extremes_and_empty():
    torch = _cuda()
    import w4a16_ext
    # all weights -8 against +-65504: |acc| = 8 * 65504 * K, the largest sums the format allows
    N, K = 32, 2048
    W = np.full((N, K // 8), np.uint32(0x88888888).view(np.int32), dtype=np.int32)
    A = np.where(np.arange(K) % 3 == 0, -65504, 65504).astype(np.float16)
    sW = np.full(N, 1e-4, np.float16)
    zW = np.zeros(N, np.float16)
    C = _run(W, A, sW, zW).cpu().numpy()
    assert np.array_equal(bits(C), bits(c_oracle.gemv(W, A, sW, zW, exact=True)))
    # K = 0: C = fp16(-z * s);  N = 0: empty
    W0, A0 = np.zeros((N, 0), np.int32), np.zeros(0, np.float16)
    zW = np.random.default_rng(0).standard_normal(N).astype(np.float16)
    C0 = w4a16_ext.w4a16_gemv(torch.zeros(N, 0, dtype=torch.int32, device="cuda"),
                              torch.zeros(0, dtype=torch.float16, device="cuda"),
                              torch.from_numpy(sW).cuda(), torch.from_numpy(zW).cuda()).cpu().numpy()
    assert np.array_equal(bits(C0), bits(c_oracle.gemv(W0, A0, sW, zW, exact=True)))
    e = w4a16_ext.w4a16_gemv(torch.zeros(0, 8, dtype=torch.int32, device="cuda"),
                             torch.zeros(64, dtype=torch.float16, device="cuda"),
                             torch.zeros(0, dtype=torch.float16, device="cuda"),
                             torch.zeros(0, dtype=torch.float16, device="cuda"))
    assert e.shape == (0,)


@pytest.mark.gpu
def test_gemv_nonfinite_inputs_follow_ieee():
    rng = np.random.default_rng(5)
    N, K = 300, 4096 + 64
    for trial in range(3):
        W, A, sW, zW = make_gemv(N, K, 50 + trial)
        W[rng.random((N, K // 8)) < 0.5] = 0
        idx = rng.choice(K, size=1 + trial, replace=False)
        A[idx] = np.array([np.inf, -np.inf, np.nan], dtype=np.float16)[:len(idx)]
        C = _run(W, A, sW, zW).cpu().numpy()
        ref = c_oracle.gemv(W, A, sW, zW, exact=True)
        assert np.array_equal(np.isnan(C), np.isnan(ref)), trial
        fin = ~np.isnan(ref)
        assert np.array_equal(bits(C[fin]), bits(ref[fin])), trial


@pytest.mark.gpu
def test_gemv_reference_error_messages():
    torch = _cuda()
    import w4a16_ext
    W = torch.zeros(16, 8, dtype=torch.int32, device="cuda")
    A = torch.zeros(64, dtype=torch.float16, device="cuda")
    s = torch.zeros(16, dtype=torch.float16, device="cuda")
    cases = [
        ((W.t(), A, s, s), "all tensors must be contiguous"),
        ((W.float(), A, s, s), "W must be int32"),
        ((W, A.float(), s, s), "A, sW, zW must be float16"),
        ((W[:, :1].contiguous(), A[:12].contiguous(), s, s), "K must be a multiple of 8"),
        ((W[:, :4].contiguous(), A, s, s), r"W must be \[N, K/8\]"),
        ((W, A, s[:8], s), r"sW, zW must be \[N\]"),
    ]
    for args, msg in cases:
        with pytest.raises(RuntimeError, match=msg):
            w4a16_ext.w4a16_gemv(*args)


@pytest.mark.gpu
def test_gemv_deterministic_and_graph_replay():
    torch = _cuda()
    import w4a16_ext
    W, A, sW, zW = (torch.from_numpy(t).cuda() for t in make_gemv(2048, 4096, 8))
    eager = w4a16_ext.w4a16_gemv(W, A, sW, zW)
    assert torch.equal(eager, w4a16_ext.w4a16_gemv(W, A, sW, zW))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = w4a16_ext.w4a16_gemv(W, A, sW, zW)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _ = (A.float() * 2).sum().item()                     # eager work between replays
