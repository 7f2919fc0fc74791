"""CPU oracle for the W4A16 GEMM: weight format, quantizer, dequantizer and fp32 reference GEMM.

TEST INFRASTRUCTURE ONLY.  Nothing on the product path may import this module: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only as the checker (or, in the bench, as the timed CPU reference path).

This is a numpy restatement of the reference's ``tests/quant.py`` (the format definition and
the fp32 oracle).  Each function cites the reference lines it follows.

Format (reference ``tests/quant.py:3-5, 34-48``):
  * codes ``q[n, k]`` are unsigned 4-bit values 0..15 with zero-point 8;
  * ``W[n, k] = (q[n, k] - 8) * scales[k // G, n]`` with ``scales`` fp16 ``[K/G, N]``;
  * packed words ``Wp`` are int32, ``N*K/8`` of them, laid out as ``[N/16][K/64][32 lanes][4]``.
    Word ``(nb, kc, lane, s)`` holds 8 nibbles; nibble ``i`` (bits ``4i..4i+3``) with
    ``p = i & 3``, ``h = i >> 2``, ``g = lane >> 2``, ``t = lane & 3`` is
    ``q[16*nb + g + 8*(p & 1), 64*kc + 16*s + 2*t + 8*(p >> 1) + h]``.

Parity status: every function here is pinned by tests/test_oracle.py (closed forms, the
independent kernel-side decoder of the reference's test_pack_matches_kernel_decode, exhaustive
fp16 checks, float64 brute force, and the C restatement in ``oracle/w4a16_oracle.c``).
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "fragment_map", "pack_int4", "unpack_int4", "quantize_w4", "dequantize_w4", "ref_gemm",
    "make_problem", "gen_codes_scales",
]


def fragment_map():
    """(n, k) inside one 16x16 (n x k) slice for every (lane 0..31, nibble 0..7).

    Follows reference ``tests/quant.py:10-25``: ``p, h = i & 3, i >> 2``;
    ``n = g + 8*(p & 1)``; ``k = 2*t + 8*(p >> 1) + h`` with ``g, t = lane >> 2, lane & 3``.
    Returns two int64 arrays of shape [32, 8].
    """
    lane = np.arange(32)[:, None]
    i = np.arange(8)[None, :]
    g, t = lane >> 2, lane & 3
    p, h = i & 3, i >> 2
    n_idx = g + 8 * (p & 1) + 0 * i
    k_idx = 2 * t + 8 * (p >> 1) + h
    return n_idx.astype(np.int64), k_idx.astype(np.int64)


# The nibble position of (a = n-half, b = k-half-of-16, h = k parity) inside a word:
# i = p + 4h with p = a + 2b  (reference tests/quant.py:21-24).
def _nibble_shifts():
    a = np.arange(2).reshape(2, 1, 1)
    b = np.arange(2).reshape(1, 2, 1)
    h = np.arange(2).reshape(1, 1, 2)
    return (4 * (a + 2 * b + 4 * h)).astype(np.uint32)          # [a, b, h]


def pack_int4(q: np.ndarray) -> np.ndarray:
    """uint8 codes [N, K] (0..15) -> int32 words [N*K/8] in kernel order.

    Reference ``tests/quant.py:34-48``: word index ``(((n/16)*(K/64) + k/64)*32 + lane)*4 + s``
    with ``s = (k % 64) / 16``; nibble i shifted by 4*i; stored as two's-complement int32.
    Implemented by splitting n = 16*nb + 8*a + g and k = 64*kc + 16*s + 8*b + 2*t + h, which is
    the same bijection as ``fragment_map`` written as a reshape (the two are cross-checked).
    """
    q = np.asarray(q)
    N, K = q.shape
    if N % 16 or K % 64:
        raise ValueError("N must be a multiple of 16 and K of 64")
    if q.dtype != np.uint8:
        q = q.astype(np.uint8)
    NB, KC = N // 16, K // 64
    # axes: nb, a, g, kc, s, b, t, h
    Q = q.reshape(NB, 2, 8, KC, 4, 2, 4, 2)
    sh = _nibble_shifts()                                      # [a, b, h]
    w = np.zeros((NB, 8, KC, 4, 4), dtype=np.uint32)          # nb, g, kc, s, t
    for a in range(2):
        for b in range(2):
            for h in range(2):
                w |= Q[:, a, :, :, :, b, :, h].astype(np.uint32) << sh[a, b, h]
    # -> [nb, kc, g, t, s] == [nb, kc, lane, s]
    w = w.transpose(0, 2, 1, 4, 3)
    return np.ascontiguousarray(w).reshape(-1).view(np.int32)


def unpack_int4(Wp: np.ndarray, N: int, K: int) -> np.ndarray:
    """Inverse of ``pack_int4`` (reference ``tests/quant.py:51-59``): int32 [N*K/8] -> uint8 [N, K]."""
    NB, KC = N // 16, K // 64
    w = np.ascontiguousarray(Wp).view(np.uint32).reshape(NB, KC, 8, 4, 4)   # nb, kc, g, t, s
    w = w.transpose(0, 2, 1, 4, 3)                                           # nb, g, kc, s, t
    sh = _nibble_shifts()
    out = np.empty((NB, 2, 8, KC, 4, 2, 4, 2), dtype=np.uint8)               # nb,a,g,kc,s,b,t,h
    for a in range(2):
        for b in range(2):
            for h in range(2):
                out[:, a, :, :, :, b, :, h] = ((w >> sh[a, b, h]) & 0xF).astype(np.uint8)
    return out.reshape(N, K)


def quantize_w4(W: np.ndarray, group_size: int):
    """Symmetric RTN, per (n, k-group) absmax/7 scale, zero-point 8 (reference ``tests/quant.py:62-74``).

    ``s = fp16(max(absmax/7, 1e-4))`` computed in fp32; ``q = clamp(round_half_even(W/s), -8, 7) + 8``.
    Returns q uint8 [N, K] and scales fp16 [K/G, N].
    """
    W = np.asarray(W, dtype=np.float32)
    N, K = W.shape
    G = group_size
    if K % G:
        raise ValueError("K must be a multiple of the group size")
    Wg = W.reshape(N, K // G, G)
    s = np.maximum(np.abs(Wg).max(-1, keepdims=True) / np.float32(7), np.float32(1e-4))
    s = s.astype(np.float16).astype(np.float32)
    q = (np.clip(np.round(Wg / s), -8, 7) + 8).astype(np.uint8).reshape(N, K)
    scales = np.ascontiguousarray(s[..., 0].T).astype(np.float16)
    return q, scales


def dequantize_w4(q: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """fp16 [N, K] = fp16_rn((q - 8) * s)  (reference ``tests/quant.py:77-80``).

    ``q - 8`` is exact in fp16; numpy's float16 multiply forms the (exact) fp32 product and
    rounds it once to nearest-even fp16, which is the reference's single fp16 multiply.
    """
    s = np.repeat(np.asarray(scales, dtype=np.float16).T, group_size, axis=1)   # [N, K]
    return (np.asarray(q).astype(np.float16) - np.float16(8)) * s


def ref_gemm(x: np.ndarray, q: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """fp32 reference ``x.float() @ dequantize_w4(q, s, G).float().T`` (reference ``tests/quant.py:83-85``)."""
    Wd = dequantize_w4(q, scales, group_size).astype(np.float32)
    return np.asarray(x, dtype=np.float16).astype(np.float32) @ Wd.T


# ----------------------------------------------------------------------------- test-data makers

def make_problem(M: int, N: int, K: int, G: int, seed: int = 0, w_std: float = 0.02):
    """Seeded mirror of the reference's ``make_problem`` (tests/test_w4a16.py:33-38).

    W ~ N(0, w_std^2), x ~ N(0, 1) as fp16, then RTN-quantize and pack.  numpy's generator is
    used instead of torch's, so the bits differ from the reference's draws; the contract is
    tolerance-based so only the distribution matters.  Returns host arrays
    ``(x fp16 [M,K], q uint8 [N,K], scales fp16 [K/G,N], Wp int32 [N*K/8])``.
    """
    rng = np.random.default_rng(seed)
    W = rng.standard_normal((N, K), dtype=np.float32) * np.float32(w_std)
    x = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    q, scales = quantize_w4(W, G)
    return x, q, scales, pack_int4(q)


def gen_codes_scales(N: int, K: int, G: int, seed: int, s_lo: float = 0.002, s_hi: float = 0.02):
    """BASELINE-style synthetic weights: q ~ U{0..15}, scales ~ U[s_lo, s_hi] fp16 [K/G, N]."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    scales = rng.uniform(s_lo, s_hi, size=(K // G, N)).astype(np.float16)
    return q, scales
