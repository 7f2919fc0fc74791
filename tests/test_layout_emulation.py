"""numpy emulation of the MI355X kernels' index math against a plain float64 matmul (CPU).

The same method as the reference's tests/layout_prefill.py (which emulates its NVIDIA fragment
layouts), applied to this build's gfx950 mapping (w4a16-gemm_amd/csrc/w4a16_device.h):
  * v_mfma_f32_16x16x32_f16 modelled as C[i][j] += sum over (lane group kb, slot) of
    A[16*kb + i][slot] * B[16*kb + j][slot]; output lane l holds C[4*(l//16) + r][l % 16];
  * A operand: lane (kb, i) reads packed lane' = 4*(i % 8) + kb, keeps its own nibble parity,
    MFMA h uses words 2h, 2h+1 (slot pair c <-> k = 32h + 8c + 2kb + {0,1});
  * B operand, prefill: the permuted LDS row layout written by lds_store_xseg and read with
    one 16-byte read at row*144 + h*64 + kb*16;
  * B operand, decode: 8 consecutive halves per lane then the 4x4 cross-row transpose made of
    v_permlane32_swap (upper half of dst <-> lower half of src) and v_permlane16_swap (odd
    rows of dst <-> even rows of src);
  * decode: waves split K, partial tiles summed in wave order, splits summed in split order.
Exact float64 arithmetic is used (dequantised values are exact), so the check is 1e-12.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import quant

XROW = 144


def permlane32_swap(dst, src):
    """v_permlane32_swap_b32: lanes 32..63 of dst <-> lanes 0..31 of src."""
    d, s = dst.copy(), src.copy()
    d[32:], s[:32] = src[:32].copy(), dst[32:].copy()
    return d, s


def permlane16_swap(dst, src):
    """v_permlane16_swap_b32: rows 1 and 3 of dst <-> rows 0 and 2 of src."""
    d, s = dst.copy(), src.copy()
    for r in (0, 2):
        d[16 * (r + 1):16 * (r + 2)], s[16 * r:16 * (r + 1)] = src[16 * r:16 * (r + 1)].copy(), dst[16 * (r + 1):16 * (r + 2)].copy()
    return d, s


def xpose_rows(v):
    """w4a16::xpose_rows on a [64 lanes, 4 dwords] array (dwords as opaque objects)."""
    a0, a1 = permlane32_swap(v[:, 0], v[:, 2])
    b0, b1 = permlane32_swap(v[:, 1], v[:, 3])
    c0, c1 = permlane16_swap(a0, b0)
    e0, e1 = permlane16_swap(a1, b1)
    return np.stack([c0, c1, e0, e1], axis=1)


def mfma(A, B, C):
    """A, B: [64 lanes, 8 slots]; C: [64 lanes, 4] in the 16x16 output layout."""
    Am = np.zeros((16, 16))
    out = C.copy()
    full = np.zeros((16, 16))
    for kb in range(4):
        full += A[16 * kb:16 * kb + 16, :] @ B[16 * kb:16 * kb + 16, :].T
    for lane in range(64):
        for r in range(4):
            out[lane, r] += full[4 * (lane // 16) + r, lane % 16]
    del Am
    return out


def a_operand(W4, Sn, nb, kc, h):
    """Dequantised A operand of one MFMA: lane (kb, i) -> 8 fp64 values.  W4: [NB,KC,32,4] uint32,
    Sn: per-(nb, kc) scale row [16] for n = 16nb + i."""
    A = np.zeros((64, 8))
    for lane in range(64):
        kb, i = lane >> 4, lane & 15
        lanep = 4 * (i & 7) + kb
        pe = i >> 3
        s = Sn[i]
        slots = []
        for word in (2 * h, 2 * h + 1):
            w = int(W4[nb, kc, lanep, word])
            for sh in (0, 8):                       # pairs p = pe (sh 0) and p = pe + 2 (sh 8)
                bits = (w >> (sh + 4 * pe)) & 0x000F000F
                slots += [((bits & 0xF) - 8) * s, ((bits >> 16) - 8) * s]
        A[lane] = slots
    return A


@pytest.mark.parametrize("M,N,K,G,BM,BN,WMs,WNs", [
    (5, 48, 192, 64, 16, 128, 1, 4), (17, 80, 256, 64, 32, 128, 1, 4),
    (33, 144, 640, 128, 64, 128, 2, 2), (70, 208, 384, 64, 128, 128, 2, 2),
])
def test_prefill_index_math(M, N, K, G, BM, BN, WMs, WNs):
    rng = np.random.default_rng(M + N)
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = rng.random((K // G, N)) * 0.05 + 0.001
    x = rng.standard_normal((M, K))
    W4 = quant.pack_int4(q).view(np.uint32).reshape(N // 16, K // 64, 32, 4)
    ref = x @ ((q.astype(np.float64) - 8) * np.repeat(s.T, G, axis=1)).T
    WM, WN = BM // WMs, BN // WNs
    TM, TN = WM // 16, WN // 16
    KC, NBLK = K // 64, N // 16
    y = np.full((M, N), np.nan)
    for tm in range(-(-M // BM)):
        for tn in range(-(-N // BN)):
            m0, n0 = tm * BM, tn * BN
            accs = {}
            for kc in range(KC):
                # x chunk -> permuted LDS (one float64 per half; index = byte offset / 2)
                lds = np.zeros(BM * XROW // 2)
                for row in range(BM):
                    for qseg in range(8):
                        v = x[m0 + row, kc * 64 + 8 * qseg: kc * 64 + 8 * qseg + 8] if m0 + row < M else np.zeros(8)
                        base = row * XROW + (qseg >> 2) * 64 + (qseg & 3) * 4
                        for e in range(4):
                            lds[(base + 16 * e) // 2:(base + 16 * e) // 2 + 2] = v[2 * e:2 * e + 2]
                for wave in range(WMs * WNs):
                    wm, wn = wave // WNs, wave % WNs
                    for b in range(TN):
                        nb = (n0 >> 4) + wn * TN + b
                        if nb >= NBLK:
                            continue
                        Sn = s[kc * 64 // G, nb * 16:nb * 16 + 16]
                        for h in range(2):
                            A = a_operand(W4, Sn, nb, kc, h)
                            for t in range(TM):
                                B = np.zeros((64, 8))
                                for lane in range(64):
                                    kb, li = lane >> 4, lane & 15
                                    off = ((wm * WM + t * 16 + li) * XROW + h * 64 + kb * 16) // 2
                                    B[lane] = lds[off:off + 8]
                                key = (wave, t, b)
                                accs[key] = mfma(A, B, accs.get(key, np.zeros((64, 4))))
            for (wave, t, b), C in accs.items():
                wm, wn = wave // WNs, wave % WNs
                nb = (n0 >> 4) + wn * TN + b
                for lane in range(64):
                    m = m0 + wm * WM + t * 16 + (lane & 15)
                    if m < M:
                        n = nb * 16 + 4 * (lane >> 4)
                        y[m, n:n + 4] = C[lane]
    assert not np.isnan(y).any()
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-12


def test_xpose_rows_is_the_b_operand_transpose():
    """Lane (row r) holding dwords D[r][0..3] ends with D[0..3][r] (w4a16_device.h mapping)."""
    D = np.array([[(r, e) for e in range(4)] for r in range(4)], dtype=object)
    v = np.empty((64, 4), dtype=object)
    for lane in range(64):
        for e in range(4):
            v[lane, e] = (lane >> 4, e, lane & 15)
    out = xpose_rows(v)
    for lane in range(64):
        r = lane >> 4
        assert [tuple(out[lane, c]) for c in range(4)] == [(c, r, lane & 15) for c in range(4)]
    del D


@pytest.mark.parametrize("M,N,K,G,NBW,WAVES,splits", [
    (1, 64, 512, 64, 1, 8, 1), (3, 128, 1024, 128, 2, 8, 2), (16, 64, 1024, 64, 4, 4, 2),
])
def test_decode_index_math(M, N, K, G, NBW, WAVES, splits):
    rng = np.random.default_rng(M * 7 + N)
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = rng.random((K // G, N)) * 0.05 + 0.001
    x = rng.standard_normal((M, K))
    W4 = quant.pack_int4(q).view(np.uint32).reshape(N // 16, K // 64, 32, 4)
    ref = x @ ((q.astype(np.float64) - 8) * np.repeat(s.T, G, axis=1)).T
    KC = K // 64
    kcw = KC // (splits * WAVES)
    y = np.full((M, N), np.nan)
    for tile in range(N // (16 * NBW)):
        parts = []
        for split in range(splits):
            red = np.zeros((WAVES, NBW, 64, 4))
            for wave in range(WAVES):
                kc0 = (split * WAVES + wave) * kcw
                for c in range(kcw):
                    kc = kc0 + c
                    Bs = []
                    for h in range(2):
                        v = np.empty((64, 4), dtype=object)
                        for lane in range(64):
                            kb, li = lane >> 4, lane & 15
                            row = min(li, M - 1)
                            base = kc * 64 + 32 * h + 8 * kb
                            for e in range(4):
                                v[lane, e] = (x[row, base + 2 * e], x[row, base + 2 * e + 1])
                        t = xpose_rows(v)
                        Bs.append(np.array([[val for dw in t[lane] for val in dw] for lane in range(64)]))
                    for b in range(NBW):
                        nb = tile * NBW + b
                        Sn = s[kc * 64 // G, nb * 16:nb * 16 + 16]
                        for h in range(2):
                            red[wave, b] = mfma(a_operand(W4, Sn, nb, kc, h), Bs[h], red[wave, b])
            tot = red[0].copy()
            for w in range(1, WAVES):
                tot += red[w]
            parts.append(tot)
        fin = parts[0].copy()
        for p in parts[1:]:
            fin += p
        for b in range(NBW):
            nb = tile * NBW + b
            for lane in range(64):
                li = lane & 15
                if li < M:
                    n = nb * 16 + 4 * (lane >> 4)
                    y[li, n:n + 4] = fin[b, lane]
    assert not np.isnan(y).any()
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-12


def mfma32(A, B, C):
    """v_mfma_f32_32x32x16_f16 model.  A, B: [64 lanes, 8 slots] (lane (kg, r) holds row r of A /
    column r of B at k = 8 kg + slot); C: [64 lanes, 16], register i of lane (kg, r) holds
    C[8 (i // 4) + 4 kg + i % 4][r]."""
    full = A[:32] @ B[:32].T + A[32:] @ B[32:].T
    out = C.copy()
    for lane in range(64):
        kg, r = lane >> 5, lane & 31
        for i in range(16):
            out[lane, i] += full[8 * (i // 4) + 4 * kg + i % 4, r]
    return out


def wide_lane_block(nb0, q, r, nblk):
    """prefill_wide_kernel: wave-uniform base block of channel block q and the lane's block offset
    (both clamped to the last n16 block; the offset is 0 or 1)."""
    qb = min(nb0 + 2 * q, nblk - 1)
    return qb, min(nb0 + 2 * q + (r >> 4), nblk - 1) - qb


@pytest.mark.parametrize("M,N,K,G,BM,BN,WMs,WNs", [
    (40, 80, 256, 64, 128, 128, 1, 2), (70, 208, 384, 128, 128, 256, 1, 4), (33, 48, 128, 64, 256, 128, 2, 2),
])
def test_wide_prefill_32x32_index_math(M, N, K, G, BM, BN, WMs, WNs):
    """prefill_wide_kernel on v_mfma_f32_32x32x16_f16: A lane (kg, r) of step (tp, h) is the
    16x16x32 A lane (kb = 2 tp + kg, i = r % 16) of n16 block 2q + r / 16; B is read from the
    permuted LDS row at h*64 + tp*32 + kg*16; D register i is channel 8(i/4) + 4kg + i%4."""
    rng = np.random.default_rng(M * N)
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = rng.random((K // G, N)) * 0.05 + 0.001
    x = rng.standard_normal((M, K))
    W4 = quant.pack_int4(q).view(np.uint32).reshape(N // 16, K // 64, 32, 4)
    ref = x @ ((q.astype(np.float64) - 8) * np.repeat(s.T, G, axis=1)).T
    WM, WN = BM // WMs, BN // WNs
    TM, TN = WM // 32, WN // 32
    KC, NBLK = K // 64, N // 16
    y = np.full((M, N), np.nan)
    for tm in range(-(-M // BM)):
        for tn in range(-(-N // BN)):
            m0, n0 = tm * BM, tn * BN
            accs = {}
            for kc in range(KC):
                lds = np.zeros(BM * XROW // 2)
                for row in range(BM):
                    for qseg in range(8):
                        v = x[min(m0 + row, M - 1), kc * 64 + 8 * qseg: kc * 64 + 8 * qseg + 8]
                        base = row * XROW + (qseg >> 2) * 64 + (qseg & 3) * 4
                        for e in range(4):
                            lds[(base + 16 * e) // 2:(base + 16 * e) // 2 + 2] = v[2 * e:2 * e + 2]
                for wave in range(WMs * WNs):
                    wm, wn = wave // WNs, wave % WNs
                    nb0 = (n0 + wn * WN) >> 4
                    for qq in range(TN):
                        for h in range(2):
                            for tp in range(2):
                                A = np.zeros((64, 8))
                                for lane in range(64):
                                    kg, r = lane >> 5, lane & 31
                                    qb, nbl = wide_lane_block(nb0, qq, r, NBLK)
                                    nb = qb + nbl
                                    Sn = s[kc * 64 // G, nb * 16:nb * 16 + 16]
                                    A[lane] = a_operand(W4, Sn, nb, kc, h)[16 * (2 * tp + kg) + (r & 15)]
                                for p in range(TM):
                                    B = np.zeros((64, 8))
                                    for lane in range(64):
                                        kg, r = lane >> 5, lane & 31
                                        off = ((wm * WM + p * 32 + r) * XROW + h * 64 + tp * 32 + kg * 16) // 2
                                        B[lane] = lds[off:off + 8]
                                    key = (wave, p, qq)
                                    accs[key] = mfma32(A, B, accs.get(key, np.zeros((64, 16))))
            for (wave, p, qq), C in accs.items():
                wm, wn = wave // WNs, wave % WNs
                nb0 = (n0 + wn * WN) >> 4
                for lane in range(64):
                    kg, r = lane >> 5, lane & 31
                    m = m0 + wm * WM + p * 32 + r
                    for g in range(4):
                        if m < M and nb0 + 2 * qq + (g >> 1) < NBLK:
                            n = (nb0 + 2 * qq) * 16 + 8 * g + 4 * kg
                            y[m, n:n + 4] = C[lane, 4 * g:4 * g + 4]
    assert not np.isnan(y).any()
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-12


# config 22 (prefill_wide_pipe_kernel) addresses memory exactly as 18
WIDE_TILES = {5: (128, 256, 1, 4), 6: (256, 128, 2, 2), 7: (128, 128, 1, 2), 18: (64, 128, 1, 4), 19: (64, 256, 1, 8),
              20: (128, 128, 1, 4), 21: (256, 256, 2, 4), 22: (64, 128, 1, 4), 23: (128, 512, 1, 8),
              24: (128, 256, 1, 8)}


@pytest.mark.parametrize("cfg", sorted(WIDE_TILES))
@pytest.mark.parametrize("M,N,K,G", [(300, 1040, 2048, 64), (129, 272, 1152, 64), (300, 80, 640, 64),
                                     (513, 208, 384, 128), (70, 16, 128, 64), (40, 4112, 4160, 64)])
def test_wide_prefill_addresses_in_bounds(cfg, M, N, K, G):
    """Every global load and store offset of prefill_wide_kernel stays inside its buffer for shapes
    whose last N tile is partial.  Regression: a per-lane block offset taken relative to an
    unclamped base went negative and, as the unsigned 32-bit offset of a saddr load, addressed
    4 GB past the weights."""
    BM, BN, WMs, WNs = WIDE_TILES[cfg]
    NT, WM, WN = WMs * WNs * 64, BM // WMs, BN // WNs
    TM, TN = WM // 32, WN // 32
    KC, NBLK, gshift = K // 64, N // 16, 1 if G == 128 else 0
    sizes = {"w": N * K // 2, "s": (K // G) * N * 2, "x": M * K * 2, "y": M * N * 2}
    for tile in range(-(-M // BM) * -(-N // BN)):
        tm, tn = tile % -(-M // BM), tile // -(-M // BM)
        m0, n0 = tm * BM, tn * BN
        for wave in range(WMs * WNs):
            wm, wn = wave // WNs, wave % WNs
            nb0 = (n0 + wn * WN) >> 4
            for lane in range(64):
                kg, r = lane >> 5, lane & 31
                for qq in range(TN):
                    qb, nbl = wide_lane_block(nb0, qq, r, NBLK)
                    assert nbl in (0, 1)
                    for tp in range(2):
                        woff = (nbl * KC * 512 + (((r & 7) << 2) | (tp << 1) | kg) * 16) & 0xFFFFFFFF
                        for kcl in (0, KC - 1):
                            assert qb * KC * 512 + kcl * 512 + woff + 16 <= sizes["w"]
                    soff = ((nbl * 16 + (r & 15)) * 2) & 0xFFFFFFFF
                    for kcl in (0, KC - 1):
                        assert qb * 32 + (kcl >> gshift) * N * 2 + soff + 2 <= sizes["s"]
                    for p in range(TM):
                        m = m0 + wm * WM + p * 32 + r
                        for g in range(4):
                            n = (nb0 + 2 * qq) * 16 + 8 * g + 4 * kg
                            if m < M and nb0 + 2 * qq + (g >> 1) < NBLK:
                                assert n + 4 <= N and (m * N + n) * 2 + 8 <= sizes["y"]
        for tid in range(NT):
            for i in range(BM * 8 // NT):
                sg = tid + i * NT
                xoff = ((min(m0 + (sg >> 3), M - 1) - m0) * K + (sg & 7) * 8) * 2
                assert m0 * K * 2 + (KC - 1) * 128 + xoff + 16 <= sizes["x"]


def ring_x_rows(x, M, K, c0, XR):
    """decode_ring_kernel x rows of the chunk pair starting at chunk c0 as they land in LDS: XR rows x 64 dwords (each dword a
    pair of fp64 halves).  XR == 1: one 4-byte load, lane j fetching dword 32*(u/8) + 16*((u/4)%2)
    + 4*(j%4) + u%4 of the pair (u = j / 4).  XR >= 4: 16-byte loads of 4 rows each, lane j of
    load q filling row (64q + j) / 16, segment j % 16 with global segment (j % 16) ^ (row % 8).
    Also returns the largest source byte offset touched within an x row and, for XR >= 4, the
    slot's LDS bytes as the loads write them (byte offset -> dword; rows 8..15 of a 16-row slot
    start 8 bytes further on)."""
    slot = np.empty((XR, 64, 2))
    phys = {}
    hi = 0
    if XR == 1:
        for lane in range(64):
            u = lane >> 2
            d = 32 * (u >> 3) + 16 * ((u >> 2) & 1) + 4 * (lane & 3) + (u & 3)
            off = c0 * 128 + 4 * d
            hi = max(hi, off + 4)
            slot[0, lane] = x[0, off // 2:off // 2 + 2]
        return slot, hi, phys
    for q in range(XR // 4):
        for lane in range(64):
            r = (64 * q + lane) >> 4
            gseg = (lane & 15) ^ (r & 7)
            off = c0 * 128 + gseg * 16
            hi = max(hi, off + 16)
            dst = q * 1024 + (8 if XR == 16 and q >= 2 else 0) + lane * 16     # the DMA's LDS bytes
            for e in range(4):
                slot[r, 4 * (lane & 15) + e] = x[min(r, M - 1), off // 2 + 2 * e:off // 2 + 2 * e + 2]
                phys[dst + 4 * e] = tuple(slot[r, 4 * (lane & 15) + e])
    return slot, hi, phys


def ring_b_operand(slot, M, XR, cc, h):
    """B operand (64 lanes x 8 halves) and the LDS byte address of each lane's first dword."""
    B = np.zeros((64, 8))
    addr = []
    for lane in range(64):
        kb, j = lane >> 4, lane & 15
        xr = min(j, M - 1)
        if XR == 1:
            pos = 8 * cc + 4 * h + kb
            B[lane] = slot[0, 4 * pos:4 * pos + 4].reshape(8)
            addr.append(pos * 16)
        else:
            dws = []
            for c in range(4):
                pos = 8 * cc + ((4 * h + c) ^ (xr & 7))
                dws.append(slot[xr, 4 * pos + kb])
            B[lane] = np.concatenate(dws)
            addr.append([xr * 256 + (8 if XR == 16 and xr >= 8 else 0) + (8 * cc + ((4 * h + c) ^ (xr & 7))) * 16 + 4 * kb
                         for c in range(4)])
    return B, addr


@pytest.mark.parametrize("M,N,K,G,NBW,WAVES,splits", [
    (1, 64, 1024, 64, 1, 8, 1), (1, 128, 2048, 128, 2, 4, 2), (2, 64, 1024, 128, 1, 4, 2),
    (3, 128, 1024, 128, 2, 4, 2), (5, 64, 1024, 64, 1, 4, 1), (9, 64, 2048, 128, 4, 4, 1),
    (16, 64, 1024, 64, 2, 4, 2),
])
def test_ring_decode_x_rows_index_math(M, N, K, G, NBW, WAVES, splits):
    """decode_ring_kernel x paths (4-byte loads in B-operand order for M = 1, swizzled 16-byte
    loads plus four 4-byte LDS reads otherwise), the waves of a workgroup interleaved over K (wave w
    takes chunk pairs w, w + WAVES, ...), the weights as in decode_kernel: the emulated
    result equals the float64 matmul, every x source offset stays inside the row, every B operand
    holds x[row][32h + 8c + 2kb + {0,1}] in slot pair c, the first-dword reads of 8 consecutive
    lanes with 8 distinct rows hit 8 distinct 16-byte bank groups, and with 16 distinct rows
    (rows 8..15 8 bytes further on) every 4-byte read hits 32 distinct banks in each half-wave (the
    LDS serves a 4-byte read 32 lanes at a time from 32 banks, measured: 0 conflict cycles at
    M <= 8, two per read at M = 16 without the shift)."""
    rng = np.random.default_rng(M * 11 + K)
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = rng.random((K // G, N)) * 0.05 + 0.001
    x = rng.standard_normal((M, K))
    W4 = quant.pack_int4(q).view(np.uint32).reshape(N // 16, K // 64, 32, 4)
    ref = x @ ((q.astype(np.float64) - 8) * np.repeat(s.T, G, axis=1)).T
    XR = 1 if M <= 1 else 4 if M <= 4 else 8 if M <= 8 else 16
    KC = K // 64
    kcw = KC // (splits * WAVES)
    y = np.full((M, N), np.nan)
    for tile in range(N // (16 * NBW)):
        fin = np.zeros((NBW, 64, 4))
        for split in range(splits):
            for wave in range(WAVES):
                kc0 = split * WAVES * kcw + 2 * wave
                acc = np.zeros((NBW, 64, 4))
                for p in range(kcw // 2):
                    c0 = kc0 + 2 * WAVES * p
                    slot, hi, phys = ring_x_rows(x, M, K, c0, XR)
                    assert hi <= 2 * K
                    for cc in range(2):
                        Bs = []
                        for h in range(2):
                            B, addr = ring_b_operand(slot, M, XR, cc, h)
                            for lane in range(64):
                                kb, j = lane >> 4, lane & 15
                                base = (c0 + cc) * 64 + 32 * h + 2 * kb
                                want = [x[min(j, M - 1), base + 8 * c + e] for c in range(4) for e in range(2)]
                                assert np.array_equal(B[lane], want)
                            if XR > 1:
                                for g0 in range(0, 64, 8):
                                    rows = {min(j, M - 1) for j in range(g0 & 15, (g0 & 15) + 8)}
                                    if len(rows) == 8:
                                        assert len({a[0] // 16 % 8 for a in addr[g0:g0 + 8]}) == 8
                                for lane in range(64):      # the read addresses find the loaded dwords
                                    for c in range(4):
                                        assert phys[addr[lane][c]] == tuple(B[lane, 2 * c:2 * c + 2])
                                if M >= 16:                 # 16 distinct rows: each half-wave on 32 distinct banks
                                    for c in range(4):
                                        for half in (addr[:32], addr[32:]):
                                            assert len({a[c] // 4 % 32 for a in half}) == 32, (cc, h, c)
                            Bs.append(B)
                        kc = c0 + cc
                        for b in range(NBW):
                            nb = tile * NBW + b
                            Sn = s[kc * 64 // G, nb * 16:nb * 16 + 16]
                            for h in range(2):
                                acc[b] = mfma(a_operand(W4, Sn, nb, kc, h), Bs[h], acc[b])
                fin += acc
        for b in range(NBW):
            nb = tile * NBW + b
            for lane in range(64):
                li = lane & 15
                if li < M:
                    n = nb * 16 + 4 * (lane >> 4)
                    y[li, n:n + 4] = fin[b, lane]
    assert not np.isnan(y).any()
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-12


def group_x_slot(x, M, K, m0, c0, TM):
    """prefill_group_kernel x rows of one chunk pair (chunks c0, c0+1) as they land in LDS:
    a dict byte offset -> fp64 half pair (one dword), for TM tiles of 16 token rows.  16-byte
    direct-to-LDS load q (4 rows) writes rows r0 = 4 (q % 4) .. r0 + 3 of tile t = q // 4 at
    t * 4352 + r0 * 256 + 8 * (r0 >= 8); lane j writes row r0 + j // 16, position j % 16, with
    global segment (j % 16) ^ (row % 8) of token min(m0 + 16 t + row, M - 1)."""
    lds = {}
    hi = 0
    for q in range(4 * TM):
        t, r0 = q // 4, 4 * (q % 4)
        base = t * 4352 + r0 * 256 + (8 if r0 >= 8 else 0)
        for lane in range(64):
            r = r0 + (lane >> 4)
            g = (lane & 15) ^ (r & 7)
            off = c0 * 128 + g * 16                         # bytes within the token's row
            hi = max(hi, off + 16)
            tok = min(m0 + 16 * t + r, M - 1)
            for e in range(4):
                lds[base + lane * 16 + 4 * e] = tuple(x[tok, off // 2 + 2 * e:off // 2 + 2 * e + 2])
    return lds, hi


@pytest.mark.parametrize("M,TM", [(17, 2), (64, 4), (100, 4), (16, 1)])
def test_group_prefill_x_rows_b_operand(M, TM):
    """prefill_group_kernel B operands without cross-lane transposes: lane (kb, li) of token tile
    t, chunk cc, half h reads four dwords at t*4352 + li*256 + 8*(li >= 8) +
    (8 cc + ((4h + c) ^ (li % 8))) * 16 + 4 kb (c = 0..3); they must hold x[token][32h + 8c + 2kb
    + {0,1}] of chunk cc, every x source offset stays inside the row, and for every (t, cc, h, c)
    each half-wave (32 lanes, served together from 32 banks) hits 32 distinct 4-byte banks."""
    rng = np.random.default_rng(M)
    K = 512
    x = rng.standard_normal((M, K))
    for m0 in range(0, M, 16 * TM):
        for c0 in range(0, K // 64, 2):
            lds, hi = group_x_slot(x, M, K, m0, c0, TM)
            assert hi <= 2 * K
            for t in range(TM):
                for cc in range(2):
                    for h in range(2):
                        for c in range(4):
                            banks = [set(), set()]
                            for lane in range(64):
                                kb, li = lane >> 4, lane & 15
                                a = t * 4352 + li * 256 + (8 if li >= 8 else 0) + (8 * cc + ((4 * h + c) ^ (li & 7))) * 16 + 4 * kb
                                banks[lane >> 5].add(a // 4 % 32)
                                tok = min(m0 + 16 * t + li, M - 1)
                                k = (c0 + cc) * 64 + 32 * h + 8 * c + 2 * kb
                                assert lds[a] == (x[tok, k], x[tok, k + 1])
                            assert len(banks[0]) == 32 and len(banks[1]) == 32


@pytest.mark.parametrize("tiles_m,tiles_n", [(16, 112), (16, 24), (3, 5), (1, 7), (5, 1), (9, 13), (16, 16)])
@pytest.mark.parametrize("group_m", [1, 2, 3, 4, 8, 16])
def test_wide_prefill_grouped_tile_order_is_a_bijection(tiles_m, tiles_n, group_m):
    """prefill_wide_kernel's block -> (tm, tn) map (XCD remap, then groups of group_m M tiles with
    the M tile fastest) visits every output tile exactly once."""
    G = tiles_m * tiles_n
    group_m = min(group_m, tiles_m)                  # as the launcher clamps it
    G8 = G >> 3
    seen = set()
    for b in range(G):
        tile = (b & 7) * G8 + (b >> 3) if b < (G8 << 3) else b
        tn_count = G // tiles_m
        gid = tile // (group_m * tn_count)
        first_m = gid * group_m
        gsz = min(tiles_m - first_m, group_m)
        rem = tile - gid * group_m * tn_count
        tm, tn = first_m + rem % gsz, rem // gsz
        assert 0 <= tm < tiles_m and 0 <= tn < tiles_n
        seen.add((tm, tn))
    assert len(seen) == G


@pytest.mark.parametrize("groups_m,cols,KC,D", [(2, 64, 224, 4), (3, 4, 130, 3), (1, 7, 448, 2), (5, 13, 192, 3)])
def test_group_split_k_covers_every_tile_segment_and_pair(groups_m, cols, KC, D):
    """prefill_group_kernel at K > 8192: block b -> (segment, tile) after the XCD remap visits every
    (segment, tile) once, and the segments' pair ranges [pair0, pair0 + npair) tile [0, KC/2) with
    at least D pairs each (the ring's prologue issues D pairs), so every load stays in the weights."""
    L = KC if KC <= 128 else 2 * -(-KC // (2 * -(-KC // 64)))
    splits = -(-KC // L)
    seg_pairs = L // 2
    tiles = groups_m * cols
    G = tiles * splits
    G8 = G >> 3
    seen = set()
    for b in range(G):
        tile_raw = (b & 7) * G8 + (b >> 3) if b < (G8 << 3) else b
        seg, tile = tile_raw // tiles, tile_raw % tiles
        assert 0 <= seg < splits and 0 <= tile < tiles
        seen.add((seg, tile))
    assert len(seen) == G
    covered = []
    for seg in range(splits):
        pair0 = seg * seg_pairs
        npair = min(seg_pairs, KC // 2 - pair0)
        assert npair >= D
        covered += list(range(pair0, pair0 + npair))
    assert covered == list(range(KC // 2))


@pytest.mark.parametrize("cfg", sorted(WIDE_TILES))
def test_wide_prefill_offsets_at_the_largest_planned_k(cfg):
    """The per-lane 32-bit byte offsets of prefill_wide_kernel (weights: second block of a pair,
    x: rows below the tile's first row) computed without wrapping at the largest K the planner
    gives the config (prefill_wide_offsets_fit): every one is below 2^32 (weights below 2^31, as
    it is formed in int).  One 128-step larger K would wrap the x offset, so the bound is tight."""
    BM, BN, WMs, WNs = WIDE_TILES[cfg]
    NT = WMs * WNs * 64
    kmax = (2**32 - 128) // (2 * (BM - 1)) // 128 * 128
    for K in (kmax, kmax + 128):
        KC = K // 64
        M = BM + 5                                     # two M tiles: the first has BM rows below m0
        wmax = max(nbl * KC * 512 + (((r & 7) << 2) | (tp << 1) | kg) * 16
                   for nbl in (0, 1) for r in range(32) for tp in (0, 1) for kg in (0, 1))
        xmax = max(((min(0 + (sg >> 3), M - 1) - 0) * K + (sg & 7) * 8) * 2 + 16
                   for tid in range(NT) for i in range(BM * 8 // NT) for sg in [tid + i * NT])
        assert wmax < 2**31
        if K == kmax:
            assert xmax <= 2**32, (cfg, K, xmax)
        else:
            assert xmax > 2**32, (cfg, K, xmax)
