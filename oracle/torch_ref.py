"""The reference's CPU path restated with torch on the CPU, for the timed CPU baseline.

Test infrastructure: only ``bench.py``'s ``cpu_baseline`` legs run it (timed) and ``tests/``
check it.  It follows the reference's own torch code path, op for op:

* ``unpack_int4``   reference ``tests/quant.py:51-59``: int32 words -> uint8 codes [N, K];
* ``dequantize_w4`` reference ``tests/quant.py:77-80``: ``(q.half() - 8) * scales`` in fp16 (the
  subtraction is exact, the multiply rounds once to nearest-even fp16);
* ``ref_gemm``      reference ``tests/quant.py:83-85``: ``x.float() @ W.float().t()`` in fp32.

The word layout is the one ``oracle/quant.py`` pins (word index
``(((n/16)*(K/64) + k/64)*32 + lane)*4 + s``, nibble ``a + 2b + 4h`` of the word holding
``n = 16 nb + 8 a + g``, ``k = 64 kc + 16 s + 8 b + 2 t + h``, lane ``4 g + t``); ``tests/test_oracle.py``
checks these functions against that numpy restatement bit for bit.
"""
from __future__ import annotations


def unpack_int4(torch, Wp, N: int, K: int):
    """int32 [N*K/8] (CPU tensor) -> uint8 [N, K] codes (reference ``tests/quant.py:51-59``)."""
    NB, KC = N // 16, K // 64
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)                      # nibble i = a + 2 b + 4 h
    w = Wp.view(NB, KC, 8, 4, 4, 1)                                          # nb, kc, g, t, s, (i)
    nib = ((w >> shifts) & 0xF).to(torch.uint8)                              # nb, kc, g, t, s, i
    nib = nib.view(NB, KC, 8, 4, 4, 2, 2, 2)                                 # ..., h, b, a
    # -> nb, a, g, kc, s, b, t, h  (n = 16 nb + 8 a + g, k = 64 kc + 16 s + 8 b + 2 t + h)
    return nib.permute(0, 7, 2, 1, 4, 6, 3, 5).reshape(N, K)


def dequantize_w4(torch, q, scales, G: int):
    """fp16 [N, K] = fp16((q - 8) * s) (reference ``tests/quant.py:77-80``)."""
    s = scales.repeat_interleave(G, dim=0).t()                               # [N, K] fp16
    return (q.half() - 8) * s


def ref_gemm(torch, x, W):
    """fp32 ``x.float() @ W.float().t()`` (reference ``tests/quant.py:83-85``)."""
    return x.float() @ W.float().t()
