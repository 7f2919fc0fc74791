"""ctypes loader for the C restatement in ``oracle/w4a16_oracle.c`` (test infrastructure only).

Build with ``make -C oracle`` (``__graft_entry__.build()`` does this).  Used by the tests as a
second, independent restatement of the reference's format and dequantisation, and by
``bench.py`` as the timed CPU reference path (unpack + dequant + fp32 GEMM).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "libw4a16_oracle.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"C oracle not built: {LIB_PATH} missing (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        L.w4a16_oracle_h2f.argtypes = [ctypes.c_uint16]
        L.w4a16_oracle_h2f.restype = ctypes.c_float
        L.w4a16_oracle_f2h.argtypes = [ctypes.c_float]
        L.w4a16_oracle_f2h.restype = ctypes.c_uint16
        L.w4a16_oracle_pack.argtypes = [P, ctypes.c_int, ctypes.c_int, P]
        L.w4a16_oracle_unpack.argtypes = [P, ctypes.c_int, ctypes.c_int, P]
        L.w4a16_oracle_dequant.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
        L.w4a16_oracle_forward.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, P, P, ctypes.c_int]
        L.w4a16_oracle_max_threads.restype = ctypes.c_int
        L.w4a16_oracle_gemv.argtypes = [P, P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def pack_int4(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    N, K = q.shape
    out = np.empty(N * K // 8, dtype=np.int32)
    if lib().w4a16_oracle_pack(_p(q), N, K, _p(out)):
        raise ValueError("N must be a multiple of 16 and K of 64")
    return out


def unpack_int4(Wp: np.ndarray, N: int, K: int) -> np.ndarray:
    Wp = np.ascontiguousarray(Wp, dtype=np.int32)
    out = np.empty((N, K), dtype=np.uint8)
    if lib().w4a16_oracle_unpack(_p(Wp), N, K, _p(out)):
        raise ValueError("bad shape")
    return out


def dequant_packed(Wp: np.ndarray, scales: np.ndarray, N: int, K: int, G: int) -> np.ndarray:
    """fp16 [N, K] dequantised weights, decoded word by word like the kernel (common.cuh:45-55)."""
    Wp = np.ascontiguousarray(Wp, dtype=np.int32)
    s = np.ascontiguousarray(scales, dtype=np.float16)
    out = np.empty((N, K), dtype=np.float16)
    if lib().w4a16_oracle_dequant(_p(Wp), _p(s), N, K, G, _p(out)):
        raise ValueError("bad shape")
    return out


def forward(Wp: np.ndarray, x: np.ndarray, scales: np.ndarray, N: int, K: int, G: int,
            nthreads: int = 0):
    """Reference CPU path: returns (y32 fp32 [M, N], y16 fp16 [M, N])."""
    Wp = np.ascontiguousarray(Wp, dtype=np.int32)
    x = np.ascontiguousarray(x, dtype=np.float16)
    s = np.ascontiguousarray(scales, dtype=np.float16)
    M = x.shape[0]
    y32 = np.empty((M, N), dtype=np.float32)
    y16 = np.empty((M, N), dtype=np.float16)
    rc = lib().w4a16_oracle_forward(_p(Wp), _p(x), _p(s), M, N, K, G, _p(y32), _p(y16), int(nthreads))
    if rc:
        raise RuntimeError(f"w4a16_oracle_forward failed ({rc})")
    return y32, y16


def gemv(W: np.ndarray, A: np.ndarray, sW: np.ndarray, zW: np.ndarray, exact: bool = True) -> np.ndarray:
    """Baseline GEMV (reference src/baseline/kernel.cu:8-34): fp16 [N].

    W int32 [N, K/8]; A fp16 [K]; sW, zW fp16 [N].  exact=False sums in the reference's fp32 k
    order; exact=True rounds the exact sum once (the contract of the GPU kernel)."""
    W = np.ascontiguousarray(W, dtype=np.int32)
    A = np.ascontiguousarray(A, dtype=np.float16)
    sW = np.ascontiguousarray(sW, dtype=np.float16)
    zW = np.ascontiguousarray(zW, dtype=np.float16)
    N, K = W.shape[0], A.shape[0]
    if W.shape != (N, K // 8) or sW.shape != (N,) or zW.shape != (N,):
        raise ValueError("W must be [N, K/8], sW and zW [N]")
    out = np.empty(N, dtype=np.float16)
    rc = lib().w4a16_oracle_gemv(_p(W), _p(A), _p(sW), _p(zW), N, K, int(bool(exact)), _p(out))
    if rc:
        raise ValueError(f"w4a16_oracle_gemv failed ({rc}): K must be a multiple of 8 (and <= 2^20 when exact)")
    return out


def h2f(bits: int) -> float:
    return float(lib().w4a16_oracle_h2f(bits))


def f2h(v: float) -> int:
    return int(lib().w4a16_oracle_f2h(v))


def max_threads() -> int:
    return int(lib().w4a16_oracle_max_threads())
