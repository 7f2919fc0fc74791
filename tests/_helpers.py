"""Shared helpers for the GPU parity tests: problem makers, the oracle comparison, the op."""
from __future__ import annotations

import functools
import os

import numpy as np
import pytest

from oracle import quant

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "w4a16-gemm_amd")


def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")
    return torch


def gemm(*a, **kw):
    """The op under test: the in-tree HIP extension (no fallback: ImportError if not built)."""
    from w4a16_opt import w4a16_gemm
    return w4a16_gemm(*a, **kw)


def ext_module_path() -> str:
    import w4a16_opt
    return os.path.realpath(w4a16_opt.__file__)


@functools.lru_cache(maxsize=4)
def _host_problem(N, K, G, seed, w_std):
    rng = np.random.default_rng(seed)
    W = rng.standard_normal((N, K), dtype=np.float32) * np.float32(w_std)
    q, scales = quant.quantize_w4(W, G)
    Wp = quant.pack_int4(q)
    return q, scales, Wp, rng.bit_generator.state


@functools.lru_cache(maxsize=3)
def dequant_f32(key):
    """fp32 copy of the oracle's dequantised weights for a cached problem key."""
    q, scales, _, _ = _host_problem(*key)
    return quant.dequantize_w4(q, scales, key[2]).astype(np.float32)


def make_problem(M, N, K, G, seed=0, w_std=0.02):
    """Mirror of the reference's make_problem (tests/test_w4a16.py:33-38) on numpy's generator.

    Returns device tensors (x fp16, scales fp16, Wp int32), the host codes q and the problem key
    (for the cached dequantised weights).  W ~ N(0, w_std^2) is RTN-quantized by the oracle;
    x ~ N(0, 1) uses a generator seeded from (seed, M) so different M get different rows.
    """
    torch = torch_cuda()
    key = (N, K, G, seed, w_std)
    q, scales, Wp, _ = _host_problem(*key)
    xr = np.random.default_rng([seed, M, 1]).standard_normal((M, K), dtype=np.float32).astype(np.float16)
    x = torch.from_numpy(xr).cuda()
    return x, q, torch.from_numpy(scales.copy()).cuda(), torch.from_numpy(Wp.copy()).cuda(), key


def ref_gemm(x, q, scales, G, key=None):
    """Oracle fp32 reference of the op (oracle.quant.ref_gemm), on host, for device inputs."""
    xh = x.detach().cpu().numpy().astype(np.float16)
    if key is not None:
        Wd = dequant_f32(key)
    else:
        sh = scales.detach().cpu().numpy() if hasattr(scales, "detach") else scales
        qh = q.detach().cpu().numpy() if hasattr(q, "detach") else q
        Wd = quant.dequantize_w4(qh, sh, G).astype(np.float32)
    return xh.astype(np.float32) @ Wd.T


def assert_close(y, ref, tol=2e-3):
    """Reference contract (tests/test_w4a16.py:41-44): finite and max|y-ref|/max|ref| < tol."""
    yh = y.detach().float().cpu().numpy()
    assert np.isfinite(yh).all(), "NaN/Inf in output"
    denom = float(np.abs(ref).max())
    rel = float(np.abs(yh - ref).max()) / denom if denom > 0 else float(np.abs(yh).max())
    assert rel < tol, f"max-abs error / max|ref| = {rel:.3e} (tol {tol:.0e})"
