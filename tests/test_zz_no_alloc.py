"""GPU test of w4a16_launch_noalloc (include/w4a16.h): the allocation-free launch, called through
the C ABI, against the existing entry point w4a16_launch on the same plan.

Both are called through ctypes on torch's current stream; w4a16_launch gets a torch workspace and
a zeroed counter buffer, w4a16_launch_noalloc only the inputs and y.  Two calls in a row, the
second with a smaller input, must each equal w4a16_launch bit for bit (same kernels, same
reduction order) and the oracle within the reference tolerance.
"""
from __future__ import annotations

import ctypes
import os

import pytest

from tests._helpers import PKG, assert_close, gemm, make_problem, ref_gemm, torch_cuda
from tests.test_abi_host import Limits, Plan, Problem

pytestmark = pytest.mark.gpu

W4A16_ERR_WORKSPACE = 4


def _lib():
    import w4a16_opt  # noqa: F401  (loads libw4a16_hip.so through its rpath; ctypes gets the same copy)
    L = ctypes.CDLL(os.path.join(PKG, "libw4a16_hip.so"))
    L.w4a16_plan_create.argtypes = [ctypes.POINTER(Problem), ctypes.c_int, ctypes.POINTER(Limits),
                                    ctypes.POINTER(Plan), ctypes.c_char_p, ctypes.c_size_t]
    L.w4a16_query_device.argtypes = [ctypes.c_int, ctypes.POINTER(Limits)]
    L.w4a16_launch.argtypes = [ctypes.POINTER(Plan)] + [ctypes.c_void_p] * 7
    L.w4a16_launch_noalloc.argtypes = [ctypes.POINTER(Plan)] + [ctypes.c_void_p] * 5
    L.w4a16_last_error.restype = ctypes.c_char_p
    return L


def _plan(L, torch, Wp, x, scales, G):
    M, K = x.shape
    N = scales.shape[1]
    lim = Limits()
    assert L.w4a16_query_device(torch.cuda.current_device(), ctypes.byref(lim)) == 0
    prob = Problem(M, K, N, K // G, Wp.numel(), Wp.data_ptr(), x.data_ptr(), scales.data_ptr())
    plan = Plan()
    err = ctypes.create_string_buffer(512)
    rc = L.w4a16_plan_create(ctypes.byref(prob), -1, ctypes.byref(lim), ctypes.byref(plan), err, 512)
    assert rc == 0, err.value
    return plan


def _both(L, torch, Wp, x, scales, G):
    """(y from w4a16_launch_noalloc, y from w4a16_launch, plan)."""
    plan = _plan(L, torch, Wp, x, scales, G)
    st = torch.cuda.current_stream().cuda_stream
    M, N = x.shape[0], scales.shape[1]
    y_na = torch.empty(M, N, dtype=torch.half, device="cuda")
    rc = L.w4a16_launch_noalloc(ctypes.byref(plan), Wp.data_ptr(), x.data_ptr(), scales.data_ptr(),
                                y_na.data_ptr(), st)
    assert rc == 0, L.w4a16_last_error()
    y = torch.empty_like(y_na)
    ws = torch.empty(max(1, plan.workspace_bytes), dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(max(1, plan.counter_slots), dtype=torch.int32, device="cuda")
    rc = L.w4a16_launch(ctypes.byref(plan), Wp.data_ptr(), x.data_ptr(), scales.data_ptr(), y.data_ptr(),
                        ws.data_ptr(), cnt.data_ptr(), st)
    assert rc == 0, L.w4a16_last_error()
    torch.cuda.synchronize()
    return y_na, y, plan


def test_noalloc_matches_launch_two_calls():
    torch = torch_cuda()
    L = _lib()
    G = 128
    x, q, scales, Wp, key = make_problem(16, 256, 14336, G, seed=51)
    print("noalloc call 1: M=16 N=256 K=14336", flush=True)
    y_na, y, plan = _both(L, torch, Wp, x, scales, G)
    assert plan.kernel == 0 and plan.splits > 1 and plan.workspace_bytes > 0, (plan.splits, plan.workspace_bytes)
    assert torch.equal(y_na, y)
    assert_close(y_na, ref_gemm(x, q, scales, G, key))
    x2 = x[:5].contiguous()
    print("noalloc call 2: M=5 N=256 K=14336", flush=True)
    y2_na, y2, plan2 = _both(L, torch, Wp, x2, scales, G)
    assert plan2.splits > 1 and 0 < plan2.workspace_bytes < plan.workspace_bytes
    assert torch.equal(y2_na, y2)
    assert_close(y2_na, ref_gemm(x2, q, scales, G, key))
    assert torch.equal(y2_na, gemm(Wp, x2, scales))


def test_noalloc_long_k_prefill_split_by_segment():
    """A long-K prefill plan that runs one K segment per workgroup (fp32 partials and counters
    in the scratch), twice in a row, the second smaller: equal to w4a16_launch bit for bit."""
    torch = torch_cuda()
    L = _lib()
    G = 128
    x, q, scales, Wp, key = make_problem(48, 1024, 14336, G, seed=53)
    for m in (48, 20):
        print(f"noalloc prefill split: M={m} N=1024 K=14336", flush=True)
        xm = x[:m].contiguous()
        y_na, y, plan = _both(L, torch, Wp, xm, scales, G)
        assert plan.kernel >= 1 and plan.splits == 4 and plan.workspace_bytes == 4 * m * 1024 * 4, plan.splits
        assert torch.equal(y_na, y)
        assert torch.equal(y_na, gemm(Wp, xm, scales))
        assert_close(y_na, ref_gemm(xm, q, scales, G, key))


def test_noalloc_prefill_and_unsplit_decode():
    """Plans without a workspace run through the same entry point unchanged."""
    torch = torch_cuda()
    L = _lib()
    for M, N, K, G in ((40, 512, 2048, 64), (1, 4096, 4096, 128)):
        print(f"noalloc M={M} N={N} K={K} G={G}", flush=True)
        x, q, scales, Wp, key = make_problem(M, N, K, G, seed=52)
        y_na, y, plan = _both(L, torch, Wp, x, scales, G)
        assert plan.workspace_bytes == 0
        assert torch.equal(y_na, y)
        assert_close(y_na, ref_gemm(x, q, scales, G, key))


def test_noalloc_rejects_plans_beyond_the_scratch(monkeypatch):
    """A plan whose partials exceed the static scratch is refused before any launch."""
    torch = torch_cuda()
    L = _lib()
    monkeypatch.setenv("W4A16_DECODE", "4,4")           # register decode kernel, 4 K splits
    M, N, K, G = 16, 32768, 4096, 128
    lim = Limits()
    assert L.w4a16_query_device(torch.cuda.current_device(), ctypes.byref(lim)) == 0
    prob = Problem(M, K, N, K // G, N * K // 8, 0, 0, 0)
    plan = Plan()
    err = ctypes.create_string_buffer(512)
    assert L.w4a16_plan_create(ctypes.byref(prob), -1, ctypes.byref(lim), ctypes.byref(plan), err, 512) == 0
    assert plan.splits == 4 and plan.workspace_bytes == 4 * M * N * 4 > 4 << 20
    rc = L.w4a16_launch_noalloc(ctypes.byref(plan), 0, 0, 0, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == W4A16_ERR_WORKSPACE
    assert b"static scratch" in L.w4a16_last_error()


def test_noalloc_long_k_moderate_m_runs_scratch_free():
    """Long K at moderate M: the auto plan splits K over workgroups and its partials (8 and 16 MiB)
    exceed the static scratch; the entry point runs a scratch-free config of the same problem
    instead, bit for bit equal to w4a16_launch with a workspace, allocating nothing."""
    torch = torch_cuda()
    L = _lib()
    G = 128
    x, q, scales, Wp, key = make_problem(256, 4096, 14336, G, seed=54)
    # the first call on a device sets up (and has the runtime load the library's GPU code): the
    # allocation-free guarantee is for the calls after it
    warm = torch.empty(128, 4096, dtype=torch.half, device="cuda")
    assert L.w4a16_launch_noalloc(ctypes.byref(_plan(L, torch, Wp, x[:128].contiguous(), scales, G)), Wp.data_ptr(),
                                  x.data_ptr(), scales.data_ptr(), warm.data_ptr(),
                                  torch.cuda.current_stream().cuda_stream) == 0
    for m in (128, 256):
        print(f"noalloc long-K prefill beyond the scratch: M={m} N=4096 K=14336", flush=True)
        xm = x[:m].contiguous()
        plan = _plan(L, torch, Wp, xm, scales, G)
        assert plan.kernel >= 1 and plan.splits > 1 and plan.workspace_bytes > 4 << 20, (plan.kernel, plan.splits)
        y_na = torch.empty(m, 4096, dtype=torch.half, device="cuda")
        st = torch.cuda.current_stream().cuda_stream
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        rc = L.w4a16_launch_noalloc(ctypes.byref(plan), Wp.data_ptr(), xm.data_ptr(), scales.data_ptr(),
                                    y_na.data_ptr(), st)
        torch.cuda.synchronize()
        assert rc == 0, L.w4a16_last_error()
        assert torch.cuda.mem_get_info()[0] == free0
        y_na2, y, _ = _both(L, torch, Wp, xm, scales, G)
        assert torch.equal(y_na, y) and torch.equal(y_na2, y)
        assert torch.equal(y, gemm(Wp, xm, scales))
        assert_close(y_na, ref_gemm(xm, q, scales, G, key))


def test_noalloc_replayed_under_graph_capture():
    """After one eager call on the device, noalloc launches captured into a HIP graph (a split-K
    decode plan whose counters and partials sit in the static scratch, and a long-K prefill plan)
    replay correctly: three replays with eager work between them, each bit for bit equal to the
    eager result; an eager call allocates no device memory."""
    torch = torch_cuda()
    L = _lib()
    G = 128
    xd, qd, sd, Wd, keyd = make_problem(16, 256, 14336, G, seed=55)
    xp, qp, sp, Wpp, keyp = make_problem(40, 1024, 14336, G, seed=56)
    pd = _plan(L, torch, Wd, xd, sd, G)
    pp = _plan(L, torch, Wpp, xp, sp, G)
    assert pd.kernel == 0 and pd.splits > 1 and pp.kernel >= 1 and pp.splits > 1
    st = torch.cuda.current_stream().cuda_stream
    yd_e = torch.empty(16, 256, dtype=torch.half, device="cuda")
    yp_e = torch.empty(40, 1024, dtype=torch.half, device="cuda")
    print("noalloc eager calls before capture", flush=True)
    assert L.w4a16_launch_noalloc(ctypes.byref(pd), Wd.data_ptr(), xd.data_ptr(), sd.data_ptr(), yd_e.data_ptr(), st) == 0
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    assert L.w4a16_launch_noalloc(ctypes.byref(pp), Wpp.data_ptr(), xp.data_ptr(), sp.data_ptr(), yp_e.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    yd_g = torch.empty_like(yd_e)
    yp_g = torch.empty_like(yp_e)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    print("noalloc capture", flush=True)
    with torch.cuda.graph(g, stream=s):
        cs = torch.cuda.current_stream().cuda_stream
        assert L.w4a16_launch_noalloc(ctypes.byref(pd), Wd.data_ptr(), xd.data_ptr(), sd.data_ptr(), yd_g.data_ptr(), cs) == 0
        assert L.w4a16_launch_noalloc(ctypes.byref(pp), Wpp.data_ptr(), xp.data_ptr(), sp.data_ptr(), yp_g.data_ptr(), cs) == 0
    for r in range(3):
        print(f"noalloc replay {r}", flush=True)
        yd_g.zero_()
        yp_g.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yd_g, yd_e) and torch.equal(yp_g, yp_e), r
        # eager work between replays, through the same scratch
        assert L.w4a16_launch_noalloc(ctypes.byref(pd), Wd.data_ptr(), xd.data_ptr(), sd.data_ptr(),
                                      yd_e.data_ptr(), st) == 0
        torch.cuda.synchronize()
    assert_close(yd_e, ref_gemm(xd, qd, sd, G, keyd))
    assert_close(yp_e, ref_gemm(xp, qp, sp, G, keyp))
