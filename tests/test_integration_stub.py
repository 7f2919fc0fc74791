"""GPU test of the reference-side ctypes binding documented in INTEGRATION.md ("Option 2: ctypes
stub"): the code block is taken from INTEGRATION.md as written (only the library path is made
absolute) and run on two streams at once with split-K plans, and under graph capture; every
result must equal w4a16_opt's bit for bit (same plans, same kernels)."""
from __future__ import annotations

import os
import re

import pytest

from tests._helpers import PKG, ROOT, gemm, make_problem, torch_cuda

pytestmark = pytest.mark.gpu


def _stub():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = text[text.index("**Option 2: ctypes stub**"):]
    code = re.search(r"```python\n(.*?)```", sec, re.S).group(1)
    assert 'ctypes.CDLL("libw4a16_hip.so")' in code
    code = code.replace('ctypes.CDLL("libw4a16_hip.so")',
                        f'ctypes.CDLL({os.path.join(PKG, "libw4a16_hip.so")!r})')
    import w4a16_opt  # noqa: F401  (the same library copy, through the module's rpath)
    ns = {}
    exec(compile(code, "INTEGRATION.md:ctypes-stub", "exec"), ns)
    return ns


def test_documented_ctypes_stub_two_streams_split_k():
    torch = torch_cuda()
    import w4a16_opt
    stub = _stub()
    G = 128
    cases = [(16, 256, 14336), (40, 1024, 14336)]            # decode split-K, long-K prefill segments
    probs = []
    for i, (M, N, K) in enumerate(cases):
        assert w4a16_opt.plan_info(M, N, K, G)["splits"] > 1
        probs.append(make_problem(M, N, K, G, seed=61 + i))
    want = [gemm(Wp, x, s) for x, q, s, Wp, key in probs]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for rep in range(4):
        outs = {}
        for st, i in ((s1, 0), (s2, 1), (s1, 1), (s2, 0)):
            with torch.cuda.stream(st):
                x, q, s, Wp, key = probs[i]
                outs[(st, i)] = [stub["w4a16_gemm"](Wp, x, s) for _ in range(3)]
        torch.cuda.synchronize()
        for (st, i), ys in outs.items():
            for y in ys:
                assert torch.equal(y, want[i]), (rep, i)


def test_documented_ctypes_stub_under_graph_capture():
    torch = torch_cuda()
    stub = _stub()
    G = 128
    x, q, s, Wp, key = make_problem(12, 256, 14336, G, seed=63)
    want = gemm(Wp, x, s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = stub["w4a16_gemm"](Wp, x, s)
    for rep in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), rep
        assert torch.equal(stub["w4a16_gemm"](Wp, x, s), want)
