"""GPU parity tests of the MI355X W4A16 op against the CPU oracle.

Mirrors the contract of the reference suite (tests/test_w4a16.py, every test function, same
parametrisations and tolerances) plus the BASELINE configurations.  The op is called through
the PyTorch binding, which calls the C ABI of libw4a16_hip.so.  The expected values come from
the oracle (oracle/quant.py: numpy restatement of tests/quant.py), computed on the host.

    python -u -m pytest tests -m gpu -x -v --timeout 120 --timeout-method thread
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import quant
from tests._helpers import (PKG, assert_close, dequant_f32, ext_module_path, gemm, make_problem,
                            ref_gemm, torch_cuda)

pytestmark = pytest.mark.gpu

GS = [64, 128]
DECODE_SHAPES = [
    (64, 512), (128, 1024), (256, 2048), (512, 4096),
    (4096, 4096), (6144, 4096), (4096, 14336), (28672, 4096),
]
DECODE_BATCHES = [1, 2, 3, 7, 8, 9, 15, 16]
PREFILL_VARIANTS = [1, 2, 3, 4]
PREFILL_M = [17, 31, 32, 33, 63, 64, 65, 100, 127, 128, 129, 300, 512, 1000]
RAGGED = [(16, 64), (48, 192), (80, 640), (208, 384), (272, 1152)]


def test_extension_is_in_tree_hip_build():
    """The op must be the in-tree HIP build (no silent fallback)."""
    torch_cuda()
    import os
    path = ext_module_path()
    assert os.path.dirname(path) == os.path.realpath(PKG), path
    import w4a16_opt
    info = w4a16_opt.plan_info(1, 4096, 4096, 128)
    assert info["gcn_arch"] == 950, info


# ------------------------------------------------------------------ reference contract mirror

@pytest.mark.parametrize("G", GS)
@pytest.mark.parametrize("M", DECODE_BATCHES)
@pytest.mark.parametrize("N,K", DECODE_SHAPES[:4])
def test_shapes(M, N, K, G):
    x, q, scales, Wp, key = make_problem(M, N, K, G)
    assert_close(gemm(Wp, x, scales), ref_gemm(x, q, scales, G, key))


@pytest.mark.parametrize("G", [128])
@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("N,K", DECODE_SHAPES[4:])
def test_llama3_8b_shapes(M, N, K, G):
    x, q, scales, Wp, key = make_problem(M, N, K, G)
    assert_close(gemm(Wp, x, scales), ref_gemm(x, q, scales, G, key))


@pytest.mark.parametrize("G", GS)
@pytest.mark.parametrize("M", PREFILL_M)
@pytest.mark.parametrize("N,K", DECODE_SHAPES[:4])
def test_prefill_auto(M, N, K, G):
    x, q, scales, Wp, key = make_problem(M, N, K, G)
    assert_close(gemm(Wp, x, scales), ref_gemm(x, q, scales, G, key))


@pytest.mark.parametrize("G", GS)
@pytest.mark.parametrize("M", [1, 3, 16, 17, 70, 200])
@pytest.mark.parametrize("N,K", RAGGED)
def test_ragged_shapes_auto(M, N, K, G):
    if K % G:
        pytest.skip("K must be a multiple of the group size")
    x, q, scales, Wp, key = make_problem(M, N, K, G)
    assert_close(gemm(Wp, x, scales), ref_gemm(x, q, scales, G, key))


@pytest.mark.parametrize("variant", PREFILL_VARIANTS)
@pytest.mark.parametrize("G", GS)
@pytest.mark.parametrize("M", [1, 7, 16, 17, 33, 129])
@pytest.mark.parametrize("N,K", [(64, 512), (208, 384), (512, 4096)])
def test_forced_prefill_variants(variant, M, N, K, G):
    if K % G:
        pytest.skip("K must be a multiple of the group size")
    x, q, scales, Wp, key = make_problem(M, N, K, G)
    assert_close(gemm(Wp, x, scales, variant=variant), ref_gemm(x, q, scales, G, key))


@pytest.mark.parametrize("G", GS)
def test_prefill_variants_bitwise_equal(G):
    """Every prefill config accumulates K in the same order -> identical bits."""
    torch = torch_cuda()
    x, q, scales, Wp, key = make_problem(200, 384, 2048, G, seed=5)
    ys = [gemm(Wp, x, scales, variant=v) for v in PREFILL_VARIANTS]
    for y in ys[1:]:
        assert torch.equal(ys[0], y)
    assert_close(ys[0], ref_gemm(x, q, scales, G, key))


@pytest.mark.parametrize("G", GS)
def test_prefill_rows_independent_of_batch(G):
    torch = torch_cuda()
    x, q, scales, Wp, key = make_problem(150, 256, 1024, G, seed=9)
    full = gemm(Wp, x, scales)
    for m in (17, 40, 64, 99):
        assert torch.equal(gemm(Wp, x[:m].contiguous(), scales), full[:m])


@pytest.mark.parametrize("G", [128])
@pytest.mark.parametrize("M", [17, 128, 1024])
@pytest.mark.parametrize("N,K", DECODE_SHAPES[4:7])
def test_llama3_8b_prefill_shapes(M, N, K, G):
    x, q, scales, Wp, key = make_problem(M, N, K, G)
    assert_close(gemm(Wp, x, scales), ref_gemm(x, q, scales, G, key))


def test_decode_variant_matches_prefill():
    x, q, scales, Wp, key = make_problem(8, 1024, 2048, 128)
    ref = ref_gemm(x, q, scales, 128, key)
    assert_close(gemm(Wp, x, scales, variant=0), ref)
    assert_close(gemm(Wp, x, scales, variant=3), ref)


def test_decode_variant_rejects_unsupported_shapes():
    x, q, scales, Wp, key = make_problem(32, 64, 512, 64)
    with pytest.raises(RuntimeError, match="decode kernel needs"):
        gemm(Wp, x, scales, variant=0)
    x, q, scales, Wp, key = make_problem(4, 80, 640, 64)
    with pytest.raises(RuntimeError, match="decode kernel needs"):
        gemm(Wp, x, scales, variant=0)


@pytest.mark.parametrize("G", GS)
@pytest.mark.parametrize("scale_mode", ["tiny", "large", "mixed"])
def test_hard_scale_and_activation_ranges(G, scale_mode):
    M, N, K = 16, 256, 2048
    x, q, scales, Wp, key = make_problem(M, N, K, G, seed=23)
    if scale_mode == "tiny":
        scales.fill_(2.0 ** -14)
        x.mul_(128)
    elif scale_mode == "large":
        scales.fill_(16.0)
        x.mul_(8)
    else:
        scales[:, ::2] = 2.0 ** -10
        scales[:, 1::2] = 8.0
        x[::2].mul_(0.125)
        x[1::2].mul_(8)
    ref = ref_gemm(x, q, scales, G)
    for v in [-1, 0] + PREFILL_VARIANTS:
        assert_close(gemm(Wp, x, scales, variant=v), ref, tol=4e-3)


@pytest.mark.parametrize("G", GS)
def test_onehot_k_mapping(G):
    """x = e_k -> y equals column k of the dequantised W exactly (reference :221-236)."""
    torch = torch_cuda()
    N, K = 128, 1024
    _, q, scales, Wp, key = make_problem(1, N, K, G)
    Wd = quant.dequantize_w4(q, scales.cpu().numpy(), G)
    ks = [0, 1, 2, 7, 8, 15, 16, 17, 63, 64, 65, 127, 128, 255, 256, 511, 512, 513, 1022, 1023]
    for i in range(0, len(ks), 16):
        chunk = ks[i:i + 16]
        x = torch.zeros(len(chunk), K, dtype=torch.half, device="cuda")
        for m, k in enumerate(chunk):
            x[m, k] = 1
        want = np.ascontiguousarray(Wd[:, chunk].T)
        for v in [-1, 0] + PREFILL_VARIANTS:
            y = gemm(Wp, x, scales, variant=v).cpu().numpy()
            assert np.array_equal(y.view(np.uint16), want.view(np.uint16)), \
                f"k-mapping wrong for k in {chunk}, variant {v}"


@pytest.mark.parametrize("fill", ["zeros", "fifteens", "random"])
def test_nibble_extremes(fill):
    torch = torch_cuda()
    M, N, K, G = 4, 128, 1024, 64
    rng = np.random.default_rng(1)
    q = {"zeros": np.zeros((N, K), np.uint8),
         "fifteens": np.full((N, K), 15, np.uint8),
         "random": rng.integers(0, 16, (N, K), dtype=np.uint8)}[fill]
    scales = (rng.random((K // G, N)) * 0.05 + 0.001).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float16)
    Wp = torch.from_numpy(quant.pack_int4(q)).cuda()
    xt, st = torch.from_numpy(x).cuda(), torch.from_numpy(scales).cuda()
    for v in [-1, 0] + PREFILL_VARIANTS:
        assert_close(gemm(Wp, xt, st, variant=v), quant.ref_gemm(x, q, scales, G))


def test_zero_input():
    torch = torch_cuda()
    x, q, scales, Wp, key = make_problem(5, 128, 1024, 64)
    for v in [-1, 0] + PREFILL_VARIANTS:
        assert not gemm(Wp, torch.zeros_like(x), scales, variant=v).any()


def test_deterministic():
    torch = torch_cuda()
    x, q, scales, Wp, key = make_problem(8, 1024, 2048, 128)
    assert torch.equal(gemm(Wp, x, scales), gemm(Wp, x, scales))
    for v in PREFILL_VARIANTS:
        assert torch.equal(gemm(Wp, x, scales, variant=v), gemm(Wp, x, scales, variant=v))


@pytest.mark.parametrize("M", [1, 12, 40, 300])
def test_cuda_graph_capture(M):
    """Graph capture and replay (reference :264-278), replayed several times with eager work and
    synchronisation between replays; every replay is checked."""
    torch = torch_cuda()
    x, q, scales, Wp, key = make_problem(M, 512, 1024, 128)
    gemm(Wp, x, scales)                                   # warm up (creates decode counters)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = gemm(Wp, x, scales)
    for rep in range(3):
        x2 = torch.randn(x.shape, device="cuda").half()
        x.copy_(x2)
        g.replay()
        torch.cuda.synchronize()
        assert_close(y, ref_gemm(x2, q, scales, 128, key))
        eager = gemm(Wp, x2, scales)
        torch.cuda.synchronize()
        assert torch.equal(eager, y), f"replay {rep} differs from the eager result"


def test_rejects_bad_inputs():
    torch = torch_cuda()

    def args(**kw):
        p = dict(M=2, N=64, K=512, G=64)
        p.update(kw)
        x, q, s, Wp, key = make_problem(p["M"], p["N"], p["K"], p["G"])
        return Wp, x, s

    Wp, x, s = args()
    with pytest.raises(RuntimeError, match="fp16"):
        gemm(Wp, x.float(), s)
    with pytest.raises(RuntimeError, match="int32"):
        gemm(Wp.to(torch.int64), x, s)
    with pytest.raises(RuntimeError, match="CUDA"):
        gemm(Wp.cpu(), x.cpu(), s.cpu())
    with pytest.raises(RuntimeError, match="contiguous"):
        gemm(Wp, torch.empty(512, 2, dtype=torch.half, device="cuda").t(), s)
    with pytest.raises(RuntimeError, match="variant"):
        gemm(Wp, x, s, variant=7)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        gemm(Wp[: 64 * 32 // 8], torch.zeros(2, 32, dtype=torch.half, device="cuda"), s[:1, :64].contiguous())
    with pytest.raises(RuntimeError, match="multiple of 16"):
        gemm(Wp[: 24 * 512 // 8], x, s[:, :24].contiguous())
    with pytest.raises(RuntimeError, match="unsupported group size"):
        gemm(*args(G=32))
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        gemm(Wp, torch.zeros(2 * 512 + 1, dtype=torch.half, device="cuda")[1:].view(2, 512), s)
    with pytest.raises(RuntimeError, match="N\\*K/8"):
        gemm(Wp[:-4], x, s)


# ----------------------------------------------------------------- beyond the reference suite

@pytest.mark.parametrize("G", GS)
def test_onehot_every_k(G):
    """Exhaustive k mapping on a small shape: e_k for every k, all kernels, bit-exact."""
    torch = torch_cuda()
    N, K = 64, 512
    _, q, scales, Wp, key = make_problem(1, N, K, G, seed=3)
    Wd = quant.dequantize_w4(q, scales.cpu().numpy(), G)
    for k0 in range(0, K, 16):
        x = torch.zeros(16, K, dtype=torch.half, device="cuda")
        x[torch.arange(16), torch.arange(k0, k0 + 16)] = 1
        want = np.ascontiguousarray(Wd[:, k0:k0 + 16].T)
        for v in [0] + PREFILL_VARIANTS:
            y = gemm(Wp, x, scales, variant=v).cpu().numpy()
            assert np.array_equal(y.view(np.uint16), want.view(np.uint16)), (k0, v)


def test_subnormal_scales_bit_exact():
    """fp16 subnormal products must not be flushed: one-hot columns with scales 2^-20..2^-15."""
    torch = torch_cuda()
    N, K, G = 128, 512, 64
    rng = np.random.default_rng(7)
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    scales = (2.0 ** rng.integers(-24, -14, (K // G, N))).astype(np.float16)
    Wd = quant.dequantize_w4(q, scales, G)
    assert (np.abs(Wd.astype(np.float32)) < 2.0 ** -14).any()
    Wp = torch.from_numpy(quant.pack_int4(q)).cuda()
    st = torch.from_numpy(scales).cuda()
    for k0 in (0, 37, 255, 496):
        x = torch.zeros(16, K, dtype=torch.half, device="cuda")
        x[torch.arange(16), torch.arange(k0, k0 + 16)] = 1
        want = np.ascontiguousarray(Wd[:, k0:k0 + 16].T)
        for v in [0] + PREFILL_VARIANTS:
            y = gemm(Wp, x, st, variant=v).cpu().numpy()
            assert np.array_equal(y.view(np.uint16), want.view(np.uint16)), (k0, v)


def _baseline_problem(M, N, K, G, seed, ragged=False):
    torch = torch_cuda()
    if ragged:
        q, scales = quant.gen_codes_scales(N, K, G, seed, 1e-4, 0.05)
        rng = np.random.default_rng([seed, 2])
        xf = rng.standard_normal((M, K)) * 2.0
        mask = rng.random((M, K)) < 0.01
        xf[mask] = np.where(rng.random(mask.sum()) < 0.5, -60.0, 60.0)
        x = xf.astype(np.float16)
    else:
        q, scales = quant.gen_codes_scales(N, K, G, seed)
        x = np.random.default_rng([seed, 2]).standard_normal((M, K)).astype(np.float16)
    Wp = quant.pack_int4(q)
    return (torch.from_numpy(x).cuda(), torch.from_numpy(scales).cuda(), torch.from_numpy(Wp).cuda(),
            x, q, scales)


BASELINE_SPECS = {"c1": (1, 4096, 4096, 128), "c3": (128, 14336, 4096, 64)}
BASELINE_SPECS.update({f"c2_gate_up_{m}": (m, 14336, 4096, 128) for m in (1, 4, 8, 16)})
BASELINE_SPECS.update({f"c2_down_{m}": (m, 4096, 14336, 128) for m in (1, 4, 8, 16)})


@pytest.mark.parametrize("cfg", sorted(BASELINE_SPECS))
def test_baseline_configs(cfg):
    """BASELINE.json configs 1-3 (all eight configs[1] cases) with their stated distributions,
    through the auto planner, against the oracle; configs[2]: the auto result and every forced
    variant bitwise equal."""
    torch = torch_cuda()
    import w4a16_opt
    M, N, K, G = BASELINE_SPECS[cfg]
    print(f"{cfg}: M={M} N={N} K={K} G={G} -> {w4a16_opt.plan_info(M, N, K, G)['kernel_name']}", flush=True)
    xt, st, Wt, x, q, scales = _baseline_problem(M, N, K, G, seed=11)
    ref = quant.ref_gemm(x, q, scales, G)
    y = gemm(Wt, xt, st)
    assert_close(y, ref)
    if cfg == "c3":
        for v in PREFILL_VARIANTS:
            assert torch.equal(gemm(Wt, xt, st, variant=v), y), v


def test_baseline_c4_prefill_full_size():
    """BASELINE configs[3] at full size (M=2048, K=8192, N=28672, G=128) through the auto planner:
    the oracle on the first and last 512 channels of all 2048 rows, bitwise equality with forced
    variant 4 over the whole output, and rows independent of the batch size (1000-row prefix)."""
    torch = torch_cuda()
    import w4a16_opt
    M, N, K, G = 2048, 28672, 8192, 128
    info = w4a16_opt.plan_info(M, N, K, G)
    print(f"configs[3]: {info['kernel_name']} grid={info['grid']}", flush=True)
    assert "prefill_wide_kernel" in info["kernel_name"], info
    xt, st, Wt, x, q, scales = _baseline_problem(M, N, K, G, seed=17)
    y = gemm(Wt, xt, st)
    for lo, hi in ((0, 512), (N - 512, N)):
        assert_close(y[:, lo:hi], quant.ref_gemm(x, q[lo:hi], np.ascontiguousarray(scales[:, lo:hi]), G))
    assert torch.equal(y, gemm(Wt, xt, st, variant=4))
    assert torch.equal(gemm(Wt, xt[:1000].contiguous(), st), y[:1000])


def test_golden_small_problem():
    """The committed fixture tests/golden/small_problem.npz (M=5, N=64, K=512, G=64): the op on its
    inputs against its oracle output, through decode and every forced prefill variant (bitwise
    equal to each other)."""
    torch = torch_cuda()
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "small_problem.npz"))
    Wp, x, s = (torch.from_numpy(np.ascontiguousarray(d[k])).cuda() for k in ("Wp", "x", "scales"))
    assert_close(gemm(Wp, x, s, variant=0), d["y_ref"])
    ys = [gemm(Wp, x, s, variant=v) for v in PREFILL_VARIANTS]
    for y in ys:
        assert torch.equal(y, ys[0])
    assert_close(ys[0], d["y_ref"])


@pytest.mark.parametrize("M", [16, 40])
def test_decode_split_k_concurrent_streams(M):
    """Split-K calls (decode at M = 16, the long-K prefill segments at M = 40) enqueued
    alternately on two streams (overlapping in time) give the single-stream results bit for bit:
    each stream has its own counter buffer."""
    torch = torch_cuda()
    import w4a16_opt
    N, K, G = 256, 14336, 128
    info = w4a16_opt.plan_info(M, N, K, G)
    assert info["splits"] > 1, info
    _, q, scales, Wp, key = make_problem(M, N, K, G, seed=41)
    gen = torch.Generator(device="cuda").manual_seed(41)
    xs = [torch.randn(M, K, device="cuda", generator=gen).half() for _ in range(8)]
    want = [gemm(Wp, x, scales) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(4):
        got = [None] * len(xs)
        for i, x in enumerate(xs):
            with torch.cuda.stream(streams[i % 2]):
                got[i] = gemm(Wp, x, scales)
        torch.cuda.synchronize()
        for i in range(len(xs)):
            assert torch.equal(got[i], want[i]), (rep, i)
    assert_close(want[0], ref_gemm(xs[0], q, scales, G, key))


@pytest.mark.parametrize("M", [12, 33])
def test_cuda_graph_capture_split_k(M):
    """Graph capture of a split-K plan (decode at M = 12, long-K prefill segments at M = 33):
    every replay (with eager split-K calls between them) equals the eager result."""
    torch = torch_cuda()
    import w4a16_opt
    N, K, G = 256, 14336, 128
    assert w4a16_opt.plan_info(M, N, K, G)["splits"] > 1
    x, q, scales, Wp, key = make_problem(M, N, K, G, seed=43)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = gemm(Wp, x, scales)
    for rep in range(3):
        x.copy_(torch.randn(x.shape, device="cuda").half())
        g.replay()
        torch.cuda.synchronize()
        eager = gemm(Wp, x, scales)
        torch.cuda.synchronize()
        assert torch.equal(eager, y), f"replay {rep} differs from the eager result"
    assert_close(y, ref_gemm(x, q, scales, G, key))


@pytest.mark.parametrize("M", [12, 33])
def test_graph_capture_without_warm_up_call(M):
    """Capture with no capture pool on the device (as in a process whose first call is captured):
    the captured split-K call zeroes counters of its own with a fill kernel recorded in the graph.
    Three replays, with eager split-K calls (which recreate the pool) between them, each equal to
    the eager result."""
    torch = torch_cuda()
    import w4a16_opt
    N, K, G = 256, 14336, 128
    assert w4a16_opt.plan_info(M, N, K, G)["splits"] > 1
    x, q, scales, Wp, key = make_problem(M, N, K, G, seed=47)
    torch.cuda.synchronize()
    w4a16_opt._debug_drop_capture_pool(torch.cuda.current_device())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = gemm(Wp, x, scales)
    for rep in range(3):
        x.copy_(torch.randn(x.shape, device="cuda").half())
        g.replay()
        torch.cuda.synchronize()
        eager = gemm(Wp, x, scales)
        torch.cuda.synchronize()
        assert torch.equal(eager, y), f"replay {rep} differs from the eager result"
    assert_close(y, ref_gemm(x, q, scales, G, key))


@pytest.mark.parametrize("G", [64])
def test_baseline_c5_ragged_rows_independent(G):
    """Config 5: N=4112 (N%64 != 0), K=4160, 65 groups, outliers; rows independent of M."""
    torch = torch_cuda()
    N, K = 4112, 4160
    xt, st, Wt, x, q, scales = _baseline_problem(513, N, K, G, seed=13, ragged=True)
    full = gemm(Wt, xt, st)
    assert_close(full, quant.ref_gemm(x, q, scales, G))
    for m in (1, 17, 37, 100):
        assert torch.equal(gemm(Wt, xt[:m].contiguous(), st), full[:m]), m


def test_decode_split_consistency_large_k():
    """Decode at K=14336 (many K slabs) vs prefill on the same inputs: both within tolerance."""
    x, q, scales, Wp, key = make_problem(16, 4096, 14336, 128, seed=4)
    ref = ref_gemm(x, q, scales, 128, key)
    assert_close(gemm(Wp, x, scales, variant=0), ref)
    assert_close(gemm(Wp, x, scales, variant=2), ref)


# Every decode kernel shape of the planner's table, forced through W4A16_DECODE="v,splits"
# (read by the planner on each call), on shapes whose K range divides evenly.
# (variant, splits, N, K, G): register kernels (kind 0, ids 0-7), streaming rings (kind 2, ids 8-15),
# refill-ahead rings (kind 3, ids 16-31), both group sizes (one or two groups per chunk pair).
DECODE_FORCED_G = [
    (0, 1, 256, 4096, 128), (1, 2, 256, 4096, 128), (2, 1, 256, 4096, 128), (3, 4, 256, 4096, 128),
    (4, 2, 256, 4096, 128), (5, 1, 256, 4096, 128), (6, 8, 256, 4096, 128), (7, 1, 256, 4096, 128),
    (6, 4, 256, 14336, 128), (0, 14, 256, 14336, 128), (8, 1, 256, 4096, 128), (9, 1, 256, 4096, 128),
    (10, 2, 256, 4096, 128), (11, 1, 256, 4096, 128), (12, 4, 256, 4096, 128), (13, 1, 256, 4096, 128),
    (14, 1, 256, 4096, 128), (15, 2, 256, 4096, 128), (12, 2, 256, 14336, 128), (8, 7, 256, 14336, 128),
    (16, 1, 256, 4096, 128), (17, 2, 256, 4096, 128), (18, 1, 256, 4096, 128), (19, 1, 256, 4096, 128),
    (20, 1, 256, 4096, 128), (21, 1, 256, 4096, 128), (22, 2, 256, 4096, 128), (16, 7, 256, 14336, 128),
    (19, 1, 256, 14336, 128), (20, 2, 256, 14336, 128), (21, 7, 256, 14336, 128), (16, 1, 256, 4096, 64),
    (19, 2, 256, 4096, 64), (18, 1, 512, 2048, 64), (22, 2, 256, 4096, 64), (20, 2, 256, 14336, 64),
    (26, 1, 256, 4096, 128), (28, 1, 256, 4096, 128), (28, 7, 256, 14336, 128), (26, 2, 256, 14336, 64),
    (28, 2, 256, 4096, 64),
]
# Ring shapes whose LDS ring holds fewer than 16 token rows: forced only up to their row limit
# (the planner refuses them above it).  (variant, splits, N, K, G, largest M)
DECODE_FORCED_SMALL_M = [
    (23, 1, 256, 4096, 128, 8), (23, 2, 256, 4096, 64, 8), (24, 1, 256, 4096, 128, 8),
    (24, 1, 256, 14336, 128, 8), (24, 1, 256, 4096, 64, 8), (25, 1, 256, 4096, 128, 8),
    (25, 2, 256, 14336, 128, 8), (25, 1, 256, 4096, 64, 8), (27, 1, 256, 14336, 128, 1),
    (27, 1, 512, 14336, 64, 1), (29, 1, 256, 4096, 128, 8), (29, 2, 256, 14336, 128, 8),
    (30, 1, 256, 14336, 128, 4), (30, 1, 512, 14336, 64, 4), (31, 1, 256, 4096, 128, 8),
    (31, 2, 256, 14336, 64, 8),
]


@pytest.mark.parametrize("v,splits,N,K,G", DECODE_FORCED_G)
def test_decode_shapes_forced(v, splits, N, K, G, monkeypatch):
    torch = torch_cuda()
    import w4a16_opt
    monkeypatch.setenv("W4A16_DECODE", f"{v},{splits}")
    info = w4a16_opt.plan_info(16, N, K, G, 0)
    assert info["decode_variant"] == v and info["splits"] == splits, info
    x, q, scales, Wp, key = make_problem(16, N, K, G, seed=v + 31)
    Wd = dequant_f32(key)
    for M in (1, 2, 3, 5, 9, 16):
        xm = x[:M].contiguous()
        assert_close(gemm(Wp, xm, scales, variant=0), ref_gemm(xm, q, scales, G, key))
    _onehot_decode_check(Wp, scales, Wd, K, v, splits, 16)


@pytest.mark.parametrize("v,splits,N,K,G,mmax", DECODE_FORCED_SMALL_M)
def test_decode_shapes_forced_small_m(v, splits, N, K, G, mmax, monkeypatch):
    torch = torch_cuda()
    import w4a16_opt
    monkeypatch.setenv("W4A16_DECODE", f"{v},{splits}")
    info = w4a16_opt.plan_info(mmax, N, K, G, 0)
    assert info["decode_variant"] == v and info["splits"] == splits, info
    assert w4a16_opt.plan_info(mmax + 1, N, K, G, 0)["decode_variant"] != v    # does not fit: not planned
    x, q, scales, Wp, key = make_problem(mmax, N, K, G, seed=v + 37)
    for M in sorted({1, min(2, mmax), (mmax + 1) // 2, mmax}):
        xm = x[:M].contiguous()
        assert_close(gemm(Wp, xm, scales, variant=0), ref_gemm(xm, q, scales, G, key))
    _onehot_decode_check(Wp, scales, dequant_f32(key), K, v, splits, mmax)


def _onehot_decode_check(Wp, scales, Wd, K, v, splits, m):
    """x = e_k rows (m of them, spread over K): y must be the dequantised columns, bit-exact."""
    torch = torch_cuda()
    ks = list(range(0, K, K // m))[:m]
    xo = torch.zeros(m, K, dtype=torch.half, device="cuda")
    xo[torch.arange(m), torch.tensor(ks)] = 1
    y = gemm(Wp, xo, scales, variant=0).float().cpu().numpy()
    assert np.array_equal(y, Wd[:, ks].T), f"one-hot mismatch for decode shape {v} splits {splits}"
    assert torch.equal(gemm(Wp, xo, scales, variant=0), gemm(Wp, xo, scales, variant=0))


# Wide-tile prefill configs (5..7 and 18..24, chosen automatically for moderate and large
# problems; 22 is 18 software-pipelined) forced through W4A16_PREFILL:
# bit-identical to the reference-API variants and within the reference tolerance, including M and
# N tails (rows past M and blocks past N load clamped data and are not stored).
@pytest.mark.parametrize("cfg", [5, 6, 7, 18, 19, 20, 21, 22, 23, 24])
@pytest.mark.parametrize("M,N,K,G", [(2048, 4096, 4096, 128), (300, 1040, 2048, 64), (129, 272, 1024, 128),
                                     (17, 16, 256, 64)])
def test_prefill_wide_configs_bitwise_equal(cfg, M, N, K, G, monkeypatch):
    torch = torch_cuda()
    import w4a16_opt
    monkeypatch.setenv("W4A16_PREFILL", str(cfg))
    assert ("prefill_wide_pipe_kernel" if cfg == 22 else "prefill_wide_kernel") in w4a16_opt.plan_info(M, N, K, G)["kernel_name"]
    x, q, scales, Wp, key = make_problem(M, N, K, G, seed=cfg)
    y = gemm(Wp, x, scales)
    assert torch.equal(y, gemm(Wp, x, scales, variant=4))
    assert torch.equal(y, gemm(Wp, x, scales, variant=1))
    assert_close(y, ref_gemm(x, q, scales, G, key))
    assert torch.equal(gemm(Wp, x[:M // 2 + 1].contiguous(), scales), y[:M // 2 + 1])


# One-wave-per-block prefill (configs 8, 9: forced only since 16-token groups took over small M):
# bit-identical to the reference-API variants, rows past M not stored.
@pytest.mark.parametrize("cfg,M,N,K,G", [(8, 17, 4096, 4096, 128), (8, 32, 1040, 2048, 64), (8, 20, 16, 1024, 64),
                                         (9, 40, 512, 14336, 128), (9, 64, 272, 1024, 64), (9, 33, 256, 1024, 128)])
def test_prefill_stream_configs_bitwise_equal(cfg, M, N, K, G, monkeypatch):
    torch = torch_cuda()
    import w4a16_opt
    monkeypatch.setenv("W4A16_PREFILL", str(cfg))
    info = w4a16_opt.plan_info(M, N, K, G)
    assert info["kernel"] == cfg and "prefill_stream_kernel" in info["kernel_name"], info
    x, q, scales, Wp, key = make_problem(M, N, K, G, seed=M + cfg)
    y = gemm(Wp, x, scales)
    assert torch.equal(y, gemm(Wp, x, scales, variant=4))
    assert torch.equal(y, gemm(Wp, x, scales, variant=1))
    assert_close(y, ref_gemm(x, q, scales, G, key))


# Small-M prefill (M = 17..64, chosen automatically): token groups of 16 rows sharing x, one wave
# per n16 block over the whole K, bit-identical to the reference-API variants.
@pytest.mark.parametrize("M,N,K,G", [(17, 4096, 4096, 128), (32, 1040, 2048, 64), (33, 256, 1024, 128),
                                     (64, 272, 1024, 64), (20, 16, 1024, 64), (40, 512, 14336, 128)])
def test_prefill_small_m_bitwise_equal(M, N, K, G):
    torch = torch_cuda()
    import w4a16_opt
    name = w4a16_opt.plan_info(M, N, K, G)["kernel_name"]
    assert "prefill_stream_kernel" in name or "prefill_group_kernel" in name, name
    x, q, scales, Wp, key = make_problem(M, N, K, G, seed=M)
    y = gemm(Wp, x, scales)
    assert torch.equal(y, gemm(Wp, x, scales, variant=4))
    assert torch.equal(y, gemm(Wp, x, scales, variant=1))
    assert_close(y, ref_gemm(x, q, scales, G, key))
    for m in (17, M - 1):
        if 17 <= m < M:
            assert torch.equal(gemm(Wp, x[:m].contiguous(), scales), y[:m]), m


# Token-group prefill (configs 10..15, forced through W4A16_PREFILL): 4 waves, 1..4 n16 blocks each, share the x rows of
# a group of 32 or 64 tokens; any M, N tails (waves past N compute clamped data and store nothing).
@pytest.mark.parametrize("cfg", [10, 11, 12, 13, 14, 15, 16, 17])
@pytest.mark.parametrize("M,N,K,G", [(17, 4096, 4096, 128), (33, 1040, 2048, 64), (100, 272, 1024, 64),
                                     (300, 4112, 4224, 64), (1000, 512, 2048, 128), (64, 16, 1024, 128),
                                     (129, 6144, 4096, 128)])
def test_prefill_token_groups_bitwise_equal(monkeypatch, cfg, M, N, K, G):
    torch = torch_cuda()
    import w4a16_opt
    print(f"token-group prefill cfg={cfg} M={M} N={N} K={K} G={G}", flush=True)
    x, q, scales, Wp, key = make_problem(M, N, K, G, seed=M + cfg)
    ref4 = gemm(Wp, x, scales, variant=4)
    monkeypatch.setenv("W4A16_PREFILL", str(cfg))
    info = w4a16_opt.plan_info(M, N, K, G)
    assert info["kernel"] == cfg and "prefill_group_kernel" in info["kernel_name"], info
    y = gemm(Wp, x, scales)
    assert torch.equal(y, ref4)
    assert torch.equal(y, gemm(Wp, x, scales, variant=1))
    assert_close(y, ref_gemm(x, q, scales, G, key))
    m = max(17, M // 3)                                       # M <= 16 would route to decode
    if m < M:
        assert torch.equal(gemm(Wp, x[:m].contiguous(), scales), y[:m])


# The planner's occupancy table (resident workgroups per CU of each prefill config, which its
# selection rules and fit checks use) agrees with the compiled kernels on this device.
def test_planner_occupancy_matches_the_compiled_kernels():
    import ctypes
    import os
    torch_cuda()
    import w4a16_opt

    class Limits(ctypes.Structure):
        _fields_ = [("cu_count", ctypes.c_int32), ("lds_bytes_per_block", ctypes.c_int32),
                    ("max_threads_per_block", ctypes.c_int32), ("gcn_arch", ctypes.c_int32)]

    lib = ctypes.CDLL(os.path.join(PKG, "libw4a16_hip.so"))
    lib.w4a16_debug_kernel_occupancy.argtypes = [ctypes.c_int]
    lib.w4a16_debug_prefill_occupancy.argtypes = [ctypes.c_int, ctypes.POINTER(Limits)]
    info = w4a16_opt.plan_info(2048, 4096, 4096, 128)
    lim = Limits(info["cu_count"], info["lds_bytes_per_block"], 1024, info["gcn_arch"])
    got = {cfg: lib.w4a16_debug_kernel_occupancy(cfg) for cfg in range(1, 25)}
    planned = {cfg: lib.w4a16_debug_prefill_occupancy(cfg, ctypes.byref(lim)) for cfg in range(1, 25)}
    print("compiled occupancy:", got, flush=True)
    assert got == planned


# Long K (K > 8192) uses the canonical segmented accumulation order (w4a16_internal.h): the
# token-group and one-wave configs run one K segment per workgroup and add the fp32 partials in
# segment order, the others keep a second accumulator set.  Every config gives the same bits as
# the reference-API variants, rows are independent of M, and the result is within tolerance.
@pytest.mark.parametrize("M,N,K,G", [(32, 4096, 14336, 128), (100, 272, 8320, 64), (17, 512, 28672, 128),
                                     (300, 1040, 12288, 64)])
def test_long_k_segmented_order_bitwise_equal_across_configs(M, N, K, G, monkeypatch):
    torch = torch_cuda()
    import w4a16_opt
    x, q, scales, Wp, key = make_problem(M, N, K, G, seed=M + 7)
    want = gemm(Wp, x, scales, variant=4)
    assert_close(want, ref_gemm(x, q, scales, G, key))
    seen = []
    for cfg in range(1, 25):
        monkeypatch.setenv("W4A16_PREFILL", str(cfg))
        info = w4a16_opt.plan_info(M, N, K, G)
        if info["kernel"] != cfg:
            continue
        print(f"long K M={M} N={N} K={K} config {cfg} {info['kernel_name']} splits {info['splits']}", flush=True)
        seen.append(cfg)
        assert torch.equal(gemm(Wp, x, scales), want), cfg
    monkeypatch.delenv("W4A16_PREFILL")
    assert {10, 14, 17}.issubset(seen) and len(seen) >= 12, seen
    for v in (1, 2, 3):
        assert torch.equal(gemm(Wp, x, scales, variant=v), want), v
    assert torch.equal(gemm(Wp, x, scales), want)
    for m in sorted({17, M // 2 + 1, M - 1}):
        if 17 <= m < M:
            assert torch.equal(gemm(Wp, x[:m].contiguous(), scales), want[:m]), m
