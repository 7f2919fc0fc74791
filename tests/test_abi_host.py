"""CPU tests of the C ABI (include/w4a16.h) of libw4a16_hip.so: exports, validation, routing,
planning.  Only pure host entry points are called (no device work), plus w4a16_launch with plans
it refuses before any HIP call, so these run without a GPU.

The validation order and messages mirror the reference op (src/vectorized/kernel.cu:219-249) and
the substrings its tests match (tests/test_w4a16.py:188-195, 281-305).
"""
from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "w4a16-gemm_amd", "libw4a16_hip.so")
HEADER = os.path.join(ROOT, "include", "w4a16.h")


class Problem(ctypes.Structure):
    _fields_ = [("M", ctypes.c_int64), ("K", ctypes.c_int64), ("N", ctypes.c_int64),
                ("groups", ctypes.c_int64), ("wp_words", ctypes.c_int64),
                ("Wp", ctypes.c_void_p), ("x", ctypes.c_void_p), ("scales", ctypes.c_void_p)]


class Limits(ctypes.Structure):
    _fields_ = [("cu_count", ctypes.c_int32), ("lds_bytes_per_block", ctypes.c_int32),
                ("max_threads_per_block", ctypes.c_int32), ("gcn_arch", ctypes.c_int32)]


class Plan(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("M", "N", "K", "G", "kernel", "splits", "slab_chunks", "tile_n",
                                              "grid", "block", "counter_slots", "decode_variant")] + \
               [("workspace_bytes", ctypes.c_uint64)]


MI355X = Limits(256, 160 * 1024, 1024, 950)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} not built (python w4a16-gemm_amd/build.py)")
    L = ctypes.CDLL(LIB)
    L.w4a16_plan_create.argtypes = [ctypes.POINTER(Problem), ctypes.c_int, ctypes.POINTER(Limits),
                                    ctypes.POINTER(Plan), ctypes.c_char_p, ctypes.c_size_t]
    L.w4a16_plan_create.restype = ctypes.c_int
    L.w4a16_max_counter_slots.restype = ctypes.c_int32
    L.w4a16_last_error.restype = ctypes.c_char_p
    return L


def plan(lib, M, N, K, G=None, variant=-1, groups=None, wp_words=None, ptrs=(0, 0, 0), limits=MI355X):
    if groups is None:
        groups = K // G if G else 1
    if wp_words is None:
        wp_words = N * K // 8
    p = Problem(M, K, N, groups, wp_words, *ptrs)
    out = Plan()
    err = ctypes.create_string_buffer(512)
    rc = lib.w4a16_plan_create(ctypes.byref(p), variant, ctypes.byref(limits), ctypes.byref(out), err, 512)
    return rc, out, err.value.decode()


def test_library_exports_every_declared_symbol(lib):
    text = open(HEADER).read()
    names = re.findall(r"^\s*(?:int|int32_t|const char\*|void)\s+(w4a16_\w+)\s*\(", text, re.M)
    assert len(names) >= 6, names
    for n in names:
        assert hasattr(lib, n), f"libw4a16_hip.so does not export {n}"
    assert lib.w4a16_abi_version() == 2


def test_wave_stamps_only_in_the_instrumented_library(lib):
    """The per-wave timestamps of wave_timeline.py live in libw4a16_hip_stamps.so (-DW4A16_WAVE_STAMPS);
    the product library carries none of them and both export the same C ABI."""
    assert not hasattr(lib, "w4a16_debug_wave_stamps")
    stamps = os.path.join(ROOT, "w4a16-gemm_amd", "libw4a16_hip_stamps.so")
    if not os.path.exists(stamps):
        pytest.skip("libw4a16_hip_stamps.so not built (w4a16-gemm_amd/build.py)")
    S = ctypes.CDLL(stamps)
    assert hasattr(S, "w4a16_debug_wave_stamps") and hasattr(S, "w4a16_debug_wave_stamps_clear")
    for n in re.findall(r"^\s*(?:int|int32_t|const char\*|void)\s+(w4a16_\w+)\s*\(", open(HEADER).read(), re.M):
        assert hasattr(S, n), n
    assert S.w4a16_abi_version() == lib.w4a16_abi_version()
    # argument checks, refused before any HIP call
    S.w4a16_debug_wave_stamps.argtypes = [ctypes.c_void_p, ctypes.c_int32]
    buf = (ctypes.c_uint32 * 8)()
    assert S.w4a16_debug_wave_stamps(buf, 0) == 1
    assert S.w4a16_debug_wave_stamps(buf, 8193) == 1
    assert S.w4a16_debug_wave_stamps(None, 1) == 1


def test_plan_struct_layout_matches_header(lib):
    text = open(HEADER).read()
    body = text[text.index("typedef struct w4a16_plan"):text.index("} w4a16_plan;")]
    fields = re.findall(r"(?:int32_t|uint64_t)\s+([\w, ]+);", body)
    flat = [f.strip() for grp in fields for f in grp.split(",")]
    assert flat == [f[0] for f in Plan._fields_]


@pytest.mark.parametrize("kw,msg", [
    (dict(M=2, N=64, K=512, G=64, variant=7), "variant"),
    (dict(M=2, N=64, K=512, G=64, variant=-2), "variant"),
    (dict(M=0, N=64, K=512, G=64), "M must be at least 1"),
    (dict(M=1 << 31, N=64, K=512, G=64), "dimensions must fit in int32"),
    (dict(M=2, N=64, K=32, G=32), "multiple of 64"),
    (dict(M=2, N=24, K=512, G=64), "multiple of 16"),
    (dict(M=2, N=64, K=512, groups=3), "divisible by the number of groups"),
    (dict(M=2, N=64, K=512, groups=0), "divisible by the number of groups"),
    (dict(M=2, N=64, K=512, G=64, wp_words=10), "N\\*K/8"),
    (dict(M=2, N=64, K=512, G=64, ptrs=(16, 8, 16)), "16-byte aligned"),
    (dict(M=2, N=64, K=512, G=32), "unsupported group size 32"),
    (dict(M=2, N=64, K=512, G=256), "unsupported group size 256"),
    (dict(M=32, N=64, K=512, G=64, variant=0), "decode kernel needs"),
    (dict(M=4, N=80, K=640, G=64, variant=0), "decode kernel needs"),
    (dict(M=4, N=64, K=576, G=64, variant=0), "decode kernel needs"),
])
def test_validation_messages(lib, kw, msg):
    rc, _, err = plan(lib, **kw)
    assert rc == 1, (kw, rc, err)
    assert re.search(msg, err), (kw, err)


def test_validation_order_follows_reference(lib):
    """kernel.cu checks variant, M, int32, K%64, N%16, groups, numel, alignment, G in this order."""
    assert "variant" in plan(lib, M=0, N=24, K=32, G=32, variant=9)[2]
    assert "M must" in plan(lib, M=0, N=24, K=32, G=32)[2]
    assert "multiple of 64" in plan(lib, M=1, N=24, K=32, G=32)[2]
    assert "multiple of 16" in plan(lib, M=1, N=24, K=512, G=32)[2]
    assert "groups" in plan(lib, M=1, N=32, K=512, groups=3, wp_words=1)[2]
    assert "N*K/8" in plan(lib, M=1, N=32, K=512, G=32, wp_words=1, ptrs=(1, 1, 1))[2]
    assert "aligned" in plan(lib, M=1, N=32, K=512, G=32, ptrs=(1, 1, 1))[2]
    assert "group size" in plan(lib, M=1, N=32, K=512, G=32)[2]


@pytest.mark.parametrize("M,N,K,kernel", [
    (1, 4096, 4096, 0), (16, 14336, 4096, 0), (16, 4096, 14336, 0),       # decode contract
    (17, 4096, 4096, None), (1, 4112, 4160, None), (4, 80, 640, None),     # prefill
    (3, 48, 192, None), (128, 14336, 4096, None), (2048, 28672, 8192, None),
])
def test_routing(lib, M, N, K, kernel):
    rc, p, err = plan(lib, M=M, N=N, K=K, G=64)
    assert rc == 0, err
    if kernel == 0:
        assert p.kernel == 0
    else:
        assert 1 <= p.kernel <= 24


@pytest.mark.parametrize("v", [1, 2, 3, 4])
def test_forced_prefill_variant_is_used(lib, v):
    rc, p, err = plan(lib, M=3, N=64, K=512, G=64, variant=v)
    assert rc == 0 and p.kernel == v


@pytest.mark.parametrize("M", [1, 4, 8, 16])
@pytest.mark.parametrize("N,K", [(64, 512), (4096, 4096), (14336, 4096), (4096, 14336), (28672, 4096),
                                 (6144, 4096), (1024, 2048), (512, 4096), (4096, 11264)])
def test_decode_plan_invariants(lib, M, N, K):
    rc, p, err = plan(lib, M=M, N=N, K=K, G=128)
    assert rc == 0 and p.kernel == 0, err
    KC = K // 64
    waves = p.block // 64
    assert p.splits * waves * p.slab_chunks == KC
    assert N % p.tile_n == 0 and p.grid == (N // p.tile_n) * p.splits
    assert 0 < p.block <= 1024
    if p.splits > 1:
        assert p.workspace_bytes == p.splits * M * N * 4
        assert p.counter_slots == N // p.tile_n <= lib.w4a16_max_counter_slots()
    else:
        assert p.workspace_bytes == 0 and p.counter_slots == 0


@pytest.mark.parametrize("M", [1, 17, 100, 513, 2048, 70000])
@pytest.mark.parametrize("N", [16, 4112, 28672])
def test_prefill_plan_invariants(lib, M, N):
    rc, p, err = plan(lib, M=M, N=N, K=4160, G=64)
    assert rc == 0, err
    tiles = PREFILL_TILES[p.kernel]
    assert p.grid == -(-M // tiles[0]) * -(-N // tiles[1])
    assert p.workspace_bytes == 0 and p.counter_slots == 0


PREFILL_TILES = {1: (16, 128), 2: (32, 128), 3: (64, 128), 4: (128, 128), 5: (128, 256), 6: (256, 128), 7: (128, 128),
                 8: (32, 16), 9: (64, 16), 10: (32, 64), 11: (64, 64), 12: (32, 128), 13: (64, 128), 14: (32, 128),
                 15: (32, 256), 16: (16, 64), 17: (16, 64), 18: (64, 128), 19: (64, 256), 20: (128, 128),
                 21: (256, 256), 22: (64, 128), 23: (128, 512),
                 24: (128, 256)}


@pytest.mark.parametrize("M,N,K,want", [
    (2048, 28672, 8192, 5), (1280, 28672, 4096, 5), (4096, 6144, 4096, 5),   # 128x512 last round half full or less
    (1024, 6144, 4096, 24), (512, 14336, 4096, 24), (2048, 4096, 4096, 24),  # one round of 128x256 8-wave tiles
    (256, 28672, 8192, 24),
    (2048, 14336, 4096, 23), (512, 28672, 8192, 23), (2048, 6144, 4096, 23), # 128x512: last round > half full
    (1024, 28672, 8192, 23), (4096, 4096, 4096, 23), (1536, 28672, 4096, 23), (768, 14336, 4096, 23),
    (768, 28672, 4096, 5),
    (1024, 4096, 4096, 20), (1024, 4096, 14336, 20),                         # 128 tiles of 128x256: 128x128
    (512, 6144, 4096, 20), (256, 14336, 4096, 20), (128, 28672, 4096, 20),   # 128x128, four 128x32 waves
    (128, 14336, 4096, 22), (512, 4096, 4096, 22), (64, 28672, 4096, 22),    # 64x128, four 64x32 waves, pipelined
    (2048, 28672, 8256, None),                                               # odd chunk count: classic only
    (17, 4096, 14336, 17), (32, 6144, 4096, 17), (32, 14336, 4096, 17),     # token groups of 16
    (33, 4096, 4096, 17), (64, 4096, 4096, 17), (48, 14336, 4096, 10), (128, 6144, 4096, 10),
    (32, 28672, 4096, 10),                                                   # token groups of 32
    (256, 4096, 4096, 10), (128, 8192, 4096, 10), (64, 16384, 4096, 10),     # exactly 4 two-block waves per CU
    (256, 4160, 4096, 14),                                                   # just above: two blocks per wave
    # long K (4 or 7 segments): split-K token groups, larger groups sooner
    (64, 4096, 14336, 10), (128, 4096, 14336, 12), (256, 4096, 14336, 13), (512, 4096, 14336, 18),
    (17, 8192, 28672, 12), (192, 8192, 28672, 13), (384, 8192, 28672, 19),
    (64, 8192, 28672, 13), (96, 8192, 28672, 12), (100, 14336, 14336, 13),  # 64-token groups when they pad no more
    (2048, 4096, 14336, 24), (1024, 8192, 28672, 24), (2048, 8192, 28672, 24),  # long K, 128 x 256: last round > half full
    (768, 8192, 28672, 24), (1536, 4096, 14336, 24), (512, 8192, 28672, 19), (1024, 4096, 14336, 20),
    (3072, 4096, 14336, 7), (1536, 8192, 28672, 7),                         # long K, >= 2 rounds of 128 x 128: two 128 x 64 waves
    (2048, 5120, 13824, 20),                                                 # 2.5 rounds: last round half empty
    (40, 4096, 4160, None)])                                                 # odd chunk count: classic
def test_prefill_wide_selection(lib, M, N, K, want):
    rc, p, err = plan(lib, M=M, N=N, K=K, G=64)
    assert rc == 0, err
    if want is None:
        assert 1 <= p.kernel <= 4, p.kernel
    else:
        assert p.kernel == want
    tiles = PREFILL_TILES[p.kernel]
    assert p.grid == -(-M // tiles[0]) * -(-N // tiles[1]) * max(p.splits, 1)
    assert p.block == 64 * {1: 4, 2: 4, 3: 4, 4: 4, 5: 4, 6: 4, 7: 2, 8: 1, 9: 1, 10: 4, 11: 4, 12: 4, 13: 4, 14: 4,
                            15: 4, 16: 4, 17: 4, 18: 4, 19: 8, 20: 4, 21: 8, 22: 4, 23: 8, 24: 8}[p.kernel]


def test_prefill_override(lib, monkeypatch):
    for cfg in range(1, 8):
        monkeypatch.setenv("W4A16_PREFILL", str(cfg))
        rc, p, err = plan(lib, M=2048, N=4096, K=4096, G=128)
        assert rc == 0 and p.kernel == cfg, (cfg, p.kernel, err)
    monkeypatch.setenv("W4A16_PREFILL", "5")                  # wide config, odd chunk count: ignored
    rc, p, err = plan(lib, M=2048, N=4096, K=4160, G=64)
    assert rc == 0 and 1 <= p.kernel <= 4
    monkeypatch.setenv("W4A16_PREFILL", "8")                  # small-M config: only when M fits
    rc, p, err = plan(lib, M=40, N=4096, K=4096, G=128)
    assert rc == 0 and p.kernel != 8
    rc, p, err = plan(lib, M=20, N=4096, K=4096, G=128)
    assert rc == 0 and p.kernel == 8 and p.grid == 4096 // 16 and p.block == 64
    monkeypatch.setenv("W4A16_PREFILL", "3")                  # a forced variant wins over the override
    rc, p, err = plan(lib, M=2048, N=4096, K=4096, G=128, variant=2)
    assert rc == 0 and p.kernel == 2


def test_empty_n_plans_nothing(lib):
    rc, p, err = plan(lib, M=4, N=0, K=512, G=64)
    assert rc == 0


def test_injected_small_lds_limit_reports_no_config(lib):
    tiny = Limits(256, 1024, 1024, 950)
    rc, _, err = plan(lib, M=1, N=4096, K=4096, G=128, limits=tiny)
    assert rc == 2 and "no pipeline configuration fits in 1024 B of shared memory" in err
    rc, _, err = plan(lib, M=300, N=4096, K=4096, G=128, limits=tiny)
    assert rc == 2 and "no prefill configuration fits" in err
    rc, _, err = plan(lib, M=300, N=4096, K=4096, G=128, variant=4, limits=Limits(256, 30000, 1024, 950))
    assert rc == 2 and "no prefill configuration fits" in err


def test_torch_binding_imports_and_rejects_host_tensors():
    """The extension module loads on CPU and rejects non-device tensors first (kernel.cu:219)."""
    torch = pytest.importorskip("torch")
    import w4a16_opt
    with pytest.raises(RuntimeError, match="CUDA"):
        w4a16_opt.w4a16_gemm(torch.zeros(8, dtype=torch.int32), torch.zeros(1, 64, dtype=torch.half),
                             torch.zeros(1, 16, dtype=torch.half))


@pytest.mark.parametrize("N,K,G,ptrs,msg", [
    (24, 128, 64, (4096, 4096, 4096), "N must be a multiple of 16"),
    (16, 96, 64, (4096, 4096, 4096), "K a multiple of 64"),
    (16, 256, 32, (4096, 4096, 4096), "unsupported group size"),
    (16, 256, 256, (4096, 4096, 4096), "unsupported group size"),
    (-16, 256, 64, (4096, 4096, 4096), "dimensions out of range"),
    (16, 1 << 31, 64, (4096, 4096, 4096), "dimensions out of range"),
    (16, 128, 64, (0, 4096, 4096), "null pointer"),
    (16, 128, 64, (4104, 4096, 4096), "16-byte aligned"),
    (16, 128, 64, (4096, 4100, 4096), "16-byte aligned"),
    (16, 128, 64, (4096, 4096, 4097), "2-byte aligned"),
])
def test_quantize_pack_validation(lib, N, K, G, ptrs, msg):
    """w4a16_quantize_pack rejects bad arguments on the host, before touching the device."""
    f = lib.w4a16_quantize_pack
    f.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    rc = f(ptrs[0], 0, N, K, G, ptrs[1], ptrs[2], None)
    assert rc == 1 and msg in lib.w4a16_last_error().decode()


def test_quantize_pack_empty_is_a_no_op(lib):
    f = lib.w4a16_quantize_pack
    f.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    assert f(None, 0, 0, 128, 64, None, None, None) == 0
    assert f(None, 1, 16, 0, 128, None, None, None) == 0


def test_torch_quantize_pack_rejects_host_tensors():
    torch = pytest.importorskip("torch")
    import w4a16_opt
    with pytest.raises(RuntimeError, match="CUDA"):
        w4a16_opt.quantize_pack(torch.zeros(16, 128, dtype=torch.half), 64)


def test_bandwidth_probe_loads_and_rejects_bad_arguments():
    """The read and copy probes behind measure_bw.py: exported, and they refuse arguments they
    cannot launch on (null pointers, an empty or non-16-byte-multiple size, a misaligned
    buffer) before touching the device."""
    path = os.path.join(ROOT, "w4a16-gemm_amd", "libw4a16_bwprobe.so")
    if not os.path.exists(path):
        pytest.fail(f"{path} not built (python w4a16-gemm_amd/build.py)")
    L = ctypes.CDLL(path)
    rd, cp = L.w4a16_bw_read, L.w4a16_bw_copy
    rd.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    cp.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    rd.restype = cp.restype = ctypes.c_int
    assert rd(None, 1024, 16, None) == 1
    assert rd(16, 1024, None, None) == 1
    assert rd(16, 0, 16, None) == 1
    assert rd(16, 1000, 16, None) == 1
    assert rd(8, 1024, 16, None) == 1
    assert cp(None, 16, 1024, None) == 1
    assert cp(16, None, 1024, None) == 1
    assert cp(16, 32, 0, None) == 1
    assert cp(16, 32, 1000, None) == 1
    assert cp(16, 40, 1024, None) == 1


def test_planner_occupancy_hook_covers_every_prefill_config(lib):
    lib.w4a16_debug_prefill_occupancy.argtypes = [ctypes.c_int, ctypes.POINTER(Limits)]
    occ = [lib.w4a16_debug_prefill_occupancy(cfg, ctypes.byref(MI355X)) for cfg in range(1, 25)]
    assert all(o >= 1 for o in occ), occ
    assert lib.w4a16_debug_prefill_occupancy(0, ctypes.byref(MI355X)) == -1
    assert lib.w4a16_debug_prefill_occupancy(25, ctypes.byref(MI355X)) == -1
    older = Limits(256, 64 * 1024, 1024, 942)                # 64 KB of LDS per CU bounds every config
    assert all(lib.w4a16_debug_prefill_occupancy(cfg, ctypes.byref(older)) <= o for cfg, o in zip(range(1, 25), occ))


@pytest.mark.parametrize("name,want", [
    (b"gfx950:sramecc+:xnack-", 950), (b"gfx950", 950), (b"gfx942:sramecc+:xnack-", 942), (b"gfx90a:xnack-", 910),
    (b"gfx1100", 1100), (b"gfx1201", 1201), (b"gfx908", 908),
    (b"", 0), (b"sm_90", 0), (b"gfx9", 0), (b"gfx9x0", 0), (b"gfx95g", 0), (None, 0)])
def test_gcn_arch_name_parse(lib, name, want):
    """hipDeviceProp_t.gcnArchName -> w4a16_device_limits.gcn_arch (major*100 + minor*10 + stepping,
    the last two characters hex digits); only 950 selects the 160 KB LDS per CU."""
    lib.w4a16_debug_parse_gcn_arch.argtypes = [ctypes.c_char_p]
    lib.w4a16_debug_parse_gcn_arch.restype = ctypes.c_int32
    assert lib.w4a16_debug_parse_gcn_arch(name) == want


@pytest.mark.parametrize("M,N,K,want", [
    (1, 14336, 4096, (20, 1)), (4, 14336, 4096, (20, 1)), (6, 14336, 4096, (20, 1)), (7, 14336, 4096, (18, 1)),
    (8, 14336, 4096, (18, 1)), (16, 14336, 4096, (18, 1)), (8, 18944, 3584, (20, 1)),
    (1, 4096, 14336, (29, 1)), (4, 4096, 14336, (29, 1)), (8, 4096, 14336, (19, 1)), (16, 4096, 14336, (20, 2)),
    (1, 28672, 4096, (21, 1)), (4, 28672, 4096, (21, 1)),                    # fused gate/up: twice as wide
    (1, 10240, 8192, (29, 1)), (4, 10240, 8192, (19, 1)), (8, 10240, 8192, (31, 1)),  # 70B qkv: K = 8192, 640 blocks
    (16, 10240, 8192, (16, 1)), (4, 8192, 8192, (26, 1)), (16, 8192, 8192, (20, 1)),  # 70B o: two-block tiles fit
    (16, 28672, 4096, (12, 1)),                                              # ring tiles would need two rounds
    (1, 4096, 4096, (19, 1)), (16, 4096, 4096, (19, 1)),                     # configs[0]: two pairs in flight
    (16, 6144, 4096, (20, 1)),                                               # qkv: 384 single-block rings = 2 rounds
    (1, 6144, 4096, (29, 1)), (4, 6144, 4096, (26, 1)), (6, 6144, 4096, (22, 1)),  # qkv: two-block rings below 16 rows,
    (8, 6144, 4096, (22, 1)),                                                # one pair in flight from 5 rows
    (1, 8192, 28672, (26, 1)), (4, 8192, 28672, (30, 1)), (8, 8192, 28672, (26, 1)),  # 70B down: 512 single blocks
    (16, 8192, 28672, (16, 2)),
    (1, 3584, 18944, (21, 1)), (16, 3584, 18944, (21, 1)),                  # odd chunks per 8-wave ring: generic rings
    (1, 5120, 13824, (21, 1)), (8, 5120, 13824, (20, 1)), (16, 18944, 3584, (20, 1))])
def test_decode_selection(lib, M, N, K, want):
    """The decode shapes the planner picks for the Llama-3 projections (BASELINE configs[1] first)."""
    rc, p, err = plan(lib, M=M, N=N, K=K, G=128)
    assert rc == 0, err
    assert (p.decode_variant, p.splits) == want


@pytest.mark.parametrize("M,N,K", [(32, 4096, 14336), (17, 4096, 14336), (100, 4096, 8320), (64, 8192, 28672)])
def test_long_k_plans_split_token_group_configs_by_segment(lib, monkeypatch, M, N, K):
    """K > 8192: the token-group (kind 3) and one-wave (kind 2) configs run one canonical K
    segment per workgroup (grid = tiles x segments, one counter per tile, fp32 partials of every
    segment); the other kinds keep the segments in-kernel (no workspace)."""
    KC = K // 64
    s = -(-KC // 64)
    L = 2 * -(-KC // (2 * s))
    segs = -(-KC // L)
    for cfg, kind in [(17, 3), (14, 3), (9, 2), (4, 0), (18, 1), (20, 1), (22, 1), (24, 1)]:
        monkeypatch.setenv("W4A16_PREFILL", str(cfg))
        rc, p, err = plan(lib, M=M, N=N, K=K, G=64)
        assert rc == 0, err
        if p.kernel != cfg:                        # the config does not fit this shape
            assert cfg in (9, 4, 18, 20, 22, 24) and (cfg != 9 or M > 64), (cfg, p.kernel)
            continue
        bm, bn = PREFILL_TILES[cfg]
        tiles = -(-M // bm) * -(-N // bn)
        assert p.slab_chunks == L
        if kind >= 2:
            assert (p.splits, p.grid, p.counter_slots, p.workspace_bytes) == (segs, tiles * segs, tiles, segs * M * N * 4)
        else:
            assert (p.splits, p.grid, p.counter_slots, p.workspace_bytes) == (1, tiles, 0, 0)
    for cfg in (5, 21, 22, 23):                    # no registers for the second set
        monkeypatch.setenv("W4A16_PREFILL", str(cfg))
        rc, p, err = plan(lib, M=2048, N=4096, K=14336, G=128)
        assert rc == 0 and p.kernel != cfg


def test_canonical_segments():
    """The segment rule of the accumulation order: one chain up to K = 8192, then balanced even
    segments of at most 64 chunks; every segment non-empty."""
    def segs(KC):
        if KC <= 128:
            return KC, 1
        s = -(-KC // 64)
        L = 2 * -(-KC // (2 * s))
        return L, -(-KC // L)
    assert segs(64) == (64, 1) and segs(128) == (128, 1)
    assert segs(224) == (56, 4) and segs(448) == (64, 7) and segs(130) == (44, 3)
    for KC in range(129, 5000):
        L, S = segs(KC)
        assert L % 2 == 0 and L <= 64 + 1 and 0 < KC - (S - 1) * L <= L


def _launch(lib, p, workspace=16, counters=16):
    """w4a16_launch with dummy pointers that are never dereferenced: a plan that fails the
    launch-side check returns before any HIP call, so this runs without a GPU."""
    lib.w4a16_launch.argtypes = [ctypes.POINTER(Plan)] + [ctypes.c_void_p] * 7
    lib.w4a16_launch.restype = ctypes.c_int
    return lib.w4a16_launch(ctypes.byref(p), 16, 16, 16, 16, workspace, counters, None)


@pytest.mark.parametrize("field,delta", [("grid", 1), ("grid", -1), ("slab_chunks", 1), ("slab_chunks", -1),
                                          ("block", 64), ("decode_variant", 40), ("splits", 1), ("M", 16),
                                          ("N", 48), ("K", 512), ("G", 64)])
def test_launch_rejects_decode_plan_not_matching_its_shape(lib, field, delta):
    """A decode plan whose grid, chunks per wave, block, shape id, split count or shape disagree
    is refused (W4A16_ERR_INVALID) before anything is launched: the kernels index the weights,
    x and y by the plan, so a stale or edited plan must not reach them."""
    for M, N, K in [(1, 14336, 4096), (8, 4096, 14336), (16, 4096, 14336)]:
        rc, p, err = plan(lib, M=M, N=N, K=K, G=128)
        assert rc == 0 and p.kernel == 0, err
        setattr(p, field, getattr(p, field) + delta)
        assert _launch(lib, p) == 1, (M, N, K, field)


def test_launch_checks_split_buffers_of_decode_plans(lib):
    rc, p, err = plan(lib, M=16, N=4096, K=14336, G=128)
    assert rc == 0 and p.kernel == 0 and p.splits == 2, (err, p.splits)
    for field in ("workspace_bytes", "counter_slots"):
        q = Plan.from_buffer_copy(p)
        setattr(q, field, getattr(q, field) - 1)
        assert _launch(lib, q) == 4, field                      # W4A16_ERR_WORKSPACE
    assert _launch(lib, Plan.from_buffer_copy(p), workspace=None) == 4
    assert _launch(lib, Plan.from_buffer_copy(p), counters=None) == 4


def test_launch_rejects_prefill_plan_not_matching_its_shape(lib):
    rc, p, err = plan(lib, M=300, N=4096, K=4096, G=64)
    assert rc == 0 and p.kernel >= 1, err
    for field, delta in (("grid", 1), ("kernel", 100), ("G", 32)):
        q = Plan.from_buffer_copy(p)
        setattr(q, field, getattr(q, field) + delta)
        assert _launch(lib, q) == 1, field


def _check(lib, p):
    lib.w4a16_debug_check_plan.argtypes = [ctypes.POINTER(Plan)]
    lib.w4a16_debug_check_plan.restype = ctypes.c_int
    return lib.w4a16_debug_check_plan(ctypes.byref(p))


def test_every_planned_shape_passes_the_launch_check(lib, monkeypatch):
    """The launch-side check (w4a16_debug_check_plan runs it without launching) accepts every
    plan the planner makes: auto plans over decode and prefill shapes, every forced decode shape
    and split count the planner takes, every forced prefill config."""
    n = 0
    for G in (64, 128):
        for K in (512, 1024, 4096, 8192, 8320, 14336, 28672):
            if K % G:
                continue
            for N in (64, 256, 4096, 6144, 14336, 28672):
                for M in (1, 2, 4, 5, 8, 9, 16):
                    rc, p, err = plan(lib, M=M, N=N, K=K, G=G)
                    assert rc == 0, err
                    assert _check(lib, p) == 0, (M, N, K, G, p.kernel, p.decode_variant, p.splits)
                    n += 1
                    for v in range(32):
                        for sp in (1, 2, 3, 4, 8):
                            monkeypatch.setenv("W4A16_DECODE", f"{v},{sp}")
                            rc, p, err = plan(lib, M=M, N=N, K=K, G=G)
                            assert rc == 0, err
                            assert _check(lib, p) == 0, (M, N, K, G, v, sp)
                            n += 1
                    monkeypatch.delenv("W4A16_DECODE")
    for G in (64, 128):
        for K in (64, 128, 4096, 4160, 8192, 8320, 14336):
            if K % G:
                continue
            for N in (16, 4112, 28672):
                for M in (1, 17, 100, 513, 2048):
                    for cfg in [None] + list(range(1, 25)):
                        if cfg is None:
                            monkeypatch.delenv("W4A16_PREFILL", raising=False)
                        else:
                            monkeypatch.setenv("W4A16_PREFILL", str(cfg))
                        rc, p, err = plan(lib, M=M, N=N, K=K, G=G, variant=-1 if M > 16 or N % 64 or K % 512 else 1)
                        assert rc == 0, err
                        assert _check(lib, p) == 0, (M, N, K, G, cfg, p.kernel)
                        n += 1
    assert n > 10000


# Wide-tile configs (kind 1) address x and the weights with 32-bit per-lane byte offsets from a
# 64-bit base: (bm - 1) * K * 2 + 112 bytes into the tile's x rows and K * 8 + 496 bytes into the
# second n16 block of a pair.  The planner must never hand them a K for which these wrap (the
# contract allows any K that fits int32, kernel.cu:228).
WIDE_BM = {5: 128, 6: 256, 7: 128, 18: 64, 19: 64, 20: 128, 21: 256, 22: 64, 23: 128, 24: 128}


def _wide_offsets_fit(bm, K):
    return (bm - 1) * K * 2 + 128 <= 2**32 and K * 8 + 512 <= 2**31 - 1


@pytest.mark.parametrize("cfg", sorted(WIDE_BM))
def test_wide_configs_refused_where_32bit_offsets_wrap(lib, monkeypatch, cfg):
    bm = WIDE_BM[cfg]
    kmax = (2**32 - 128) // (2 * (bm - 1)) // 128 * 128          # largest K (multiple of 128) that fits
    monkeypatch.setenv("W4A16_PREFILL", str(cfg))
    for K in (kmax - 128 * 64, kmax, kmax + 128, kmax + 128 * 64, 2**23 + 2**16, 2**24 + 2**16):
        rc, p, err = plan(lib, M=2 * bm + 1, N=4096, K=K, G=128)
        assert rc == 0, err
        if p.kernel == cfg:
            assert _wide_offsets_fit(bm, K), (cfg, K)
        if not _wide_offsets_fit(bm, K):
            assert p.kernel != cfg and _check(lib, p) == 0, (cfg, K, p.kernel)
        chosen_bm = WIDE_BM.get(p.kernel)
        assert chosen_bm is None or _wide_offsets_fit(chosen_bm, K), (cfg, K, p.kernel)


# Waves of the refill-ahead ring shapes (kind 3) of the decode table (w4a16_internal.h,
# kDecodeTable ids 16..31).  Those of 8 or more waves address x with 32-bit per-lane byte offsets
# of up to 15 token rows (15 * K * 2 + 256 bytes from a 64-bit base), so the planner keeps them
# to K < 2^27.
RING_WAVES = {16: 4, 17: 4, 18: 8, 19: 8, 20: 4, 21: 4, 22: 8, 23: 4, 24: 16, 25: 8, 26: 8, 27: 16, 28: 4, 29: 8,
              30: 16, 31: 8}


def test_wide_decode_rings_refused_where_32bit_x_offsets_wrap(lib, monkeypatch):
    assert 15 * (2**27) * 2 + 256 < 2**32 < 15 * (2**28) * 2
    taken = 0
    for K in (2**27 - 4096, 2**27, 2**27 + 4096):
        for M in (1, 4, 16):
            rc, p, err = plan(lib, M=M, N=64, K=K, G=128)
            assert rc == 0 and p.kernel == 0, err
            assert _check(lib, p) == 0
            if K >= 2**27:
                assert RING_WAVES.get(p.decode_variant, 0) < 8, (K, M, p.decode_variant)
            for v, waves in RING_WAVES.items():
                if waves < 8:
                    continue
                monkeypatch.setenv("W4A16_DECODE", f"{v},1")
                rc, p, err = plan(lib, M=M, N=64, K=K, G=128)
                assert rc == 0 and _check(lib, p) == 0, err
                if K >= 2**27:
                    assert p.decode_variant != v, (K, M, v)
                elif p.decode_variant == v:               # taken below the bound (LDS permitting)
                    taken += 1
                    q = Plan.from_buffer_copy(p)          # the same plan moved past the bound
                    q.K = 2**27
                    q.slab_chunks = (2**27 // 64) // waves
                    assert _check(lib, q) == 1, (M, v)
                monkeypatch.delenv("W4A16_DECODE")
    assert taken >= 6


def test_auto_plan_at_k_beyond_the_256_row_wide_tiles(lib):
    """K = 2^23 + 2^16: the 256-row wide tiles (configs 6, 21) would wrap their x offsets; the auto
    plan takes a config whose addresses fit, and passes the launch-side check."""
    K = 2**23 + 2**16
    assert not _wide_offsets_fit(256, K) and _wide_offsets_fit(128, K)
    for M in (17, 300, 2048):
        rc, p, err = plan(lib, M=M, N=4096, K=K, G=128)
        assert rc == 0, err
        assert _check(lib, p) == 0
        assert WIDE_BM.get(p.kernel, 0) != 256
    rc, p, err = plan(lib, M=2048, N=4096, K=2**24 + 128, G=128)
    assert rc == 0 and _check(lib, p) == 0
    assert p.kernel not in WIDE_BM or _wide_offsets_fit(WIDE_BM[p.kernel], 2**24 + 128)


def test_random_problems_plan_and_pass_the_launch_check(lib):
    """Seeded random problems (any M up to 8192, N and K on their 16 / 64 grids, both group sizes)
    on the MI355X and on its compute partitions (SPX 256 CUs, DPX 128, QPX 64, CPX 32): every
    valid problem gets a plan that the launch-side check accepts, with consistent scratch fields."""
    import numpy as np
    rng = np.random.default_rng(20261202)
    max_slots = lib.w4a16_max_counter_slots()
    n = 0
    for _ in range(2500):
        G = int(rng.choice([64, 128]))
        K = G * int(rng.integers(1, 300))
        N = 16 * int(rng.integers(1, 2400))
        M = int(np.exp(rng.uniform(0, np.log(8192))))
        cus = int(rng.choice([256, 128, 64, 32]))
        rc, p, err = plan(lib, M=M, N=N, K=K, G=G, limits=Limits(cus, 160 * 1024, 1024, 950))
        assert rc == 0, (M, N, K, G, cus, err)
        assert _check(lib, p) == 0, (M, N, K, G, cus, p.kernel, p.decode_variant, p.splits)
        assert p.grid >= 1 and p.splits >= 1 and 0 <= p.counter_slots <= max_slots, (M, N, K, G, cus)
        assert (p.M, p.N, p.K, p.G) == (M, N, K, G)
        if p.kernel == 0:
            assert 0 <= p.decode_variant < 32
        else:
            assert 1 <= p.kernel <= 24
        if p.splits == 1 and p.kernel == 0:
            assert p.workspace_bytes == 0 and p.counter_slots == 0, (M, N, K, G, cus, p.decode_variant)
        n += 1
    assert n == 2500
