// Host-side validation, routing and tile selection for the W4A16 GEMM (pure host code: the
// planner touches no device, so it is unit-tested on CPU through the C ABI).
//
// Validation order and message text follow the reference op w4a16_gemm_cuda
// (src/vectorized/kernel.cu:224-249); the tensor-level checks that precede them in the
// reference (device, contiguity, dtypes, ranks: kernel.cu:219-223) live in the torch binding,
// which owns the tensors.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <map>
#include <mutex>
#include <string>

#include "w4a16.h"
#include "w4a16_internal.h"

using namespace w4a16;

namespace {

thread_local std::string g_last_error;

int fail(int code, char* err, size_t errlen, const char* fmt, ...) {
    if (err && errlen) {
        va_list ap;
        va_start(ap, fmt);
        std::vsnprintf(err, errlen, fmt, ap);
        va_end(ap);
    }
    return code;
}

bool debug_enabled() {
    static const bool on = std::getenv("W4A16_DEBUG_PREFILL") != nullptr;
    return on;
}

// LDS per CU: 160 KB on gfx950 (CDNA4), 64 KB on earlier CDNA parts.
int lds_per_cu(const w4a16_device_limits& lim) {
    return lim.gcn_arch == 950 ? 160 * 1024 : 64 * 1024;
}

// Resident workgroups per CU for a prefill config: the compiled kernel's occupancy on gfx950
// (the table's occ field, which a GPU test checks against the HIP occupancy query), bounded by
// the device's LDS per CU; 0 when the config does not fit the device at all.
int prefill_occupancy(int cfg, const w4a16_device_limits& lim) {
    const int lds = prefill_lds_bytes(cfg);
    if (lds > lim.lds_bytes_per_block) return 0;
    if (prefill_threads(cfg) > lim.max_threads_per_block) return 0;
    return std::max(0, std::min(kPrefillTable[cfg].occ, lds_per_cu(lim) / lds));
}

// Auto prefill selection (replaces pf_select, kernel.cu:142-156).  Cost = full-device waves of
// tiles x per-wave work, where a tile's work is BN * (BM + D): the MFMA work plus the per-tile
// dequantisation overhead D, paid once per weight column block and wave row (D = 32 rows for
// prefill_kernel, 16 for the wide wave tiles whose dequantised operands feed twice as many
// MFMAs).
// The launch fields of a prefill plan for config `cfg` (p->M, N, K, G set): kinds 2 and 3 run one
// canonical K segment per workgroup (split-K partials and one counter per tile), the others all
// of K.  False when the grid does not fit int32.
bool fill_prefill_plan(int cfg, w4a16_plan* p) {
    const int KC = p->K / 64;
    const int segs = prefill_segments(KC);
    const PrefillTile& t = kPrefillTable[cfg];
    const int64_t tiles = ((int64_t)(p->M + t.bm - 1) / t.bm) * ((p->N + t.bn - 1) / t.bn);
    const int splits = t.kind >= 2 ? segs : 1;
    if (tiles * splits > std::numeric_limits<int32_t>::max()) return false;
    p->kernel = cfg;
    p->block = prefill_threads(cfg);
    p->grid = (int32_t)(tiles * splits);
    p->splits = splits;
    p->slab_chunks = prefill_segment_chunks(KC);
    p->counter_slots = splits > 1 ? (int32_t)tiles : 0;
    p->workspace_bytes = splits > 1 ? (uint64_t)splits * p->M * p->N * sizeof(float) : 0;
    return true;
}

int prefill_select(int M, int N, int K, const w4a16_device_limits& lim) {
    int best = 0;
    double best_cost = std::numeric_limits<double>::infinity();
    const double cus = lim.cu_count > 0 ? lim.cu_count : 1;
    // Tiles of a wide-tile config, or -1 when it does not fit the device or the shape.
    auto wide_tiles = [&](int cfg) {
        if (prefill_occupancy(cfg, lim) < 1 || !prefill_shape_ok(cfg, M, K)) return -1.0;
        const PrefillTile& t = kPrefillTable[cfg];
        const double tiles = std::ceil((double)M / t.bm) * std::ceil((double)N / t.bn);
        return tiles <= (double)std::numeric_limits<int32_t>::max() ? tiles : -1.0;
    };
    // Rules measured on MI355X (w4a16-gemm_amd/route_sweep.py: every config forced, graph-timed,
    // on the Llama-3-8B projections and the BASELINE shapes, M = 17..2048):
    //  * the wide 32x32x16 tiles first, largest first, once the M tile is filled:
    //    - 128 x 512 (eight 128 x 64 waves sharing the x rows, one workgroup per CU) when the last
    //      round of its tiles is more than half full (tiles / CUs in (k + 1/2, k + 1]): a full
    //      round of it runs ~5-9% faster than the same work as 128 x 256 tiles two per CU, but a
    //      128 x 256 tile alone on a CU finishes a sparse last round in about half a round.
    //      Measured at M = 256..4096, N = 4096..28672, K = 4096 and 8192 on every shape of both
    //      kinds, e.g. N = 28672, K = 8192, M = 512 (0.875 rounds): 219.6 us against 228.0 for
    //      256 x 256 in 2 x 4 waves (config 21, which this rule replaced: 3.6-4.4% slower on all
    //      six shapes it took) and 241 for 128 x 256; N = 28672, K = 4096, M = 1536 (2.6 rounds):
    //      330 vs 347; M = 4096 (7 rounds): 830 vs 847; but M = 1280 (2.2 rounds): 322 vs 290
    //      and configs[3] (3.5 rounds): 864 vs 856 for 128 x 256;
    //    - 128 x 256 tiles of eight 128 x 32 waves sharing the x rows (config 24, one workgroup
    //      per CU) when they make one round more than half full, e.g. BASELINE configs[2]'s shape
    //      at M = 512: 64.1 vs 69.9 us for 128 x 256 tiles two per CU, N = 4096, K = 4096,
    //      M = 2048: 69.5 vs 73.8, N = 28672, K = 8192, M = 256: 124.1 vs 129.5; over several
    //      rounds the 128 x 32 wave tiles lose to the 128 x 64 ones (N = 28672, M = 2048: 465 vs
    //      425 at K = 4096);
    //    - then, once their tiles number at least 3/4 of the CUs: 128 x 256 (two workgroups per
    //      CU); then 128 x 128 with four waves of 128 x 32 (M >= 128), e.g. N = 28672, M = 128:
    //      43.4 vs 55.4 us for two waves of 128 x 64, N = 4096, K = 14336, M = 1024: 137 vs 171;
    //      then 64 x 128 with four waves of 64 x 32 (M >= 64), software-pipelined across chunks
    //      (config 22; the unpipelined config 18 on long K), e.g. configs[2] (M = 128,
    //      N = 14336, G = 64): 27.6 us against 30.7 for config 18 and 36.4 for token groups of
    //      32, N = 4096, M = 512: 27.6 vs 29.2 (config 18);
    //  * token groups of 16 rows, one n16 block per wave, 4 pairs in flight, while their waves
    //    (M/16 groups x N/16 blocks) are at most 8 per CU: every small-M shape measured, e.g.
    //    K = 14336, N = 4096, M = 32: 42.8 vs 52.6 us for one wave per block over 32 rows
    //    (prefill_stream_kernel, now forced-only); at 12 per CU token groups of 32 rows are
    //    faster (N = 6144, M = 128: 19.0 vs 21.3 us);
    //  * token groups of 32 rows with two n16 blocks per wave (every x operand read feeds two
    //    MFMAs) while their waves (M/32 groups x N/32 block pairs) number 4..12 per CU, 3 pairs
    //    in flight up to 8 per CU, else 2;
    //  * token groups of 32 rows, one n16 block per wave, while the waves (M/32 groups x N/16
    //    blocks) are at most 12 per CU: e.g. N = 28672, M = 32: 25.6 vs 49 us;
    //  * token groups of 64 rows while those waves are at most 8 per CU;
    //  * else the 128 x 128 wide tiles.
    // Long K (several canonical segments): the token-group configs run one segment per workgroup,
    // so their waves multiply by the segment count and larger token groups pay off sooner, and the
    // 128 x 256 tiles are out (no registers for the second accumulator set).  Measured on the
    // down projections (K = 14336, 28672) and K = 12288, M = 17..2048, every choice within 6% of
    // the fastest forced config: e.g. K = 14336, N = 4096, M = 32: 19.2 us (42.8 us before the
    // segments), M = 64: 25.9 (groups of 32, one block per wave), M = 128: 38.8 (groups of 32,
    // two blocks per wave), M = 256: 58.1 (groups of 64), M = 512: 94.6 (64 x 128 wide tiles).
    // At M >= 512: 128 x 256 tiles of eight 128 x 32 waves sharing the x rows (config 24, one
    // workgroup per CU) when the last round of its tiles is more than half full, as for the
    // 128 x 512 tiles above (K = 14336, N = 4096, M = 2048: 234.5 vs 240 us for config 7,
    // M = 1536: 191 vs 201, M = 4096: 453 vs 470; K = 28672, N = 8192, M = 768: 387 vs 493 for
    // the 64 x 256 tiles, M = 1024: 457 vs 469, M = 2048: 912 vs 946, M = 4096: 1815 vs 1905;
    // but M = 512 (half a round): 339 vs 283 for the 64 x 256 tiles); else two waves of 128 x 64
    // per 128 x 128 tile (config 7, one wave per SIMD) once its tiles fill two rounds of the CUs'
    // workgroup slots (K = 14336, N = 4096, M = 2048: 237 vs 252 us for four waves of 128 x 32;
    // K = 28672, N = 8192, M = 1024: 472 vs 499), else the four 128 x 32 waves (K = 14336,
    // N = 4096, M = 1024: 143 vs 180 us).
    const int segs = prefill_segments(K / 64);
    if (segs > 1) {
        auto group_waves = [&](int cfg) {
            const PrefillTile& t = kPrefillTable[cfg];
            return std::ceil((double)M / t.bm) * std::ceil((double)N / t.bn) * t.waves_n * segs;
        };
        auto group_ok = [&](int cfg) { return prefill_occupancy(cfg, lim) > 0 && prefill_shape_ok(cfg, M, K); };
        if (M >= 512) {
            const double rounds = wide_tiles(24) / cus;
            if (rounds > 0.5 && std::ceil(rounds) - rounds < 0.5) return 24;
        }
        // Config 7 once its tiles fill two rounds of the CUs and its last round is more than half full,
        // as for the 128 x 512 and 128 x 256 tiles (Llama-2-13B down, N = 5120, K = 13824, M = 2048:
        // 2.5 rounds, 394 us against 343 for config 20).
        if (M >= 1024) {
            const double rounds7 = wide_tiles(7) / cus;
            if (rounds7 >= 2.0 && std::ceil(rounds7) - rounds7 < 0.5) return 7;
        }
        if (M >= 1024 && wide_tiles(20) >= 0.75 * cus) return 20;
        // From 0.6 of the CUs, as the K <= 8192 wide tiles (Llama-2-13B down, N = 5120, K = 13824,
        // M = 512, 160 tiles of 64 x 256: 109.8 vs 136.8 us for the 64-token groups).
        if (M >= 384 && wide_tiles(19) >= 0.6 * cus) return 19;
        if (M >= 256 && wide_tiles(18) >= 0.75 * cus) return 18;
        if (group_ok(17) && group_waves(17) <= 9.0 * cus) return 17;
        // 64-token groups once config 12's waves exceed 13 per CU, from M = 64 when they pad no more
        // rows than 32-token groups (M = 64: 61.9-62.2 vs 69.2-70.4 us at N = K = 14336, 68.5-69.0 vs
        // 70.4-71.3 at N = 8192, K = 28672; M = 96, a half-empty second group: 105 vs 95.5).
        const bool pad64_ok = M >= 128 || (M >= 64 && (M + 63) / 64 * 64 == (M + 31) / 32 * 32);
        if (pad64_ok && group_ok(13) && group_waves(12) >= 13.0 * cus) return 13;
        if (group_ok(12) && group_waves(12) >= 5.0 * cus) return 12;
        if (group_ok(10) && group_waves(10) <= 8.0 * cus) return 10;
        if (wide_tiles(20) >= 0.75 * cus) return 20;
        if (group_ok(12)) return 12;
    }
    if (M >= 256) {
        const double rounds = wide_tiles(23) / cus;
        if (rounds > 0.5 && std::ceil(rounds) - rounds < 0.5) return 23;
        const double rounds24 = wide_tiles(24) / cus;
        if (rounds24 > 0.5 && rounds24 <= 1.0) return 24;
    }
    if (wide_tiles(5) >= 0.75 * cus) return 5;
    // The 128 x 128 and pipelined 64 x 128 tiles from 0.6 of the CUs: at 62.5% (Llama-3-70B qkv,
    // N = 10240, K = 8192) they beat the token groups (M = 128: 43.4 vs 57.5 us; M = 256: 64.9 vs
    // 69.5 for the 64 x 128 tiles); at 50% (70B o, N = 8192, M = 128) they lose (43.3 vs 38.0).
    if (M >= 128 && wide_tiles(20) >= 0.6 * cus) return 20;
    if (M >= 64 && wide_tiles(22) >= 0.6 * cus) return 22;
    const double blocks = std::ceil(N / 16.0);
    if (prefill_occupancy(17, lim) > 0 && prefill_shape_ok(17, M, K) &&
        std::ceil(M / 16.0) * blocks <= 8.0 * cus)
        return 17;
    // Two blocks per wave from just above 4 such waves per CU: at exactly 4 per CU the one-block
    // groups (8 waves per CU) are ~7% faster (o, N = K = 4096, M = 256: 19.3 vs 20.8 us, and 22.5
    // vs 24.2 in an earlier sweep).
    const double waves2 = std::ceil(M / 32.0) * std::ceil(N / 32.0);
    if (waves2 > 4.0 * cus && waves2 <= 12.0 * cus) {
        const int cfg = waves2 <= 8.0 * cus ? 14 : 12;
        if (prefill_occupancy(cfg, lim) > 0 && prefill_shape_ok(cfg, M, K)) return cfg;
    }
    if (prefill_occupancy(10, lim) > 0 && prefill_shape_ok(10, M, K) &&
        std::ceil(M / 32.0) * blocks <= 12.0 * cus)
        return 10;
    if (prefill_occupancy(11, lim) > 0 && prefill_shape_ok(11, M, K) &&
        std::ceil(M / 64.0) * blocks <= 8.0 * cus)
        return 11;
    if (wide_tiles(20) > 0) return 20;
    for (int cfg = kNumPrefillTable; cfg >= 1; --cfg) {    // descending: ties go to the later config
        const int occ = prefill_occupancy(cfg, lim);
        if (occ < 1 || !prefill_shape_ok(cfg, M, K) || kPrefillTable[cfg].kind >= 1) continue;   // other kinds: rules above
        const PrefillTile& t = kPrefillTable[cfg];
        const double tiles = std::ceil((double)M / t.bm) * std::ceil((double)N / t.bn);
        if (tiles > (double)std::numeric_limits<int32_t>::max()) continue;
        const double waves = std::ceil(tiles / (cus * occ));
        const double cost = waves * occ * t.bn * (t.bm + (t.kind ? 16.0 : 32.0));
        if (cost < best_cost) { best_cost = cost; best = cfg; }
    }
    return best;
}

}  // namespace

extern "C" void w4a16_set_last_error(const char* msg) { g_last_error = msg ? msg : ""; }
extern "C" const char* w4a16_last_error(void) { return g_last_error.c_str(); }
extern "C" int w4a16_abi_version(void) { return W4A16_ABI_VERSION; }

// Test hook (no counterpart in the reference): the planner's occupancy for prefill config `cfg`.
// gcn_arch of an architecture name "gfx<major><minor><stepping>[:features]": minor and stepping are
// the last two characters before ':' (hex digits), major the decimal digits before them;
// encoded major * 100 + minor * 10 + stepping (gfx950 -> 950, gfx942 -> 942, gfx90a -> 910,
// gfx1100 -> 1100); 0 when the name does not parse.
static int32_t parse_gcn_arch(const char* a) {
    if (!a || std::strncmp(a, "gfx", 3) != 0) return 0;
    const char* s = a + 3;
    size_t n = std::strcspn(s, ":");
    if (n < 3) return 0;
    int32_t major = 0;
    for (size_t i = 0; i + 2 < n; ++i) {
        if (s[i] < '0' || s[i] > '9') return 0;
        major = major * 10 + (s[i] - '0');
    }
    auto hex = [](char c) { return c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10 : -1; };
    const int minor = hex(s[n - 2]), stepping = hex(s[n - 1]);
    if (minor < 0 || stepping < 0) return 0;
    return major * 100 + minor * 10 + stepping;
}

extern "C" int32_t w4a16_debug_parse_gcn_arch(const char* name) { return parse_gcn_arch(name); }

extern "C" int w4a16_debug_prefill_occupancy(int cfg, const w4a16_device_limits* lim) {
    if (!lim || cfg < 1 || cfg > kNumPrefillTable) return -1;
    return prefill_occupancy(cfg, *lim);
}
extern "C" int32_t w4a16_max_counter_slots(void) { return kMaxCounterSlots; }

extern "C" int w4a16_plan_create(const w4a16_problem* prob, int variant, const w4a16_device_limits* lim,
                                 w4a16_plan* plan, char* err, size_t errlen) {
    if (err && errlen) err[0] = '\0';
    if (!prob || !lim || !plan) return fail(W4A16_ERR_INVALID, err, errlen, "null argument");
    const w4a16_problem& p = *prob;

    // kernel.cu:224-240, in the same order and with the same messages.
    if (variant < -1 || variant > kNumPrefillCfg)
        return fail(W4A16_ERR_INVALID, err, errlen, "variant must be -1 (auto), 0 (decode) or 1..%d", kNumPrefillCfg);
    if (p.M < 1) return fail(W4A16_ERR_INVALID, err, errlen, "M must be at least 1");
    const int64_t lim32 = (int64_t)1 << 31;
    if (!(p.M < lim32 && p.K < lim32 && p.N < lim32) || p.K < 0 || p.N < 0)
        return fail(W4A16_ERR_INVALID, err, errlen, "dimensions must fit in int32");
    const int M = (int)p.M, K = (int)p.K, N = (int)p.N;
    if (K % 64 != 0) return fail(W4A16_ERR_INVALID, err, errlen, "K must be a multiple of 64");
    if (N % 16 != 0) return fail(W4A16_ERR_INVALID, err, errlen, "N must be a multiple of 16");
    if (!(p.groups > 0 && K % p.groups == 0))
        return fail(W4A16_ERR_INVALID, err, errlen, "K must be divisible by the number of groups");
    if (p.wp_words != (int64_t)N * K / 8) return fail(W4A16_ERR_INVALID, err, errlen, "Wp must hold N*K/8 words");
    if ((reinterpret_cast<uintptr_t>(p.Wp) | reinterpret_cast<uintptr_t>(p.x) |
         reinterpret_cast<uintptr_t>(p.scales)) % 16 != 0)
        return fail(W4A16_ERR_INVALID, err, errlen, "Wp, x and scales must be 16-byte aligned");
    const int G = K / (int)p.groups;
    if (G != 64 && G != 128)
        return fail(W4A16_ERR_INVALID, err, errlen, "unsupported group size %d, supported: 64, 128", G);

    // Routing (kernel.cu:242-249): the decode kernel keeps its shape contract.
    const bool decode_ok = (M <= 16) && (N % 64 == 0) && (K % 512 == 0);
    int v = variant;
    if (v == -1 && decode_ok) v = 0;
    if (v == 0 && !decode_ok)
        return fail(W4A16_ERR_INVALID, err, errlen,
                    "decode kernel needs M in [1, 16], N a multiple of 64 and K a multiple of 512 "
                    "(use variant=-1 or 1..4 for other shapes)");

    w4a16_plan out;
    std::memset(&out, 0, sizeof(out));
    out.M = M; out.N = N; out.K = K; out.G = G;

    if (v == 0) {
        // Decode.  Column tiles of 16*NBW channels; the workgroup's WAVES waves split its K
        // range (kcw chunks each); `splits` workgroups split K further only when there are too
        // few column tiles to give every CU a workgroup.  NBW grows with M so that the x
        // fragments each wave loads stay below ~2x its weight bytes.
        const int KC = K / 64;
        const int cus = lim->cu_count > 0 ? lim->cu_count : 1;
        int var = -1, splits = 0;
        if (const char* o = std::getenv("W4A16_DECODE")) {          // tuning override "v,splits"
            int ov = -1, os = 0;
            if (std::sscanf(o, "%d,%d", &ov, &os) == 2 && ov >= 0 && ov < kNumDecodeCfg &&
                decode_shape_fits(ov, KC, os, G) && decode_lds_bytes(ov, M) <= lim->lds_bytes_per_block &&
                kDecodeTable[ov].waves * 64 <= lim->max_threads_per_block) {
                var = ov; splits = os;
            }
        }
        if (var < 0) {
            // Shapes measured fastest on MI355X (graph-timed sweeps over the whole table,
            // w4a16-gemm_amd/route_sweep.py) for the Llama-3 decode projections, tried in order;
            // the first that fits wins:
            //  * N alone fills the device with 4-block tiles (gate/up, N = 14336): refill-ahead
            //    rings of 4 waves, 2 blocks while the x rows are few (M <= 6), else 4 blocks on 8
            //    waves with one pair in flight each (M = 16: 9.42-9.48 vs 9.75-9.81 us for 4 waves
            //    with two pairs, three alternating runs; 10.05 vs 11.16 for 2 blocks; since the
            //    8-wave rings issue their DMAs with SGPR bases, also M = 7, 8: M = 8 8.48-8.54 vs
            //    8.70-8.79 us on two boxes, M = 7 8.50 vs 8.59, while M = 5, 6 stay 0.06-0.11 us
            //    faster on 2 blocks); no split.  Twice as wide (fused gate/up, N = 28672): single-block rings
            //    of 4 waves with 4 pairs in flight at M <= 4 (M = 1 in four sweeps at K = 4096 and 8192:
            //    14.27-15.05 vs 15.15-15.33 us and 25.69-25.86 vs 25.83-27.58 for 8 waves with 3 pairs);
            //  * long K, moderate N (down, K = 14336): single-block refill-ahead rings of 8 waves,
            //    3 pairs in flight up to 4 token rows and 2 up to 8 rows; above 8 rows, where the x
            //    traffic per block grows, two-block tiles of 4 waves split in two (M = 16: 11.95
            //    vs 12.57 us for 8 waves, in two sweeps);
            //  * short K, moderate N (K = N = 4096): single-block rings of 8 waves, else two-block
            //    rings of 4; at one token row with two pairs in flight up to K = 4096 where the
            //    single-block tiles fit one per CU (configs[0]: 4.03-4.04 vs 4.09-4.10 us for three
            //    pairs, G = 128 and 64, order-rotated on two boxes) and three above (qkv, N = 6144:
            //    5.33 vs 5.57 us);
            //  * more single-block tiles than CUs (qkv N = 6144, Llama-3-70B down N = 8192): two-block
            //    rings of 8 waves from 2 token rows up, which give every CU one tile (70B down
            //    M = 8: 28.5 vs 33.2 us for the single-block rings; qkv M = 8: 6.08 vs 6.46 us), on
            //    short K with one pair in flight from 5 rows (qkv M = 8: 5.48 vs 5.85 us, M = 6: 5.37
            //    vs 5.67, order-rotated; M = 4 level);
            //    16 waves at M <= 4 on long K (70B down M = 4: 26.3 vs 27.7 us), 4-block rings of 4
            //    waves split in two above 8 rows (70B down M = 16: 30.6 vs 35.6 us).
            // Above 8 token rows a ring's LDS allows one or two workgroups per CU, so a shape is
            // taken only if all its workgroups are resident at once (qkv, N = 6144, M = 16: 6.7
            // vs 9.4 us for the single-block rings, whose 384 workgroups ran in two rounds).
            auto ok = [&](int cand, int sp) {
                return decode_shape_fits(cand, KC, sp, G) && decode_lds_bytes(cand, M) <= lim->lds_bytes_per_block &&
                       kDecodeTable[cand].waves * 64 <= lim->max_threads_per_block;
            };
            auto ntiles_of = [&](int cand) { return N / (16 * kDecodeTable[cand].nbw); };
            auto one_round = [&](int cand, int sp) {
                const int per_cu = std::min(lds_per_cu(*lim) / decode_lds_bytes(cand, M), 32 / kDecodeTable[cand].waves);
                return (int64_t)ntiles_of(cand) * sp <= (int64_t)per_cu * cus;
            };
            struct Cand { int v, sp; };
            Cand vwide_m1[] = {{21, 1}, {29, 1}, {20, 1}};
            Cand vwide_small_m[] = {{21, 1}, {20, 1}, {12, 1}};
            Cand wide_small_m[] = {{20, 1}, {12, 1}, {7, 1}};
            Cand wide[] = {{16, 1}, {12, 1}, {7, 1}};
            Cand wide_mid_m[] = {{18, 1}, {20, 1}, {12, 1}};
            Cand wide_large_m[] = {{18, 1}, {16, 1}, {12, 1}};
            Cand longk_m4[] = {{29, 1}, {19, 1}, {22, 2}};
            Cand longk_small_m[] = {{19, 1}, {22, 2}, {22, 2}};
            Cand longk_large_m[] = {{20, 2}, {22, 2}, {19, 1}};
            Cand shortk_m1[] = {{29, 1}, {19, 1}, {14, 1}};
            Cand shortk_m1_fit[] = {{19, 1}, {29, 1}, {14, 1}};
            Cand shortk[] = {{19, 1}, {20, 1}, {21, 1}};
            Cand many_m1[] = {{26, 1}, {29, 1}, {19, 1}};
            Cand many_longk_m4[] = {{30, 1}, {26, 1}, {29, 1}};
            Cand many_small_m[] = {{26, 1}, {22, 1}, {19, 1}};
            Cand many_mid_m[] = {{22, 1}, {26, 1}, {19, 1}};
            Cand many_longk_large_m[] = {{16, 2}, {26, 1}, {20, 2}};
            // K = 8192 with many blocks (Llama-3-70B o, qkv): shorter streams than the 70B down
            // projection the lists above come from, so no split; two-block tiles while they fit one
            // per CU (o, N = 8192: M = 4 9.28 vs 9.93 us, M = 16 10.84 vs 13.15), else single-block
            // rings below 8 rows and four-block tiles above (qkv, N = 10240: M = 1 12.07 vs 14.03,
            // M = 4 12.87 vs 16.38, M = 8 14.34 vs 16.66, M = 16 15.60 vs 28.25).
            Cand k8k_fit_small_m[] = {{26, 1}, {29, 1}, {19, 1}};
            Cand k8k_fit_large_m[] = {{20, 1}, {28, 1}, {26, 1}};
            Cand k8k_m1[] = {{29, 1}, {25, 1}, {19, 1}};
            Cand k8k_m4[] = {{19, 1}, {29, 1}, {22, 1}};
            Cand k8k_m8[] = {{31, 1}, {19, 1}, {18, 1}};
            Cand k8k_large_m[] = {{16, 1}, {18, 1}, {17, 1}};
            Cand* list;
            const int n = 3;
            const bool very_wide = (int64_t)ntiles_of(12) * 2 >= 3LL * cus;
            const bool many_blocks = N / 16 > cus;                      // single-block tiles: over one per CU
            if ((int64_t)ntiles_of(12) * 8 >= 7LL * cus && very_wide)
                list = M <= 1 ? vwide_m1 : M <= 4 ? vwide_small_m : wide;
            else if ((int64_t)ntiles_of(12) * 8 >= 7LL * cus)
                list = M <= 6 ? wide_small_m : M <= 8 ? wide_mid_m : wide_large_m;
            else if (KC == 128 && many_blocks && ntiles_of(26) <= cus)
                list = M <= 8 ? k8k_fit_small_m : k8k_fit_large_m;
            else if (KC == 128 && many_blocks)
                list = M <= 1 ? k8k_m1 : M <= 4 ? k8k_m4 : M <= 8 ? k8k_m8 : k8k_large_m;
            else if (KC >= 128 && many_blocks)
                list = M <= 1 ? many_m1 : M <= 4 ? many_longk_m4 : M <= 8 ? many_small_m : many_longk_large_m;
            else if (KC >= 128) list = M <= 4 ? longk_m4 : M <= 8 ? longk_small_m : longk_large_m;
            else list = M <= 1 ? (!many_blocks && KC <= 64 ? shortk_m1_fit : shortk_m1)
                               : M <= 8 && many_blocks ? (M <= 4 ? many_small_m : many_mid_m) : shortk;
            for (int i = 0; i < n && var < 0; ++i)
                if (ok(list[i].v, list[i].sp) && (int64_t)ntiles_of(list[i].v) * list[i].sp * 2 >= cus &&
                    (M <= 8 || one_round(list[i].v, list[i].sp))) {
                    var = list[i].v; splits = list[i].sp;
                }
            // Shapes the lists above do not fit (a K whose chunks per wave are odd for 8-wave rings,
            // e.g. 13824 and 18944, or rings that would need two rounds above 8 rows): the ring
            // kernels still beat the fallbacks below by 1.7-3.5x.  Single-block 4-wave rings with 4
            // pairs in flight up to 4 rows, and above while single-block tiles fit one per CU;
            // two-block rings otherwise (Qwen2-7B down, N = 3584, K = 18944, M = 1..16: 11.2-15.9 us
            // against 39-49 for the fallback; Llama-2-13B down, N = 5120, K = 13824, M = 1..16:
            // 12.3-16.2 against 22.6-27.8; Qwen2-7B gate, N = 18944, K = 3584, M = 16: 13.6 vs 23.8).
            if (var < 0) {
                Cand gen_fit[] = {{21, 1}, {28, 1}, {20, 1}};
                Cand gen_many[] = {{20, 1}, {28, 1}, {21, 1}};
                Cand* gen = (M <= 4 || N / 16 <= cus) ? gen_fit : gen_many;
                for (int i = 0; i < 3 && var < 0; ++i)
                    if (ok(gen[i].v, gen[i].sp) && (int64_t)ntiles_of(gen[i].v) * gen[i].sp * 2 >= cus) {
                        var = gen[i].v; splits = gen[i].sp;
                    }
            }
            if (var < 0 && KC >= 128) {
                for (int sp = 1; sp <= KC; ++sp)
                    if (ok(6, sp) && ((int64_t)ntiles_of(6) * sp >= cus || KC / (sp * 8) <= 4)) {
                        var = 6; splits = sp; break;
                    }
            } else if (var < 0) {
                const int cand = M <= 4 ? 0 : 4;
                if (ok(cand, 1)) { var = cand; splits = 1; }
            }
            if (var < 0) {                                               // any valid shape
                for (int cand = 0; cand < kNumDecodeCfg && var < 0; ++cand)
                    if (kDecodeTable[cand].kind == 0)
                    for (int sp = 1; sp <= KC; ++sp)
                        if (ok(cand, sp)) { var = cand; splits = sp; break; }
            }
        }
        if (var < 0 || decode_lds_bytes(var, M) > lim->lds_bytes_per_block ||
            kDecodeTable[var].waves * 64 > lim->max_threads_per_block)
            return fail(W4A16_ERR_NO_CONFIG, err, errlen, "no pipeline configuration fits in %d B of shared memory",
                        lim->lds_bytes_per_block);
        const DecodeCfg& c = kDecodeTable[var];
        const int ntiles = N / (16 * c.nbw);
        if (splits > 1 && ntiles > kMaxCounterSlots)
            return fail(W4A16_ERR_NO_CONFIG, err, errlen, "N too large for the decode kernel");
        out.kernel = 0;
        out.decode_variant = var;
        out.slab_chunks = KC / (splits * c.waves);             // chunks per wave
        out.splits = splits;
        out.tile_n = 16 * c.nbw;
        out.block = c.waves * 64;
        out.grid = ntiles * splits;
        out.counter_slots = splits > 1 ? ntiles : 0;
        out.workspace_bytes = splits > 1 ? (uint64_t)splits * M * N * sizeof(float) : 0;
        if (debug_enabled())
            std::fprintf(stderr, "decode dispatch G=%d M=%d N=%d K=%d shape=%d (nbw=%d waves=%d depth=%d) "
                         "kcw=%d splits=%d grid=%d\n", G, M, N, K, var, c.nbw, c.waves, c.d,
                         out.slab_chunks, splits, out.grid);
    } else {
        int cfg = v;                                          // 1..4 forced, or -1 = auto
        if (cfg < 0) {
            if (const char* o = std::getenv("W4A16_PREFILL")) {   // tuning override: prefill config id
                const int oc = std::atoi(o);
                if (oc >= 1 && oc <= kNumPrefillTable && prefill_occupancy(oc, *lim) > 0 && prefill_shape_ok(oc, M, K)) cfg = oc;
            }
        }
        if (cfg < 0) cfg = prefill_select(M, N, K, *lim);
        if (!(cfg >= 1 && cfg <= kNumPrefillTable && prefill_occupancy(cfg, *lim) > 0))
            return fail(W4A16_ERR_NO_CONFIG, err, errlen,
                        "no prefill configuration fits (shared memory limit %d B, M=%d)", lim->lds_bytes_per_block, M);
        // Kinds 2 and 3 run one canonical K segment per workgroup: with several segments their
        // tiles need a split-K counter each, else the forced variant 4 (segments in-kernel).
        const int KC = K / 64;
        const int segs = prefill_segments(KC);
        auto tiles_of = [&](int c) {
            const PrefillTile& t = kPrefillTable[c];
            return ((int64_t)(M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
        };
        if (kPrefillTable[cfg].kind >= 2 && segs > 1 && tiles_of(cfg) > kMaxCounterSlots) cfg = 4;
        if (!fill_prefill_plan(cfg, &out))
            return fail(W4A16_ERR_INVALID, err, errlen, "M too large for prefill config %d", cfg);
        if (debug_enabled())
            std::fprintf(stderr, "prefill dispatch G=%d M=%d N=%d K=%d cfg=%d occ=%d tiles=%d\n",
                         G, M, N, K, cfg, prefill_occupancy(cfg, *lim), out.grid);
    }
    *plan = out;
    return W4A16_OK;
}

namespace w4a16 {
// A plan for the same prefill problem whose config needs no split-K scratch (every prefill config
// gives the same bits): the wide tiles or the tiled kernel, which keep the canonical K segments
// in registers, sized by M.  False when `in` is not a prefill plan.
bool prefill_plan_no_scratch(const w4a16_plan& in, const w4a16_device_limits& lim, w4a16_plan* out) {
    if (in.kernel < 1 || in.kernel > kNumPrefillTable) return false;
    const int M = in.M, K = in.K;
    static const int small_m[] = {2, 1, 4}, m64[] = {18, 3, 4}, m128[] = {20, 18, 4}, m256[] = {20, 7, 4},
                     large_m[] = {24, 20, 7, 4};
    const int* order = M <= 32 ? small_m : M <= 64 ? m64 : M <= 128 ? m128 : M <= 256 ? m256 : large_m;
    const int n = order == large_m ? 4 : 3;
    *out = in;
    for (int i = 0; i < n; ++i) {
        const int cfg = order[i];
        if (kPrefillTable[cfg].kind <= 1 && prefill_occupancy(cfg, lim) > 0 && prefill_shape_ok(cfg, M, K) &&
            fill_prefill_plan(cfg, out))
            return true;
    }
    return false;
}
}  // namespace w4a16

extern "C" int w4a16_query_device(int device, w4a16_device_limits* lim) {
    static std::mutex mu;
    static std::map<int, w4a16_device_limits> cache;
    if (!lim) return W4A16_ERR_INVALID;
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(device);
    if (it != cache.end()) { *lim = it->second; return W4A16_OK; }
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        w4a16_set_last_error(hipGetErrorString(e));
        return W4A16_ERR_HIP;
    }
    w4a16_device_limits l;
    l.cu_count = prop.multiProcessorCount;
    l.lds_bytes_per_block = (int32_t)prop.sharedMemPerBlock;
    l.max_threads_per_block = prop.maxThreadsPerBlock;
    l.gcn_arch = parse_gcn_arch(prop.gcnArchName);         // e.g. "gfx950:sramecc+:xnack-" -> 950
    cache[device] = l;
    *lim = l;
    return W4A16_OK;
}
