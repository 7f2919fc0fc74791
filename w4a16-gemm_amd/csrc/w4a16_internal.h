// Internal tables shared by the host planner (w4a16_plan.cpp) and the launcher
// (w4a16_kernels.hip).  Host-only constants; no device code.
#pragma once
#include <stdint.h>

#include "w4a16.h"

namespace w4a16 {

// Prefill tile configurations.  Ids 1..4 are the forced variants of the reference API (its
// PfCfg<1..4>, src/vectorized/kernel.cu:59-63, re-tiled for 64-wide wavefronts and 256 CUs) and
// run prefill_kernel (kind 0); ids 5..7 and 18..21 run prefill_wide_kernel (kind 1, 32x32x16
// wave tiles of 64 or 128 tokens x 32 or 64 channels); ids 8..9 run prefill_stream_kernel (kind
// 2: one wave per n16 block over the whole K, for M <= bm, ring of `depth` chunk pairs); ids
// 10..17 run prefill_group_kernel (kind 3: waves_n waves, one or more n16 blocks each, share the
// x rows of a group of bm tokens in the ring; any M, one token group per grid row).  The auto
// planner (or the W4A16_PREFILL override) picks among all of them; all give bit-identical output.
//   depth: kinds 2 and 3: chunk pairs in flight in the ring; kind 1: register sets of prefetched
//          chunks (2 or 4: loads issued that many chunks ahead; K/64 must be a multiple);
//   wpe: waves per SIMD the kind-1 kernels' registers are budgeted for (amdgpu_waves_per_eu);
//   occ: resident workgroups per CU of the compiled kernel on gfx950 (registers, LDS and wave
//        slots), the value hipOccupancyMaxActiveBlocksPerMultiprocessor reports for it
//        (tests/test_w4a16_gpu.py::test_planner_occupancy_matches_the_compiled_kernels).
struct PrefillTile {
    int bm, bn, waves_m, waves_n, kind, depth, wpe, occ, pipe;
};
constexpr PrefillTile kPrefillTable[25] = {
    {0, 0, 0, 0, 0, 0, 0, 0},
    {16, 128, 1, 4, 0, 0, 0, 7},     // 1: small batches: 4 waves across N, wave tile 16 x 32
    {32, 128, 1, 4, 0, 0, 0, 6},     // 2: wave tile 32 x 32
    {64, 128, 2, 2, 0, 0, 0, 3},     // 3: wave tile 32 x 64
    {128, 128, 2, 2, 0, 0, 0, 2},    // 4: wave tile 64 x 64
    {128, 256, 1, 4, 1, 2, 2, 2},    // 5: wave tile 128 x 64, 4 waves across N
    {256, 128, 2, 2, 1, 2, 1, 1},    // 6: wave tile 128 x 64, 2 x 2 waves
    {128, 128, 1, 2, 1, 2, 1, 2},    // 7: wave tile 128 x 64, 2 waves
    {32, 16, 1, 1, 2, 6, 0, 2},      // 8: M <= 32, one wave per n16 block, 6 pairs in flight
    {64, 16, 1, 1, 2, 3, 0, 2},      // 9: M <= 64, one wave per n16 block, 3 pairs in flight
    {32, 64, 1, 4, 3, 3, 0, 3},      // 10: groups of 32 tokens, 4 n16 blocks per workgroup, 3 pairs
    {64, 64, 1, 4, 3, 2, 0, 2},      // 11: groups of 64 tokens, 4 n16 blocks per workgroup, 2 pairs
    {32, 128, 1, 4, 3, 2, 0, 3},     // 12: groups of 32 tokens, 2 n16 blocks per wave, 2 pairs
    {64, 128, 1, 4, 3, 2, 0, 2},     // 13: groups of 64 tokens, 2 n16 blocks per wave, 2 pairs (forced only)
    {32, 128, 1, 4, 3, 3, 0, 2},     // 14: groups of 32 tokens, 2 n16 blocks per wave, 3 pairs
    {32, 256, 1, 4, 3, 2, 0, 2},     // 15: groups of 32 tokens, 4 n16 blocks per wave, 2 pairs (forced only)
    {16, 64, 1, 4, 3, 3, 0, 4},      // 16: groups of 16 tokens, 1 n16 block per wave, 3 pairs
    {16, 64, 1, 4, 3, 4, 0, 3},      // 17: groups of 16 tokens, 1 n16 block per wave, 4 pairs
    {64, 128, 1, 4, 1, 4, 2, 2},     // 18: wave tile 64 x 32, 4 waves across N
    {64, 256, 1, 8, 1, 2, 2, 2},     // 19: wave tile 64 x 32, 8 waves across N share the x rows
    {128, 128, 1, 4, 1, 4, 2, 2},    // 20: wave tile 128 x 32, 4 waves across N
    {256, 256, 2, 4, 1, 2, 2, 1},    // 21: wave tile 128 x 64, 2 x 4 waves (forced only)
    {64, 128, 1, 4, 1, 4, 2, 2, 1},  // 22: config 18 software-pipelined across chunks (three x buffers)
    {128, 512, 1, 8, 1, 2, 2, 1},    // 23: wave tile 128 x 64, 8 waves across N share the x rows
    {128, 256, 1, 8, 1, 4, 2, 1},    // 24: wave tile 128 x 32, 8 waves across N share the x rows
};
constexpr int kNumPrefillCfg = 4;        // forced variants 1..4 (reference API)
constexpr int kNumPrefillTable = 24;     // all prefill configs

// Bytes of one LDS row (128 B of a 64-wide fp16 chunk + 16 B pad); must match kXRow.
constexpr int kLdsRowBytes = 144;

// Bytes of one 16-row token tile in a prefill_group_kernel slot: 16 rows x 256 B, rows 8..15
// shifted by 8 B (bank spread), rounded up to a multiple of 256.
constexpr int kGroupXTileBytes = 16 * 256 + 256;

// Ring slot of kinds 2 and 3: kind 2 per wave 1 KB of weights and 1 KB of scales, plus the x rows
// of the token group (bm rows x 256 B); kind 3 per n16 block 1 KB of weights and 64 B of scales,
// plus the x rows with the tile padding above.
constexpr int prefill_lds_bytes(int cfg) {
    return kPrefillTable[cfg].kind == 3
               ? (kPrefillTable[cfg].depth + 1) *
                     (1088 * kPrefillTable[cfg].bn / 16 + kPrefillTable[cfg].bm / 16 * kGroupXTileBytes)
           : kPrefillTable[cfg].kind == 2
               ? (kPrefillTable[cfg].depth + 1) *
                     (2048 * kPrefillTable[cfg].waves_n + kPrefillTable[cfg].bm / 4 * 1024)   // ring slots
               : (kPrefillTable[cfg].pipe ? 3 : 2) * kPrefillTable[cfg].bm * kLdsRowBytes;
}
// Canonical prefill accumulation order.  Every prefill config sums the K range in the same
// order, so all of them give bit-identical results and token rows are independent of M:
//  * K <= 8192 (KC = K/64 <= 128 chunks): one fp32 MFMA chain over the chunks in order;
//  * longer K: S = ceil(KC / 64) segments of L = 2 ceil(KC / 2S) chunks (the last one shorter),
//    each an MFMA chain from zero, added in fp32 in segment order (total = p0, then
//    total = total + p_s).  The split-K configs compute one segment per workgroup and the last
//    workgroup of a tile adds the partials; the others keep a second accumulator set.
// 8192 keeps the BASELINE prefill shape (K = 8192) on one chain, where the 128 x 256 tiles have
// no registers for a second set; Llama-3 down projections (K = 14336) get 4 segments of 3584.
constexpr int kMaxSegmentChunks = 64;       // longest canonical segment above K = 8192 (chunks of 64)
constexpr int prefill_segment_chunks(int KC) {
    if (KC <= 128) return KC;
    const int s = (KC + kMaxSegmentChunks - 1) / kMaxSegmentChunks;
    return 2 * ((KC + 2 * s - 1) / (2 * s));
}
constexpr int prefill_segments(int KC) {
    return KC <= 0 ? 1 : (KC + prefill_segment_chunks(KC) - 1) / prefill_segment_chunks(KC);
}
// Whether a kind-1 config has the registers for a second accumulator set: not the 128 x 64
// wave tiles budgeted for two waves per SIMD (configs 5, 21 and 23: 128 accumulators in 256 registers).
constexpr bool prefill_wide_segmentable(int cfg) {
    return kPrefillTable[cfg].kind == 1 && !kPrefillTable[cfg].pipe &&
           !(kPrefillTable[cfg].wpe == 2 &&
             (kPrefillTable[cfg].bm / kPrefillTable[cfg].waves_m) * (kPrefillTable[cfg].bn / kPrefillTable[cfg].waves_n) >=
                 128 * 64);
}
// Chunks a kind-1 kernel walks per loop step (its register sets of prefetched chunks): `depth`,
// except with the second accumulator set of the long-K segments on the 128 x 32 wave tiles
// budgeted for two waves per SIMD, which then have registers for two sets only.
constexpr int prefill_wide_steps(int cfg, bool seg) {
    return seg && kPrefillTable[cfg].wpe == 2 &&
                   (kPrefillTable[cfg].bm / kPrefillTable[cfg].waves_m) * (kPrefillTable[cfg].bn / kPrefillTable[cfg].waves_n) >=
                       128 * 32
               ? 2
               : kPrefillTable[cfg].depth;
}
// The wide kernels (kind 1) address x and the weights with 32-bit per-lane byte offsets from a
// wave-uniform 64-bit base: x rows up to bm - 1 below the tile's first row ((bm - 1) * K * 2 + 112
// bytes) and the second n16 block of a 32-channel pair (K * 8 + 496 bytes, formed in int).  Longer
// K goes to the other kinds, whose addresses are 64-bit throughout.
constexpr bool prefill_wide_offsets_fit(int cfg, int K) {
    return (int64_t)(kPrefillTable[cfg].bm - 1) * K * 2 + 128 <= ((int64_t)1 << 32) &&
           (int64_t)K * 8 + 512 <= ((int64_t)1 << 31) - 1;
}
// Kinds 1..3 walk K two chunks at a time; kinds 2 and 3 need at least `depth` chunk pairs in
// every segment and kind 2 covers all M in one tile; kind 1 walks K `depth` chunks at a time
// and, with several segments, needs the registers of a second accumulator set and segments of
// a whole number of steps.
constexpr bool prefill_shape_ok(int cfg, int M, int K) {
    return kPrefillTable[cfg].kind == 0 ||
           ((K / 64) % 2 == 0 &&
            (kPrefillTable[cfg].kind == 1
                 ? prefill_wide_offsets_fit(cfg, K) && (prefill_segments(K / 64) == 1
                        ? (K / 64) % prefill_wide_steps(cfg, false) == 0
                        : prefill_wide_segmentable(cfg) && (K / 64) % prefill_wide_steps(cfg, true) == 0 &&
                              prefill_segment_chunks(K / 64) % prefill_wide_steps(cfg, true) == 0)
                 : ((kPrefillTable[cfg].kind == 3 || M <= kPrefillTable[cfg].bm) &&
                    (K / 64 - (prefill_segments(K / 64) - 1) * prefill_segment_chunks(K / 64)) / 2 >=
                        kPrefillTable[cfg].depth)));
}
constexpr int prefill_threads(int cfg) { return 64 * kPrefillTable[cfg].waves_m * kPrefillTable[cfg].waves_n; }

// Decode kernel shapes.  A workgroup covers NBW n16 blocks (16*NBW output channels) with WAVES
// waves splitting its K range.
//   kind 0: decode_kernel         weights streamed into VGPRs, pipeline depth d chunks, any
//                                  chunk count per wave;
//   kind 2: decode_stream_kernel  per-wave ring of d chunk pairs in LDS (the pairs per wave must
//                                  be a multiple of d);
//   kind 3: decode_ring_kernel    ring of d + 1 chunk-pair slots (weights, x rows and the pair's
//                                  scales), d pairs in flight also while computing (pairs per
//                                  wave >= d).
struct DecodeCfg {
    int kind, nbw, waves, d;
};
constexpr DecodeCfg kDecodeTable[32] = {
    {0, 1, 16, 4}, {0, 1, 16, 2}, {0, 2, 16, 4}, {0, 2, 16, 2},     // 0-3
    {0, 1, 8, 4},  {0, 2, 8, 4},  {0, 4, 8, 4},  {0, 4, 16, 2},     // 4-7
    {2, 4, 4, 4},  {2, 4, 8, 4},  {2, 2, 4, 4},  {2, 1, 4, 4},      // 8-11
    {2, 4, 4, 2},  {2, 2, 8, 4},  {2, 1, 8, 4},  {2, 4, 8, 2},      // 12-15
    {3, 4, 4, 2},  {3, 4, 4, 3},  {3, 4, 8, 1},  {3, 1, 8, 2},      // 16-19
    {3, 2, 4, 2},  {3, 1, 4, 4},  {3, 2, 8, 1},  {3, 4, 4, 4},      // 20-23
    {3, 1, 16, 2}, {3, 1, 8, 4},  {3, 2, 8, 2},  {3, 1, 16, 4},     // 24-27
    {3, 2, 4, 4},  {3, 1, 8, 3},  {3, 2, 16, 2}, {3, 4, 8, 2},      // 28-31
};
constexpr int kNumDecodeCfg = 32;

// Token rows per chunk-pair slot of the kind-3 kernel: one row for M = 1 (4-byte x loads in
// B-operand order), else 4, 8 or 16 rows (16-byte x loads of 4 rows each).
constexpr int decode_ring_xr(int M) { return M <= 1 ? 1 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

constexpr int decode_lds_bytes(int v, int M) {
    return kDecodeTable[v].kind == 0   ? kDecodeTable[v].waves * kDecodeTable[v].nbw * 64 * 16 + 16
           : kDecodeTable[v].kind == 2 ? kDecodeTable[v].waves * kDecodeTable[v].nbw * kDecodeTable[v].d * 1024 + 16
                                       : kDecodeTable[v].waves * (kDecodeTable[v].d + 1) *
                                             (kDecodeTable[v].nbw * 1088 + decode_ring_xr(M) * 256 +
                                              (decode_ring_xr(M) == 16 ? 16 : 0)) + 16;
}
// Whether a decode shape can cover K (in 64-wide chunks, group size G) with `splits` workgroups
// per column tile.  The 8- and 16-wave rings address x with 32-bit per-lane byte offsets of up to
// 15 rows (15 * K * 2 + 256 bytes), so they take K < 2^27 (KC < 2^21).
constexpr int kDecodeRingSbaseMaxKC = 1 << 21;
constexpr bool decode_shape_fits(int v, int KC, int splits, int G) {
    return splits >= 1 && KC % (splits * kDecodeTable[v].waves) == 0 &&
           (kDecodeTable[v].kind != 2 || ((KC / (splits * kDecodeTable[v].waves)) % (2 * kDecodeTable[v].d) == 0)) &&
           (kDecodeTable[v].kind != 3 ||
            ((KC / (splits * kDecodeTable[v].waves)) % 2 == 0 &&
             KC / (splits * kDecodeTable[v].waves) >= 2 * kDecodeTable[v].d &&
             (kDecodeTable[v].waves < 8 || KC < kDecodeRingSbaseMaxKC)));
}

// Counter buffer size (ints) the library may ask for: one per decode column tile.
constexpr int32_t kMaxCounterSlots = 1 << 18;

// A plan for the same prefill problem as `in` whose config needs no split-K scratch (prefill
// configs all give the same bits); false when `in` is not a prefill plan or none fits.
// Defined in w4a16_plan.cpp; used by w4a16_launch_noalloc.
bool prefill_plan_no_scratch(const w4a16_plan& in, const w4a16_device_limits& lim, w4a16_plan* out);

}  // namespace w4a16

extern "C" void w4a16_set_last_error(const char* msg);
