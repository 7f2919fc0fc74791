// Internal tables shared by the host planner (w4a16_plan.cpp) and the launcher
// (w4a16_kernels.hip).  Host-only constants; no device code.
#pragma once
#include <stdint.h>

namespace w4a16 {

// Prefill tile configurations, variant ids 1..4 (the reference's PfCfg<1..4>,
// src/vectorized/kernel.cu:59-63, re-tiled for 64-wide wavefronts and 256 CUs).
struct PrefillTile {
    int bm, bn, waves_m, waves_n;
};
constexpr PrefillTile kPrefillTable[5] = {
    {0, 0, 0, 0},
    {16, 128, 1, 4},    // 1: small batches: 4 waves across N, wave tile 16 x 32
    {32, 128, 1, 4},    // 2: wave tile 32 x 32
    {64, 128, 2, 2},    // 3: wave tile 32 x 64
    {128, 128, 2, 2},   // 4: wave tile 64 x 64
};
constexpr int kNumPrefillCfg = 4;

// Bytes of one LDS row (128 B of a 64-wide fp16 chunk + 16 B pad); must match kXRow.
constexpr int kLdsRowBytes = 144;

constexpr int prefill_lds_bytes(int cfg) { return 2 * kPrefillTable[cfg].bm * kLdsRowBytes; }
constexpr int prefill_threads(int cfg) { return 64 * kPrefillTable[cfg].waves_m * kPrefillTable[cfg].waves_n; }

// Decode kernel shapes: NBW n16 blocks (16*NBW output channels) per workgroup, WAVES waves
// splitting the workgroup's K range, software-pipeline depth D (chunks in flight per wave).
struct DecodeCfg {
    int nbw, waves, depth;
};
constexpr DecodeCfg kDecodeTable[8] = {
    {1, 16, 4},   // 0
    {1, 16, 2},   // 1
    {2, 16, 4},   // 2
    {2, 16, 2},   // 3
    {1, 8, 4},    // 4
    {2, 8, 4},    // 5
    {4, 8, 4},    // 6
    {4, 16, 2},   // 7
};
constexpr int kNumDecodeCfg = 8;
constexpr int decode_lds_bytes(int v) { return kDecodeTable[v].waves * kDecodeTable[v].nbw * 64 * 16 + 16; }

// Counter buffer size (ints) the library may ask for: one per decode column tile.
constexpr int32_t kMaxCounterSlots = 1 << 18;

}  // namespace w4a16

extern "C" void w4a16_set_last_error(const char* msg);
