// Device building blocks shared by the decode and prefill kernels (gfx950 / CDNA4).
//
// Operand mapping onto v_mfma_f32_16x16x32_f16 (64-wide wavefront).  The MFMA contracts
// over (lane group kb = lane / 16, slot 0..7): lane (kb, i) of operand A holds 8 fp16 of row
// i, lane (kb, j) of operand B holds the 8 fp16 of column j with the SAME k in the same
// slot.  Any bijection k <-> (kb, slot) gives the exact dot product, so the kernels pick the
// one the packed weight format already provides and stage x to match it:
//
//   A = dequantised weights, row i = output channel n (16 per n16 block).
//       Lane (kb, i) reads the 16-byte word quad of packed lane' = 4*(i % 8) + kb, i.e. the
//       codes of n in {g, g+8} (g = i % 8) at k = 16s + 2kb + {0,1} and 16s + 2kb + 8 + {0,1}
//       (reference tests/quant.py:19-24, :37).  It keeps the nibbles of its own n (even
//       nibble pairs p = 0, 2 for i < 8, odd pairs p = 1, 3 for i >= 8, common.cuh:45-55).
//       MFMA h (h = 0, 1 covers the 64-wide chunk) uses words s = 2h, 2h+1, giving slot
//       pair c (c = 0..3) the k values 32h + 8c + 2kb + {0, 1}.
//   B = activations x, column j = token.  Lane (kb, j) needs x[j][32h + 8c + 2kb + {0,1}],
//       c = 0..3: dwords d = 16h + 4c + kb of the chunk.  The LDS copy of x stores dword d
//       at position 16h + 4kb + c (a 4x4 transpose of the (c, kb) fields), so the lane's
//       B operand is one 16-byte LDS read.
//   C (16x16 fp32): lane l holds rows 4*(l/16) + r (r = 0..3) of column l % 16, i.e. four
//       consecutive output channels of one token: one 8-byte fp16 store per lane.
//
// Dequantisation is bit-identical to the reference's dequant8 (common.cuh:45-55):
//   (bits & mask) | 0x64006400 gives fp16 1024 + q (mask 0x000F000F) or 1024 + 16q (mask
//   0x00F000F0); one fp16 FMA with per-lane constants (1, -1032) or (1/16, -72) gives q - 8
//   exactly; one round-to-nearest-even fp16 multiply by the scale gives fp16((q - 8) * s).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a16 {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// Bytes of one token row of one 64-wide K chunk in LDS: 128 B of data + 16 B pad, so that the
// 16 lanes of a B-operand read (16 consecutive tokens) hit 16 distinct 16-byte bank groups.
constexpr int kXRow = 144;

__device__ __forceinline__ f4 mfma16x16x32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_f16: lane l supplies A[l % 32][8 (l / 32) + i] and B[8 (l / 32) + i][l % 32]
// (i = 0..7); D register i of lane l is D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32].  Measured on
// MI355X: one 16x16x32 MFMA over k-slots 0..31 equals two chained 16x16x16 MFMAs over slots
// 0..15 then 16..31, and each of those equals the 32x32x16 MFMA over the same 16 slots, bit for
// bit (the hardware rounds in the same k groups).  So kernels that feed the same k-slot sets in
// the same order produce identical results whichever of the two shapes they use.
typedef float f32x16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ f32x16 mfma32x32x16(h8 a, h8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Per-lane dequantisation constants (row i = lane % 16 selects the nibble parity).
struct Dq {
    uint32_t mask;
    h2 mul;
    h2 add;
};

__device__ __forceinline__ Dq dq_setup(int lane) {
    const bool odd = (lane & 8) != 0;               // i >= 8  ->  n = g + 8  ->  odd pairs
    Dq d;
    d.mask = odd ? 0x00F000F0u : 0x000F000Fu;
    const _Float16 m = odd ? (_Float16)0.0625f : (_Float16)1.0f;
    const _Float16 a = odd ? (_Float16)-72.0f : (_Float16)-1032.0f;
    d.mul = h2{m, m};
    d.add = h2{a, a};
    return d;
}

// Two codes (k, k+1) of one output channel -> fp16x2 (q - 8) * s, bit-exact.
__device__ __forceinline__ uint32_t dq_pair(uint32_t bits, const Dq& d, h2 s) {
    const uint32_t v = (bits & d.mask) | 0x64006400u;
    const h2 qm8 = __builtin_elementwise_fma(__builtin_bit_cast(h2, v), d.mul, d.add);
    const h2 r = qm8 * s;
    return __builtin_bit_cast(uint32_t, r);
}

// A operand of one MFMA from two packed words (s = 2h and 2h + 1).
__device__ __forceinline__ h8 dq_frag(uint32_t w0, uint32_t w1, const Dq& d, h2 s) {
    u4 r;
    r.x = dq_pair(w0, d, s);
    r.y = dq_pair(w0 >> 8, d, s);
    r.z = dq_pair(w1, d, s);
    r.w = dq_pair(w1 >> 8, d, s);
    return __builtin_bit_cast(h8, r);
}

__device__ __forceinline__ h2 scale2(uint16_t bits) {
    const _Float16 s = __builtin_bit_cast(_Float16, bits);
    return h2{s, s};
}

// Store one 16-byte global segment q (halves 8q..8q+7 of a 64-wide chunk) of a token row into
// the permuted LDS layout: dword e of the segment (kb = e, c = q & 3, h = q >> 2) goes to
// dword position 16h + 4e + c.
__device__ __forceinline__ void lds_store_xseg(char* row, int q, u4 v) {
    char* b = row + (q >> 2) * 64 + (q & 3) * 4;
    *reinterpret_cast<uint32_t*>(b) = v.x;
    *reinterpret_cast<uint32_t*>(b + 16) = v.y;
    *reinterpret_cast<uint32_t*>(b + 32) = v.z;
    *reinterpret_cast<uint32_t*>(b + 48) = v.w;
}

// fp32 x4 -> fp16 x4 (round to nearest even, like __floats2half2_rn), packed for an 8-byte store.
__device__ __forceinline__ u2 pack_f16x4(f4 v) {
    const h2 lo = h2{(_Float16)v.x, (_Float16)v.y};
    const h2 hi = h2{(_Float16)v.z, (_Float16)v.w};
    return u2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}

}  // namespace w4a16
