// On-device group-wise RTN quantisation + packing into the GEMM's int32 nibble format.
//
// Replaces the reference's host-side test-data path quantize_w4 + pack_int4
// (tests/quant.py:62-74, 34-48) for weight loading: from W [N, K] (fp16 or fp32, row-major) it
// writes scales fp16 [K/G, N] and the packed words Wp int32 [N*K/8] that w4a16_launch reads.
//
//   s[g, n] = fp16(max(absmax(W[n, gG .. gG+G-1]) / 7, 1e-4))        (fp32 arithmetic)
//   q[n, k] = clamp(round_half_even(W[n, k] / float(s[k/G, n])), -8, 7) + 8
//   word (((n/16)*(K/64) + k/64)*32 + lane)*4 + (k%64)/16, nibble i = p + 4h:
//       n = 16*(n/16) + lane/4 + 8*(p & 1),  k = 64*(k/64) + 16*s + 2*(lane % 4) + 8*(p >> 1) + h
//
// Every operation is an IEEE fp32 operation (correctly rounded division, round-half-even) or an
// exact conversion, so the result is bit-identical to the reference's fp32 torch arithmetic.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w4a16.h"
#include "w4a16_device.h"
#include "w4a16_internal.h"

namespace w4a16 {

// Group-local position of code k in a row of the LDS code tile.  Within a 64-wide chunk the
// codes of packed lane t' = 4g + tt (tt = (k >> 1) & 3) occupy 16 consecutive bytes, one dword
// per word s = (k >> 4) & 3, with bytes ordered (k, k + 1, k + 8, k + 9) = (b, h) = (0, 0),
// (0, 1), (1, 0), (1, 1) for b = (k >> 3) & 1, h = k & 1.  Codes k, k + 1 (k even) are adjacent.
__device__ __forceinline__ int code_pos(int k) {
    return (k >> 6) * 64 + 16 * ((k >> 1) & 3) + 4 * ((k >> 4) & 3) + 2 * ((k >> 3) & 1) + (k & 1);
}

// Workgroup = 64 threads on one (n16 block, quantisation group) tile of 16 rows x G columns.
// Phase 1: thread t owns row r = t / 4 and, in load j, the V = 16 / sizeof(T) consecutive values
// at column 4Vj + V(t % 4) of the group (each load instruction reads 64 contiguous bytes of 16
// rows).  The 4 threads of a row reduce their absolute maxima with two lane swaps; every one of
// them derives the row's scale, quantises its values in registers and stores the code pairs into
// LDS at code_pos.  Phase 2: thread t < G/2 reads the 16 code bytes of packed lane t % 32 of the
// 64-wide chunk t / 32 for rows g and g + 8 and writes the 4 words with one 16-byte store.
//
// Quotient.  The code is rint(fl(v / s)) with fl() the correctly rounded fp32 division.  The fast
// path forms y = v * rcp(s) (v_rcp_f32: 1 ulp), so |y - v/s| <= 1.5 ulp(y) and
// |y - fl(v/s)| < 2 ulp(y) <= 2^-20 because |v / s| <= 7.0034 (s is absmax/7 rounded to fp16, or
// larger when clamped to 1e-4, or +inf).  Adding 2^23 + 8 rounds y + 8 to an integer with ties to
// even and leaves rint(y) + 8 in the low mantissa byte.  When y lies within 2^-18 of a half-
// integer the lane recomputes every value with the IEEE division (v / s), so exact and near ties
// are decided as the reference decides them; otherwise rint(y) == rint(fl(v/s)) and the fast code
// is exact.  |rint(v / s)| <= 7 for finite inputs, so the reference's clamp to [-8, 7] is a no-op
// on the fast path; the slow path applies it.
template <typename T, int G>
__global__ void __launch_bounds__(64)
quantize_pack_kernel(const T* __restrict__ W, int N, int K, int32_t* __restrict__ Wp,
                     uint16_t* __restrict__ scales) {
    constexpr int V = 16 / (int)sizeof(T);                   // values per 16-byte load
    constexpr int L = G / (4 * V);                           // loads per thread
    constexpr int S = G + 16;                                // LDS row stride (bytes)
    constexpr float kMagic = 8388616.0f;                     // 2^23 + 8
    constexpr float kTieBand = 0.5f - 0x1p-18f;
    __shared__ __align__(16) uint8_t codes[16 * S];
    const int t = threadIdx.x;
    const int groups = K / G;
    const int nb = blockIdx.x / groups;
    const int grp = blockIdx.x - nb * groups;
    const int r = t >> 2;
    const int part = t & 3;

    const char* src = reinterpret_cast<const char*>(W + (size_t)(nb * 16 + r) * K + (size_t)grp * G) + part * 16;
    u4 raw[L];
#pragma unroll
    for (int j = 0; j < L; ++j) raw[j] = *reinterpret_cast<const u4*>(src + 64 * j);
    float v[L * V];
#pragma unroll
    for (int j = 0; j < L; ++j) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t d = e == 0 ? raw[j].x : e == 1 ? raw[j].y : e == 2 ? raw[j].z : raw[j].w;
            if constexpr (sizeof(T) == 2) {
                v[j * V + 2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(d & 0xFFFFu));
                v[j * V + 2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(d >> 16));
            } else {
                v[j * V + e] = __builtin_bit_cast(float, d);
            }
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < L * V; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    const _Float16 s16 = (_Float16)fmaxf(amax / 7.0f, 1e-4f);
    const float s = (float)s16;
    if (part == 0) scales[(size_t)grp * N + nb * 16 + r] = __builtin_bit_cast(uint16_t, s16);

    const float rs = __builtin_amdgcn_rcpf(s);
    uint32_t cbits[L * V];
    bool near_tie = false;
#pragma unroll
    for (int i = 0; i < L * V; ++i) {
        const float y = v[i] * rs;
        const float m = y + kMagic;
        near_tie |= fabsf(y - (m - kMagic)) > kTieBand;
        cbits[i] = __builtin_bit_cast(uint32_t, m);
    }
    if (near_tie) {
#pragma unroll
        for (int i = 0; i < L * V; ++i) {
            const float q = fminf(fmaxf(rintf(v[i] / s), -8.f), 7.f);
            cbits[i] = __builtin_bit_cast(uint32_t, q + kMagic);
        }
    }
    uint8_t* row = codes + r * S;
#pragma unroll
    for (int j = 0; j < L; ++j) {
#pragma unroll
        for (int e = 0; e < V; e += 2) {
            const int k = 4 * V * j + V * part + e;
            const uint32_t pair = __builtin_amdgcn_perm(cbits[j * V + e + 1], cbits[j * V + e], 0x0c0c0400u);
            *reinterpret_cast<uint16_t*>(row + code_pos(k)) = (uint16_t)pair;
        }
    }
    __syncthreads();

    if (t < G / 2) {
        const int cl = t >> 5;                               // 64-wide chunk within the group
        const int lanep = t & 31;
        const int g = lanep >> 2;
        const int off = cl * 64 + 16 * (lanep & 3);
        const u4 a = *reinterpret_cast<const u4*>(codes + g * S + off);
        const u4 b = *reinterpret_cast<const u4*>(codes + (g + 8) * S + off);
        // dword bytes (k, k+1, k+8, k+9) -> nibbles (0, 4, 2, 6) of rows g and (1, 5, 3, 7) of g + 8:
        // reorder to (k, k+8, k+1, k+9) so byte i sits at nibble 2i, then interleave the rows.
        auto word = [](uint32_t x, uint32_t y) {
            return __builtin_amdgcn_perm(x, x, 0x03010200u) | (__builtin_amdgcn_perm(y, y, 0x03010200u) << 4);
        };
        int32_t* dst = Wp + (((size_t)nb * (K >> 6) + (size_t)grp * (G / 64) + cl) * 32 + lanep) * 4;
        *reinterpret_cast<u4*>(dst) = u4{word(a.x, b.x), word(a.y, b.y), word(a.z, b.z), word(a.w, b.w)};
    }
}

template <typename T>
static hipError_t launch_quantize(const void* W, int N, int K, int G, int32_t* Wp, uint16_t* s, hipStream_t st) {
    const dim3 grid((unsigned)((N / 16) * (K / G)));
    if (G == 64)
        hipLaunchKernelGGL((quantize_pack_kernel<T, 64>), grid, dim3(64), 0, st, (const T*)W, N, K, Wp, s);
    else
        hipLaunchKernelGGL((quantize_pack_kernel<T, 128>), grid, dim3(64), 0, st, (const T*)W, N, K, Wp, s);
    return hipGetLastError();
}

}  // namespace w4a16

using namespace w4a16;

extern "C" int w4a16_quantize_pack(const void* W, int w_is_fp32, int64_t N, int64_t K, int64_t G, int32_t* Wp,
                                   uint16_t* scales, void* stream) {
    if (N < 0 || K < 0 || N >= (int64_t)1 << 31 || K >= (int64_t)1 << 31 || N * K >= (int64_t)1 << 40) {
        w4a16_set_last_error("dimensions out of range");
        return W4A16_ERR_INVALID;
    }
    if (N % 16 != 0 || K % 64 != 0) {
        w4a16_set_last_error("N must be a multiple of 16 and K a multiple of 64");
        return W4A16_ERR_INVALID;
    }
    if (G != 64 && G != 128) {
        w4a16_set_last_error("unsupported group size, supported: 64, 128");
        return W4A16_ERR_INVALID;
    }
    if (N == 0 || K == 0) return W4A16_OK;
    if (!W || !Wp || !scales) {
        w4a16_set_last_error("null pointer");
        return W4A16_ERR_INVALID;
    }
    if ((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(Wp)) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(scales) % 2 != 0) {
        w4a16_set_last_error("W and Wp must be 16-byte aligned, scales 2-byte aligned");
        return W4A16_ERR_INVALID;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const hipError_t e = w_is_fp32 ? launch_quantize<float>(W, (int)N, (int)K, (int)G, Wp, scales, st)
                                   : launch_quantize<_Float16>(W, (int)N, (int)K, (int)G, Wp, scales, st);
    if (e != hipSuccess) {
        w4a16_set_last_error(hipGetErrorString(e));
        return W4A16_ERR_HIP;
    }
    return W4A16_OK;
}
