// Baseline W4A16 GEMV (the reference's second extension, w4a16_ext.w4a16_gemv):
//
//   C[n] = fp16_rn((acc[n] - zW[n]) * sW[n]),   acc[n] = sum_k wv(n, k) * A[k]
//
// W int32 [N, K/8] row-major; nibble j (bits 4j..4j+3) of word k/8 of row n is the signed 4-bit
// weight wv(n, k) at k = 8*(k/8) + j (src/baseline/kernel.cu:19-28).  A fp16 [K]; sW, zW fp16 [N];
// fp32 epilogue (kernel.cu:31-33).
//
// Exact accumulation on the int8 matrix cores.  Every finite fp16 value a is an integer multiple
// of 2^-24 with |a * 2^24| < 2^40, so X = a * 2^24 is an exact integer.  Written in six signed
// base-256 digits, X = sum_j L_j * 256^j with L_j in [-128, 127] (the bytes of X + 0x808080808080,
// each minus 128), the dot product becomes six integer dot products
//     acc * 2^24 = sum_j 256^j * P_j,   P_j = sum_k wv(n, k) * L_j(k),
// and P_j is exact in int32 for K <= 2^20 (|wv * L| <= 1024).  One v_mfma_i32_16x16x64_i8 takes
// 16 rows of signed weight bytes (A operand) against a B operand whose columns 0..5 are the digit
// planes L_0..L_5 (columns 6..15 zero).  The int64 sum is rounded once to fp32, so the result is
// the exact dot product correctly rounded, whatever the split of K.  The reference accumulates in
// fp32 in k order (kernel.cu:22-30); its result differs from this one by that order's rounding
// error only.  Non-finite inputs follow IEEE semantics, which for this sum do not depend on the
// order: a NaN term, 0 * inf, or +inf together with -inf give NaN, otherwise any infinite term
// gives that infinity.
//
// Workgroup = 8 waves on 16 or 32 rows.  K is processed in segments of 4096: each of the 512 threads
// converts 8 A values into the digit table in LDS (laid out as the B operands), then each wave
// multiplies a contiguous eighth of the segment's 128-wide superchunks.  Lane (r, g) = (lane %
// 16, lane / 16) loads 16 bytes of row r per superchunk: the 32 weights at k = 128p + 32g .. +31,
// two MFMAs' worth (k offsets 0..15 and 16..31 of its group).  The MFMA output tiles of the 8
// waves (row 4g + i, digit r in lane (r, g), element i) are summed in LDS (exact integers).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "w4a16.h"
#include "w4a16_device.h"
#include "w4a16_internal.h"

namespace w4a16 {

namespace {

typedef int32_t i4v __attribute__((ext_vector_type(4)));

constexpr int kRows = 16;                  // rows per MFMA row tile
constexpr int kWaves = 8;                  // waves per workgroup, splitting each segment's k range
constexpr int kThreads = kWaves * 64;
constexpr int kSeg = 4096;                 // k per digit-table segment
constexpr int kSuper = 128;                // k per superchunk (16 bytes of a row per lane)
constexpr int kDigits = 6;                 // base-256 digits of a * 2^24
constexpr int kSuperBytes = 2 * 4 * kDigits * 16;   // table bytes per superchunk (768)
constexpr int kPerWave = kSeg / kSuper / kWaves;   // superchunks per wave and segment (4)
constexpr uint64_t kDigitBias = 0x808080808080ull;  // 128 * sum_j 256^j

static_assert(kSeg % (kSuper * kWaves) == 0, "segment must split evenly over the waves");
static_assert(kSeg / 8 == kThreads, "the table build gives each thread one 8-k unit");

// a * 2^24 + kDigitBias for a finite fp16 a (callers pass 0 for inputs that must count as 0).
// Branch-free: the hidden bit is min(e, 1), the mantissa is shifted by e - min(e, 1), and the
// sign is applied as (mag ^ s) - s = (mag ^ s) + (s & 1) with s = 0 or all ones, folded into the
// bias.
__device__ __forceinline__ uint64_t biased_fixed(uint32_t h) {
    const uint32_t e = (h >> 10) & 31u;
    const uint32_t hid = min(e, 1u);
    const uint32_t mant = (h & 1023u) | (hid << 10);
    const uint64_t mag = (uint64_t)mant << (e - hid);
    const uint32_t s = 0u - ((h >> 15) & 1u);
    const uint64_t sx = ((uint64_t)s << 32) | s;
    return (mag ^ sx) + (kDigitBias + (s & 1u));
}

// 4x4 byte transpose: out[j] byte i = byte j of in[i] (v_perm_b32 picks bytes of {src0, src1},
// selector values 0..3 = src1, 4..7 = src0).
__device__ __forceinline__ void byte_transpose(const uint32_t (&in)[4], uint32_t (&out)[4]) {
    const uint32_t u01l = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);
    const uint32_t u01h = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);
    const uint32_t u23l = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
    const uint32_t u23h = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
    out[0] = __builtin_amdgcn_perm(u23l, u01l, 0x05040100u);
    out[1] = __builtin_amdgcn_perm(u23l, u01l, 0x07060302u);
    out[2] = __builtin_amdgcn_perm(u23h, u01h, 0x05040100u);
    out[3] = __builtin_amdgcn_perm(u23h, u01h, 0x07060302u);
}

// Digit dwords of four biased values: d[j] byte i = digit j of value i as a signed byte
// (the byte of X + kDigitBias minus 128, i.e. XOR 0x80), j = 0..5.
__device__ __forceinline__ void digit_dwords(const uint64_t (&v)[4], uint32_t (&d)[kDigits]) {
    const uint32_t lo[4] = {(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
    uint32_t t[4];
    byte_transpose(lo, t);
#pragma unroll
    for (int j = 0; j < 4; ++j) d[j] = t[j] ^ 0x80808080u;
    const uint32_t h0 = (uint32_t)(v[0] >> 32), h1 = (uint32_t)(v[1] >> 32);
    const uint32_t h2 = (uint32_t)(v[2] >> 32), h3 = (uint32_t)(v[3] >> 32);
    const uint32_t v01 = __builtin_amdgcn_perm(h1, h0, 0x05010400u);
    const uint32_t v23 = __builtin_amdgcn_perm(h3, h2, 0x05010400u);
    d[4] = __builtin_amdgcn_perm(v23, v01, 0x05040100u) ^ 0x80808080u;
    d[5] = __builtin_amdgcn_perm(v23, v01, 0x07060302u) ^ 0x80808080u;
}

// Signed bytes of the even (shift 0) or odd (shift 4) nibbles of a word: nibble n becomes
// n - 16 * (n >= 8).  With u = n ^ 8 (in 0..15), (u + 0x78) ^ 0x80 is that value as a byte and
// no byte carries into the next.
__device__ __forceinline__ uint32_t signed_nibbles(uint32_t w, int shift) {
    const uint32_t u = ((w ^ 0x88888888u) >> shift) & 0x0F0F0F0Fu;
    return (u + 0x78787878u) ^ 0x80808080u;
}

// IEEE class of the non-finite terms of row n (only called when A holds inf or NaN).
// Returns 0 (none), 1 (+inf), 2 (-inf) or 3 (NaN).
__device__ int nonfinite_class(const uint32_t* __restrict__ wrow, const uint16_t* __restrict__ A, int K) {
    bool pos = false, neg = false, nan = false;
    for (int k = 0; k < K; ++k) {
        const uint32_t h = A[k];
        if (((h >> 10) & 31u) != 31u) continue;
        const int nib = (int)((wrow[k >> 3] >> (4 * (k & 7))) & 15u);
        const int wv = nib >= 8 ? nib - 16 : nib;
        if ((h & 1023u) != 0 || wv == 0) nan = true;
        else if ((wv < 0) != ((h & 0x8000u) != 0)) neg = true;
        else pos = true;
    }
    return nan || (pos && neg) ? 3 : pos ? 1 : neg ? 2 : 0;
}

// WVEC: rows are 16-byte aligned (W 16-byte aligned and K % 32 == 0), one 16-byte load per lane
// and superchunk; otherwise four 4-byte loads.  Loads past the row's end are redirected to its
// first word: their digits are zero (the table is zero for k >= K), so they add nothing.
// XVEC: A is 16-byte aligned (one 16-byte load per 8 values); otherwise eight 2-byte loads.
//
// Segments are double-buffered: the A values and weights of segment s + 1 are requested before
// the MFMAs of segment s, so their latency overlaps that work.  Every load is issued
// unconditionally (clamped addresses) so the compiler's waits count exactly the loads in flight.
// RT: row tiles of 16 per workgroup.  Each digit-table B operand feeds RT MFMAs, so the A
// conversion (done once per workgroup and segment) is shared by 16 RT rows.
template <bool WVEC, bool XVEC, int RT>
__global__ void __launch_bounds__(kThreads)
gemv_kernel(const uint32_t* __restrict__ W, const uint16_t* __restrict__ A, const uint16_t* __restrict__ sW,
            const uint16_t* __restrict__ zW, uint16_t* __restrict__ C, int N, int K) {
    constexpr int ROWS = kRows * RT;
    __shared__ __align__(16) uint8_t table[kSeg / kSuper * kSuperBytes];
    __shared__ int32_t part[kWaves][ROWS][8];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int row0 = blockIdx.x * ROWS;
    const int kw = K >> 3;                                   // words per row
    const uint32_t* __restrict__ wrow[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) wrow[t] = W + (size_t)min(row0 + kRows * t + r, N - 1) * kw;
    i4v acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = i4v{0, 0, 0, 0};
    int nonfinite = 0;

    // superchunks of segment `seg`, and this wave's share (a contiguous range starting at p0)
    auto shape = [&](int seg, int& nsc, int& per) {
        nsc = (min(kSeg, K - seg) + kSuper - 1) / kSuper;
        per = (nsc + kWaves - 1) / kWaves;
    };
    // Request the A values of this thread's 8-k unit and this wave's weights for segment `seg`.
    auto issue = [&](int seg, u4& xa, u4 (&wq)[RT][kPerWave]) {
        int nsc, per;
        shape(seg, nsc, per);
        const int k0 = seg + 8 * tid;
        const uint16_t* src = A + (k0 < K ? k0 : 0);
        if constexpr (XVEC) {
            xa = *reinterpret_cast<const u4*>(src);
        } else {
            uint32_t d[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) d[e] = (uint32_t)src[2 * e] | ((uint32_t)src[2 * e + 1] << 16);
            xa = u4{d[0], d[1], d[2], d[3]};
        }
#pragma unroll
        for (int i = 0; i < kPerWave; ++i) {
            const int p = wave * per + min(i, per - 1);      // past the share: repeat its last one
            const int wi = ((seg + p * kSuper) >> 3) + 4 * g;   // first word of the lane's 32 weights
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                if constexpr (WVEC) {
                    wq[t][i] = *reinterpret_cast<const u4*>(wrow[t] + (wi + 4 <= kw ? wi : 0));
                } else {
                    uint32_t d[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) d[e] = wrow[t][wi + e < kw ? wi + e : 0];
                    wq[t][i] = u4{d[0], d[1], d[2], d[3]};
                }
            }
        }
    };
    // Digits of this thread's unit into the table (units past the segment's superchunks are
    // never read; units past K write zero digits).
    auto build = [&](int seg, const u4& xa) {
        int nsc, per;
        shape(seg, nsc, per);
        const int u = tid;
        if (u >= nsc * (kSuper / 8)) return;
        const bool in = seg + 8 * u < K;
        uint32_t hw[4] = {in ? xa.x : 0u, in ? xa.y : 0u, in ? xa.z : 0u, in ? xa.w : 0u};
        // inf / NaN count as 0 here (their class is applied in the epilogue); rare, so one test
        // per 8 values and the zeroing behind a branch
        bool special = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t ee = hw[q] & 0x7C007C00u;
            special |= (ee & 0xFFFFu) == 0x7C00u || (ee >> 16) == 0x7C00u;
        }
        if (special) {
            nonfinite = 1;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t ee = hw[q] & 0x7C007C00u;
                hw[q] &= ((ee & 0xFFFFu) == 0x7C00u ? 0xFFFF0000u : 0xFFFFFFFFu) &
                         ((ee >> 16) == 0x7C00u ? 0x0000FFFFu : 0xFFFFFFFFu);
            }
        }
        uint64_t ve[4], vo[4];                               // k offsets 0, 2, 4, 6 and 1, 3, 5, 7
#pragma unroll
        for (int i = 0; i < 8; ++i) (i & 1 ? vo : ve)[i >> 1] = biased_fixed((hw[i >> 1] >> (16 * (i & 1))) & 0xFFFFu);
        uint32_t de[kDigits], dd[kDigits];
        digit_dwords(ve, de);
        digit_dwords(vo, dd);
        const int p = u >> 4, rr = (u & 15) * 8;             // superchunk, k offset in it
        const int gg = rr >> 5, m = (rr >> 4) & 1, h = (rr >> 3) & 1;
        uint8_t* dst = table + p * kSuperBytes + ((m * 4 + gg) * kDigits) * 16 + 8 * h;
#pragma unroll
        for (int j = 0; j < kDigits; ++j) *reinterpret_cast<uint2*>(dst + 16 * j) = uint2{de[j], dd[j]};
    };
    auto multiply = [&](int seg, const u4 (&wq)[RT][kPerWave]) {
        int nsc, per;
        shape(seg, nsc, per);
#pragma unroll
        for (int i = 0; i < kPerWave; ++i) {
            const int p = wave * per + i;
            if (i >= per || p >= nsc) break;
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                i4v b = {0, 0, 0, 0};
                if (r < kDigits) {
                    const u4 t = *reinterpret_cast<const u4*>(table + p * kSuperBytes + ((m * 4 + g) * kDigits + r) * 16);
                    b = i4v{(int32_t)t.x, (int32_t)t.y, (int32_t)t.z, (int32_t)t.w};
                }
#pragma unroll
                for (int t = 0; t < RT; ++t) {
                    const uint32_t w0 = m ? wq[t][i].z : wq[t][i].x, w1 = m ? wq[t][i].w : wq[t][i].y;
                    const i4v a = {(int32_t)signed_nibbles(w0, 0), (int32_t)signed_nibbles(w0, 4),
                                   (int32_t)signed_nibbles(w1, 0), (int32_t)signed_nibbles(w1, 4)};
                    acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[t], 0, 0, 0);
                }
            }
        }
    };

    u4 xa0, xa1;
    u4 wq0[RT][kPerWave], wq1[RT][kPerWave];
    if (K > 0) issue(0, xa0, wq0);
    for (int seg = 0; seg < K; seg += 2 * kSeg) {
        __syncthreads();                                     // earlier table reads are done
        build(seg, xa0);
        __syncthreads();
        if (seg + kSeg < K) issue(seg + kSeg, xa1, wq1);
        multiply(seg, wq0);
        if (seg + kSeg >= K) break;
        __syncthreads();
        build(seg + kSeg, xa1);
        __syncthreads();
        if (seg + 2 * kSeg < K) issue(seg + 2 * kSeg, xa0, wq0);
        multiply(seg + kSeg, wq1);
    }

    if (r < kDigits) {
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) part[wave][kRows * t + 4 * g + i][r] = acc[t][i];
    }
    const bool any_nonfinite = __syncthreads_or(nonfinite);
    if (tid < ROWS && row0 + tid < N) {
        const int n = row0 + tid;
        int64_t total = 0;
#pragma unroll
        for (int j = 0; j < kDigits; ++j) {
            int32_t pj = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) pj += part[w][tid][j];
            total += (int64_t)pj << (8 * j);
        }
        float s = (float)total * 0x1p-24f;                   // the exact sum, rounded once
        if (any_nonfinite) {
            const int cls = nonfinite_class(W + (size_t)n * kw, A, K);
            if (cls == 3) s = __builtin_nanf("");
            else if (cls == 1) s = __builtin_inff();
            else if (cls == 2) s = -__builtin_inff();
        }
        // fp32 subtract and multiply, then fp16 rounding: two roundings, as the reference's
        // __float2half((acc - z) * s).  Left alone, the compiler folds the multiply and the
        // conversion into one v_fma_mixlo_f16, which rounds the exact product once (measured: one
        // fp16 ulp apart in 1 of 14336 outputs); the empty asm makes the fp32 product a value of
        // its own.
        const float z = (float)__builtin_bit_cast(_Float16, zW[n]);
        const float sc = (float)__builtin_bit_cast(_Float16, sW[n]);
        float prod = (s - z) * sc;
        asm volatile("" : "+v"(prod));
        C[n] = __builtin_bit_cast(uint16_t, (_Float16)prod);
    }
}

}  // namespace

}  // namespace w4a16

using namespace w4a16;

extern "C" int w4a16_gemv(const int32_t* W, const uint16_t* A, const uint16_t* sW, const uint16_t* zW,
                          uint16_t* C, int64_t N, int64_t K, void* stream) {
    if (N < 0 || K < 0 || N >= (int64_t)1 << 31) {
        w4a16_set_last_error("dimensions out of range");
        return W4A16_ERR_INVALID;
    }
    if (K % 8 != 0) {
        w4a16_set_last_error("K must be a multiple of 8");
        return W4A16_ERR_INVALID;
    }
    if (K > W4A16_GEMV_MAX_K) {
        w4a16_set_last_error("K must be at most 1048576 (exact int32 digit sums)");
        return W4A16_ERR_INVALID;
    }
    if (N == 0) return W4A16_OK;
    if (!sW || !zW || !C || (K > 0 && (!W || !A))) {             // W and A may be empty when K == 0
        w4a16_set_last_error("null pointer");
        return W4A16_ERR_INVALID;
    }
    if (reinterpret_cast<uintptr_t>(W) % 4 != 0 ||
        (reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(sW) | reinterpret_cast<uintptr_t>(zW) |
         reinterpret_cast<uintptr_t>(C)) % 2 != 0) {
        w4a16_set_last_error("W must be 4-byte aligned, A, sW, zW and C 2-byte aligned");
        return W4A16_ERR_INVALID;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    // Two row tiles per workgroup once that still gives every CU a workgroup (N = 14336, K = 4096:
    // 448 workgroups, 10.8 -> 9.9 us); one otherwise, so a small N still keeps every CU busy.
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        w4a16_device_limits lim;
        if (w4a16_query_device(dev, &lim) == W4A16_OK && lim.cu_count > 0) cus = lim.cu_count;
    }
    const bool two = (N + 2 * kRows - 1) / (2 * kRows) >= cus;
    const dim3 grid((unsigned)((N + (two ? 2 : 1) * kRows - 1) / ((two ? 2 : 1) * kRows)));
    const bool wvec = reinterpret_cast<uintptr_t>(W) % 16 == 0 && K % 32 == 0;
    const bool xvec = reinterpret_cast<uintptr_t>(A) % 16 == 0;
    auto pick = [&](auto rt) {
        constexpr int R = decltype(rt)::value;
        return wvec ? (xvec ? gemv_kernel<true, true, R> : gemv_kernel<true, false, R>)
                    : (xvec ? gemv_kernel<false, true, R> : gemv_kernel<false, false, R>);
    };
    auto kernel = two ? pick(std::integral_constant<int, 2>{}) : pick(std::integral_constant<int, 1>{});
    hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, st, reinterpret_cast<const uint32_t*>(W), A, sW, zW, C, (int)N,
                       (int)K);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        w4a16_set_last_error(hipGetErrorString(e));
        return W4A16_ERR_HIP;
    }
    return W4A16_OK;
}
