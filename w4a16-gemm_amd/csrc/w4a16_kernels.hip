// W4A16 GEMM kernels for MI355X (gfx950): decode (M <= 16, split-K) and prefill (tiled MFMA).
//
//   y[M, N] = x[M, K] @ W^T,  W[n, k] = fp16((q[n, k] - 8) * scales[k / G, n])
//
// Both kernels read the reference's packed int32 weight format unchanged and use the operand
// mapping described in w4a16_device.h.  Host entry point: w4a16_launch (C ABI, w4a16.h).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <cstring>

#include "w4a16.h"
#include "w4a16_device.h"
#include "w4a16_internal.h"

namespace w4a16 {

// ------------------------------------------------------------------------------------ decode
// Replaces the reference decode kernel w4a16_gemm_mma (src/vectorized/decode.cuh:18-159).
//
// Grid: (N / (16*WAVES)) column tiles x `splits` K slabs, one workgroup each (slab index is the
// fastest-varying part of blockIdx.x).  Wave w of a workgroup owns n16 block
// tile*WAVES + w over KS 64-wide chunks.  All KS weight word-quads of the wave are issued up
// front (16 B per lane each) so the whole slab is in flight at once; the slab of x (M rows) is
// staged once into LDS in the permuted B-operand layout and shared by the WAVES waves.
//
// Each wave accumulates its 16 (n) x 16 (token) tile in fp32 over the slab in K order.  With
// splits > 1 the fp32 partial goes to workspace[split][m][n]; the last workgroup of a column
// tile to finish (device-scope counter) adds the partials in split order 0..splits-1 and
// writes fp16 y, then resets its counter to zero.  The summation order is therefore fixed and
// the result is deterministic run to run (reference test_deterministic, test_w4a16.py:258-261).
template <int WAVES, int KS>
__global__ void __launch_bounds__(WAVES * 64)
decode_kernel(const u4* __restrict__ Wp, const uint16_t* __restrict__ x,
              const uint16_t* __restrict__ scales, uint16_t* __restrict__ y,
              float* __restrict__ ws, int* __restrict__ counters,
              int M, int N, int K, int gshift, int splits) {
    constexpr int NT = WAVES * 64;
    constexpr int XROWB = KS * 128 + 16;            // LDS bytes per token row of the slab
    __shared__ __attribute__((aligned(16))) char xs[16 * XROWB];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int kb = lane >> 4;
    const int li = lane & 15;
    const int split = blockIdx.x % splits;
    const int tile = blockIdx.x / splits;
    const int KC = K >> 6;
    const int kc0 = split * KS;
    const int nb = tile * WAVES + wave;
    const int lanep = ((li & 7) << 2) | kb;

    // 1. the wave's weight slab: KS word quads per lane, all in flight together.
    const u4* wsrc = Wp + ((size_t)nb * KC + kc0) * 32 + lanep;
    u4 wv[KS];
#pragma unroll
    for (int c = 0; c < KS; ++c) wv[c] = __builtin_nontemporal_load(wsrc + (size_t)c * 32);
    const uint16_t* ssrc = scales + (size_t)nb * 16 + li;
    uint16_t sv[KS];
#pragma unroll
    for (int c = 0; c < KS; ++c) sv[c] = ssrc[(size_t)((kc0 + c) >> gshift) * N];

    // 2. x slab -> LDS (only the M real token rows are stored).
    const int segs = M * KS * 8;
    for (int sg = tid; sg < segs; sg += NT) {
        const int m = sg / (KS * 8);
        const int rem = sg - m * (KS * 8);
        const int c = rem >> 3;
        const int q = rem & 7;
        const u4 v = *reinterpret_cast<const u4*>(x + (size_t)m * K + (size_t)(kc0 + c) * 64 + q * 8);
        lds_store_xseg(xs + m * XROWB + c * 128, q, v);
    }
    __syncthreads();

    // 3. dequantise + MFMA over the slab in K order.
    const Dq d = dq_setup(lane);
    const bool tok_ok = li < M;
    const char* xb = xs + li * XROWB + kb * 16;
    const h8 zero8 = {};
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < KS; ++c) {
        const h2 s2 = scale2(sv[c]);
        const h8 a0 = dq_frag(wv[c].x, wv[c].y, d, s2);
        const h8 a1 = dq_frag(wv[c].z, wv[c].w, d, s2);
        const h8 b0 = tok_ok ? *reinterpret_cast<const h8*>(xb + c * 128) : zero8;
        const h8 b1 = tok_ok ? *reinterpret_cast<const h8*>(xb + c * 128 + 64) : zero8;
        acc = mfma16x16x32(a0, b0, acc);
        acc = mfma16x16x32(a1, b1, acc);
    }

    // lane holds token li, channels n .. n+3
    const int n = nb * 16 + 4 * kb;
    if (splits == 1) {
        if (tok_ok) *reinterpret_cast<u2*>(y + (size_t)li * N + n) = pack_f16x4(acc);
        return;
    }
    if (tok_ok) *reinterpret_cast<f4*>(ws + ((size_t)split * M + li) * N + n) = acc;
    __threadfence();                                  // release the partial (agent scope)
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(&counters[tile], 1) == splits - 1);
    __syncthreads();
    if (!s_last) return;
    __threadfence();                                  // acquire the other slabs' partials

    constexpr int TW4 = WAVES * 4;                    // float4 columns per tile
    const int n0 = tile * WAVES * 16;
    const size_t sstride = (size_t)M * N;
    for (int e = tid; e < M * TW4; e += NT) {
        const int m = e / TW4;
        const int c4 = e - m * TW4;
        const float* p = ws + (size_t)m * N + n0 + c4 * 4;
        f4 sum = *reinterpret_cast<const f4*>(p);
        for (int s = 1; s < splits; ++s) sum += *reinterpret_cast<const f4*>(p + (size_t)s * sstride);
        *reinterpret_cast<u2*>(y + (size_t)m * N + n0 + c4 * 4) = pack_f16x4(sum);
    }
    if (tid == 0) atomicExch(&counters[tile], 0);
}

// ----------------------------------------------------------------------------------- prefill
// Replaces the reference prefill kernel pf::w4a16_gemm_prefill (src/vectorized/prefill.cuh:27-184).
//
// Workgroup tile BM x BN (tokens x channels), WAVES_M x WAVES_N waves, wave tile WM x WN.
// K is walked sequentially in 64-wide chunks.  x chunks are double-buffered in LDS (permuted
// B layout, one barrier per chunk); each wave streams its own WN/16 weight blocks straight
// from HBM into VGPRs one chunk ahead and dequantises them in registers into MFMA A operands.
// Every accumulator receives the same MFMA sequence (chunk 0 h 0, chunk 0 h 1, chunk 1 h 0,
// ...) whatever the tile config, so all configs give bit-identical output, and token rows
// never mix (rows past M are zero-filled and not stored).
template <int BM, int BN, int WAVES_M, int WAVES_N>
__global__ void __launch_bounds__(WAVES_M * WAVES_N * 64)
prefill_kernel(const u4* __restrict__ Wp, const uint16_t* __restrict__ x,
               const uint16_t* __restrict__ scales, uint16_t* __restrict__ y,
               int M, int N, int K, int gshift, int tiles_m) {
    constexpr int NT = WAVES_M * WAVES_N * 64;
    constexpr int WM = BM / WAVES_M;
    constexpr int WN = BN / WAVES_N;
    constexpr int TM = WM / 16;
    constexpr int TN = WN / 16;
    constexpr int XBUF = BM * kXRow;
    constexpr int SEGS = BM * 8;
    constexpr int SPT = (SEGS + NT - 1) / NT;
    static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be a multiple of 16x16");
    __shared__ __attribute__((aligned(16))) char xs[2 * XBUF];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N;
    const int wn = wave - wm * WAVES_N;
    const int kb = lane >> 4;
    const int li = lane & 15;
    const int tm = blockIdx.x % tiles_m;
    const int tn = blockIdx.x / tiles_m;
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const int KC = K >> 6;
    const int NBLK = N >> 4;
    const int nb0 = (n0 >> 4) + wn * TN;
    const int lanep = ((li & 7) << 2) | kb;

    const u4* wsrc[TN];
    const uint16_t* ssrc[TN];
    bool nb_ok[TN];
#pragma unroll
    for (int b = 0; b < TN; ++b) {
        const int nb = nb0 + b;
        nb_ok[b] = nb < NBLK;
        const int nbc = nb_ok[b] ? nb : 0;
        wsrc[b] = Wp + (size_t)nbc * KC * 32 + lanep;
        ssrc[b] = scales + (size_t)nbc * 16 + li;
    }

    u4 xr[SPT];
    auto load_x = [&](int kc) {
#pragma unroll
        for (int r = 0; r < SPT; ++r) {
            const int sg = tid + r * NT;
            if (SEGS % NT == 0 || sg < SEGS) {
                const int row = sg >> 3;
                const int q = sg & 7;
                const int m = m0 + row;
                xr[r] = (m < M) ? *reinterpret_cast<const u4*>(x + (size_t)m * K + (size_t)kc * 64 + q * 8)
                                : u4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int r = 0; r < SPT; ++r) {
            const int sg = tid + r * NT;
            if (SEGS % NT == 0 || sg < SEGS)
                lds_store_xseg(xs + buf * XBUF + (sg >> 3) * kXRow, sg & 7, xr[r]);
        }
    };
    u4 wv[TN];
    uint16_t sv[TN];
    auto load_w = [&](int kc) {
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            wv[b] = nb_ok[b] ? wsrc[b][(size_t)kc * 32] : u4{0u, 0u, 0u, 0u};
            sv[b] = nb_ok[b] ? ssrc[b][(size_t)(kc >> gshift) * N] : (uint16_t)0;
        }
    };

    f4 acc[TM][TN];
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[t][b] = f4{0.f, 0.f, 0.f, 0.f};

    const Dq d = dq_setup(lane);
    load_x(0);
    load_w(0);
    store_x(0);
    __syncthreads();

    for (int kc = 0; kc < KC; ++kc) {
        u4 wc[TN];
        uint16_t sc[TN];
#pragma unroll
        for (int b = 0; b < TN; ++b) { wc[b] = wv[b]; sc[b] = sv[b]; }
        const bool more = kc + 1 < KC;
        if (more) { load_x(kc + 1); load_w(kc + 1); }

        h8 a[TN][2];
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const h2 s2 = scale2(sc[b]);
            a[b][0] = dq_frag(wc[b].x, wc[b].y, d, s2);
            a[b][1] = dq_frag(wc[b].z, wc[b].w, d, s2);
        }
        const char* xb = xs + (kc & 1) * XBUF + (wm * WM + li) * kXRow + kb * 16;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int t = 0; t < TM; ++t) {
                const h8 bf = *reinterpret_cast<const h8*>(xb + t * 16 * kXRow + h * 64);
#pragma unroll
                for (int b = 0; b < TN; ++b) acc[t][b] = mfma16x16x32(a[b][h], bf, acc[t][b]);
            }
        if (more) store_x((kc + 1) & 1);
        __syncthreads();
    }

#pragma unroll
    for (int t = 0; t < TM; ++t) {
        const int m = m0 + wm * WM + t * 16 + li;
        if (m >= M) continue;
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            if (!nb_ok[b]) continue;
            const int n = (nb0 + b) * 16 + 4 * kb;
            *reinterpret_cast<u2*>(y + (size_t)m * N + n) = pack_f16x4(acc[t][b]);
        }
    }
}

// ------------------------------------------------------------------------------------ launch

template <int CFG> struct PrefillCfg;
#define W4A16_PREFILL_CFG(ID)                                                                  \
    template <> struct PrefillCfg<ID> {                                                        \
        static constexpr int BM = kPrefillTable[ID].bm, BN = kPrefillTable[ID].bn;             \
        static constexpr int WM = kPrefillTable[ID].waves_m, WN = kPrefillTable[ID].waves_n;   \
    };
W4A16_PREFILL_CFG(1)
W4A16_PREFILL_CFG(2)
W4A16_PREFILL_CFG(3)
W4A16_PREFILL_CFG(4)
#undef W4A16_PREFILL_CFG

template <int CFG>
static hipError_t launch_prefill(const w4a16_plan& p, const u4* Wp, const uint16_t* x,
                                 const uint16_t* s, uint16_t* y, hipStream_t st) {
    using C = PrefillCfg<CFG>;
    const int gshift = p.G == 128 ? 1 : 0;
    const int tiles_m = (p.M + C::BM - 1) / C::BM;
    hipLaunchKernelGGL((prefill_kernel<C::BM, C::BN, C::WM, C::WN>), dim3(p.grid),
                       dim3(C::WM * C::WN * 64), 0, st, Wp, x, s, y, p.M, p.N, p.K, gshift, tiles_m);
    return hipGetLastError();
}

template <int KS>
static hipError_t launch_decode(const w4a16_plan& p, const u4* Wp, const uint16_t* x,
                                const uint16_t* s, uint16_t* y, float* ws, int* cnt, hipStream_t st) {
    const int gshift = p.G == 128 ? 1 : 0;
    hipLaunchKernelGGL((decode_kernel<kDecodeWaves, KS>), dim3(p.grid), dim3(kDecodeWaves * 64), 0, st,
                       Wp, x, s, y, ws, cnt, p.M, p.N, p.K, gshift, p.splits);
    return hipGetLastError();
}

}  // namespace w4a16

using namespace w4a16;

extern "C" int w4a16_launch(const w4a16_plan* plan, const int32_t* Wp, const uint16_t* x,
                            const uint16_t* scales, uint16_t* y, void* workspace, int32_t* counters,
                            void* stream) {
    if (!plan) return W4A16_ERR_INVALID;
    const w4a16_plan& p = *plan;
    if (p.grid <= 0 || p.M <= 0 || p.N <= 0 || p.K <= 0) return W4A16_OK;   // empty output
    if (p.workspace_bytes && !workspace) return W4A16_ERR_WORKSPACE;
    if (p.counter_slots && !counters) return W4A16_ERR_WORKSPACE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const u4* wp = reinterpret_cast<const u4*>(Wp);
    hipError_t e = hipSuccess;
    if (p.kernel == W4A16_VARIANT_DECODE) {
        float* ws = reinterpret_cast<float*>(workspace);
        int* cnt = reinterpret_cast<int*>(counters);
        switch (p.slab_chunks) {
            case 4:  e = launch_decode<4>(p, wp, x, scales, y, ws, cnt, st); break;
            case 8:  e = launch_decode<8>(p, wp, x, scales, y, ws, cnt, st); break;
            case 16: e = launch_decode<16>(p, wp, x, scales, y, ws, cnt, st); break;
            default: return W4A16_ERR_INVALID;
        }
    } else {
        switch (p.kernel) {
            case 1: e = launch_prefill<1>(p, wp, x, scales, y, st); break;
            case 2: e = launch_prefill<2>(p, wp, x, scales, y, st); break;
            case 3: e = launch_prefill<3>(p, wp, x, scales, y, st); break;
            case 4: e = launch_prefill<4>(p, wp, x, scales, y, st); break;
            default: return W4A16_ERR_INVALID;
        }
    }
    if (e != hipSuccess) {
        w4a16_set_last_error(hipGetErrorString(e));
        return W4A16_ERR_HIP;
    }
    return W4A16_OK;
}
