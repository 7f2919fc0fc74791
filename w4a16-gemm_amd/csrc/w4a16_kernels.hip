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
#include <mutex>

#include "w4a16.h"
#include "w4a16_asm.h"
#include "w4a16_device.h"
#include "w4a16_internal.h"

namespace w4a16 {

// Cache policy of the decode kernels' weight DMAs: nontemporal (`nt`), since a decode call reads
// every weight byte exactly once (aux operand of __builtin_amdgcn_global_load_lds: 1 = sc0,
// 2 = nt, 16 = sc1 on gfx950).
constexpr int kWeightStreamPolicy = 2;

// ------------------------------------------------------------------------------------ decode
// Replaces the reference decode kernel w4a16_gemm_mma (src/vectorized/decode.cuh:18-159).
//
// Workgroup = WAVES waves on one column tile of NBW n16 blocks (16*NBW output channels); the
// waves split the workgroup's K range, wave w taking `kcw` consecutive 64-wide chunks.  Each
// wave streams its weight word quads and its x fragments straight from memory into VGPRs
// (software pipeline of depth D chunks), dequantises in registers and accumulates with MFMA.
// The x fragment of a chunk half is one 16-byte load of 8 consecutive halves per lane followed
// by a 4x4 transpose across the four 16-lane rows (v_permlane32_swap + v_permlane16_swap),
// which yields the B operand layout of w4a16_device.h without LDS.  Token rows >= M load row
// M-1; such columns of the MFMA only feed outputs that are never stored.
//
// The WAVES partial tiles are summed through LDS in wave order.  When the K range is split
// over `splits` workgroups (grid = column tiles x splits, split fastest), each workgroup's fp32
// tile goes to workspace[split][m][n] and the last workgroup of the column tile to arrive
// (device-scope counter) adds the partials in split order and writes fp16 y.  Every sum is in a
// fixed order, so results are deterministic (reference test_deterministic, test_w4a16.py:258).

// 4x4 transpose of dwords across the four 16-lane rows: lane (row r, p) holds v[e] = D[r][e]
// on entry and D[e][r] on exit.
__device__ __forceinline__ u4 xpose_rows(u4 v) {
    const auto a = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto e = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    return u4{c[0], c[1], e[0], e[1]};
}

// Final stage shared by the decode kernels.  Thread (rb, lane) of the first NBW waves holds the
// workgroup's fp32 result for token li and channels n..n+3 of n16 block nb0+rb (`have`).  With
// one split it is rounded to fp16 and stored.  Otherwise it is handed to the last workgroup of
// the column tile through the workspace (see the decode comment above) and summed in split order.
template <int NBW, int WAVES>
__device__ __forceinline__ void decode_finish(f4 sum, bool have, int rb, int lane, int split, int tile, int nb0,
                                              uint16_t* __restrict__ y, float* __restrict__ ws,
                                              int* __restrict__ counters, int M, int N, int splits) {
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int kb = lane >> 4;
    const int li = lane & 15;
    const int n = (nb0 + rb) * 16 + 4 * kb;
    const bool mine = have && li < M;
    if (splits == 1) {
        if (mine) *reinterpret_cast<u2*>(y + (size_t)li * N + n) = pack_f16x4(sum);
        return;
    }
    // Split-K hand-off without agent-scope fences (those write back / invalidate the XCD's whole
    // L2): the partials travel through agent-scope atomic stores/loads, which are coherent at
    // device scope by themselves, and every wave waits for its stores to complete
    // (s_waitcnt vmcnt(0)) before the workgroup's counter RMW.
    if (mine) {
        unsigned long long* p = reinterpret_cast<unsigned long long*>(ws + ((size_t)split * M + li) * N + n);
        const u4 bits = __builtin_bit_cast(u4, sum);
        __hip_atomic_store(p, (unsigned long long)bits.x | ((unsigned long long)bits.y << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p + 1, (unsigned long long)bits.z | ((unsigned long long)bits.w << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // Wrapping increment (old >= splits - 1 ? 0 : old + 1): the last arrival sees splits - 1 and
    // the same instruction returns the counter to zero, so every launch leaves it zero without a
    // separate reset store.
    if (tid == 0)
        s_last = __builtin_amdgcn_atomic_inc32(reinterpret_cast<unsigned*>(&counters[tile]), (unsigned)(splits - 1),
                                               __ATOMIC_RELAXED, "agent") == (unsigned)(splits - 1);
    __syncthreads();
    if (!s_last) return;

    // Last arrival: thread (m, c4) adds the `splits` partials of its 4 channels in split order,
    // issuing the loads of up to 8 splits at once.
    constexpr int C4 = NBW * 4;                              // float4 groups per row of the tile
    if (tid < M * C4) {
        const int m = tid / C4;
        const int c4 = tid - m * C4;
        const int nn = nb0 * 16 + c4 * 4;
        const unsigned long long* p = reinterpret_cast<const unsigned long long*>(ws + (size_t)m * N + nn);
        const size_t sstride = (size_t)M * N / 2;           // in 8-byte words
        f4 tot = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < splits; s0 += 8) {
            unsigned long long lo[8], hi[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (s0 + j < splits) {
                    lo[j] = __hip_atomic_load(p + (size_t)(s0 + j) * sstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    hi[j] = __hip_atomic_load(p + (size_t)(s0 + j) * sstride + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (s0 + j < splits) {
                    const f4 v = __builtin_bit_cast(f4, u4{(uint32_t)lo[j], (uint32_t)(lo[j] >> 32),
                                                           (uint32_t)hi[j], (uint32_t)(hi[j] >> 32)});
                    tot = (s0 + j == 0) ? v : tot + v;
                }
        }
        *reinterpret_cast<u2*>(y + (size_t)m * N + nn) = pack_f16x4(tot);
    }
}

// Output of a prefill tile whose lanes hold TM x NB 16x16 fp32 fragments (lane (kb, li): token
// m0 + 16 t + li, channels 16 (nb0 + b) + 4 kb .. + 3).  One K segment per workgroup
// (splits > 1, the canonical segments of prefill_segment_chunks): the fragments go to
// ws[seg][m][n] (agent-scope atomic stores, as in decode_finish), and the last of the `splits`
// workgroups of the tile adds the partials of every segment in segment order (total = p0, then
// total + p_s) and stores fp16.  splits == 1: stored directly.  Rows past M and blocks past
// N are neither stored nor read.
template <int TM, int NB>
__device__ __forceinline__ void prefill_tile_out(const f4 (&acc)[TM][NB], int m0, int nb0, int lane,
                                                 uint16_t* __restrict__ y, float* __restrict__ ws,
                                                 int* __restrict__ counters, int M, int N, int seg, int splits,
                                                 int tile) {
    const int kb = lane >> 4;
    const int li = lane & 15;
    const int NBLK = N >> 4;
    if (splits == 1) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (nb0 + b >= NBLK) break;
#pragma unroll
            for (int t = 0; t < TM; ++t) {
                const int m = m0 + 16 * t + li;
                if (m < M) *reinterpret_cast<u2*>(y + (size_t)m * N + (nb0 + b) * 16 + 4 * kb) = pack_f16x4(acc[t][b]);
            }
        }
        return;
    }
    __shared__ int s_last;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (nb0 + b >= NBLK) break;
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const int m = m0 + 16 * t + li;
            if (m >= M) continue;
            unsigned long long* q =
                reinterpret_cast<unsigned long long*>(ws + ((size_t)seg * M + m) * N + (nb0 + b) * 16 + 4 * kb);
            const u4 bits = __builtin_bit_cast(u4, acc[t][b]);
            __hip_atomic_store(q, (unsigned long long)bits.x | ((unsigned long long)bits.y << 32), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(q + 1, (unsigned long long)bits.z | ((unsigned long long)bits.w << 32), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __builtin_amdgcn_atomic_inc32(reinterpret_cast<unsigned*>(&counters[tile]), (unsigned)(splits - 1),
                                               __ATOMIC_RELAXED, "agent") == (unsigned)(splits - 1);
    __syncthreads();
    if (!s_last) return;
    const size_t sstride = (size_t)M * N / 2;                // one segment, in 8-byte words
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (nb0 + b >= NBLK) break;
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const int m = m0 + 16 * t + li;
            if (m >= M) continue;
            const unsigned long long* q =
                reinterpret_cast<const unsigned long long*>(ws + (size_t)m * N + (nb0 + b) * 16 + 4 * kb);
            f4 tot = {0.f, 0.f, 0.f, 0.f};
            for (int sg = 0; sg < splits; ++sg) {
                const unsigned long long lo = __hip_atomic_load(q + sg * sstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const unsigned long long hi = __hip_atomic_load(q + sg * sstride + 1, __ATOMIC_RELAXED,
                                                                __HIP_MEMORY_SCOPE_AGENT);
                const f4 v = __builtin_bit_cast(f4, u4{(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)});
                tot = sg == 0 ? v : tot + v;
            }
            *reinterpret_cast<u2*>(y + (size_t)m * N + (nb0 + b) * 16 + 4 * kb) = pack_f16x4(tot);
        }
    }
}

template <int NBW, int WAVES, int D>
__global__ void __launch_bounds__(WAVES * 64)
decode_kernel(const u4* __restrict__ Wp, const uint16_t* __restrict__ x,
              const uint16_t* __restrict__ scales, int M, int N, int K, int gshift, int splits, int kcw,
              uint16_t* __restrict__ y, float* __restrict__ ws, int* __restrict__ counters) {
    __shared__ __attribute__((aligned(16))) f4 red[WAVES][NBW][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int kb = lane >> 4;
    const int li = lane & 15;
    const int split = blockIdx.x % splits;
    const int tile = blockIdx.x / splits;
    const int KC = K >> 6;
    const int kc0 = (split * WAVES + wave) * kcw;           // this wave's first chunk
    const int nb0 = tile * NBW;
    const int lanep = ((li & 7) << 2) | kb;

    const u4* wsrc[NBW];
    const uint16_t* ssrc[NBW];
#pragma unroll
    for (int b = 0; b < NBW; ++b) {
        wsrc[b] = Wp + ((size_t)(nb0 + b) * KC + kc0) * 32 + lanep;
        ssrc[b] = scales + (size_t)(nb0 + b) * 16 + li;
    }
    const uint16_t* xsrc = x + (size_t)min(li, M - 1) * K + (size_t)kc0 * 64 + kb * 8;

    u4 wq[D][NBW];
    u4 xq[D][2];
    uint16_t sq[D][NBW];
    auto issue = [&](int c, int slot) {
#pragma unroll
        for (int b = 0; b < NBW; ++b) wq[slot][b] = __builtin_nontemporal_load(wsrc[b] + (size_t)c * 32);
        xq[slot][0] = *reinterpret_cast<const u4*>(xsrc + (size_t)c * 64);
        xq[slot][1] = *reinterpret_cast<const u4*>(xsrc + (size_t)c * 64 + 32);
#pragma unroll
        for (int b = 0; b < NBW; ++b) sq[slot][b] = ssrc[b][(size_t)((kc0 + c) >> gshift) * N];
    };

    const Dq d = dq_setup(lane);
    f4 acc[NBW];
#pragma unroll
    for (int b = 0; b < NBW; ++b) acc[b] = f4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int i = 0; i < D; ++i)
        if (i < kcw) issue(i, i);
    for (int c0 = 0; c0 < kcw; c0 += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            if (c0 + i >= kcw) break;
            const h8 b0 = __builtin_bit_cast(h8, xpose_rows(xq[i][0]));
            const h8 b1 = __builtin_bit_cast(h8, xpose_rows(xq[i][1]));
#pragma unroll
            for (int b = 0; b < NBW; ++b) {
                const h2 s2 = scale2(sq[i][b]);
                const h8 a0 = dq_frag(wq[i][b].x, wq[i][b].y, d, s2);
                const h8 a1 = dq_frag(wq[i][b].z, wq[i][b].w, d, s2);
                acc[b] = mfma16x16x32(a0, b0, acc[b]);
                acc[b] = mfma16x16x32(a1, b1, acc[b]);
            }
            if (c0 + D + i < kcw) issue(c0 + D + i, i);
        }
    }

    // Cross-wave reduction in wave order.
#pragma unroll
    for (int b = 0; b < NBW; ++b) red[wave][b][lane] = acc[b];
    __syncthreads();
    f4 sum = {0.f, 0.f, 0.f, 0.f};
    const int rb = tid >> 6;                                // n16 block this thread finishes
    if (tid < NBW * 64) {
        sum = red[0][rb][lane];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) sum += red[w][rb][lane];
    }
    decode_finish<NBW, WAVES>(sum, tid < NBW * 64, rb, lane, split, tile, nb0, y, ws, counters, M, N, splits);
}


// Decode with a per-wave software pipeline over a ring of D chunk pairs in LDS.  Each wave walks
// a long K range (kcw chunks, kcw even) pair by pair: while it dequantises and multiplies pair p,
// pairs p+1..p+D-1 are in flight (weights by direct-to-LDS loads, x fragments and scales by
// untracked VGPR loads), and pair p+D is issued into the slot it just consumed.  Compute thus
// follows the memory stream instead of waiting for a wave's whole range.  Issue order per pair is
// x, scales, then the NBW weight DMAs (OPS operations), so waiting for pair p is
// s_waitcnt vmcnt(OPS * #pairs issued after p).  Reduction and split-K hand-off as above.
template <int NBW, int WAVES, int D>
__global__ void __launch_bounds__(WAVES * 64)
decode_stream_kernel(const u4* __restrict__ Wp, const uint16_t* __restrict__ x,
                     const uint16_t* __restrict__ scales, int M, int N, int K, int gshift, int splits, int kcw,
                     uint16_t* __restrict__ y, float* __restrict__ ws, int* __restrict__ counters) {
    constexpr int SLOT = NBW * 1024;                         // [n16 block][2 chunks][512 B]
    constexpr int WAVE_BYTES = D * SLOT;
    constexpr int OPS = 4 + 2 * NBW + NBW;                   // x loads + scale loads + DMAs per pair
    static_assert((D - 1) * OPS <= 63, "too many loads in flight for vmcnt");
    __shared__ __attribute__((aligned(16))) char wl[WAVES * WAVE_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int kb = lane >> 4;
    const int li = lane & 15;
    const int split = blockIdx.x % splits;
    const int tile = blockIdx.x / splits;
    const int KC = K >> 6;
    const int kc0 = (split * WAVES + wave) * kcw;
    const int nb0 = tile * NBW;
    const int lanep = ((li & 7) << 2) | kb;
    const int npair = kcw >> 1;
    char* wreg = wl + wave * WAVE_BYTES;
    const uint32_t wlds = (uint32_t)reinterpret_cast<uintptr_t>(wreg) + lanep * 16;

    const uint16_t* xsrc = x + (size_t)min(li, M - 1) * K + (size_t)kc0 * 64 + kb * 8;
    const u4* wsrc = Wp + ((size_t)nb0 * KC + kc0) * 32 + lane;
    const uint16_t* ssrc = scales + (size_t)nb0 * 16 + li;

    u4 xq[D][4];                                             // chunk 2p: h0, h1; chunk 2p+1: h0, h1
    uint32_t sq[D][NBW][2];
    auto issue = [&](int p, int slot) {
        const int c = 2 * p;
#pragma unroll
        for (int j = 0; j < 4; ++j) xq[slot][j] = gload_u4_untracked(xsrc + (size_t)c * 64 + 32 * j);
#pragma unroll
        for (int b = 0; b < NBW; ++b)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                sq[slot][b][j] = gload_u16_untracked(ssrc + (size_t)((kc0 + c + j) >> gshift) * N + b * 16);
#pragma unroll
        for (int b = 0; b < NBW; ++b) {
            auto* dst = (__attribute__((address_space(3))) void*)(wreg + slot * SLOT + b * 1024);
            __builtin_amdgcn_global_load_lds(wsrc + (size_t)b * KC * 32 + (size_t)c * 32, dst, 16, 0, kWeightStreamPolicy);
        }
        asm volatile("" ::: "memory");
    };

    const Dq d = dq_setup(lane);
    f4 acc[NBW];
#pragma unroll
    for (int b = 0; b < NBW; ++b) acc[b] = f4{0.f, 0.f, 0.f, 0.f};

    // Consume ring slot s (pair p): x/scales/weights of the pair are complete when this runs.
    auto consume = [&](int s) {
#pragma unroll
        for (int j = 0; j < 4; ++j) bind_after_wait(xq[s][j]);
#pragma unroll
        for (int b = 0; b < NBW; ++b) { bind_after_wait(sq[s][b][0]); bind_after_wait(sq[s][b][1]); }
        u4 wv[2][NBW];
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int b = 0; b < NBW; ++b) wv[cc][b] = lds_read_u4(wlds + s * SLOT + b * 1024 + cc * 512);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int b = 0; b < NBW; ++b) bind_after_wait(wv[cc][b]);
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const h8 b0 = __builtin_bit_cast(h8, xpose_rows(xq[s][2 * cc]));
            const h8 b1 = __builtin_bit_cast(h8, xpose_rows(xq[s][2 * cc + 1]));
#pragma unroll
            for (int b = 0; b < NBW; ++b) {
                const h2 s2 = scale2((uint16_t)sq[s][b][cc]);
                acc[b] = mfma16x16x32(dq_frag(wv[cc][b].x, wv[cc][b].y, d, s2), b0, acc[b]);
                acc[b] = mfma16x16x32(dq_frag(wv[cc][b].z, wv[cc][b].w, d, s2), b1, acc[b]);
            }
        }
    };

    // Straight-line prologue (npair >= D, npair % D == 0: enforced by the planner), a steady-state
    // loop that always has D-1 pairs in flight behind the one it consumes, and a straight-line
    // epilogue that drains the ring.  Every wait count is a compile-time constant.
#pragma unroll
    for (int s = 0; s < D; ++s) issue(s, s);
    for (int p0 = 0; p0 + D < npair; p0 += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            wait_vmcnt<(D - 1) * OPS>();
            consume(s);
            issue(p0 + D + s, s);
        }
    }
    static_for<0, D>([&](auto t) {
        constexpr int T = decltype(t)::value;
        wait_vmcnt<(D - 1 - T) * OPS>();
        consume(T);
    });

    // Cross-wave reduction in wave order; each wave parks its tile in its own LDS region.
    f4* red = reinterpret_cast<f4*>(wreg);
#pragma unroll
    for (int b = 0; b < NBW; ++b) red[b * 64 + lane] = acc[b];
    __syncthreads();
    f4 sum = {0.f, 0.f, 0.f, 0.f};
    const int rb = tid >> 6;
    if (tid < NBW * 64) {
        sum = reinterpret_cast<const f4*>(wl)[rb * 64 + lane];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) sum += reinterpret_cast<const f4*>(wl + w * WAVE_BYTES)[rb * 64 + lane];
    }
    decode_finish<NBW, WAVES>(sum, tid < NBW * 64, rb, lane, split, tile, nb0, y, ws, counters, M, N, splits);
}

#ifdef W4A16_WAVE_STAMPS
// Instrumented builds only (-DW4A16_WAVE_STAMPS: libw4a16_hip_stamps.so, built by build.py for
// wave_timeline.py; the product library has none of this).  Lane 0 of every decode-ring wave
// records the chip-wide 100 MHz clock (s_memrealtime) at kernel entry, after the prologue's loads
// are issued, after its first pair is consumed, when its stream is done (before the cross-wave
// reduction) and after its part of the output (y or partials) is written and acknowledged, plus
// the wave's HW_ID and XCC_ID registers and its workgroup index: kStampWords words per wave,
// indexed by blockIdx.x * WAVES + wave; waves past kStampWaves record nothing.
constexpr int kStampWaves = 8192;
constexpr int kStampWords = 8;
__device__ uint32_t g_wave_stamps[kStampWaves * kStampWords];
__device__ __forceinline__ uint32_t stamp_clock() { return (uint32_t)__builtin_amdgcn_s_memrealtime(); }
#endif

// Decode with a refill-ahead ring of chunk pairs (kind 3).
//
// Work split as in decode_stream_kernel: WAVES waves per column tile of NBW n16 blocks, each
// wave walking its kcw chunks pair by pair.  Differences:
//  * The ring has D + 1 slots and the loads of pair p + D are issued BEFORE pair p is
//    dequantised and multiplied, so the memory system always holds D pairs of every wave,
//    also while the wave computes.
//  * A pair's x rows (XR rows; rows >= M repeat row M-1) arrive in the slot by direct-to-LDS
//    loads next to the weights.  The B operand of lane (kb, j) for MFMA half h of chunk cc is
//    dwords 16h + 4c + kb (c = 0..3) of row j's chunk, a stride-4 gather:
//      - XR >= 4 (M >= 2): 16-byte loads of 4 rows each (XR/4 per pair), 16-byte segments
//        XOR-swizzled by row; the B operand is four 4-byte LDS reads from the swizzled segments
//        (a 4-byte read is served 32 lanes at a time from 32 banks: lanes (kb, j) with kb = 0, 1
//        use dwords 0, 1 of their rows' segments; the reads of 8 distinct rows hit distinct banks,
//        and with 16 rows, rows 8..15 sit 8 bytes further on, so they use the segments' dwords
//        2, 3 and the 32 lanes hit 32 distinct banks; unshifted, rows r and r + 8 shared a bank
//        and every such read cost two extra cycles, 0.46-0.92 M conflict cycles per launch);
//      - XR == 1 (M == 1): one 4-byte load per pair in which each lane picks the dword it
//        fetches so that the row lands already in B-operand order (16-byte unit 8cc + 4h + kb
//        holds dwords 16h + 4c + kb of chunk cc); the B operand is one 16-byte LDS read and the
//        pair moves 256 bytes of x instead of 4 rows' 1 KB.
//    Either way no cross-lane transpose (VALU) is needed.
//  * The pair's scales ([chunk][block][16 channels], 64*NBW bytes) ride in the same slot: one
//    16-byte direct-to-LDS load with 4*NBW active lanes per pair, so no scale traffic sits in
//    front of the first pair.  Per pair the wave issues NBW + XD + 1 memory instructions
//    (XD = 1 for XR == 1, XR / 4 otherwise).
//  * Weight segments are stored transposed (segment (i % 8) + 8*kb of a chunk holds packed lane
//    4*(i % 8) + kb), so the 16-byte A-operand reads of 8 consecutive lanes are conflict-free.
//  * The steady-state loop is unrolled by the ring size, so every slot offset is a compile-time
//    constant carried in the LDS instructions' offset fields; per-lane LDS bases and global
//    offsets are computed once, the per-pair advance is wave-uniform (scalar registers).
//    Apart from the dequantisation the loop does almost no vector arithmetic.
// Dequantisation is dq_frag, bit-identical to the reference's fp16 subtract-then-multiply.
// Every ring load runs with all 64 lanes active (clamped addresses), so each pair is exactly
// OPS vector-memory instructions and the vmcnt arithmetic is exact.
// Argument order: everything the prologue needs before its first load (the three input pointers,
// the shape, the split and the grid size, 14 dwords) comes first, so that with kernel-argument
// preloading (build.py: -amdgpu-kernarg-preload-count=16) it arrives in SGPRs with the wave and
// the first loads issue without waiting for an s_load of the argument segment; y and the split-K
// buffers, used only at the end, come last.  The grid size is an argument for the same reason
// (gridDim.x is read from the implicit arguments).  Measured: 0.1-0.3 us per call faster on the
// gate/up and long-K calls at M >= 4, level at M = 1 on down and on configs[0].
template <int NBW, int WAVES, int D, int XR>
__global__ void __launch_bounds__(WAVES * 64)
decode_ring_kernel(const u4* __restrict__ Wp, const uint16_t* __restrict__ x,
                   const uint16_t* __restrict__ scales,
                   int M, int N, int K, int gshift, int splits, int kcw, int xcd_remap, int nwg,
                   uint16_t* __restrict__ y, float* __restrict__ ws, int* __restrict__ counters) {
    constexpr int S = D + 1;                                 // ring slots
    constexpr int WSLOT = NBW * 1024;                        // [n16 block][chunk][32 x 16 B]
    constexpr int XHI = XR == 16 ? 8 : 0;                    // shift of rows 8..15 (bank spread)
    constexpr int XSLOT = XR * 256 + (XHI ? 16 : 0);         // [XR rows][16 x 16 B], 16-byte aligned
    constexpr int SCOFF = WSLOT + XSLOT;                     // [chunk][block][16 halves]
    constexpr int SLOT = SCOFF + 64 * NBW;
    constexpr int WAVE_BYTES = S * SLOT;
    constexpr int XD = XR == 1 ? 1 : XR / 4;                 // x loads per pair
    constexpr int OPS = NBW + XD + 1;
    static_assert((D - 1) * OPS <= 63, "too many loads in flight for vmcnt");
    static_assert(WAVES >= NBW && WAVE_BYTES >= NBW * 1024, "reduction layout");
    static_assert(S * SLOT < 65536, "slot offsets must fit the LDS offset field");
    static_assert(XR == 1 || XR == 4 || XR == 8 || XR == 16, "x rows per slot");
    __shared__ __attribute__((aligned(16))) char wl[WAVES * WAVE_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kb = lane >> 4;
    const int li = lane & 15;
#ifdef W4A16_WAVE_STAMPS
    const uint32_t st_entry = stamp_clock();
    uint32_t st_first = 0;
#endif
    // Workgroups are dealt to the 8 XCDs round-robin (b % 8).  With xcd_remap, give each XCD a
    // contiguous range of (tile, split) indices, so that neighbouring column tiles -- which share
    // the 128-byte lines of every scale row -- meet in one L2.  A bijection: the results do not
    // depend on it.  Without it the fetch from beyond L2 grows from 1.01-1.06x to 1.10-1.15x of
    // the algorithmic bytes on the long-K shapes (each scale line is then fetched by several
    // XCDs).  The host turns it off when the grid exceeds the CU count (gate/up, 448 workgroups):
    // there the plain order was 0.1-0.3 us faster per call in alternating runs; and for four-block
    // tiles at K <= 4096 (gate/up M = 7..16, 224 workgroups: M = 8 0.06-0.27 us and M = 16
    // 0.10-0.24 us faster plain, order-rotated runs on three boxes), while four-block tiles at
    // K = 8192 measured 0.14-0.24 us slower plain and narrower tiles at K = 4096 level.
    const int bid = xcd_remap && (nwg & 7) == 0 ? (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const int split = bid % splits;
    const int tile = bid / splits;
    const int KC = K >> 6;
    // The workgroup's waves interleave over its K range: wave w takes chunk pairs w, w + WAVES,
    // w + 2*WAVES, ..., so each step of the ring reads 1 KB x WAVES of contiguous weights per
    // block (measured faster than a contiguous range per wave, whose waves stream 1 KB pieces
    // of separate regions).
    const int kc0 = split * WAVES * kcw + 2 * wave;
    const int nb0 = tile * NBW;
    const int npair = kcw >> 1;
    char* wreg = wl + wave * WAVE_BYTES;
    const uint32_t lds_wave = (uint32_t)reinterpret_cast<uintptr_t>(wreg);

    // Ring load sources: a base that advances per pair plus a fixed per-lane byte offset.
    // Weights: lane j fills segment j & 31 of chunk j >> 5 with packed lane 4*(seg % 8) + seg / 8.
    // x, XR >= 4: lane j of load q fills row r = (64q + j) / 16, segment j % 16, with global
    // segment (j % 16) ^ (r % 8) of row min(r, M - 1); rows 8..15 start XHI bytes later.
    // x, XR == 1: lane j fills dword j of the row's 256 bytes, i.e. dword e = j % 4 of unit
    // u = j / 4 (chunk u / 8, half (u / 4) % 2, lane group u % 4), so it fetches dword
    // 32*(u/8) + 16*((u/4)%2) + 4e + u%4 of the row's pair.
    const int wseg = lane & 31;
    const uint32_t woff_g = (uint32_t)((((lane >> 5) * 32) + 4 * (wseg & 7) + (wseg >> 3)) * 16);
    const char* wbase_g = reinterpret_cast<const char*>(Wp) + ((size_t)nb0 * KC + kc0) * 512;
    // Scales: lane e < 4*NBW fills entry e = [chunk cc][block b][half] (8 channels) with the
    // scales of chunk kc0 + 2*WAVES*p + cc; the group advances by WAVES * (2 >> gshift) per pair.
    const int se = min(lane, 4 * NBW - 1);
    const char* ssrc = reinterpret_cast<const char*>(
        scales + (size_t)((kc0 + se / (2 * NBW)) >> gshift) * N + (size_t)(nb0 + (se >> 1) % NBW) * 16 + (se & 1) * 8);
    const size_t sstep = (size_t)(2 >> gshift) * N * 2;      // bytes per chunk pair
    const char* xsrc[XD];
    if constexpr (XR == 1) {
        const int u = lane >> 2;
        xsrc[0] = reinterpret_cast<const char*>(x) + (size_t)kc0 * 128 +
                  (32 * (u >> 3) + 16 * ((u >> 2) & 1) + 4 * (lane & 3) + (u & 3)) * 4;
    } else {
#pragma unroll
        for (int q = 0; q < XD; ++q) {
            const int r = (64 * q + lane) >> 4;
            const int gseg = (lane & 15) ^ (r & 7);
            xsrc[q] = reinterpret_cast<const char*>(x + (size_t)min(r, M - 1) * K + (size_t)kc0 * 64 + gseg * 8);
        }
    }
    // The same sources as a wave-uniform base plus a 32-bit lane offset, for the 8- and 16-wave
    // rings (SGPR-base DMAs below).  kc0 is even (the chunks per wave are), so the scale row of
    // chunk kc0 + cc is (kc0 >> gshift) + (cc >> gshift), cc = se / (2 * NBW) in {0, 1}.  The x
    // offset is below 15 * K * 2 + 256 bytes: decode_shape_fits keeps K < 2^27 for these rings.
    const char* sbase_g = reinterpret_cast<const char*>(scales + (size_t)(kc0 >> gshift) * N + (size_t)nb0 * 16);
    const uint32_t soff_g = (uint32_t)((((se / (2 * NBW)) >> gshift) * N + ((se >> 1) % NBW) * 16 + (se & 1) * 8) * 2);
    const char* xbase_g = reinterpret_cast<const char*>(x) + (size_t)kc0 * 128;
    uint32_t xoff_g[XD];
    if constexpr (XR == 1) {
        const int u = lane >> 2;
        xoff_g[0] = (uint32_t)((32 * (u >> 3) + 16 * ((u >> 2) & 1) + 4 * (lane & 3) + (u & 3)) * 4);
    } else {
#pragma unroll
        for (int q = 0; q < XD; ++q) {
            const int r = (64 * q + lane) >> 4;
            const int gseg = (lane & 15) ^ (r & 7);
            xoff_g[q] = (uint32_t)min(r, M - 1) * (uint32_t)K * 2u + (uint32_t)gseg * 16u;
        }
    }
    // One pair's loads into ring slot `slot`.  The 8- and 16-wave rings issue them through asm with
    // SGPR bases, which keeps the per-pair address arithmetic out of the VALU (the dequantisation
    // already keeps the VALU busy); in alternating runs on two boxes: gate/up M = 16 0.22-0.24 us
    // per call faster, down M = 1, 4, 8 0.03-0.13 us, the 70B MLP shapes 0.7-4.7%, configs[0]
    // 0.02 us slower.  The 4-wave rings measured level to 1.2% slower that way and keep the
    // builtin (64-bit per-lane pointers).
    static_assert(kWeightStreamPolicy == 2, "the asm weight DMAs below are written with the nt policy");
    auto issue = [&](int p, auto slot) {
        if constexpr (WAVES >= 8) {
            const uint32_t sl = lds_wave + decltype(slot)::value * SLOT;
#pragma unroll
            for (int b = 0; b < NBW; ++b)
                dma16_sbase_nt(wbase_g + (size_t)b * KC * 512 + (size_t)p * (1024 * WAVES), woff_g, sl + b * 1024);
            if constexpr (XR == 1) {
                dma4_sbase(xbase_g + (size_t)p * (256 * WAVES), xoff_g[0], sl + WSLOT);
            } else {
#pragma unroll
                for (int q = 0; q < XD; ++q)
                    dma16_sbase(xbase_g + (size_t)p * (256 * WAVES), xoff_g[q], sl + WSLOT + q * 1024 + (q >= 2 ? XHI : 0));
            }
            if (lane < 4 * NBW)
                dma16_sbase(sbase_g + (size_t)p * (sstep * WAVES), soff_g, sl + SCOFF);
        } else {
            char* sl = wreg + decltype(slot)::value * SLOT;
#pragma unroll
            for (int b = 0; b < NBW; ++b)
                __builtin_amdgcn_global_load_lds((const void*)(wbase_g + (size_t)b * KC * 512 + (size_t)p * (1024 * WAVES) + woff_g),
                                                 (__attribute__((address_space(3))) void*)(sl + b * 1024), 16, 0,
                                                 kWeightStreamPolicy);
            if constexpr (XR == 1) {
                __builtin_amdgcn_global_load_lds((const void*)(xsrc[0] + (size_t)p * (256 * WAVES)),
                                                 (__attribute__((address_space(3))) void*)(sl + WSLOT), 4, 0, 0);
            } else {
#pragma unroll
                for (int q = 0; q < XD; ++q)
                    __builtin_amdgcn_global_load_lds((const void*)(xsrc[q] + (size_t)p * (256 * WAVES)),
                                                     (__attribute__((address_space(3))) void*)(sl + WSLOT + q * 1024 +
                                                                                               (q >= 2 ? XHI : 0)),
                                                     16, 0, 0);
            }
            if (lane < 4 * NBW)
                __builtin_amdgcn_global_load_lds((const void*)(ssrc + (size_t)p * (sstep * WAVES)),
                                                 (__attribute__((address_space(3))) void*)(sl + SCOFF), 16, 0, 0);
            asm volatile("" ::: "memory");
        }
    };

    // Per-lane LDS bases (slot 0).  x, XR >= 4: global segment 8*cc + 4*h + c of row xr sits at
    // position 8*cc + ((4*h + c) ^ (xr % 8)); lane (kb, j) reads dword kb of it.  x, XR == 1:
    // lane (kb, j) reads unit 8*cc + 4*h + kb.  Weights: segment (li % 8) + 8*kb.  Scales:
    // channel li of [group][block].
    const int xr = min(li, M - 1);
    uint32_t xb[2][XR == 1 ? 1 : 4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if constexpr (XR == 1) {
            xb[h][0] = lds_wave + WSLOT + ((4 * h + kb) << 4);
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                xb[h][c] = lds_wave + WSLOT + xr * 256 + (xr >= 8 ? XHI : 0) + (((4 * h + c) ^ (xr & 7)) << 4) + 4 * kb;
        }
    }
    const uint32_t wb = lds_wave + (((li & 7) + 8 * kb) << 4);
    const uint32_t sb = lds_wave + SCOFF + li * 2;
    const Dq d = dq_setup(lane);

    f4 acc[NBW];
#pragma unroll
    for (int b = 0; b < NBW; ++b) acc[b] = f4{0.f, 0.f, 0.f, 0.f};

    // Pair p sits in ring slot `slot` (a compile-time constant); its loads (and the scale loads,
    // which are older) are complete.
    auto consume = [&](int p, auto slot) {
        constexpr int SO = decltype(slot)::value * SLOT;
        u4 xv[2][2], wv[2][NBW];
        uint32_t sc[2][NBW];
        static_for<0, 2>([&](auto cc) {
            static_for<0, 2>([&](auto h) {
                constexpr int O = SO + decltype(cc)::value * 128;
                constexpr int H = decltype(h)::value;
                if constexpr (XR == 1) {
                    xv[cc][h] = lds_read_u4_at<O>(xb[H][0]);
                } else {
                    xv[cc][h] = u4{lds_read_u32_at<O>(xb[H][0]), lds_read_u32_at<O>(xb[H][1]),
                                   lds_read_u32_at<O>(xb[H][2]), lds_read_u32_at<O>(xb[H][3])};
                }
            });
        });
        static_for<0, 2>([&](auto cc) {
            static_for<0, NBW>([&](auto b) {
                wv[cc][b] = lds_read_u4_at<SO + decltype(b)::value * 1024 + decltype(cc)::value * 512>(wb);
            });
        });
        static_for<0, NBW>([&](auto b) {
            sc[0][b] = lds_read_u16_at<SO + decltype(b)::value * 32>(sb);
            sc[1][b] = lds_read_u16_at<SO + (NBW + decltype(b)::value) * 32>(sb);
        });
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
            for (int h = 0; h < 2; ++h) bind_after_wait(xv[cc][h]);
#pragma unroll
            for (int b = 0; b < NBW; ++b) { bind_after_wait(wv[cc][b]); bind_after_wait(sc[cc][b]); }
        }
        if constexpr (XR == 16 || NBW == 1) {
            // Dequantise the whole pair first and pin the fragments ahead of the next step.  Left
            // to the scheduler, the next step's vmcnt wait (an asm statement the arithmetic may
            // move across) and its refill are hoisted above this pair's dequantisation, so the
            // wave waits for pair p + 1 before computing pair p.  Pinned, in alternating runs:
            // 16 rows 0.6 us per call faster on the down projection (M = 16), 0.2 on gate/up;
            // single-block tiles 0.15-0.2 us faster (down M = 1, 4, 8).  Two- and four-block tiles
            // at 1..8 rows measured slower with the whole pair pinned (gate/up M = 1 +0.85 us: with
            // two pairs in flight the refill then waits for all the compute); see the half pin below.
            // Same MFMA sequence either way.
            h8 af[2][NBW][2];
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
                for (int b = 0; b < NBW; ++b) {
                    const h2 s2 = scale2((uint16_t)sc[cc][b]);
                    const u4 w = wv[cc][b];
                    af[cc][b][0] = dq_frag(w.x, w.y, d, s2);
                    af[cc][b][1] = dq_frag(w.z, w.w, d, s2);
                    asm volatile("" ::"v"(af[cc][b][0]), "v"(af[cc][b][1]));
                }
            }
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const u4 x0 = xv[cc][0], x1 = xv[cc][1];
                const h8 b0 = __builtin_bit_cast(h8, x0);
                const h8 b1 = __builtin_bit_cast(h8, x1);
#pragma unroll
                for (int b = 0; b < NBW; ++b) {
                    acc[b] = mfma16x16x32(af[cc][b][0], b0, acc[b]);
                    acc[b] = mfma16x16x32(af[cc][b][1], b1, acc[b]);
                }
            }
        } else {
            // Partial pin (multi-block tiles at 1, 4 and 8 rows): part of the pair is dequantised
            // ahead of the next step, so the refill waits for that part of the compute instead of
            // all of it -- the first chunk of two-block tiles (half the pair), the first block of
            // four-block tiles (a quarter).  In alternating runs against no pin: gate/up M = 1
            // 0.17-0.27 us per call faster (three boxes), M = 4 0.13-0.14 (gate/up and qkv, three
            // order-rotated runs; one earlier run without rotation read it 0.24 slower), M = 8 on the
            // four-block ring 0.14 with the first chunk pinned and another 0.15 with the first block
            // instead (order-rotated, two boxes; on two-block tiles the first block measured
            // -0.03..-0.06 at gate/up M = 1, 4 and +0.04 at qkv M = 4, so they keep the chunk).
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const u4 x0 = xv[cc][0], x1 = xv[cc][1];
                const h8 b0 = __builtin_bit_cast(h8, x0);
                const h8 b1 = __builtin_bit_cast(h8, x1);
#pragma unroll
                for (int b = 0; b < NBW; ++b) {
                    const h2 s2 = scale2((uint16_t)sc[cc][b]);
                    const u4 w = wv[cc][b];
                    const h8 a0 = dq_frag(w.x, w.y, d, s2);
                    const h8 a1 = dq_frag(w.z, w.w, d, s2);
                    if (NBW >= 4 ? b == 0 : cc == 0) asm volatile("" ::"v"(a0), "v"(a1));
                    acc[b] = mfma16x16x32(a0, b0, acc[b]);
                    acc[b] = mfma16x16x32(a1, b1, acc[b]);
                }
            }
        }
    };

    // Prologue: pairs 0..D-1 in slots 0..D-1 (npair >= D, checked by the planner).  Steady
    // state, S pairs per iteration: wait for pair p (D-1 younger pairs may stay in flight), refill
    // with pair p + D, then compute pair p; pair p lives in slot p % S.  Tail: the remaining
    // (< S) steady steps, then the last D pairs with shrinking waits.
    static_for<0, D>([&](auto s) { issue(s, s); });
    const int nsteady = npair - D;
#ifdef W4A16_WAVE_STAMPS
    const uint32_t st_issued = stamp_clock();
#endif
    int p = 0;
    // Issue priority by progress.  A SIMD issues the oldest of its waves first, so of two waves
    // sharing a SIMD (8-wave workgroups, or two workgroups on one CU) the younger runs on the
    // slots the older leaves free: measured per wave on the down projection, waves 4..7 ended
    // their streams 1.3-1.5 us after waves 0..3 and the workgroup waited for them.  Every wave
    // starts at priority 1 and drops to 0 at half its pairs, so a wave that is behind wins the
    // SIMD over one that is ahead.  The work and the arithmetic of each wave are unchanged.
    // Multi-block tiles below 16 rows step down from 3 by one at each quarter instead: in
    // order-rotated runs on two boxes gate/up M = 1, 4, 8 0.06, 0.07 and 0.12 us per call faster,
    // while the single-block and 16-row tiles measured mixed to 0.1 us slower that way.
    constexpr bool quarters = NBW >= 2 && XR < 16;
    __builtin_amdgcn_s_setprio(quarters ? 3 : 1);
    const int phalf = npair >> 1;
    const int pq1 = npair >> 2, pq3 = (3 * npair) >> 2;
    for (; p + S <= nsteady; p += S) {
        static_for<0, S>([&](auto t) {
            constexpr int T = decltype(t)::value;
            wait_vmcnt<(D - 1) * OPS>();
            issue(p + T + D, std::integral_constant<int, (T + D) % S>{});
            if constexpr (quarters) {
                if (p + T == pq1) __builtin_amdgcn_s_setprio(2);
                if (p + T == phalf) __builtin_amdgcn_s_setprio(1);
                if (p + T == pq3) __builtin_amdgcn_s_setprio(0);
            } else {
                if (p + T == phalf) __builtin_amdgcn_s_setprio(0);
            }
            consume(p + T, t);
#ifdef W4A16_WAVE_STAMPS
            if (st_first == 0) st_first = stamp_clock();
#endif
        });
    }
    __builtin_amdgcn_s_setprio(0);
    static_switch<0, S>(nsteady - p, [&](auto r) {
        constexpr int R = decltype(r)::value;
        static_for<0, R>([&](auto t) {
            constexpr int T = decltype(t)::value;
            wait_vmcnt<(D - 1) * OPS>();
            issue(p + T + D, std::integral_constant<int, (T + D) % S>{});
            consume(p + T, t);
#ifdef W4A16_WAVE_STAMPS
            if (st_first == 0) st_first = stamp_clock();
#endif
        });
        static_for<0, D>([&](auto t) {
            constexpr int T = decltype(t)::value;
            wait_vmcnt<(D - 1 - T) * OPS>();
            consume(p + R + T, std::integral_constant<int, (R + T) % S>{});
#ifdef W4A16_WAVE_STAMPS
            if (st_first == 0) st_first = stamp_clock();
#endif
        });
    });

#ifdef W4A16_WAVE_STAMPS
    const uint32_t st_done = stamp_clock();
#endif
    // Cross-wave reduction in wave order; each wave parks its tile at the start of its region
    // (its own loads are complete and its LDS reads have returned).
    f4* red = reinterpret_cast<f4*>(wreg);
#pragma unroll
    for (int b = 0; b < NBW; ++b) red[b * 64 + lane] = acc[b];
    __syncthreads();
    f4 sum = {0.f, 0.f, 0.f, 0.f};
    const int rb = tid >> 6;
    if (tid < NBW * 64) {
        sum = reinterpret_cast<const f4*>(wl)[rb * 64 + lane];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) sum += reinterpret_cast<const f4*>(wl + w * WAVE_BYTES)[rb * 64 + lane];
    }
    decode_finish<NBW, WAVES>(sum, tid < NBW * 64, rb, lane, split, tile, nb0, y, ws, counters, M, N, splits);
#ifdef W4A16_WAVE_STAMPS
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const uint32_t st_stored = stamp_clock();
    uint32_t hw_id, xcc_id;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw_id));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc_id));
    const int gw = blockIdx.x * WAVES + wave;
    if (lane == 0 && gw < kStampWaves) {
        uint32_t* o = g_wave_stamps + (size_t)gw * kStampWords;
        o[0] = st_entry; o[1] = st_issued; o[2] = st_first; o[3] = st_done;
        o[4] = st_stored; o[5] = hw_id; o[6] = xcc_id; o[7] = blockIdx.x;
    }
#endif
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
template <int BM, int BN, int WAVES_M, int WAVES_N, bool SEG>
__global__ void __launch_bounds__(WAVES_M * WAVES_N * 64)
prefill_kernel(const u4* __restrict__ Wp, const uint16_t* __restrict__ x,
               const uint16_t* __restrict__ scales, uint16_t* __restrict__ y,
               int M, int N, int K, int gshift, int tiles_m, int seg_chunks) {
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

    // SEG (K split into the canonical segments of seg_chunks chunks): acc holds the running
    // segment, total the sum of the finished ones (total = p0, then total + p_s).
    f4 total[SEG ? TM : 1][SEG ? TN : 1];
    int seg_left = seg_chunks;
    bool first_seg = true;

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
        if constexpr (SEG) {
            if (--seg_left == 0 || !more) {
#pragma unroll
                for (int t = 0; t < TM; ++t)
#pragma unroll
                    for (int b = 0; b < TN; ++b) {
                        total[t][b] = first_seg ? acc[t][b] : total[t][b] + acc[t][b];
                        acc[t][b] = f4{0.f, 0.f, 0.f, 0.f};
                    }
                first_seg = false;
                seg_left = seg_chunks;
            }
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
            *reinterpret_cast<u2*>(y + (size_t)m * N + n) = pack_f16x4(SEG ? total[SEG ? t : 0][SEG ? b : 0] : acc[t][b]);
        }
    }
}

// Small-M prefill (17 <= M <= 16*TM): one wave per n16 block walks the whole K range.
//
// With few token rows the prefill tiles leave most CUs idle (N/BN workgroups) and a K-sequential
// wave is latency-bound.  Here every n16 block gets its own wave (N/16 workgroups of one wave)
// that streams its weights through a refill-ahead ring of D+1 chunk-pair slots in LDS (the
// decode_ring_kernel scheme): the loads of pair p+D are issued before pair p is multiplied.  A
// slot holds the block's two 512-byte weight chunks (segments transposed for conflict-free A
// reads) and the pair's 16*TM x rows (16-byte segments XOR-swizzled by row); the pair's scales
// come straight into VGPRs.  Every accumulator receives chunk 0 h 0, chunk 0 h 1, chunk 1 h 0,
// ... with the same A (dq_frag) and B operands (8 consecutive halves, row-transposed), so the
// output is bit-identical to every other prefill config.  All loads run with all lanes active
// (clamped addresses), so each pair is exactly OPS vector-memory instructions.
template <int TM, int D>
__global__ void __launch_bounds__(64)
prefill_stream_kernel(const u4* __restrict__ Wp, const uint16_t* __restrict__ x,
                      const uint16_t* __restrict__ scales, int M, int N, int K, int gshift, int splits,
                      int seg_pairs, uint16_t* __restrict__ y, float* __restrict__ ws, int* __restrict__ counters) {
    constexpr int S = D + 1;                                 // ring slots
    constexpr int XD = 4 * TM;                               // x loads per pair (4 rows each)
    constexpr int SLOT = 1024 + XD * 1024 + 1024;            // weights, 16*TM rows x 256 B, scales
    constexpr int SOFF = 1024 + XD * 1024;                   // scale region of a slot
    constexpr int OPS = 1 + XD + 1;                          // weights, x rows, scales
    static_assert((D - 1) * OPS <= 63, "too many loads in flight for vmcnt");
    __shared__ __attribute__((aligned(16))) char wl[S * SLOT];

    const int lane = threadIdx.x;
    const int kb = lane >> 4;
    const int li = lane & 15;
    const int NBLK = N >> 4;
    const int seg = blockIdx.x / NBLK;                       // K segment (split-K over segments)
    const int nb = blockIdx.x - seg * NBLK;
    const int KC = K >> 6;
    const int pair0 = seg * seg_pairs;
    const int npair = min(seg_pairs, (KC >> 1) - pair0);
    const uint32_t lds = (uint32_t)reinterpret_cast<uintptr_t>(wl);

    // Weights: lane j fills segment j & 31 of chunk j >> 5 with packed lane 4*(seg % 8) + seg / 8.
    const int wseg = lane & 31;
    const u4* wsrc = Wp + ((size_t)nb * KC + (lane >> 5)) * 32 + 4 * (wseg & 7) + (wseg >> 3);
    // x: lane j of load q fills row r = (64q + j) / 16, segment j % 16, with global segment
    // (j % 16) ^ (r % 8) of row min(r, M - 1).
    const uint16_t* xsrc[XD];
#pragma unroll
    for (int q = 0; q < XD; ++q) {
        const int r = (64 * q + lane) >> 4;
        xsrc[q] = x + (size_t)min(r, M - 1) * K + (((lane & 15) ^ (r & 7)) * 8);
    }
    // Scales: the pair's 2 chunks x 16 channels are 4 16-byte pieces (chunk c = (j >> 1) & 1,
    // channels 8*(j & 1)..+7); lane j loads piece j & 3, so the other lanes repeat them.
    const uint16_t* ssrc = scales + (size_t)nb * 16 + (lane & 1) * 8;
    const int scc = (lane >> 1) & 1;
    auto issue = [&](int p, int s) {
        char* sl = wl + s * SLOT;
        __builtin_amdgcn_global_load_lds((const void*)(wsrc + (size_t)p * 64),
                                         (__attribute__((address_space(3))) void*)sl, 16, 0, 0);
#pragma unroll
        for (int q = 0; q < XD; ++q)
            __builtin_amdgcn_global_load_lds((const void*)(xsrc[q] + (size_t)p * 128),
                                             (__attribute__((address_space(3))) void*)(sl + 1024 + q * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(ssrc + (size_t)((2 * p + scc) >> gshift) * N),
                                         (__attribute__((address_space(3))) void*)(sl + SOFF), 16, 0, 0);
        asm volatile("" ::: "memory");
    };

    uint32_t xoff[TM][2][2];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        const int r = min(16 * t + li, M - 1);
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int h = 0; h < 2; ++h) xoff[t][cc][h] = 1024 + r * 256 + (((cc * 8 + 4 * h + kb) ^ (r & 7)) << 4);
    }
    const uint32_t woff = ((li & 7) + 8 * kb) << 4;
    const uint32_t soff = SOFF + (li >> 3) * 16 + (li & 7) * 2;     // + 32 * chunk
    const Dq d = dq_setup(lane);
    f4 acc[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};

    auto consume = [&](int s) {
        const uint32_t base = lds + s * SLOT;
        u4 wv[2], xv[TM][2][2];
        uint32_t sv[2];
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) wv[cc] = lds_read_u4(base + cc * 512 + woff);
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) sv[cc] = lds_read_u16(base + soff + cc * 32);
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int h = 0; h < 2; ++h) xv[t][cc][h] = lds_read_u4(base + xoff[t][cc][h]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            bind_after_wait(wv[cc]);
            bind_after_wait(sv[cc]);
#pragma unroll
            for (int t = 0; t < TM; ++t) { bind_after_wait(xv[t][cc][0]); bind_after_wait(xv[t][cc][1]); }
        }
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const h2 s2 = scale2((uint16_t)sv[cc]);
            const h8 a0 = dq_frag(wv[cc].x, wv[cc].y, d, s2);
            const h8 a1 = dq_frag(wv[cc].z, wv[cc].w, d, s2);
#pragma unroll
            for (int t = 0; t < TM; ++t) acc[t] = mfma16x16x32(a0, __builtin_bit_cast(h8, xpose_rows(xv[t][cc][0])), acc[t]);
#pragma unroll
            for (int t = 0; t < TM; ++t) acc[t] = mfma16x16x32(a1, __builtin_bit_cast(h8, xpose_rows(xv[t][cc][1])), acc[t]);
        }
    };

    // Prologue: pairs 0..D-1 (npair >= D, checked by the planner).  Steady state: wait for pair
    // p, refill with pair p + D, then compute pair p.  Drain: the last D pairs.
#pragma unroll
    for (int s = 0; s < D; ++s) issue(pair0 + s, s);
    int sc = 0, si = D;
    int p = 0;
    for (; p + D < npair; ++p) {
        wait_vmcnt<(D - 1) * OPS>();
        issue(pair0 + p + D, si);
        consume(sc);
        sc = sc + 1 == S ? 0 : sc + 1;
        si = si + 1 == S ? 0 : si + 1;
    }
    static_for<0, D>([&](auto t) {
        wait_vmcnt<(D - 1 - decltype(t)::value) * OPS>();
        consume(sc);
        sc = sc + 1 == S ? 0 : sc + 1;
    });

    f4 out[TM][1];
#pragma unroll
    for (int t = 0; t < TM; ++t) out[t][0] = acc[t];
    prefill_tile_out<TM, 1>(out, 0, nb, lane, y, ws, counters, M, N, seg, splits, nb);
}

// Prefill for token groups (any M): W waves per workgroup, NB n16 blocks per wave, share the x
// rows of one group of 16*TM tokens (grid: ceil(M / 16TM) token groups x ceil(N / 16 W NB) column
// groups).
//
// prefill_stream_kernel with the x rows shared.  Each wave walks the whole K range of its NB
// n16 blocks with the refill-ahead ring of D+1 chunk-pair slots, but a slot holds the x rows of
// the pair once for the W waves: wave w issues x loads [w XD/W, (w+1) XD/W) besides its own
// weights and scales, waits for its own loads of pair p, and one barrier then publishes all of
// pair p and retires every wave's reads of pair p-1, whose slot the refill (pair p+D) reuses.  So
// the x traffic and the LDS of a group are shared W ways, and large M runs as independent token
// groups (their weights re-read from L2).  Every x operand a wave reads feeds NB MFMAs: the LDS
// reads per MFMA fall as 1/NB.  Same A and B operands and the same MFMA order per accumulator
// as every other prefill config, so the output is bit-identical.  Blocks past N are computed on
// the last block (clamped) and not stored.
//
// x layout in a slot: token tile t (16 rows) at t * XT; row r at r * 256, rows 8..15 shifted by
// 8 bytes; the 16-byte global segment g of a row sits at position g ^ (r % 8).  The B operand
// of lane (kb, j) -- dwords 16h + 4c + kb (c = 0..3) of row j's chunk cc -- is read as four 4-byte
// LDS reads, with no cross-lane transpose.  The LDS serves a 4-byte read 32 lanes at a time from
// 32 banks; lanes kb = 0, 1 (or 2, 3) read dwords kb of their rows' segments, and the 8-byte
// shift moves rows 8..15 onto the segments' other two dwords, so the 32 lanes hit 32 banks.  Per wave, a slot holds NB KB of weights and the
// pair's scales ([block][chunk][16 channels], 64 B per block).  The ring loop is unrolled by its
// size, so every LDS offset is an instruction immediate.  Arguments ordered as decode_ring_kernel's:
// what the prologue needs (14 dwords, with the grid size) first, preloaded into SGPRs.
template <int TM, int D, int W, int NB>
__global__ void __launch_bounds__(64 * W)
prefill_group_kernel(const u4* __restrict__ Wp, const uint16_t* __restrict__ x,
                     const uint16_t* __restrict__ scales,
                     int M, int N, int K, int gshift, int groups_m, int splits, int seg_pairs, int G,
                     uint16_t* __restrict__ y, float* __restrict__ ws, int* __restrict__ counters) {
    constexpr int S = D + 1;                                 // ring slots
    constexpr int XD = 4 * TM;                               // x loads per pair (4 rows each)
    constexpr int XW = XD / W;                               // x loads per wave and pair
    constexpr int WR = NB * 1024 + NB * 64;                  // per wave: weights, scales
    constexpr int XOFF = WR * W;                             // x region of a slot
    constexpr int XT = kGroupXTileBytes;                     // bytes per 16-row token tile
    constexpr int SLOT = XOFF + TM * XT;
    constexpr int OPS = NB + XW + 1;                         // weights, x share, scales
    static_assert(XD % W == 0, "x loads must split evenly over the waves");
    static_assert(4 * NB <= 64, "scale pieces of one pair must fit one load");
    static_assert((D - 1) * OPS <= 63, "too many loads in flight for vmcnt");
    static_assert((S - 1) * SLOT + (TM - 1) * XT + 128 < 65536, "x read offsets must fit the LDS offset field");
    __shared__ __attribute__((aligned(16))) char wl[S * SLOT];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kb = lane >> 4;
    const int li = lane & 15;
    // Workgroup -> (K segment, column group, token group); consecutive blocks of one XCD (b % 8)
    // share the column group's weights in that XCD's L2, and the segment varies slowest.
    const int G8 = G >> 3;
    const int bid = blockIdx.x;
    const int tile_raw = bid < (G8 << 3) ? (bid & 7) * G8 + (bid >> 3) : bid;
    const int tiles = G / splits;
    const int seg = tile_raw / tiles;
    const int tile = tile_raw - seg * tiles;
    const int tg = tile % groups_m;
    const int ng = tile / groups_m;
    const int NBLK = N >> 4;
    const int nb0_raw = (ng * W + wave) * NB;                // first n16 block of the wave
    const int m0 = tg * 16 * TM;
    const int KC = K >> 6;
    const int pair0 = seg * seg_pairs;                       // this workgroup's K segment
    const int npair = min(seg_pairs, (KC >> 1) - pair0);
    const uint32_t lds = (uint32_t)reinterpret_cast<uintptr_t>(wl);

    // Weights of block b: lane j fills segment j & 31 of chunk j >> 5 with packed lane
    // 4*(seg % 8) + seg / 8.
    const int wseg = lane & 31;
    const u4* wsrc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
        wsrc[b] = Wp + ((size_t)min(nb0_raw + b, NBLK - 1) * KC + (lane >> 5)) * 32 + 4 * (wseg & 7) + (wseg >> 3);
    // x: load q fills rows r0 = 4 (q % 4) .. r0 + 3 of token tile q / 4; lane j fills row
    // r0 + j / 16, position j % 16, with global segment (j % 16) ^ (row % 8) of token
    // min(m0 + 16 (q / 4) + row, M - 1).  This wave issues loads q = wave*XW + i.
    const uint16_t* xsrc[XW];
#pragma unroll
    for (int i = 0; i < XW; ++i) {
        const int q = wave * XW + i;
        const int r = 4 * (q & 3) + (lane >> 4);
        xsrc[i] = x + (size_t)min(m0 + 16 * (q >> 2) + r, M - 1) * K + (((lane & 15) ^ (r & 7)) * 8);
    }
    // Scales: lane e < 4 NB loads piece e & 3 of block e / 4 (chunk (e >> 1) & 1, channels
    // 8 (e & 1)..+7), 16 bytes, into byte 16 e of the wave's scale region.
    const int se = min(lane, 4 * NB - 1);
    const uint16_t* ssrc = scales + (size_t)min(nb0_raw + (se >> 2), NBLK - 1) * 16 + (se & 1) * 8;
    const int scc = (se >> 1) & 1;
    auto issue = [&](int p, auto slot) {
        char* sl = wl + decltype(slot)::value * SLOT;
#pragma unroll
        for (int b = 0; b < NB; ++b)
            __builtin_amdgcn_global_load_lds((const void*)(wsrc[b] + (size_t)p * 64),
                                             (__attribute__((address_space(3))) void*)(sl + wave * WR + b * 1024), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < XW; ++i) {
            const int q = wave * XW + i;
            const int r0 = 4 * (q & 3);
            __builtin_amdgcn_global_load_lds((const void*)(xsrc[i] + (size_t)p * 128),
                                             (__attribute__((address_space(3))) void*)(sl + XOFF + (q >> 2) * XT + r0 * 256 +
                                                                                       (r0 >= 8 ? 8 : 0)),
                                             16, 0, 0);
        }
        if (lane < 4 * NB)
            __builtin_amdgcn_global_load_lds((const void*)(ssrc + (size_t)((2 * p + scc) >> gshift) * N),
                                             (__attribute__((address_space(3))) void*)(sl + wave * WR + NB * 1024), 16, 0, 0);
        asm volatile("" ::: "memory");
    };

    // Per-lane LDS bases (slot 0, token tile 0, chunk 0, block 0): x dword kb of global segment
    // 4h + c of row li; weights segment (li % 8) + 8 kb; scales of channel li.
    uint32_t xb[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int c = 0; c < 4; ++c)
            xb[h][c] = lds + XOFF + li * 256 + (li >> 3) * 8 + (((4 * h + c) ^ (li & 7)) << 4) + 4 * kb;
    const uint32_t wb = lds + wave * WR + (((li & 7) + 8 * kb) << 4);
    const uint32_t sb = lds + wave * WR + NB * 1024 + (li >> 3) * 16 + (li & 7) * 2;   // + 64 block + 32 chunk
    const Dq d = dq_setup(lane);
    f4 acc[TM][NB];
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[t][b] = f4{0.f, 0.f, 0.f, 0.f};

    auto consume = [&](auto slot) {
        constexpr int SO = decltype(slot)::value * SLOT;
        u4 wv[NB][2], xv[TM][2][2];
        uint32_t sv[NB][2];
        static_for<0, NB>([&](auto b) {
            static_for<0, 2>([&](auto cc) {
                constexpr int B = decltype(b)::value, C = decltype(cc)::value;
                wv[B][C] = lds_read_u4_at<SO + B * 1024 + C * 512>(wb);
                sv[B][C] = lds_read_u16_at<SO + B * 64 + C * 32>(sb);
            });
        });
        static_for<0, TM>([&](auto t) {
            static_for<0, 2>([&](auto cc) {
                static_for<0, 2>([&](auto h) {
                    constexpr int O = SO + decltype(t)::value * XT + decltype(cc)::value * 128;
                    constexpr int H = decltype(h)::value;
                    xv[decltype(t)::value][decltype(cc)::value][H] =
                        u4{lds_read_u32_at<O>(xb[H][0]), lds_read_u32_at<O>(xb[H][1]),
                           lds_read_u32_at<O>(xb[H][2]), lds_read_u32_at<O>(xb[H][3])};
                });
            });
        });
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
            for (int b = 0; b < NB; ++b) { bind_after_wait(wv[b][cc]); bind_after_wait(sv[b][cc]); }
#pragma unroll
            for (int t = 0; t < TM; ++t) { bind_after_wait(xv[t][cc][0]); bind_after_wait(xv[t][cc][1]); }
        }
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            h8 a0[NB], a1[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const h2 s2 = scale2((uint16_t)sv[b][cc]);
                const u4 w = wv[b][cc];
                a0[b] = dq_frag(w.x, w.y, d, s2);
                a1[b] = dq_frag(w.z, w.w, d, s2);
            }
#pragma unroll
            for (int t = 0; t < TM; ++t) {
                const u4 b0 = xv[t][cc][0];
#pragma unroll
                for (int b = 0; b < NB; ++b) acc[t][b] = mfma16x16x32(a0[b], __builtin_bit_cast(h8, b0), acc[t][b]);
            }
#pragma unroll
            for (int t = 0; t < TM; ++t) {
                const u4 b1 = xv[t][cc][1];
#pragma unroll
                for (int b = 0; b < NB; ++b) acc[t][b] = mfma16x16x32(a1[b], __builtin_bit_cast(h8, b1), acc[t][b]);
            }
        }
    };

    // Prologue: pairs 0..D-1 in slots 0..D-1 (npair >= D, checked by the planner).  Steady state,
    // S pairs per iteration: wait for this wave's loads of pair p, barrier (all of pair p landed;
    // every wave is done with pair p-1), refill pair p-1's slot with pair p + D, compute pair p;
    // pair p lives in slot p % S.  Tail: the remaining (< S) steady steps, then the last D pairs.
    // The barrier is a bare s_barrier: the explicit vmcnt wait has completed this wave's loads of
    // pair p (a completed direct-to-LDS load is in LDS) and consume() ends with lgkmcnt(0), which
    // is all the ordering the ring needs; __syncthreads() would also wait for vmcnt(0), draining
    // the loads of the next D pairs at every step.
    static_for<0, D>([&](auto s) { issue(pair0 + decltype(s)::value, s); });
    const int nsteady = npair - D;
    int p = 0;
    for (; p + S <= nsteady; p += S) {
        static_for<0, S>([&](auto t) {
            constexpr int T = decltype(t)::value;
            wait_vmcnt<(D - 1) * OPS>();
            __builtin_amdgcn_s_barrier();
            issue(pair0 + p + T + D, std::integral_constant<int, (T + D) % S>{});
            consume(t);
        });
    }
    static_switch<0, S>(nsteady - p, [&](auto r) {
        constexpr int R = decltype(r)::value;
        static_for<0, R>([&](auto t) {
            constexpr int T = decltype(t)::value;
            wait_vmcnt<(D - 1) * OPS>();
            __builtin_amdgcn_s_barrier();
            issue(pair0 + p + T + D, std::integral_constant<int, (T + D) % S>{});
            consume(t);
        });
        static_for<0, D>([&](auto t) {
            constexpr int T = decltype(t)::value;
            wait_vmcnt<(D - 1 - T) * OPS>();
            __builtin_amdgcn_s_barrier();
            consume(std::integral_constant<int, (R + T) % S>{});
        });
    });

    prefill_tile_out<TM, NB>(acc, m0, nb0_raw, lane, y, ws, counters, M, N, seg, splits, tile);
}

// ------------------------------------------------------------------------------------ launch

// Wide prefill configs (kind 1) live in their own translation unit (w4a16_prefill_wide.hip),
// compiled with a different instruction-scheduling strategy.
hipError_t launch_prefill_wide(int cfg, const w4a16_plan& p, const u4* Wp, const uint16_t* x, const uint16_t* s,
                               uint16_t* y, hipStream_t st);
int prefill_wide_occupancy(int cfg);
hipError_t prefill_wide_load_code(hipStream_t st);

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
W4A16_PREFILL_CFG(5)
W4A16_PREFILL_CFG(6)
W4A16_PREFILL_CFG(7)
W4A16_PREFILL_CFG(8)
W4A16_PREFILL_CFG(9)
W4A16_PREFILL_CFG(10)
W4A16_PREFILL_CFG(11)
W4A16_PREFILL_CFG(12)
W4A16_PREFILL_CFG(13)
W4A16_PREFILL_CFG(14)
W4A16_PREFILL_CFG(15)
W4A16_PREFILL_CFG(16)
W4A16_PREFILL_CFG(17)
W4A16_PREFILL_CFG(18)
W4A16_PREFILL_CFG(19)
W4A16_PREFILL_CFG(20)
W4A16_PREFILL_CFG(21)
W4A16_PREFILL_CFG(22)
W4A16_PREFILL_CFG(23)
W4A16_PREFILL_CFG(24)
#undef W4A16_PREFILL_CFG

template <int CFG>
static hipError_t launch_prefill(const w4a16_plan& p, const u4* Wp, const uint16_t* x,
                                 const uint16_t* s, uint16_t* y, float* ws, int* counters, hipStream_t st) {
    using C = PrefillCfg<CFG>;
    const int gshift = p.G == 128 ? 1 : 0;
    const int tiles_m = (p.M + C::BM - 1) / C::BM;
    // Kinds 2 and 3 run one canonical K segment per workgroup (p.splits of them per tile).
    const int seg_pairs = prefill_segment_chunks(p.K >> 6) >> 1;
    const int splits = p.splits > 1 ? p.splits : 1;
    if constexpr (kPrefillTable[CFG].kind == 3)
        hipLaunchKernelGGL((prefill_group_kernel<C::BM / 16, kPrefillTable[CFG].depth, C::WN, C::BN / (16 * C::WN)>),
                           dim3(p.grid), dim3(64 * C::WN), 0, st, Wp, x, s, p.M, p.N, p.K, gshift, tiles_m, splits,
                           seg_pairs, p.grid, y, ws, counters);
    else if constexpr (kPrefillTable[CFG].kind == 2)
        hipLaunchKernelGGL((prefill_stream_kernel<C::BM / 16, kPrefillTable[CFG].depth>), dim3(p.grid), dim3(64), 0, st,
                           Wp, x, s, p.M, p.N, p.K, gshift, splits, seg_pairs, y, ws, counters);
    else if constexpr (kPrefillTable[CFG].kind == 1)
        return launch_prefill_wide(CFG, p, Wp, x, s, y, st);
    else
    {
        const int seg_chunks = prefill_segment_chunks(p.K >> 6);
        if (prefill_segments(p.K >> 6) > 1)
            hipLaunchKernelGGL((prefill_kernel<C::BM, C::BN, C::WM, C::WN, true>), dim3(p.grid),
                               dim3(C::WM * C::WN * 64), 0, st, Wp, x, s, y, p.M, p.N, p.K, gshift, tiles_m, seg_chunks);
        else
            hipLaunchKernelGGL((prefill_kernel<C::BM, C::BN, C::WM, C::WN, false>), dim3(p.grid),
                               dim3(C::WM * C::WN * 64), 0, st, Wp, x, s, y, p.M, p.N, p.K, gshift, tiles_m, seg_chunks);
    }
    return hipGetLastError();
}

// Resident workgroups per CU of a prefill config's compiled kernel (HIP occupancy query on the
// current device), -1 on error.
template <int CFG>
static int prefill_occupancy_of() {
    using C = PrefillCfg<CFG>;
    int n = 0;
    hipError_t e = hipSuccess;
    if constexpr (kPrefillTable[CFG].kind == 3)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, prefill_group_kernel<C::BM / 16, kPrefillTable[CFG].depth, C::WN, C::BN / (16 * C::WN)>, 64 * C::WN, 0);
    else if constexpr (kPrefillTable[CFG].kind == 2)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_stream_kernel<C::BM / 16, kPrefillTable[CFG].depth>,
                                                         64, 0);
    else if constexpr (kPrefillTable[CFG].kind == 1)
        return prefill_wide_occupancy(CFG);
    else
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_kernel<C::BM, C::BN, C::WM, C::WN, false>,
                                                         C::WM * C::WN * 64, 0);
    return e == hipSuccess ? n : -1;
}

// Decode launches go through a function handle resolved once per device (hipGetFuncBySymbol) and
// hipModuleLaunchKernel: the runtime then skips its per-call lookup of the kernel by its host
// stub.  Measured through the library in an alternating host loop: 0.15-0.2 us less host time per
// call (about 4.4 -> 4.2 us with ctypes), which is what an eager call of a ~4 us decode kernel
// (configs[0]) is bound by; device time per call unchanged.
constexpr int kMaxLaunchDevices = 64;
template <auto Kern, typename... Args>
static hipError_t launch_cached(unsigned grid, unsigned block, hipStream_t st, Args... args) {
    static hipFunction_t fn[kMaxLaunchDevices] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxLaunchDevices) return hipErrorInvalidDevice;
    hipFunction_t f = __atomic_load_n(&fn[dev], __ATOMIC_ACQUIRE);
    if (!f) {
        const hipError_t e = hipGetFuncBySymbol(&f, reinterpret_cast<const void*>(Kern));
        if (e != hipSuccess) return e;
        __atomic_store_n(&fn[dev], f, __ATOMIC_RELEASE);
    }
    void* params[] = {static_cast<void*>(&args)...};
    return hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, 0, st, params, nullptr);
}

template <int V>
static hipError_t launch_decode_v(const w4a16_plan& p, const u4* Wp, const uint16_t* x, const uint16_t* s,
                                  uint16_t* y, float* ws, int* cnt, hipStream_t st) {
    constexpr DecodeCfg c = kDecodeTable[V];
    const int gshift = p.G == 128 ? 1 : 0;
    if constexpr (c.kind == 0) {
        return launch_cached<decode_kernel<c.nbw, c.waves, c.d>>((unsigned)p.grid, (unsigned)(c.waves * 64), st, Wp, x, s,
                                                                 (int)p.M, (int)p.N, (int)p.K, gshift, (int)p.splits,
                                                                 (int)p.slab_chunks, y, ws, cnt);
    } else if constexpr (c.kind == 2) {
        return launch_cached<decode_stream_kernel<c.nbw, c.waves, c.d>>((unsigned)p.grid, (unsigned)(c.waves * 64), st, Wp,
                                                                        x, s, (int)p.M, (int)p.N, (int)p.K, gshift,
                                                                        (int)p.splits, (int)p.slab_chunks, y, ws, cnt);
    } else if constexpr (c.kind == 3) {
        const int xr = decode_ring_xr(p.M);
        int dev = 0;
        w4a16_device_limits lim{};
        const int remap = hipGetDevice(&dev) == hipSuccess && w4a16_query_device(dev, &lim) == W4A16_OK
                              ? (p.grid <= lim.cu_count && !(c.nbw >= 4 && p.K <= 4096) ? 1 : 0) : 1;
#define W4A16_RING(XR)                                                                                   \
        return launch_cached<decode_ring_kernel<c.nbw, c.waves, c.d, XR>>(                               \
            (unsigned)p.grid, (unsigned)(c.waves * 64), st, Wp, x, s, (int)p.M, (int)p.N, (int)p.K, gshift, \
            (int)p.splits, (int)p.slab_chunks, remap, (int)p.grid, y, ws, cnt)
        // Shapes whose ring does not fit in LDS for a row count are never planned for it.
        if (xr == 1) {
            if constexpr (decode_lds_bytes(V, 1) <= 163840) W4A16_RING(1); else return hipErrorInvalidValue;
        } else if (xr == 4) {
            if constexpr (decode_lds_bytes(V, 4) <= 163840) W4A16_RING(4); else return hipErrorInvalidValue;
        } else if (xr == 8) {
            if constexpr (decode_lds_bytes(V, 8) <= 163840) W4A16_RING(8); else return hipErrorInvalidValue;
        } else {
            if constexpr (decode_lds_bytes(V, 16) <= 163840) W4A16_RING(16); else return hipErrorInvalidValue;
        }
#undef W4A16_RING
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

static hipError_t launch_decode(const w4a16_plan& p, const u4* Wp, const uint16_t* x, const uint16_t* s,
                                uint16_t* y, float* ws, int* cnt, hipStream_t st) {
    switch (p.decode_variant) {   // the planner only emits entries of kDecodeTable
#define W4A16_DEC_CASE(I) case I: return launch_decode_v<I>(p, Wp, x, s, y, ws, cnt, st);
        W4A16_DEC_CASE(0) W4A16_DEC_CASE(1) W4A16_DEC_CASE(2) W4A16_DEC_CASE(3)
        W4A16_DEC_CASE(4) W4A16_DEC_CASE(5) W4A16_DEC_CASE(6) W4A16_DEC_CASE(7)
        W4A16_DEC_CASE(8) W4A16_DEC_CASE(9) W4A16_DEC_CASE(10) W4A16_DEC_CASE(11)
        W4A16_DEC_CASE(12) W4A16_DEC_CASE(13) W4A16_DEC_CASE(14) W4A16_DEC_CASE(15)
        W4A16_DEC_CASE(16) W4A16_DEC_CASE(17) W4A16_DEC_CASE(18) W4A16_DEC_CASE(19)
        W4A16_DEC_CASE(20) W4A16_DEC_CASE(21) W4A16_DEC_CASE(22) W4A16_DEC_CASE(23)
        W4A16_DEC_CASE(24) W4A16_DEC_CASE(25) W4A16_DEC_CASE(26) W4A16_DEC_CASE(27)
        W4A16_DEC_CASE(28) W4A16_DEC_CASE(29) W4A16_DEC_CASE(30) W4A16_DEC_CASE(31)
#undef W4A16_DEC_CASE
        default: return hipErrorInvalidValue;
    }
}

}  // namespace w4a16

using namespace w4a16;

// ------------------------------------------------------------------ allocation-free launches
// Scratch of w4a16_launch_noalloc: the split-K counters (first W4A16_NOALLOC_MAX_COUNTER_SLOTS
// ints) followed by the fp32 partials (W4A16_NOALLOC_MAX_WORKSPACE_BYTES).  Each device holds its
// own copy for the life of the process.  The counters start at zero (zero-initialised storage,
// and cleared once more when a device is first used) and every launch leaves them zero (the
// wrapping increment in decode_finish).
namespace {
constexpr size_t kScratchCounterBytes = (size_t)W4A16_NOALLOC_MAX_COUNTER_SLOTS * sizeof(int32_t);
constexpr size_t kScratchBytes = kScratchCounterBytes + (size_t)W4A16_NOALLOC_MAX_WORKSPACE_BYTES;
static_assert(kScratchCounterBytes % 256 == 0, "partials start 256-byte aligned");
static __device__ __align__(256) char scratch[kScratchBytes];

__global__ void __launch_bounds__(256) scratch_clear_kernel(u4* __restrict__ p, int n16) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n16) p[i] = u4{0u, 0u, 0u, 0u};
}

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kMaxScratchDevices];      // device address of `scratch` per device, or null

// The device address of this device's scratch, or null with the message set.  The first call on a
// device resolves it, clears its counters and launches a no-op kernel of the wide prefill unit:
// the HIP runtime loads a unit's GPU code (allocating device memory) on the first launch of one of
// its kernels, and these two launches load both units a noalloc call can run, so later calls
// allocate nothing.
char* scratch_for_current_device(hipStream_t st) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
        w4a16_set_last_error("w4a16_launch_noalloc: no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            w4a16_set_last_error(e != hipSuccess ? hipGetErrorString(e) : "hipGetSymbolAddress returned null");
            return nullptr;
        }
        constexpr int n16 = (int)(kScratchCounterBytes / 16);
        hipLaunchKernelGGL(scratch_clear_kernel, dim3((n16 + 255) / 256), dim3(256), 0, st,
                           static_cast<u4*>(ptr), n16);
        hipError_t le = hipGetLastError();
        if (le == hipSuccess) le = prefill_wide_load_code(st);
        if (le != hipSuccess) {
            w4a16_set_last_error(hipGetErrorString(le));
            return nullptr;
        }
        g_scratch_ptr[dev] = static_cast<char*>(ptr);
    }
    return g_scratch_ptr[dev];
}
}  // namespace

namespace {
int check_plan(const w4a16_plan& p);
}  // namespace

extern "C" int w4a16_launch_noalloc(const w4a16_plan* plan, const int32_t* Wp, const uint16_t* x,
                                    const uint16_t* scales, uint16_t* y, void* stream) {
    if (!plan) return W4A16_ERR_INVALID;
    // Per-device set-up on the first call, whatever the plan (see scratch_for_current_device).
    char* const scratch_base = scratch_for_current_device(reinterpret_cast<hipStream_t>(stream));
    if (!scratch_base) return W4A16_ERR_HIP;
    // A prefill plan that needs more scratch than the static array (long K at moderate M splits
    // K over workgroups) runs as a scratch-free config of the same problem: every prefill config
    // gives the same bits.
    w4a16_plan alt;
    if (plan->kernel != W4A16_VARIANT_DECODE &&
        (plan->workspace_bytes > (uint64_t)W4A16_NOALLOC_MAX_WORKSPACE_BYTES ||
         plan->counter_slots > W4A16_NOALLOC_MAX_COUNTER_SLOTS) &&
        check_plan(*plan) == W4A16_OK) {
        int dev = 0;
        w4a16_device_limits lim;
        if (hipGetDevice(&dev) == hipSuccess && w4a16_query_device(dev, &lim) == W4A16_OK &&
            prefill_plan_no_scratch(*plan, lim, &alt))
            plan = &alt;
    }
    if (plan->workspace_bytes > (uint64_t)W4A16_NOALLOC_MAX_WORKSPACE_BYTES ||
        plan->counter_slots > W4A16_NOALLOC_MAX_COUNTER_SLOTS) {
        char msg[256];
        std::snprintf(msg, sizeof(msg),
                      "w4a16_launch_noalloc: the plan needs %llu bytes of partials and %d counters; the static "
                      "scratch holds %llu bytes and %d counters (use w4a16_launch with a workspace)",
                      (unsigned long long)plan->workspace_bytes, plan->counter_slots,
                      (unsigned long long)W4A16_NOALLOC_MAX_WORKSPACE_BYTES, W4A16_NOALLOC_MAX_COUNTER_SLOTS);
        w4a16_set_last_error(msg);
        return W4A16_ERR_WORKSPACE;
    }
    char* const base = plan->workspace_bytes || plan->counter_slots ? scratch_base : nullptr;
    return w4a16_launch(plan, Wp, x, scales, y, base ? base + kScratchCounterBytes : nullptr,
                        base ? reinterpret_cast<int32_t*>(base) : nullptr, stream);
}

namespace {
// Whether a plan matches what its kernel derives from (M, N, K, G): W4A16_OK, W4A16_ERR_INVALID,
// or W4A16_ERR_WORKSPACE when a split plan declares buffers too small for its partials and
// counters.  Pure host code.
int check_plan(const w4a16_plan& p) {
    if ((p.G != 64 && p.G != 128) || p.K % 64 != 0 || p.N % 16 != 0 || p.K % p.G != 0) return W4A16_ERR_INVALID;
    if (p.kernel == W4A16_VARIANT_DECODE) {
        // The grid, the chunks per wave and the block size bound every weight, x and y index
        // the decode kernels form.
        if (p.decode_variant < 0 || p.decode_variant >= kNumDecodeCfg) return W4A16_ERR_INVALID;
        const DecodeCfg& c = kDecodeTable[p.decode_variant];
        const int KC = p.K >> 6;
        const int ntiles = p.N / (16 * c.nbw);
        if (p.M > 16 || p.N % 64 != 0 || p.K % 512 != 0 || p.N % (16 * c.nbw) != 0 ||
            !decode_shape_fits(p.decode_variant, KC, p.splits, p.G) ||
            p.slab_chunks != KC / (p.splits * c.waves) || p.block != c.waves * 64 ||
            (int64_t)p.grid != (int64_t)ntiles * p.splits)
            return W4A16_ERR_INVALID;
        if (p.splits > 1 && (p.counter_slots < ntiles ||
                             p.workspace_bytes < (uint64_t)p.splits * p.M * p.N * sizeof(float)))
            return W4A16_ERR_WORKSPACE;
        return W4A16_OK;
    }
    if (p.kernel < 1 || p.kernel > kNumPrefillTable) return W4A16_ERR_INVALID;
    // The grid (tiles x K segments of the split-K kinds) bounds every segment and tile index a
    // prefill kernel touches.
    const PrefillTile& t = kPrefillTable[p.kernel];
    const int segs = t.kind >= 2 ? prefill_segments(p.K >> 6) : 1;
    const int64_t tiles = ((int64_t)(p.M + t.bm - 1) / t.bm) * ((p.N + t.bn - 1) / t.bn);
    if (!prefill_shape_ok(p.kernel, p.M, p.K) || (p.splits > 1 ? p.splits : 1) != segs ||
        (int64_t)p.grid != tiles * segs)
        return W4A16_ERR_INVALID;
    if (segs > 1 && ((int64_t)p.counter_slots < tiles ||
                     p.workspace_bytes < (uint64_t)segs * p.M * p.N * sizeof(float)))
        return W4A16_ERR_WORKSPACE;
    return W4A16_OK;
}
}  // namespace

// Test hook (no counterpart in the reference): the launch-side plan check alone, without a launch.
extern "C" int w4a16_debug_check_plan(const w4a16_plan* plan) {
    return plan ? check_plan(*plan) : W4A16_ERR_INVALID;
}

extern "C" int w4a16_launch(const w4a16_plan* plan, const int32_t* Wp, const uint16_t* x,
                            const uint16_t* scales, uint16_t* y, void* workspace, int32_t* counters,
                            void* stream) {
    if (!plan) return W4A16_ERR_INVALID;
    const w4a16_plan& p = *plan;
    if (p.grid <= 0 || p.M <= 0 || p.N <= 0 || p.K <= 0) return W4A16_OK;   // empty output
    if (p.workspace_bytes && !workspace) return W4A16_ERR_WORKSPACE;
    if (p.counter_slots && !counters) return W4A16_ERR_WORKSPACE;
    if (const int rc = check_plan(p); rc != W4A16_OK) return rc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const u4* wp = reinterpret_cast<const u4*>(Wp);
    hipError_t e = hipSuccess;
    if (p.kernel == W4A16_VARIANT_DECODE) {
        float* ws = reinterpret_cast<float*>(workspace);
        int* cnt = reinterpret_cast<int*>(counters);
        e = launch_decode(p, wp, x, scales, y, ws, cnt, st);
    } else {
        switch (p.kernel) {
            case 1: e = launch_prefill<1>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 2: e = launch_prefill<2>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 3: e = launch_prefill<3>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 4: e = launch_prefill<4>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 5: e = launch_prefill<5>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 6: e = launch_prefill<6>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 7: e = launch_prefill<7>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 8: e = launch_prefill<8>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 9: e = launch_prefill<9>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 10: e = launch_prefill<10>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 11: e = launch_prefill<11>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 12: e = launch_prefill<12>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 13: e = launch_prefill<13>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 14: e = launch_prefill<14>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 15: e = launch_prefill<15>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 16: e = launch_prefill<16>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 17: e = launch_prefill<17>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 18: e = launch_prefill<18>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 19: e = launch_prefill<19>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 20: e = launch_prefill<20>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 21: e = launch_prefill<21>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 22: e = launch_prefill<22>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 23: e = launch_prefill<23>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            case 24: e = launch_prefill<24>(p, wp, x, scales, y, reinterpret_cast<float*>(workspace), counters, st); break;
            default: return W4A16_ERR_INVALID;
        }
    }
    if (e != hipSuccess) {
        w4a16_set_last_error(hipGetErrorString(e));
        return W4A16_ERR_HIP;
    }
    return W4A16_OK;
}

// Test hook (no counterpart in the reference): the compiled occupancy of prefill config `cfg`
// on the current device, which the planner's table must match.
extern "C" int w4a16_debug_kernel_occupancy(int cfg) {
    switch (cfg) {
        case 1: return prefill_occupancy_of<1>();
        case 2: return prefill_occupancy_of<2>();
        case 3: return prefill_occupancy_of<3>();
        case 4: return prefill_occupancy_of<4>();
        case 5: return prefill_occupancy_of<5>();
        case 6: return prefill_occupancy_of<6>();
        case 7: return prefill_occupancy_of<7>();
        case 8: return prefill_occupancy_of<8>();
        case 9: return prefill_occupancy_of<9>();
        case 10: return prefill_occupancy_of<10>();
        case 11: return prefill_occupancy_of<11>();
        case 12: return prefill_occupancy_of<12>();
        case 13: return prefill_occupancy_of<13>();
        case 14: return prefill_occupancy_of<14>();
        case 15: return prefill_occupancy_of<15>();
        case 16: return prefill_occupancy_of<16>();
        case 17: return prefill_occupancy_of<17>();
        case 18: return prefill_occupancy_of<18>();
        case 19: return prefill_occupancy_of<19>();
        case 20: return prefill_occupancy_of<20>();
        case 21: return prefill_occupancy_of<21>();
        case 22: return prefill_occupancy_of<22>();
        case 23: return prefill_occupancy_of<23>();
        case 24: return prefill_occupancy_of<24>();
        default: return -1;
    }
}

#ifdef W4A16_WAVE_STAMPS
// Instrumented builds only: copy out the stamps of the first `waves` waves (kStampWords words
// each; at most kStampWaves) / clear them.  Synchronous: call outside graph capture, after the
// launch has completed.  W4A16_OK, W4A16_ERR_INVALID or W4A16_ERR_HIP.
extern "C" int w4a16_debug_wave_stamps(uint32_t* dst, int32_t waves) {
    if (waves <= 0 || waves > w4a16::kStampWaves || !dst) return W4A16_ERR_INVALID;
    if (hipMemcpyFromSymbol(dst, HIP_SYMBOL(w4a16::g_wave_stamps), (size_t)waves * w4a16::kStampWords * 4, 0,
                            hipMemcpyDeviceToHost) != hipSuccess)
        return W4A16_ERR_HIP;
    return W4A16_OK;
}
extern "C" int w4a16_debug_wave_stamps_clear(void) {
    static uint32_t zeros[w4a16::kStampWaves * w4a16::kStampWords];
    return hipMemcpyToSymbol(HIP_SYMBOL(w4a16::g_wave_stamps), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice) ==
                   hipSuccess ? W4A16_OK : W4A16_ERR_HIP;
}
#endif
