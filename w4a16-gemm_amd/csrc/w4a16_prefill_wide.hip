// Wide-tile prefill (configs 5..7 and 18..24 of kPrefillTable, kind 1) in its own translation unit.
//
// Built with -mllvm -amdgpu-sched-strategy=max-memory-clause (build.py): with the default
// scheduler the register allocator gives most MFMAs a destination other than their accumulator
// input and rotates the 128 accumulators through copies (96 v_accvgpr_mov plus 56 AGPR<->VGPR
// transfers per two chunks, which serialise the MFMA pipe); with this strategy every
// accumulator stays in place in 128 AGPRs and the loop body is ~30% shorter.  The decode and
// other prefill kernels keep the default scheduler (the strategy does not help them).
// Kernel arguments: the first 16 dwords are preloaded into SGPRs (build.py), and the kernels take
// what their prologue needs first (the grid size included, instead of gridDim.x), y last.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstdlib>

#include "w4a16.h"
#include "w4a16_asm.h"
#include "w4a16_device.h"
#include "w4a16_internal.h"

namespace w4a16 {

// Prefill with large wave tiles on v_mfma_f32_32x32x16_f16.
//
// Wave tile WM x WN (tokens x channels) = TM x TN blocks of 32 x 32.  Per 64-wide K chunk and
// chunk half h the k-slots of the 16x16x32 formulation (k = 32h + 8c + 2t + e, t = 0..3) are fed
// as two 32x32x16 steps, t in {0, 1} then t in {2, 3}: lane (kg = l / 32, r = l % 32) supplies
// t = 2 tp + kg.  Measured on MI355X, this gives every accumulator bit for bit the same value as
// the 16x16x32 kernels (see mfma32x32x16), so all prefill configs stay bit-identical.  One
// 32x32x16 instruction does the work of two 16x16x32 ones, which halves the MFMA issue slots per
// chunk: with one wave per SIMD the wave's instruction stream (MFMA issue + dequantisation VALU +
// memory) and not the matrix pipe limited the 16x16x32 version.
//  * A (weights, rows = channels): lane (kg, r) reads the 16-byte word quad of packed lane
//    4 (r % 8) + 2 tp + kg of n16 block 2q + r / 16 and keeps the nibbles of its own channel
//    (odd pairs for r % 16 >= 8), exactly as the 16x16x32 kernels do; the word quad gives the A
//    operands of both halves of the chunk.
//  * B (x, columns = tokens): one 16-byte LDS read per (token block, tp, h) from the permuted x
//    layout shared with the other prefill kernels (dword 16h + 4t + c).
//  * D: register i of lane (kg, r) holds channel 8 (i / 4) + 4 kg + i % 4 of token r: four runs
//    of four consecutive channels, each one 8-byte fp16 store.
//  * The weights of chunk kc+2 are loaded while chunk kc is multiplied, into two named register
//    sets used alternately (the loop is unrolled by two chunks, K/64 must be even).
//  * Rows past M and channels past N load clamped, in-bounds data instead of branching (their
//    results are never stored and rows never mix).
//  * XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs, so block b is
//    given tile (b % 8) * (G / 8) + b / 8: each XCD walks consecutive tiles through its own L2.
//    Consecutive tiles run in groups of group_m M tiles: within a group the M tile varies
//    fastest, then the N tile, so the workgroups resident at one time share group_m M tiles of x
//    and their weight tiles.  Measured on configs[3] (M = 2048, 16 M tiles): group_m = 4 fetches
//    0.94 GB per launch from beyond L2 against 2.01 GB with all 16 M tiles of a weight tile
//    first, and runs 2-3% faster (931 vs 953-962 us); 2 and 8 are within 1% of 4.
// Waves per SIMD the wide kernels' registers are budgeted for (WPE, the table's wpe field).
// 128 x 256 tiles (1 x 4 waves): 2, i.e. two workgroups per CU, so one workgroup's MFMAs run
// while the other dequantises, stages x and waits at its barrier (at 1, the default for its 328
// registers, the matrix cores idled ~48% of the time).  The compiler then keeps the 128
// accumulators in VGPRs and spills three registers outside the loop.  256 x 128 and 128 x 128
// (1 x 2) stay at 1: at 2, 256 x 128 spills 67 times inside its loop and 128 x 128 spills a
// pending asm-load destination (tests/test_isa_hazards.py rejects that).  The 32-channel wave
// tiles (configs 18..20, 24) and the 8-wave tiles of 128 x 64 waves (256 x 256 and 128 x 512) fit
// 2 without spills.
// SEG: K longer than one canonical segment (seg_chunks chunks, even): acc holds the running
// segment and total the sum of the finished ones (total = p0, then total + p_s), closed after
// every seg_chunks chunks of the two-chunk loop.
template <int BM, int BN, int WAVES_M, int WAVES_N, int WPE, bool SEG, int R>
__global__ void __launch_bounds__(WAVES_M * WAVES_N * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
prefill_wide_kernel(const u4* __restrict__ Wp, const uint16_t* __restrict__ x,
                    const uint16_t* __restrict__ scales,
                    int M, int N, int K, int gshift, int tiles_m, int group_m, int seg_chunks, int G,
                    uint16_t* __restrict__ y) {
    constexpr int NT = WAVES_M * WAVES_N * 64;
    constexpr int WM = BM / WAVES_M;
    constexpr int WN = BN / WAVES_N;
    constexpr int TM = WM / 32;
    constexpr int TN = WN / 32;
    constexpr int XBUF = BM * kXRow;
    constexpr int SEGS = BM * 8;
    constexpr int SPT = SEGS / NT;
    static_assert(WM % 32 == 0 && WN % 32 == 0 && SEGS % NT == 0, "tile shape");
    __shared__ __attribute__((aligned(16))) char xs[2 * XBUF];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);      // wave-uniform (SGPR)
    const int wm = wave / WAVES_N;
    const int wn = wave - wm * WAVES_N;
    const int kg = lane >> 5;
    const int r = lane & 31;

    // XCD-aware tile order (a bijection on [0, G), G = gridDim.x).
    const int G8 = G >> 3;
    const int b = blockIdx.x;
    const int tile = b < (G8 << 3) ? (b & 7) * G8 + (b >> 3) : b;
    const int tiles_n = G / tiles_m;
    const int gid = tile / (group_m * tiles_n);
    const int first_m = gid * group_m;
    const int gsz = min(tiles_m - first_m, group_m);
    const int rem = tile - gid * group_m * tiles_n;
    const int tm = first_m + rem % gsz;
    const int tn = rem / gsz;
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const int KC = K >> 6;
    const int NBLK = N >> 4;
    const int nb0 = (n0 + wn * WN) >> 4;                            // first n16 block of the wave

    // All global loads are issued through asm with a wave-uniform base (SGPRs, advanced per
    // chunk) and a constant 32-bit per-lane byte offset, and waited for with explicit counts: the
    // compiler's own wait placement drained every prefetch at the loop back-edge.
    // The wave-uniform base is the first n16 block of the 32-channel block q and the lane adds 0
    // or 1 block (r / 16), both clamped to the last block of N, so the unsigned 32-bit lane offset
    // is never negative (blocks past N re-read the last block; their results are never stored).
    const char* wbase[TN];
    const char* sbase[TN];
    int qblk[TN];
#pragma unroll
    for (int q = 0; q < TN; ++q) {
        qblk[q] = min(nb0 + 2 * q, NBLK - 1);
        wbase[q] = reinterpret_cast<const char*>(Wp + (size_t)qblk[q] * KC * 32);
        sbase[q] = reinterpret_cast<const char*>(scales + (size_t)qblk[q] * 16);
    }
    uint32_t woff[TN][2];
    uint32_t soff[TN];
#pragma unroll
    for (int q = 0; q < TN; ++q) {
        const int nbl = min(nb0 + 2 * q + (r >> 4), NBLK - 1) - qblk[q];          // 0 or 1
#pragma unroll
        for (int tp = 0; tp < 2; ++tp)
            woff[q][tp] = (uint32_t)(nbl * KC * 512 + (((r & 7) << 2) | (tp << 1) | kg) * 16);
        soff[q] = (uint32_t)((nbl * 16 + (r & 15)) * 2);
    }
    const char* xbase = reinterpret_cast<const char*>(x + (size_t)m0 * K);
    uint32_t xoff[SPT];                                        // bytes, relative to row m0, chunk 0
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
        const int sg = tid + i * NT;
        xoff[i] = ((uint32_t)(min(m0 + (sg >> 3), M - 1) - m0) * (uint32_t)K + (sg & 7) * 8) * 2;
    }

    u4 xr[R][SPT];                                            // R register sets of prefetched chunks
    auto load_x = [&](int kc, u4 (&xr)[SPT]) __attribute__((always_inline)) {
        const char* xb = xbase + (size_t)min(kc, KC - 1) * 128;   // past the end: harmless reload
#pragma unroll
        for (int i = 0; i < SPT; ++i) xr[i] = gload_u4_sbase(xb, xoff[i]);
    };
    auto store_x = [&](int buf, u4 (&xr)[SPT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < SPT; ++i) bind_after_wait(xr[i]);
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const int sg = tid + i * NT;
            lds_store_xseg(xs + buf * XBUF + (sg >> 3) * kXRow, sg & 7, xr[i]);
        }
    };
    u4 wr[R][TN][2];
    uint32_t sr[R][TN];
    auto load_w = [&](int kc, u4 (&w)[TN][2], uint32_t (&s)[TN]) __attribute__((always_inline)) {
        const int kcl = min(kc, KC - 1);
#pragma unroll
        for (int q = 0; q < TN; ++q)
#pragma unroll
            for (int tp = 0; tp < 2; ++tp) w[q][tp] = gload_u4_sbase(wbase[q] + (size_t)kcl * 512, woff[q][tp]);
#pragma unroll
        for (int q = 0; q < TN; ++q) s[q] = gload_u16_sbase(sbase[q] + (size_t)(kcl >> gshift) * N * 2, soff[q]);
    };
    // Per chunk: SPT x loads and 3 TN weight/scale loads.  In flight when chunk c starts, oldest
    // first: x c+1, weights c, x c+2, weights c+1, ..., x c+R, weights c+R-1.  Younger than x of
    // chunk c+1: weights c and R-1 chunks' loads; younger than the weights of chunk c once x of
    // chunk c+1+R is issued: R-1 chunks' loads and that x.
    constexpr int WAIT_X = 3 * TN + (R - 1) * (SPT + 3 * TN);
    constexpr int WAIT_W = (R - 1) * (SPT + 3 * TN) + SPT;
    static_assert(R == 2 || R == 4, "register sets: the x LDS buffer parity must be static in the unrolled loop");
    static_assert(WAIT_X <= 63 && WAIT_W <= 63, "vmcnt range");

    f32x16 acc[TM][TN];
#pragma unroll
    for (int p = 0; p < TM; ++p)
#pragma unroll
        for (int q = 0; q < TN; ++q)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[p][q][i] = 0.f;

    f32x16 total[SEG ? TM : 1][SEG ? TN : 1];
    int seg_left = seg_chunks;
    bool first_seg = true;

    const Dq d = dq_setup(r);                                  // nibble parity of channel r % 16
    const uint32_t xrow = (uint32_t)reinterpret_cast<uintptr_t>(xs) + (wm * WM + r) * kXRow + kg * 16;
    // One chunk: for each half h, the 2 TM B operands are read from LDS through asm (the compiler
    // would follow each read with a full lgkmcnt wait), the 2 TN A operands are dequantised
    // while the reads are in flight, then one wait and the 4 TM TN MFMAs (tp = 0 before tp = 1).
    // The buffer and every B-operand offset are compile-time constants carried in the ds_read
    // offset field (no address arithmetic per read).
    auto compute = [&](auto buf, u4 (&w)[TN][2], uint32_t (&s)[TN]) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < TN; ++q) {
            bind_after_wait(w[q][0]); bind_after_wait(w[q][1]); bind_after_wait(s[q]);
        }
        static_for<0, 2>([&](auto hh) {
            constexpr int h = decltype(hh)::value;
            u4 bv[TM][2];
            static_for<0, TM>([&](auto pp) {
                constexpr int P = decltype(pp)::value;
                constexpr int O = decltype(buf)::value * XBUF + P * 32 * kXRow + h * 64;
                bv[P][0] = lds_read_u4_at<O>(xrow);
                bv[P][1] = lds_read_u4_at<O + 32>(xrow);
            });
            h8 a[TN][2];
#pragma unroll
            for (int q = 0; q < TN; ++q) {
                const h2 s2 = scale2((uint16_t)s[q]);
#pragma unroll
                for (int tp = 0; tp < 2; ++tp)
                    a[q][tp] = h ? dq_frag(w[q][tp].z, w[q][tp].w, d, s2) : dq_frag(w[q][tp].x, w[q][tp].y, d, s2);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int p = 0; p < TM; ++p) { bind_after_wait(bv[p][0]); bind_after_wait(bv[p][1]); }
#pragma unroll
            for (int tp = 0; tp < 2; ++tp)
#pragma unroll
                for (int p = 0; p < TM; ++p) {
                    const h8 bf = __builtin_bit_cast(h8, bv[p][tp]);
#pragma unroll
                    for (int q = 0; q < TN; ++q) acc[p][q] = mfma32x32x16(a[q][tp], bf, acc[p][q]);
                }
        });
    };

    // Issue order: prologue x0 | x1 w0 x2 w1 ... x(R) w(R-1); then chunk c issues x(c+1+R) and
    // w(c+R).  Chunk c uses x buffer c & 1, and register set c % R for its weights and for x of
    // chunk c+1 (the loop is unrolled by R chunks; K/64 is a multiple of R, checked by the
    // planner).  x of chunk c+1 is written to the other LDS buffer first, so those LDS writes
    // overlap the MFMAs.  One barrier per chunk orders both buffers.  Loads past the end re-read
    // the last chunk into registers nobody uses again.  SEG: a segment closes after every
    // seg_chunks chunks (and at the end), a multiple of R (checked by the planner).
    load_x(0, xr[0]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    store_x(0, xr[0]);
    static_for<1, R + 1>([&](auto j) {
        constexpr int J = decltype(j)::value;
        load_x(J, xr[J % R]);
        load_w(J - 1, wr[(J - 1) % R], sr[(J - 1) % R]);
    });
    __syncthreads();
    for (int kc = 0; kc < KC; kc += R) {
        static_for<0, R>([&](auto t) {
            constexpr int T = decltype(t)::value;
            const int c = kc + T;
            wait_vmcnt<WAIT_X>();
            store_x((T + 1) & 1, xr[(T + 1) % R]);
            load_x(c + 1 + R, xr[(T + 1) % R]);
            wait_vmcnt<WAIT_W>();
            compute(std::integral_constant<int, T & 1>{}, wr[T], sr[T]);
            load_w(c + R, wr[T], sr[T]);
            __syncthreads();
        });
        if constexpr (SEG) {
            seg_left -= R;
            if (seg_left == 0 || kc + R >= KC) {
#pragma unroll
                for (int p = 0; p < TM; ++p)
#pragma unroll
                    for (int q = 0; q < TN; ++q) {
                        total[p][q] = first_seg ? acc[p][q] : total[p][q] + acc[p][q];
#pragma unroll
                        for (int i = 0; i < 16; ++i) acc[p][q][i] = 0.f;
                    }
                first_seg = false;
                seg_left = seg_chunks;
            }
        }
    }
    // No load in flight at exit.  The registers of the last (unused) prefetches are re-bound
    // after the wait: otherwise the compiler, seeing them dead, reuses them before it.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
        for (int i = 0; i < SPT; ++i) bind_after_wait(xr[j][i]);
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
        for (int q = 0; q < TN; ++q) {
            bind_after_wait(wr[j][q][0]); bind_after_wait(wr[j][q][1]); bind_after_wait(sr[j][q]);
        }

    // The lane id again, from v_mbcnt (opaque to the compiler): keeping r and kg live across the
    // loop would cost two registers, which at two waves per SIMD the allocator spills.
    int lane_e;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_e));
    const int r_e = lane_e & 31;
    const int kg_e = lane_e >> 5;
#pragma unroll
    for (int p = 0; p < TM; ++p) {
        const int m = m0 + wm * WM + p * 32 + r_e;
        if (m >= M) continue;
#pragma unroll
        for (int q = 0; q < TN; ++q) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int nbk = nb0 + 2 * q + (g >> 1);
                const int n = (nb0 + 2 * q) * 16 + 8 * g + 4 * kg_e;
                if (nbk < NBLK)
                    *reinterpret_cast<u2*>(y + (size_t)m * N + n) =
                        pack_f16x4(SEG ? f4{total[SEG ? p : 0][SEG ? q : 0][4 * g], total[SEG ? p : 0][SEG ? q : 0][4 * g + 1],
                                            total[SEG ? p : 0][SEG ? q : 0][4 * g + 2], total[SEG ? p : 0][SEG ? q : 0][4 * g + 3]}
                                       : f4{acc[p][q][4 * g], acc[p][q][4 * g + 1], acc[p][q][4 * g + 2], acc[p][q][4 * g + 3]});
            }
        }
    }
}

// The same tiles software-pipelined across chunks, for the 32-channel wave tiles that run one wave
// per SIMD (few tiles: moderate M).  prefill_wide_kernel serialises each chunk -- x store, B reads
// after the barrier, dequantisation, then the MFMAs -- and with no second wave on the SIMD every
// latency in that chain is exposed (configs[2]: ~1000 cycles per chunk for 256 cycles of MFMA).
// Here x has three LDS buffers, so the barrier that ends chunk c-1 has already published x of
// chunk c+1, and during chunk c's MFMAs each wave
//  * reads chunk c+1's B operands from LDS into a second register set,
//  * dequantises chunk c+1's weights (loaded R chunks ahead) into a second set of A operands,
//  * stores x of chunk c+2 into the third buffer and issues the loads R chunks ahead.
// Chunk c uses x buffer c % 3 (a wave-uniform rotation) and register sets c % R (static: the loop
// is unrolled by R).  In flight when chunk c starts, oldest first: x c+2, weights c+1, x c+3,
// weights c+2, ..., x c+1+R, weights c+R.  Each accumulator receives exactly the MFMA sequence of
// prefill_wide_kernel (chunk by chunk, h = 0 then 1, tp = 0 then 1, same A and B operands), so
// the output is bit-identical to every other prefill config.  One K chain only (K <= 8192): the
// second register sets leave no room for the long-K segments' second accumulator set.
// Measured on MI355X against the same tiles unpipelined: 6-10% faster at M = 64..512 (configs[2]:
// 30.7 -> 27.6 us); loads eight chunks ahead, or MFMAs and dequantisation interleaved one by one
// (sched_group_barrier), were no faster.
template <int BM, int BN, int WAVES_M, int WAVES_N, int WPE, bool SEG, int R>
__global__ void __launch_bounds__(WAVES_M * WAVES_N * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
prefill_wide_pipe_kernel(const u4* __restrict__ Wp, const uint16_t* __restrict__ x,
                         const uint16_t* __restrict__ scales,
                         int M, int N, int K, int gshift, int tiles_m, int group_m, int seg_chunks, int G,
                         uint16_t* __restrict__ y) {
    constexpr int NT = WAVES_M * WAVES_N * 64;
    constexpr int WM = BM / WAVES_M;
    constexpr int WN = BN / WAVES_N;
    constexpr int TM = WM / 32;
    constexpr int TN = WN / 32;
    constexpr int XBUF = BM * kXRow;
    constexpr int SEGS = BM * 8;
    constexpr int SPT = SEGS / NT;
    static_assert(WM % 32 == 0 && WN % 32 == 0 && SEGS % NT == 0, "tile shape");
    static_assert(R == 2 || R == 4, "register sets: the A/B operand sets alternate with the chunk parity");
    static_assert(!SEG, "one K chain only: the pipelined tiles are not used above K = 8192 (no registers for a second set)");
    __shared__ __attribute__((aligned(16))) char xs[3 * XBUF];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N;
    const int wn = wave - wm * WAVES_N;
    const int kg = lane >> 5;
    const int r = lane & 31;

    // Tile order as in prefill_wide_kernel (XCD-contiguous, groups of group_m M tiles).
    const int G8 = G >> 3;
    const int b = blockIdx.x;
    const int tile = b < (G8 << 3) ? (b & 7) * G8 + (b >> 3) : b;
    const int tiles_n = G / tiles_m;
    const int gid = tile / (group_m * tiles_n);
    const int first_m = gid * group_m;
    const int gsz = min(tiles_m - first_m, group_m);
    const int rem = tile - gid * group_m * tiles_n;
    const int tm = first_m + rem % gsz;
    const int tn = rem / gsz;
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const int KC = K >> 6;
    const int NBLK = N >> 4;
    const int nb0 = (n0 + wn * WN) >> 4;

    // Load addressing as in prefill_wide_kernel: wave-uniform bases, constant per-lane offsets,
    // rows past M and blocks past N clamped in bounds.
    const char* wbase[TN];
    const char* sbase[TN];
    int qblk[TN];
#pragma unroll
    for (int q = 0; q < TN; ++q) {
        qblk[q] = min(nb0 + 2 * q, NBLK - 1);
        wbase[q] = reinterpret_cast<const char*>(Wp + (size_t)qblk[q] * KC * 32);
        sbase[q] = reinterpret_cast<const char*>(scales + (size_t)qblk[q] * 16);
    }
    uint32_t woff[TN][2];
    uint32_t soff[TN];
#pragma unroll
    for (int q = 0; q < TN; ++q) {
        const int nbl = min(nb0 + 2 * q + (r >> 4), NBLK - 1) - qblk[q];
#pragma unroll
        for (int tp = 0; tp < 2; ++tp)
            woff[q][tp] = (uint32_t)(nbl * KC * 512 + (((r & 7) << 2) | (tp << 1) | kg) * 16);
        soff[q] = (uint32_t)((nbl * 16 + (r & 15)) * 2);
    }
    const char* xbase = reinterpret_cast<const char*>(x + (size_t)m0 * K);
    uint32_t xoff[SPT];
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
        const int sg = tid + i * NT;
        xoff[i] = ((uint32_t)(min(m0 + (sg >> 3), M - 1) - m0) * (uint32_t)K + (sg & 7) * 8) * 2;
    }

    u4 xr[R][SPT];
    auto load_x = [&](int kc, u4 (&xv)[SPT]) __attribute__((always_inline)) {
        const char* xb = xbase + (size_t)min(kc, KC - 1) * 128;
#pragma unroll
        for (int i = 0; i < SPT; ++i) xv[i] = gload_u4_sbase(xb, xoff[i]);
    };
    auto store_x = [&](int buf, u4 (&xv)[SPT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < SPT; ++i) bind_after_wait(xv[i]);
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const int sg = tid + i * NT;
            lds_store_xseg(xs + buf * XBUF + (sg >> 3) * kXRow, sg & 7, xv[i]);
        }
    };
    u4 wr[R][TN][2];
    uint32_t sr[R][TN];
    auto load_w = [&](int kc, u4 (&w)[TN][2], uint32_t (&s)[TN]) __attribute__((always_inline)) {
        const int kcl = min(kc, KC - 1);
#pragma unroll
        for (int q = 0; q < TN; ++q)
#pragma unroll
            for (int tp = 0; tp < 2; ++tp) w[q][tp] = gload_u4_sbase(wbase[q] + (size_t)kcl * 512, woff[q][tp]);
#pragma unroll
        for (int q = 0; q < TN; ++q) s[q] = gload_u16_sbase(sbase[q] + (size_t)(kcl >> gshift) * N * 2, soff[q]);
    };
    constexpr int WAIT_X = 3 * TN + (R - 1) * (SPT + 3 * TN);
    constexpr int WAIT_W = (R - 1) * (SPT + 3 * TN) + SPT;
    static_assert(WAIT_X <= 63 && WAIT_W <= 63, "vmcnt range");

    f32x16 acc[TM][TN];
#pragma unroll
    for (int p = 0; p < TM; ++p)
#pragma unroll
        for (int q = 0; q < TN; ++q)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[p][q][i] = 0.f;

    const Dq d = dq_setup(r);
    const uint32_t xrow = (uint32_t)reinterpret_cast<uintptr_t>(xs) + (wm * WM + r) * kXRow + kg * 16;
    u4 bv[2][TM][2][2];                                        // B operands [set][p][h][tp]
    h8 av[2][TN][2][2];                                        // A operands [set][q][h][tp]
    auto read_b = [&](int buf, u4 (&bo)[TM][2][2]) __attribute__((always_inline)) {
        const uint32_t xb = xrow + buf * XBUF;                 // the offsets within the buffer are immediates
        static_for<0, TM>([&](auto pp) {
            constexpr int P = decltype(pp)::value;
            bo[P][0][0] = lds_read_u4_at<P * 32 * kXRow>(xb);
            bo[P][0][1] = lds_read_u4_at<P * 32 * kXRow + 32>(xb);
            bo[P][1][0] = lds_read_u4_at<P * 32 * kXRow + 64>(xb);
            bo[P][1][1] = lds_read_u4_at<P * 32 * kXRow + 96>(xb);
        });
    };
    auto bind_b = [&](u4 (&bo)[TM][2][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < TM; ++p)
#pragma unroll
            for (int h = 0; h < 2; ++h) { bind_after_wait(bo[p][h][0]); bind_after_wait(bo[p][h][1]); }
    };
    auto bind_w = [&](u4 (&w)[TN][2], uint32_t (&s)[TN]) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < TN; ++q) {
            bind_after_wait(w[q][0]); bind_after_wait(w[q][1]); bind_after_wait(s[q]);
        }
    };
    auto dequant = [&](u4 (&w)[TN][2], uint32_t (&s)[TN], h8 (&a)[TN][2][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < TN; ++q) {
            const h2 s2 = scale2((uint16_t)s[q]);
#pragma unroll
            for (int tp = 0; tp < 2; ++tp) {
                a[q][0][tp] = dq_frag(w[q][tp].x, w[q][tp].y, d, s2);
                a[q][1][tp] = dq_frag(w[q][tp].z, w[q][tp].w, d, s2);
            }
        }
    };
    auto mma = [&](u4 (&bo)[TM][2][2], h8 (&a)[TN][2][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int tp = 0; tp < 2; ++tp)
#pragma unroll
                for (int p = 0; p < TM; ++p) {
                    const h8 bf = __builtin_bit_cast(h8, bo[p][h][tp]);
#pragma unroll
                    for (int q = 0; q < TN; ++q) acc[p][q] = mfma32x32x16(a[q][h][tp], bf, acc[p][q]);
                }
    };

    // Prologue: x of chunks 0 and 1 into buffers 0 and 1, chunk 0's operands into set 0, then
    // the loads x 2, w 1, ..., x R+1, w R (register sets 2 % R.. and 1.. once their data is used).
    load_x(0, xr[0]);
    load_x(1, xr[1]);
    load_w(0, wr[0], sr[0]);
    wait_vmcnt<0>();
    store_x(0, xr[0]);
    store_x(1, xr[1]);
    __syncthreads();
    read_b(0, bv[0]);
    bind_w(wr[0], sr[0]);
    dequant(wr[0], sr[0], av[0]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    bind_b(bv[0]);
    static_for<2, R + 2>([&](auto j) {
        constexpr int J = decltype(j)::value;
        load_x(J, xr[J % R]);
        load_w(J - 1, wr[(J - 1) % R], sr[(J - 1) % R]);
    });
    int b1 = 1, b2 = 2;                                        // x buffers of chunks c+1, c+2
    for (int kc = 0; kc < KC; kc += R) {
        static_for<0, R>([&](auto t) {
            constexpr int T = decltype(t)::value;
            constexpr int CUR = T & 1;
            const int c = kc + T;
            read_b(b1, bv[CUR ^ 1]);                           // B of chunk c+1
            wait_vmcnt<WAIT_X>();                              // x of chunk c+2 has landed
            store_x(b2, xr[(T + 2) % R]);
            load_x(c + 2 + R, xr[(T + 2) % R]);
            wait_vmcnt<WAIT_W>();                              // weights of chunk c+1 have landed
            bind_w(wr[(T + 1) % R], sr[(T + 1) % R]);
            mma(bv[CUR], av[CUR]);                             // chunk c
            dequant(wr[(T + 1) % R], sr[(T + 1) % R], av[CUR ^ 1]);
            load_w(c + 1 + R, wr[(T + 1) % R], sr[(T + 1) % R]);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            bind_b(bv[CUR ^ 1]);
            __builtin_amdgcn_s_barrier();                      // publishes x c+2, retires reads of x c+1's predecessor
            b1 = b2;
            b2 = b2 == 2 ? 0 : b2 + 1;
        });
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
        for (int i = 0; i < SPT; ++i) bind_after_wait(xr[j][i]);
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
        for (int q = 0; q < TN; ++q) {
            bind_after_wait(wr[j][q][0]); bind_after_wait(wr[j][q][1]); bind_after_wait(sr[j][q]);
        }

    int lane_e;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_e));
    const int r_e = lane_e & 31;
    const int kg_e = lane_e >> 5;
#pragma unroll
    for (int p = 0; p < TM; ++p) {
        const int m = m0 + wm * WM + p * 32 + r_e;
        if (m >= M) continue;
#pragma unroll
        for (int q = 0; q < TN; ++q) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int nbk = nb0 + 2 * q + (g >> 1);
                const int n = (nb0 + 2 * q) * 16 + 8 * g + 4 * kg_e;
                if (nbk < NBLK)
                    *reinterpret_cast<u2*>(y + (size_t)m * N + n) =
                        pack_f16x4(f4{acc[p][q][4 * g], acc[p][q][4 * g + 1], acc[p][q][4 * g + 2], acc[p][q][4 * g + 3]});
            }
        }
    }
}

constexpr int kWideGroupM = 4;                                 // M tiles per group of the tile order

template <int CFG, bool SEG>
static void launch_wide_kernel(const w4a16_plan& p, const u4* Wp, const uint16_t* x, const uint16_t* s, uint16_t* y,
                               hipStream_t st, int gshift, int tiles_m, int group_m, int seg_chunks) {
    constexpr PrefillTile c = kPrefillTable[CFG];
    constexpr int R = prefill_wide_steps(CFG, SEG);
    if constexpr (c.pipe)
        hipLaunchKernelGGL((prefill_wide_pipe_kernel<c.bm, c.bn, c.waves_m, c.waves_n, c.wpe, SEG, R>), dim3(p.grid),
                           dim3(c.waves_m * c.waves_n * 64), 0, st, Wp, x, s, p.M, p.N, p.K, gshift, tiles_m,
                           group_m, seg_chunks, p.grid, y);
    else
        hipLaunchKernelGGL((prefill_wide_kernel<c.bm, c.bn, c.waves_m, c.waves_n, c.wpe, SEG, R>), dim3(p.grid),
                           dim3(c.waves_m * c.waves_n * 64), 0, st, Wp, x, s, p.M, p.N, p.K, gshift, tiles_m,
                           group_m, seg_chunks, p.grid, y);
}

template <int CFG>
static hipError_t launch_wide(const w4a16_plan& p, const u4* Wp, const uint16_t* x, const uint16_t* s, uint16_t* y,
                              hipStream_t st) {
    constexpr PrefillTile c = kPrefillTable[CFG];
    static_assert(c.kind == 1, "wide prefill configs only");
    const int gshift = p.G == 128 ? 1 : 0;
    const int tiles_m = (p.M + c.bm - 1) / c.bm;
    int group_m = std::min(kWideGroupM, tiles_m);
    if (const char* o = std::getenv("W4A16_WIDE_GROUP_M")) {      // tuning override, read per call
        const int g = std::atoi(o);
        if (g >= 1) group_m = std::min(g, tiles_m);
    }
    const int KC = p.K >> 6;
    const int seg_chunks = prefill_segment_chunks(KC);
    if (prefill_segments(KC) > 1) {
        if constexpr (prefill_wide_segmentable(CFG))
            launch_wide_kernel<CFG, true>(p, Wp, x, s, y, st, gshift, tiles_m, group_m, seg_chunks);
        else
            return hipErrorInvalidValue;                      // no registers for a second set (planner never asks)
    } else {
        launch_wide_kernel<CFG, false>(p, Wp, x, s, y, st, gshift, tiles_m, group_m, seg_chunks);
    }
    return hipGetLastError();
}

// A kernel that does nothing.  The HIP runtime loads each unit's GPU code on the first launch of
// one of its kernels, and that load allocates device memory; w4a16_launch_noalloc launches this
// once per device in its first call, so that its later calls running wide configs allocate nothing.
__global__ void __launch_bounds__(64) wide_unit_load_kernel() {}

hipError_t prefill_wide_load_code(hipStream_t st) {
    hipLaunchKernelGGL(wide_unit_load_kernel, dim3(1), dim3(64), 0, st);
    return hipGetLastError();
}

hipError_t launch_prefill_wide(int cfg, const w4a16_plan& p, const u4* Wp, const uint16_t* x, const uint16_t* s,
                               uint16_t* y, hipStream_t st) {
    switch (cfg) {
        case 5: return launch_wide<5>(p, Wp, x, s, y, st);
        case 6: return launch_wide<6>(p, Wp, x, s, y, st);
        case 7: return launch_wide<7>(p, Wp, x, s, y, st);
        case 18: return launch_wide<18>(p, Wp, x, s, y, st);
        case 19: return launch_wide<19>(p, Wp, x, s, y, st);
        case 20: return launch_wide<20>(p, Wp, x, s, y, st);
        case 21: return launch_wide<21>(p, Wp, x, s, y, st);
        case 22: return launch_wide<22>(p, Wp, x, s, y, st);
        case 23: return launch_wide<23>(p, Wp, x, s, y, st);
        case 24: return launch_wide<24>(p, Wp, x, s, y, st);
        default: return hipErrorInvalidValue;
    }
}

// Resident workgroups per CU of a wide config's compiled kernel (HIP occupancy query), -1 on
// error; a test hook that checks the planner's table.
template <int CFG>
static int occupancy_wide() {
    constexpr PrefillTile c = kPrefillTable[CFG];
    constexpr int R = prefill_wide_steps(CFG, false);
    int n = 0;
    hipError_t e;
    if constexpr (c.pipe)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, prefill_wide_pipe_kernel<c.bm, c.bn, c.waves_m, c.waves_n, c.wpe, false, R>, c.waves_m * c.waves_n * 64, 0);
    else
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, prefill_wide_kernel<c.bm, c.bn, c.waves_m, c.waves_n, c.wpe, false, R>, c.waves_m * c.waves_n * 64, 0);
    return e == hipSuccess ? n : -1;
}

int prefill_wide_occupancy(int cfg) {
    switch (cfg) {
        case 5: return occupancy_wide<5>();
        case 6: return occupancy_wide<6>();
        case 7: return occupancy_wide<7>();
        case 18: return occupancy_wide<18>();
        case 19: return occupancy_wide<19>();
        case 20: return occupancy_wide<20>();
        case 21: return occupancy_wide<21>();
        case 22: return occupancy_wide<22>();
        case 23: return occupancy_wide<23>();
        case 24: return occupancy_wide<24>();
        default: return -1;
    }
}

}  // namespace w4a16
