/*
 * w4a16.h -- C ABI of the MI355X (gfx950) W4A16 GEMM library ``libw4a16_hip.so``.
 *
 *   y[M, N] = x[M, K] @ W^T,   W[n, k] = (q[n, k] - 8) * scales[k / G, n]
 *
 * x: fp16 [M, K] row-major.  scales: fp16 [K/G, N] row-major, G = K / (rows of scales) in {64, 128}.
 * Wp: int32 [N*K/8] packed nibbles in the reference's layout [N/16][K/64][32][4]
 * (reference tests/quant.py:34-48), read unchanged.  y: fp16 [M, N] row-major.
 *
 * Plain C types only (no torch, no HIP headers): device buffers are passed as pointers,
 * the HIP stream as an opaque ``void*`` (a ``hipStream_t``).
 *
 * Reference interfaces replaced (paths relative to the reference repository root):
 *   w4a16_plan_create      validation + routing + tile selection of
 *                          w4a16_gemm_cuda (src/vectorized/kernel.cu:218-249),
 *                          dispatch_prefill / pf_select (kernel.cu:142-156, 174-201)
 *   w4a16_launch           the launches of dispatch<G> / try_launch (kernel.cu:19-53) and
 *                          pf_launch / pf_launch_st (kernel.cu:117-138)
 *   w4a16_query_device     the device-attribute queries and occupancy probe cache
 *                          (kernel.cu:39-41, 72-115, 177-182)
 *   w4a16_gemm (pybind11, src/vectorized/extension.cpp:5-9) is re-exposed by the torch
 *   extension module ``w4a16_opt`` built on top of this ABI.
 *   w4a16_gemv             the launch of the baseline extension's w4a16_gemv_cuda
 *                          (src/baseline/kernel.cu:36-72); its pybind11 entry point
 *                          (src/baseline/extension.cpp:6-8) is re-exposed by ``w4a16_ext``.
 */
#ifndef W4A16_H_
#define W4A16_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version.  2: prefill plans may split K over workgroups (splits > 1, counter_slots and
 * workspace_bytes set, kernel ids 1..24), and the decode shape ids behind W4A16_DECODE were
 * renumbered; a caller written for version 1 (scratch only for decode split-K) must size the
 * workspace and counters from every plan. */
#define W4A16_ABI_VERSION 2

/* Status codes. */
#define W4A16_OK            0
#define W4A16_ERR_INVALID   1   /* argument / shape contract violated (message in err buffer) */
#define W4A16_ERR_NO_CONFIG 2   /* no kernel configuration fits the device limits            */
#define W4A16_ERR_HIP       3   /* a HIP runtime call failed                                   */
#define W4A16_ERR_WORKSPACE 4   /* workspace / counter buffer missing or too small            */

/* Variant ids (kernel.cu:217-224): -1 auto, 0 decode kernel, 1..4 prefill tile configs. */
#define W4A16_VARIANT_AUTO   (-1)
#define W4A16_VARIANT_DECODE 0
#define W4A16_NUM_PREFILL_CFG 4

/* Problem description.  Pointer values are used only for the 16-byte alignment check. */
typedef struct w4a16_problem {
    int64_t M, K, N;          /* x is [M, K]; scales is [groups, N]                     */
    int64_t groups;           /* rows of scales (K / G)                                  */
    int64_t wp_words;         /* number of int32 words in Wp (must be N*K/8)             */
    const void* Wp;
    const void* x;
    const void* scales;
} w4a16_problem;

/* Device limits the selector uses.  Fill with w4a16_query_device, or by hand on the host
 * (CPU tests inject small limits to exercise the "no configuration fits" path). */
typedef struct w4a16_device_limits {
    int32_t cu_count;             /* compute units (256 on MI355X)                      */
    int32_t lds_bytes_per_block;  /* max LDS bytes one workgroup may allocate            */
    int32_t max_threads_per_block;
    int32_t gcn_arch;             /* major*100 + minor*10 + stepping: 950 for gfx950,    */
                                  /* 910 for gfx90a, 1100 for gfx1100; 0 = unknown        */
} w4a16_device_limits;

/* A launch plan: the result of validation + routing + selection.  Plain data; copyable. */
typedef struct w4a16_plan {
    int32_t M, N, K, G;
    int32_t kernel;           /* 0 = decode, 1..24 = prefill tile config (1..4 forced)   */
    int32_t splits;           /* K ranges reduced across workgroups (decode split-K;
                                 prefill token-group configs: the K segments, K > 8192)  */
    int32_t slab_chunks;      /* decode: 64-wide K chunks per wave; prefill: chunks per
                                 K segment of the fixed accumulation order               */
    int32_t tile_n;           /* decode: output columns per workgroup                    */
    int32_t grid;             /* workgroups launched by the main kernel                  */
    int32_t block;            /* threads per workgroup                                   */
    int32_t counter_slots;    /* ints of the counter buffer used (split-K fixup)         */
    int32_t decode_variant;   /* decode: kernel shape id (waves, n16 blocks per wave)     */
    uint64_t workspace_bytes; /* bytes of fp32 partials the launch needs (0 if none)     */
} w4a16_plan;

/* Validate a problem and build a plan.  Pure host code: touches no device.
 * variant: -1 auto, 0 decode, 1..4 prefill config.  On failure returns W4A16_ERR_INVALID or
 * W4A16_ERR_NO_CONFIG and writes the reference's error message into err (NUL-terminated).
 * The messages (and their order) follow kernel.cu:224-249, 52, 196-198. */
int w4a16_plan_create(const w4a16_problem* prob, int variant, const w4a16_device_limits* lim,
                      w4a16_plan* plan, char* err, size_t errlen);

/* Launch a plan on a HIP stream (asynchronous; no host synchronisation, no allocation, so it
 * may be captured into a HIP graph).
 *   workspace : device buffer of >= plan->workspace_bytes bytes (may be NULL when 0).
 *   counters  : device int32 buffer of >= plan->counter_slots ints (may be NULL when 0).
 *               It must be all-zero before the first launch that uses it; every launch leaves
 *               it all-zero again.  Launches that share one counter buffer must not overlap
 *               in time (use one buffer per concurrently running stream).
 * The plan is checked against what its kernel derives from (M, N, K, G) before anything is
 * launched: a plan that does not match (grid, chunks per wave, block, shape id, split count)
 * returns W4A16_ERR_INVALID, a split plan whose buffers are declared too small
 * W4A16_ERR_WORKSPACE.
 * Returns W4A16_OK, W4A16_ERR_INVALID, W4A16_ERR_WORKSPACE or W4A16_ERR_HIP. */
int w4a16_launch(const w4a16_plan* plan, const int32_t* Wp, const uint16_t* x,
                 const uint16_t* scales, uint16_t* y, void* workspace, int32_t* counters,
                 void* stream);

/* Scratch limits of w4a16_launch_noalloc: fp32 partials and split-K counters it can hold. */
#define W4A16_NOALLOC_MAX_WORKSPACE_BYTES (4u << 20)
#define W4A16_NOALLOC_MAX_COUNTER_SLOTS   16384

/* w4a16_launch without a caller-provided workspace: the same kernels, with the split-K partials
 * and counters in a static device array of the library (4 MiB + 64 KiB per GPU, held until the
 * process ends).  No counterpart in the reference (its decode path needs no scratch); it is for
 * callers that cannot allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  It allocates nothing (no hipMalloc, no allocating library
 * call); the caller passes only the inputs and y.  Runs on the current HIP device, on `stream`.
 * The first call on a device, whatever its plan, resolves the array's address, clears its counters
 * with a small kernel on `stream` and launches a no-op kernel of the wide prefill code, so that the
 * HIP runtime loads the library's GPU code then (it does so on a unit's first kernel launch, and
 * that load allocates device memory); make that first call outside graph capture and before any
 * region that must not allocate.  Later calls allocate nothing and may be captured: the graph
 * replays them against the same array.  Every call on one GPU shares that GPU's array: calls whose
 * plans have workspace_bytes > 0 must not overlap in time on one GPU (they race on the partials and
 * counters); plans without a workspace (unsplit prefill and decode) use no scratch.
 * A prefill plan whose partials or counters exceed the array (long K at moderate M, which splits K
 * over workgroups) runs as a scratch-free config of the same problem instead: every prefill
 * config gives the same bits.
 * Returns W4A16_OK, W4A16_ERR_WORKSPACE when a decode plan's workspace_bytes exceeds
 * W4A16_NOALLOC_MAX_WORKSPACE_BYTES or its counter_slots exceed W4A16_NOALLOC_MAX_COUNTER_SLOTS
 * (message via w4a16_last_error), or W4A16_ERR_HIP. */
int w4a16_launch_noalloc(const w4a16_plan* plan, const int32_t* Wp, const uint16_t* x,
                         const uint16_t* scales, uint16_t* y, void* stream);

/* Quantise and pack a weight matrix on the device (asynchronous, no allocation).
 * Replaces the reference's torch-side quantize_w4 + pack_int4 (tests/quant.py:62-74, 34-48),
 * the producer of the Wp and scales that w4a16_gemm consumes:
 *   W      : [N, K] row-major, fp16 (w_is_fp32 = 0) or fp32 (w_is_fp32 = 1), device memory.
 *   Wp     : int32 [N*K/8] packed nibbles in the layout w4a16_launch reads.
 *   scales : fp16 bits [K/G, N], s = fp16(max(absmax(group) / 7, 1e-4)).
 * Codes q = clamp(round_half_even(W / s), -8, 7) + 8 with fp32 arithmetic, bit-identical to
 * the reference's torch fp32 path.  N % 16 == 0, K % 64 == 0, G in {64, 128}; W and Wp
 * 16-byte aligned.  Inputs must be finite (a NaN in a group gives unspecified codes).
 * Returns W4A16_OK, W4A16_ERR_INVALID (message via w4a16_last_error) or W4A16_ERR_HIP. */
int w4a16_quantize_pack(const void* W, int w_is_fp32, int64_t N, int64_t K, int64_t G,
                        int32_t* Wp, uint16_t* scales, void* stream);

/* Largest K that w4a16_gemv accepts: its per-digit int32 sums are exact up to this size. */
#define W4A16_GEMV_MAX_K (1 << 20)

/* Baseline W4A16 GEMV of the reference's second extension (src/baseline/kernel.cu:8-72), a
 * different weight format from w4a16_launch's:
 *   W  : int32 [N, K/8] row-major; nibble j (bits 4j..4j+3) of word k/8 of row n is the signed
 *        4-bit weight wv(n, k) (values 8..15 are -8..-1), k = 8*(k/8) + j   (kernel.cu:19-28)
 *   A  : fp16 bits [K];  sW, zW : fp16 bits [N] per-row scale and zero;  C : fp16 bits [N]
 *   C[n] = fp16_rn((acc - zW[n]) * sW[n]) in fp32                          (kernel.cu:31-33)
 * acc is the exact sum of wv(n, k) * A[k] rounded once to fp32 (the reference sums in fp32 in k
 * order; the two differ by that order's rounding error only).  Inf and NaN inputs give the IEEE
 * result of the sum.  K % 8 == 0, 0 <= K <= W4A16_GEMV_MAX_K; W 4-byte aligned, the others 2-byte
 * aligned (16-byte alignment of W with K % 32 == 0, and of A, selects wider loads).  Asynchronous
 * on `stream`, allocates nothing.  Returns W4A16_OK, W4A16_ERR_INVALID (message via
 * w4a16_last_error) or W4A16_ERR_HIP. */
int w4a16_gemv(const int32_t* W, const uint16_t* A, const uint16_t* sW, const uint16_t* zW, uint16_t* C,
               int64_t N, int64_t K, void* stream);

/* Query the limits of HIP device `device` (cached per device, thread-safe). */
int w4a16_query_device(int device, w4a16_device_limits* lim);

/* Largest counter_slots any plan may request (size of a counter buffer that fits all plans). */
int32_t w4a16_max_counter_slots(void);

/* Message of the last failing HIP call on this thread ("" if none). */
const char* w4a16_last_error(void);

/* ABI version (W4A16_ABI_VERSION). */
int w4a16_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* W4A16_H_ */
