/*
 * C restatement of the W4A16 reference algorithm -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library
 * (through oracle/c_oracle.py).  It is the checker and the timed CPU reference path; it is
 * never part of the product path.
 *
 * What it restates (reference paths relative to the reference repository root):
 *   - pack / unpack of the int32 nibble format      tests/quant.py:34-59 (word index :37,
 *                                                    nibble order :19-24, int32 wrap :47)
 *   - dequantisation, written the way the kernel     src/vectorized/common.cuh:45-55
 *     does it: ((w >> 4p) & 0x000F000F) | 0x64006400 gives fp16 1024+q, minus 1032 gives q-8
 *     exactly, then one round-to-nearest-even fp16 multiply by the scale
 *   - the fp32 reference GEMM over dequantised      tests/quant.py:83-85
 *     weights (y = x.float() @ Wdeq.float().T), and the fp16 output rounding of the op
 *     (src/vectorized/prefill.cuh:178-181, __floats2half2_rn)
 *   - the baseline GEMV of the second extension     src/baseline/kernel.cu:8-34
 *     (w4a16_ext.w4a16_gemv): in the reference's fp32 k order, and as the exact sum rounded once
 *
 * fp16 <-> fp32 conversions are written here from the IEEE 754 binary16 definition.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

float w4a16_oracle_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    float f;
    if (e == 0) {
        f = (float)m * 0x1p-24f;                       /* zero or subnormal: m * 2^-24, exact */
        return sign ? -f : f;
    }
    if (e == 31) bits = sign | 0x7F800000u | (m << 13);                /* inf / nan */
    else bits = sign | ((e + 112u) << 23) | (m << 13);                 /* rebias 15 -> 127 */
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t w4a16_oracle_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return sign | 0x7E00u;                       /* nan */
    if (ax >= 0x47800000u) return sign | 0x7C00u;                      /* |f| >= 2^16 -> inf */
    if (ax < 0x38800000u) {                                            /* |f| < 2^-14 */
        float af;
        memcpy(&af, &ax, 4);
        double r = nearbyint((double)af * 16777216.0);                 /* units of 2^-24, RNE */
        return sign | (uint16_t)r;                                     /* r == 1024 encodes 2^-14 */
    }
    uint32_t h = ((ax >> 23) - 112u) << 10 | ((ax & 0x7FFFFFu) >> 13);
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;        /* RNE; carry may reach inf */
    return sign | (uint16_t)h;
}

/* Word index of code (n, k) and its nibble position (tests/quant.py:19-24, :37). */
static inline void locate(int n, int k, int K, size_t* word, int* nib) {
    const int nb = n >> 4, nr = n & 15, kc = k >> 6, kr = k & 63;
    const int s = kr >> 4, kk = kr & 15;
    const int a = nr >> 3, g = nr & 7;                 /* n = g + 8a            */
    const int b = kk >> 3, t = (kk & 7) >> 1, h = kk & 1;  /* k = 2t + 8b + h   */
    const int lane = 4 * g + t, p = a + 2 * b;
    *word = (((size_t)nb * (size_t)(K >> 6) + (size_t)kc) * 32u + (size_t)lane) * 4u + (size_t)s;
    *nib = p + 4 * h;
}

int w4a16_oracle_pack(const uint8_t* q, int N, int K, int32_t* Wp) {
    if (N % 16 || K % 64) return 1;
    memset(Wp, 0, (size_t)N * K / 8 * sizeof(int32_t));
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) {
            size_t w; int i;
            locate(n, k, K, &w, &i);
            uint32_t v = (uint32_t)Wp[w] | ((uint32_t)(q[(size_t)n * K + k] & 0xF) << (4 * i));
            Wp[w] = (int32_t)v;
        }
    return 0;
}

int w4a16_oracle_unpack(const int32_t* Wp, int N, int K, uint8_t* q) {
    if (N % 16 || K % 64) return 1;
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) {
            size_t w; int i;
            locate(n, k, K, &w, &i);
            q[(size_t)n * K + k] = (uint8_t)(((uint32_t)Wp[w] >> (4 * i)) & 0xFu);
        }
    return 0;
}

/* dequant8 (common.cuh:45-55) on one word: out[p] = {low half, high half} for p = 0..3.
 * Low half of nibble pair p is nibble p (bits 4p..4p+3), high half is nibble p+4. */
static inline void dequant_word(uint32_t word, uint16_t s_even, uint16_t s_odd, uint16_t out[4][2]) {
    for (int p = 0; p < 4; ++p) {
        uint32_t bits = ((word >> (4 * p)) & 0x000F000Fu) | 0x64006400u;
        uint16_t s = (p & 1) ? s_odd : s_even;
        for (int half = 0; half < 2; ++half) {
            uint16_t hv = (uint16_t)(bits >> (16 * half));
            float qm8 = w4a16_oracle_h2f(hv) - 1032.0f;                 /* exact: q - 8 */
            uint16_t qh = w4a16_oracle_f2h(qm8);                        /* __hsub2 result */
            out[p][half] = w4a16_oracle_f2h(w4a16_oracle_h2f(qh) * w4a16_oracle_h2f(s)); /* __hmul2 */
        }
    }
}

/* Dequantise a whole packed matrix into fp16 [N, K] by walking the packed words in kernel
 * order (each word is decoded the way the kernel's lane decodes it). */
int w4a16_oracle_dequant(const int32_t* Wp, const uint16_t* scales, int N, int K, int G, uint16_t* Wd) {
    if (N % 16 || K % 64 || G <= 0 || K % G || G % 64) return 1;
    const int NB = N / 16, KC = K / 64, GPC = G / 64;
    for (int nb = 0; nb < NB; ++nb)
        for (int kc = 0; kc < KC; ++kc) {
            const uint16_t* srow = scales + (size_t)(kc / GPC) * N + (size_t)nb * 16;
            for (int lane = 0; lane < 32; ++lane) {
                const int g = lane >> 2, t = lane & 3;
                for (int s = 0; s < 4; ++s) {
                    uint32_t word = (uint32_t)Wp[(((size_t)nb * KC + kc) * 32 + lane) * 4 + s];
                    uint16_t out[4][2];
                    dequant_word(word, srow[g], srow[g + 8], out);
                    for (int p = 0; p < 4; ++p) {
                        const int n = nb * 16 + g + 8 * (p & 1);
                        const int k = kc * 64 + s * 16 + 2 * t + 8 * (p >> 1);
                        Wd[(size_t)n * K + k] = out[p][0];
                        Wd[(size_t)n * K + k + 1] = out[p][1];
                    }
                }
            }
        }
    return 0;
}

/* y32[m, n] = sum_k fp32(x[m, k]) * fp32(Wd[n, k]).  Eight interleaved fp32 partial sums
 * combined in a fixed order (deterministic; any fp32 summation order is a valid reference,
 * tests/test_w4a16.py:41-44 compares with a 2e-3 relative tolerance). */
static void gemm_rows(const float* xf, const uint16_t* wrow_h, float* wrow_f, int M, int K, float* yrow, size_t ldy) {
    for (int k = 0; k < K; ++k) wrow_f[k] = w4a16_oracle_h2f(wrow_h[k]);
    for (int m = 0; m < M; ++m) {
        const float* xr = xf + (size_t)m * K;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int k = 0; k < K; k += 8)
            for (int j = 0; j < 8; ++j) acc[j] += xr[k + j] * wrow_f[k + j];
        yrow[(size_t)m * ldy] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    }
}

/* The reference's CPU path end to end (unpack + dequant + fp32 GEMM), optionally also the fp16
 * rounding of the op's output.  y32 is [M, N] fp32 (may be NULL), y16 is [M, N] fp16 (may be
 * NULL).  nthreads <= 0 uses the OpenMP default.  Returns 0 on success. */
int w4a16_oracle_forward(const int32_t* Wp, const uint16_t* x, const uint16_t* scales,
                         int M, int N, int K, int G, float* y32, uint16_t* y16, int nthreads) {
    if (M < 1 || N % 16 || K % 64 || G <= 0 || K % G || G % 64) return 1;
    uint16_t* Wd = (uint16_t*)malloc((size_t)N * K * sizeof(uint16_t));
    float* xf = (float*)malloc((size_t)M * K * sizeof(float));
    float* yt = (float*)malloc((size_t)M * N * sizeof(float));
    if (!Wd || !xf || !yt) { free(Wd); free(xf); free(yt); return 2; }
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    const int NB = N / 16, KC = K / 64, GPC = G / 64;
    /* dequant, parallel over n16 blocks (same arithmetic as w4a16_oracle_dequant) */
#pragma omp parallel for schedule(static)
    for (int nb = 0; nb < NB; ++nb)
        for (int kc = 0; kc < KC; ++kc) {
            const uint16_t* srow = scales + (size_t)(kc / GPC) * N + (size_t)nb * 16;
            for (int lane = 0; lane < 32; ++lane) {
                const int g = lane >> 2, t = lane & 3;
                for (int s = 0; s < 4; ++s) {
                    uint32_t word = (uint32_t)Wp[(((size_t)nb * KC + kc) * 32 + lane) * 4 + s];
                    uint16_t out[4][2];
                    dequant_word(word, srow[g], srow[g + 8], out);
                    for (int p = 0; p < 4; ++p) {
                        const int n = nb * 16 + g + 8 * (p & 1);
                        const int k = kc * 64 + s * 16 + 2 * t + 8 * (p >> 1);
                        Wd[(size_t)n * K + k] = out[p][0];
                        Wd[(size_t)n * K + k + 1] = out[p][1];
                    }
                }
            }
        }
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < (size_t)M * K; ++i) xf[i] = w4a16_oracle_h2f(x[i]);
#pragma omp parallel
    {
        float* wf = (float*)malloc((size_t)K * sizeof(float));
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) gemm_rows(xf, Wd + (size_t)n * K, wf, M, K, yt + n, (size_t)N);
        free(wf);
    }
    if (y32) memcpy(y32, yt, (size_t)M * N * sizeof(float));
    if (y16)
        for (size_t i = 0; i < (size_t)M * N; ++i) y16[i] = w4a16_oracle_f2h(yt[i]);
    free(Wd); free(xf); free(yt);
    return 0;
}

int w4a16_oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/*
 * Baseline GEMV of the reference's second extension, w4a16_ext.w4a16_gemv
 * (src/baseline/kernel.cu:8-34).  W int32 [N, K/8] row-major; nibble j of word k/8 of row n is
 * the weight at k = 8*(k/8) + j, read as a signed 4-bit value (kernel.cu:26-27).  A fp16 [K];
 * sW, zW fp16 [N];  C[n] = fp16_rn((acc - z) * s) with fp32 arithmetic (kernel.cu:31-33).
 *
 *   exact = 0: acc in the reference's order, acc += wv * a for k = 0 .. K-1 in fp32
 *              (kernel.cu:20-30; each product is exact in fp32, so an fma gives the same acc).
 *   exact = 1: acc = the exact sum rounded once to fp32 (the GPU kernel's contract).  Finite fp16
 *              values are integers in units of 2^-24 below 2^40 in magnitude, so the sum is an
 *              exact int64 for K <= 2^20.  Non-finite terms take their IEEE class, which for a
 *              sum does not depend on the order: NaN, 0 * inf, or +inf with -inf give NaN.
 */
static inline int gemv_weight(const int32_t* W, int n, int k, int K) {
    const uint32_t word = (uint32_t)W[(size_t)n * (size_t)(K / 8) + (size_t)(k / 8)];
    const int nib = (int)((word >> (4 * (k % 8))) & 15u);
    return nib >= 8 ? nib - 16 : nib;
}

int w4a16_oracle_gemv(const int32_t* W, const uint16_t* A, const uint16_t* sW, const uint16_t* zW,
                      int N, int K, int exact, uint16_t* C) {
    if (N < 0 || K < 0 || K % 8 != 0 || (exact && K > (1 << 20))) return 1;
    int64_t* fx = NULL;
    if (exact && K > 0) {
        fx = (int64_t*)malloc((size_t)K * sizeof(int64_t));
        if (!fx) return 2;
        for (int k = 0; k < K; ++k) {
            const uint32_t h = A[k], e = (h >> 10) & 31u, m = h & 1023u;
            const int64_t mag = e == 0 ? (int64_t)m : (int64_t)(1024u | m) << (e - 1);   /* a * 2^24 */
            fx[k] = e == 31 ? 0 : (h & 0x8000u) ? -mag : mag;
        }
    }
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int n = 0; n < N; ++n) {
        float acc = 0.0f;
        if (!exact) {
            for (int k = 0; k < K; ++k) acc += (float)gemv_weight(W, n, k, K) * w4a16_oracle_h2f(A[k]);
        } else {
            int64_t sum = 0;
            int pos = 0, neg = 0, nan = 0;
            for (int k = 0; k < K; ++k) {
                const int wv = gemv_weight(W, n, k, K);
                const uint32_t h = A[k];
                if (((h >> 10) & 31u) == 31u) {
                    if ((h & 1023u) || wv == 0) nan = 1;
                    else if ((wv < 0) != ((h & 0x8000u) != 0)) neg = 1;
                    else pos = 1;
                }
                sum += (int64_t)wv * fx[k];
            }
            acc = (float)sum * 0x1p-24f;                  /* int64 -> fp32 rounds to nearest even */
            if (nan || (pos && neg)) acc = NAN;
            else if (pos) acc = INFINITY;
            else if (neg) acc = -INFINITY;
        }
        const float t = acc - w4a16_oracle_h2f(zW[n]);
        C[n] = w4a16_oracle_f2h(t * w4a16_oracle_h2f(sW[n]));
    }
    free(fx);
    return 0;
}
