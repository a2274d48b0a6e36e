/*
 * oracle.c -- CPU oracle for asmllm's quantized matvec path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  The checker for the HIP path and
 * the reported CPU baseline; never called by the product.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so that every fused
 * multiply-add below is one the reference also fuses).  SIMD kernels carry
 * their own target attributes and are selected at run time.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#define AVX2_FN __attribute__((target("avx2,fma")))
#define AVX512_FN __attribute__((target("avx512f,avx512bw,avx2,fma")))
#define FMA_FN __attribute__((target("fma")))

/* ======================================================================== */
/* fp16 <-> fp32, round to nearest even (portable; no F16C needed).          */
/* ======================================================================== */

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / nan (quiet the nan) */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? (0x200u | ((ax >> 13) & 0x3FFu)) : 0u));
    if (ax >= 0x477FF000u) /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) { /* below 2^-14: fp16 subnormal or zero */
        uint32_t e = ax >> 23;
        if (e < 102u) return (uint16_t)sign;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (ax >> 13) - (112u << 10);
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (e == 0) {
        float f = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        memcpy(&x, &f, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static inline float load_f16(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return oracle_f16_to_f32(h);
}

int oracle_has_avx512(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw");
}

/* ======================================================================== */
/* a1: Q4 AVX2 kernel, matmul_q4_avx2.asm:92-262                            */
/* ======================================================================== */

/* One block: the four vcvtdq2ps/vsubps nibble vectors (:132-153) folded into
 * a fresh accumulator with four vfmadd231ps (:159-164). */
AVX2_FN static inline __m256 q4_block_avx2(const uint8_t* qs, const float* xb) {
    const __m128i m0f = _mm_set1_epi8(0x0F);
    const __m256 eight = _mm256_set1_ps(8.0f);
    __m128i raw = _mm_loadu_si128((const __m128i*)qs);
    __m128i lo = _mm_and_si128(raw, m0f);
    __m128i hi = _mm_and_si128(_mm_srli_epi16(raw, 4), m0f);
    __m256 w0 = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(lo)), eight);
    __m256 w1 = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(lo, 8))), eight);
    __m256 w2 = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(hi)), eight);
    __m256 w3 = _mm256_sub_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(hi, 8))), eight);
    __m256 t = _mm256_setzero_ps();
    t = _mm256_fmadd_ps(w0, _mm256_loadu_ps(xb), t);
    t = _mm256_fmadd_ps(w1, _mm256_loadu_ps(xb + 8), t);
    t = _mm256_fmadd_ps(w2, _mm256_loadu_ps(xb + 16), t);
    t = _mm256_fmadd_ps(w3, _mm256_loadu_ps(xb + 24), t);
    return t;
}

/* Horizontal sum, matmul_q4_avx2.asm:251-256: ((l0+h0)+(l2+h2))+((l1+h1)+(l3+h3)). */
AVX2_FN static inline float hsum8(__m256 v) {
    __m128 a = _mm_add_ps(_mm256_extractf128_ps(v, 1), _mm256_castps256_ps128(v));
    a = _mm_add_ps(a, _mm_permute_ps(a, 0x0E));
    a = _mm_add_ss(a, _mm_permute_ps(a, 0x01));
    return _mm_cvtss_f32(a);
}

/* Rows [r0, r1) of the split-layout kernel.  K % 32 tails are not restated:
 * the reference's tail path (:180-246) reads the next row's first block and
 * no configuration or reference test exercises it. */
AVX2_FN static void q4_avx2_rows(const uint8_t* q, const float* s, const float* x, float* y,
                                 int64_t r0, int64_t r1, int64_t K) {
    int64_t nb = K / 32;
    for (int64_t m = r0; m < r1; ++m) {
        __m256 acc = _mm256_setzero_ps();
        for (int64_t b = 0; b < nb; ++b) {
            __m256 t = q4_block_avx2(q + (m * nb + b) * 16, x + b * 32);
            acc = _mm256_fmadd_ps(t, _mm256_set1_ps(s[m * nb + b]), acc); /* :172-175 */
        }
        y[m] = hsum8(acc);
    }
}

AVX2_FN static void q4_0_gguf_avx2_rows(const uint8_t* blocks, const float* x, float* y,
                                        int64_t r0, int64_t r1, int64_t K) {
    int64_t nb = K / 32;
    for (int64_t m = r0; m < r1; ++m) {
        __m256 acc = _mm256_setzero_ps();
        const uint8_t* row = blocks + m * nb * 18;
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * 18;
            __m256 t = q4_block_avx2(blk + 2, x + b * 32);
            acc = _mm256_fmadd_ps(t, _mm256_set1_ps(load_f16(blk)), acc);
        }
        y[m] = hsum8(acc);
    }
}

void oracle_matmul_q4_avx2(const uint8_t* q, const float* s, const float* x, float* y,
                           int64_t M, int64_t K) {
    q4_avx2_rows(q, s, x, y, 0, M, K);
}

/* The same arithmetic as eight scalar lanes: lane l of block b sees weights
 * l, 8+l (low nibbles of bytes l, 8+l) and 16+l, 24+l (high nibbles). */
FMA_FN void oracle_matmul_q4_lanes(const uint8_t* q, const float* s, const float* x, float* y,
                                   int64_t M, int64_t K) {
    int64_t nb = K / 32;
    for (int64_t m = 0; m < M; ++m) {
        float acc[8] = {0};
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* qs = q + (m * nb + b) * 16;
            const float* xb = x + b * 32;
            float sc = s[m * nb + b];
            for (int l = 0; l < 8; ++l) {
                float w0 = (float)(qs[l] & 15) - 8.0f;
                float w1 = (float)(qs[8 + l] & 15) - 8.0f;
                float w2 = (float)(qs[l] >> 4) - 8.0f;
                float w3 = (float)(qs[8 + l] >> 4) - 8.0f;
                float t = fmaf(w0, xb[l], 0.0f);
                t = fmaf(w1, xb[8 + l], t);
                t = fmaf(w2, xb[16 + l], t);
                t = fmaf(w3, xb[24 + l], t);
                acc[l] = fmaf(t, sc, acc[l]);
            }
        }
        float a0 = acc[4] + acc[0], a1 = acc[5] + acc[1], a2 = acc[6] + acc[2], a3 = acc[7] + acc[3];
        y[m] = (a0 + a2) + (a1 + a3);
    }
}

/* ======================================================================== */
/* a2: Q4 AVX-512 kernel, matmul_q4_avx512.asm:92-254                       */
/* ======================================================================== */

AVX512_FN static void q4_avx512_rows(const uint8_t* q, const float* s, const float* x, float* y,
                                     int64_t r0, int64_t r1, int64_t K) {
    int64_t nb = K / 32;
    const __m128i m0f = _mm_set1_epi8(0x0F);
    const __m512 eight = _mm512_set1_ps(8.0f);
    for (int64_t m = r0; m < r1; ++m) {
        __m512 acc = _mm512_setzero_ps();
        for (int64_t b = 0; b < nb; ++b) {
            __m128i raw = _mm_loadu_si128((const __m128i*)(q + (m * nb + b) * 16));
            __m128i lo = _mm_and_si128(raw, m0f);
            __m128i hi = _mm_and_si128(_mm_srli_epi16(raw, 4), m0f);
            __m512 wl = _mm512_sub_ps(_mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(lo)), eight);
            __m512 wh = _mm512_sub_ps(_mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(hi)), eight);
            const float* xb = x + b * 32;
            __m512 t = _mm512_setzero_ps();
            t = _mm512_fmadd_ps(wl, _mm512_loadu_ps(xb), t);      /* :144-147 */
            t = _mm512_fmadd_ps(wh, _mm512_loadu_ps(xb + 16), t); /* :148-150 */
            acc = _mm512_fmadd_ps(t, _mm512_set1_ps(s[m * nb + b]), acc);
        }
        /* :239-246: (hi256 + lo256), then (lo128 + hi128), then the 4-lane tail. */
        __m256 hi8 = _mm256_castpd_ps(_mm512_extractf64x4_pd(_mm512_castps_pd(acc), 1));
        __m256 h = _mm256_add_ps(hi8, _mm512_castps512_ps256(acc));
        __m128 a = _mm_add_ps(_mm256_castps256_ps128(h), _mm256_extractf128_ps(h, 1));
        a = _mm_add_ps(a, _mm_permute_ps(a, 0x0E));
        a = _mm_add_ss(a, _mm_permute_ps(a, 0x01));
        y[m] = _mm_cvtss_f32(a);
    }
}

FMA_FN static void q4_avx512_lanes_rows(const uint8_t* q, const float* s, const float* x, float* y,
                                        int64_t r0, int64_t r1, int64_t K) {
    int64_t nb = K / 32;
    for (int64_t m = r0; m < r1; ++m) {
        float acc[16] = {0};
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* qs = q + (m * nb + b) * 16;
            const float* xb = x + b * 32;
            float sc = s[m * nb + b];
            for (int l = 0; l < 16; ++l) {
                float t = fmaf((float)(qs[l] & 15) - 8.0f, xb[l], 0.0f);
                t = fmaf((float)(qs[l] >> 4) - 8.0f, xb[16 + l], t);
                acc[l] = fmaf(t, sc, acc[l]);
            }
        }
        float h[8], a[4];
        for (int i = 0; i < 8; ++i) h[i] = acc[8 + i] + acc[i];
        for (int i = 0; i < 4; ++i) a[i] = h[i] + h[4 + i];
        y[m] = (a[0] + a[2]) + (a[1] + a[3]);
    }
}

void oracle_matmul_q4_avx512_lanes(const uint8_t* q, const float* s, const float* x, float* y,
                                   int64_t M, int64_t K) {
    q4_avx512_lanes_rows(q, s, x, y, 0, M, K);
}

void oracle_matmul_q4_avx512(const uint8_t* q, const float* s, const float* x, float* y,
                             int64_t M, int64_t K) {
    if (oracle_has_avx512())
        q4_avx512_rows(q, s, x, y, 0, M, K);
    else
        q4_avx512_lanes_rows(q, s, x, y, 0, M, K);
}

/* ======================================================================== */
/* a3: Q8 AVX2 kernel, matmul_q8_avx2.asm:86-169                            */
/* ======================================================================== */

AVX2_FN static inline __m256 q8_block_avx2(const int8_t* qs, const float* xb) {
    __m128i r0 = _mm_loadu_si128((const __m128i*)qs);
    __m128i r1 = _mm_loadu_si128((const __m128i*)(qs + 16));
    __m256 w0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(r0));
    __m256 w1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(r0, 8)));
    __m256 w2 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(r1));
    __m256 w3 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(r1, 8)));
    __m256 t = _mm256_setzero_ps();
    t = _mm256_fmadd_ps(w0, _mm256_loadu_ps(xb), t);
    t = _mm256_fmadd_ps(w1, _mm256_loadu_ps(xb + 8), t);
    t = _mm256_fmadd_ps(w2, _mm256_loadu_ps(xb + 16), t);
    t = _mm256_fmadd_ps(w3, _mm256_loadu_ps(xb + 24), t);
    return t;
}

/* :159-164 reduces lo+hi, then [2,3,0,1], then [1,0,3,2]: the same order as hsum8. */
AVX2_FN static void q8_avx2_rows(const int8_t* q, const float* s, const float* x, float* y,
                                 int64_t r0, int64_t r1, int64_t K) {
    int64_t nb = K / 32;
    for (int64_t m = r0; m < r1; ++m) {
        __m256 acc = _mm256_setzero_ps();
        for (int64_t b = 0; b < nb; ++b) {
            __m256 t = q8_block_avx2(q + (m * nb + b) * 32, x + b * 32);
            acc = _mm256_fmadd_ps(t, _mm256_set1_ps(s[m * nb + b]), acc);
        }
        y[m] = hsum8(acc);
    }
}

AVX2_FN static void q8_0_gguf_avx2_rows(const uint8_t* blocks, const float* x, float* y,
                                        int64_t r0, int64_t r1, int64_t K) {
    int64_t nb = K / 32;
    for (int64_t m = r0; m < r1; ++m) {
        __m256 acc = _mm256_setzero_ps();
        const uint8_t* row = blocks + m * nb * 34;
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * 34;
            __m256 t = q8_block_avx2((const int8_t*)(blk + 2), x + b * 32);
            acc = _mm256_fmadd_ps(t, _mm256_set1_ps(load_f16(blk)), acc);
        }
        y[m] = hsum8(acc);
    }
}

void oracle_matmul_q8_avx2(const int8_t* q, const float* s, const float* x, float* y,
                           int64_t M, int64_t K) {
    q8_avx2_rows(q, s, x, y, 0, M, K);
}

FMA_FN void oracle_matmul_q8_lanes(const int8_t* q, const float* s, const float* x, float* y,
                                   int64_t M, int64_t K) {
    int64_t nb = K / 32;
    for (int64_t m = 0; m < M; ++m) {
        float acc[8] = {0};
        for (int64_t b = 0; b < nb; ++b) {
            const int8_t* qs = q + (m * nb + b) * 32;
            const float* xb = x + b * 32;
            float sc = s[m * nb + b];
            for (int l = 0; l < 8; ++l) {
                float t = fmaf((float)qs[l], xb[l], 0.0f);
                t = fmaf((float)qs[8 + l], xb[8 + l], t);
                t = fmaf((float)qs[16 + l], xb[16 + l], t);
                t = fmaf((float)qs[24 + l], xb[24 + l], t);
                acc[l] = fmaf(t, sc, acc[l]);
            }
        }
        float a0 = acc[0] + acc[4], a1 = acc[1] + acc[5], a2 = acc[2] + acc[6], a3 = acc[3] + acc[7];
        y[m] = (a0 + a2) + (a1 + a3);
    }
}

/* ======================================================================== */
/* Q5_0 AVX2 kernel, matmul_q5_avx2.asm:93-210                              */
/* ======================================================================== */

/* One block (:104-193): the 16 ql bytes split into low nibbles (weights
 * 0..15) and high nibbles (16..31, :117-124); slice k of eight weights takes
 * qh byte k, broadcast and tested against 1,2,4,..,128 (:134-140), so that
 * lane l adds 16.0 when bit l is set; the weight is cvt(nibble) + that - 16.0
 * (:142-145), folded into a fresh accumulator by vfmadd231ps (:146). */
AVX2_FN static inline __m256 q5_block_avx2(const uint8_t* ql, const uint8_t* qh, const float* xb) {
    const __m128i m0f = _mm_set1_epi8(0x0F);
    const __m256 sixteen = _mm256_set1_ps(16.0f);
    const __m256i lane_bit = _mm256_setr_epi32(1, 2, 4, 8, 16, 32, 64, 128);
    __m128i raw = _mm_loadu_si128((const __m128i*)ql);
    __m128i lo = _mm_and_si128(raw, m0f);
    __m128i hi = _mm_and_si128(_mm_srli_epi16(raw, 4), m0f);
    const __m128i slice[4] = {lo, _mm_srli_si128(lo, 8), hi, _mm_srli_si128(hi, 8)};
    __m256 t = _mm256_setzero_ps();
    for (int k = 0; k < 4; ++k) {
        __m256i sel = _mm256_and_si256(_mm256_set1_epi32(qh[k]), lane_bit);
        __m256 add = _mm256_and_ps(_mm256_castsi256_ps(_mm256_cmpeq_epi32(sel, lane_bit)), sixteen);
        __m256 w = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(slice[k]));
        w = _mm256_sub_ps(_mm256_add_ps(w, add), sixteen);
        t = _mm256_fmadd_ps(w, _mm256_loadu_ps(xb + 8 * k), t);
    }
    return t;
}

/* Rows [r0, r1): per-block scale FMA (:196-197), then the horizontal sum of
 * :202-210, the same order as hsum8. */
AVX2_FN static void q5_avx2_rows(const uint8_t* ql, const uint8_t* qh, const float* s, const float* x, float* y,
                                 int64_t r0, int64_t r1, int64_t K) {
    int64_t nb = K / 32;
    for (int64_t m = r0; m < r1; ++m) {
        __m256 acc = _mm256_setzero_ps();
        for (int64_t b = 0; b < nb; ++b) {
            int64_t blk = m * nb + b;
            __m256 t = q5_block_avx2(ql + blk * 16, qh + blk * 4, x + b * 32);
            acc = _mm256_fmadd_ps(t, _mm256_set1_ps(s[blk]), acc);
        }
        y[m] = hsum8(acc);
    }
}

/* GGUF Q5_0 blocks (22 B: fp16 d, qh[4], qs[16]) with the same arithmetic,
 * the scale widened fp16 -> fp32 first. */
AVX2_FN static void q5_0_gguf_avx2_rows(const uint8_t* blocks, const float* x, float* y, int64_t r0, int64_t r1,
                                        int64_t K) {
    int64_t nb = K / 32;
    for (int64_t m = r0; m < r1; ++m) {
        __m256 acc = _mm256_setzero_ps();
        const uint8_t* row = blocks + m * nb * 22;
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * 22;
            __m256 t = q5_block_avx2(blk + 6, blk + 2, x + b * 32);
            acc = _mm256_fmadd_ps(t, _mm256_set1_ps(load_f16(blk)), acc);
        }
        y[m] = hsum8(acc);
    }
}

void oracle_matmul_q5_avx2(const uint8_t* ql, const uint8_t* qh, const float* s, const float* x, float* y,
                           int64_t M, int64_t K) {
    q5_avx2_rows(ql, qh, s, x, y, 0, M, K);
}

/* The same arithmetic as eight scalar lanes: lane l of block b sees weights
 * l, 8+l (low nibbles of bytes l, 8+l) and 16+l, 24+l (high nibbles), whose
 * fifth bits are bit l of qh bytes 0, 1, 2, 3. */
FMA_FN void oracle_matmul_q5_lanes(const uint8_t* ql, const uint8_t* qh, const float* s, const float* x, float* y,
                                   int64_t M, int64_t K) {
    int64_t nb = K / 32;
    for (int64_t m = 0; m < M; ++m) {
        float acc[8] = {0};
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* q = ql + (m * nb + b) * 16;
            const uint8_t* h = qh + (m * nb + b) * 4;
            const float* xb = x + b * 32;
            float sc = s[m * nb + b];
            for (int l = 0; l < 8; ++l) {
                float t = 0.0f;
                for (int k = 0; k < 4; ++k) {
                    int byte = (k & 1) * 8 + l;
                    int nib = k < 2 ? (q[byte] & 15) : (q[byte] >> 4);
                    float high = ((h[k] >> l) & 1) ? 16.0f : 0.0f;
                    float w = ((float)nib + high) - 16.0f;
                    t = fmaf(w, xb[8 * k + l], t);
                }
                acc[l] = fmaf(t, sc, acc[l]);
            }
        }
        float a0 = acc[0] + acc[4], a1 = acc[1] + acc[5], a2 = acc[2] + acc[6], a3 = acc[3] + acc[7];
        y[m] = (a0 + a2) + (a1 + a3);
    }
}

/* ======================================================================== */
/* a6/a7: GGUF block conversion and exact dequant                           */
/* ======================================================================== */

void oracle_split_q4_0(const uint8_t* blocks, uint8_t* qs, float* scales, int64_t rows, int64_t K) {
    int64_t n = rows * (K / 32);
    for (int64_t i = 0; i < n; ++i) {
        scales[i] = load_f16(blocks + i * 18);
        memcpy(qs + i * 16, blocks + i * 18 + 2, 16);
    }
}

void oracle_split_q8_0(const uint8_t* blocks, int8_t* qs, float* scales, int64_t rows, int64_t K) {
    int64_t n = rows * (K / 32);
    for (int64_t i = 0; i < n; ++i) {
        scales[i] = load_f16(blocks + i * 34);
        memcpy(qs + i * 32, blocks + i * 34 + 2, 32);
    }
}

/* ops.py:24-29: (nibble - 8) * scale, low nibbles are weights 0..15. */
void oracle_dequantize_q4_0(const uint8_t* blocks, float* w, int64_t rows, int64_t K) {
    int64_t n = rows * (K / 32);
    for (int64_t i = 0; i < n; ++i) {
        const uint8_t* blk = blocks + i * 18;
        float d = load_f16(blk);
        for (int j = 0; j < 16; ++j) {
            w[i * 32 + j] = ((float)(blk[2 + j] & 15) - 8.0f) * d;
            w[i * 32 + 16 + j] = ((float)(blk[2 + j] >> 4) - 8.0f) * d;
        }
    }
}

/* ops.py:52: q * scale. */
void oracle_dequantize_q8_0(const uint8_t* blocks, float* w, int64_t rows, int64_t K) {
    int64_t n = rows * (K / 32);
    for (int64_t i = 0; i < n; ++i) {
        const uint8_t* blk = blocks + i * 34;
        float d = load_f16(blk);
        for (int j = 0; j < 32; ++j) w[i * 32 + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

/* GGUF Q5_0 blocks -> the split layout asm_matmul_q5 reads (ql, qh planes,
 * fp32 scales): the byte planes are copied, the scale widened exactly. */
void oracle_split_q5_0(const uint8_t* blocks, uint8_t* ql, uint8_t* qh, float* scales, int64_t rows, int64_t K) {
    int64_t n = rows * (K / 32);
    for (int64_t i = 0; i < n; ++i) {
        const uint8_t* b = blocks + i * 22;
        scales[i] = load_f16(b);
        memcpy(qh + i * 4, b + 2, 4);
        memcpy(ql + i * 16, b + 6, 16);
    }
}

/* ops.py:67-92 applied to GGUF Q5_0 blocks. */
void oracle_dequantize_q5_0(const uint8_t* blocks, float* w, int64_t rows, int64_t K) {
    int64_t n = rows * (K / 32);
    for (int64_t i = 0; i < n; ++i) {
        const uint8_t* b = blocks + i * 22;
        float d = load_f16(b);
        uint32_t h = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
        for (int j = 0; j < 16; ++j) {
            int lo = (b[6 + j] & 15) | (int)(((h >> j) & 1u) << 4);
            int hi = (b[6 + j] >> 4) | (int)(((h >> (j + 16)) & 1u) << 4);
            w[i * 32 + j] = ((float)lo - 16.0f) * d;
            w[i * 32 + 16 + j] = ((float)hi - 16.0f) * d;
        }
    }
}

/* ======================================================================== */
/* Quantizers                                                                */
/* ======================================================================== */

void oracle_quantize_q4_0(const float* w, uint8_t* blocks, int64_t rows, int64_t K) {
    int64_t n = rows * (K / 32);
    for (int64_t i = 0; i < n; ++i) {
        const float* v = w + i * 32;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 32; ++j) {
            float a = fabsf(v[j]);
            if (a > amax) {
                amax = a;
                mx = v[j];
            }
        }
        float d = mx / -8.0f;
        float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        uint16_t dh = oracle_f32_to_f16(d);
        uint8_t* blk = blocks + i * 18;
        memcpy(blk, &dh, 2);
        for (int j = 0; j < 16; ++j) {
            float x0 = v[j] * id, x1 = v[16 + j] * id;
            int q0 = (int)(x0 + 8.5f), q1 = (int)(x1 + 8.5f);
            if (q0 > 15) q0 = 15;
            if (q1 > 15) q1 = 15;
            blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

void oracle_quantize_q8_0(const float* w, uint8_t* blocks, int64_t rows, int64_t K) {
    int64_t n = rows * (K / 32);
    for (int64_t i = 0; i < n; ++i) {
        const float* v = w + i * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j])); /* fabs/fmax/fmaxv */
        float d = amax / 127.0f;                                      /* fdiv s18 */
        float inv = (amax == 0.0f) ? 0.0f : 127.0f / amax;            /* fdiv s17 / movi 0 */
        uint16_t dh = oracle_f32_to_f16(d);
        uint8_t* blk = blocks + i * 34;
        memcpy(blk, &dh, 2);
        for (int j = 0; j < 32; ++j) {
            float t = v[j] * inv;                 /* fmul */
            float r = nearbyintf(t);              /* fcvtns: nearest, ties to even */
            if (r > 127.0f) r = 127.0f;           /* sqxtn saturation */
            if (r < -128.0f) r = -128.0f;
            blk[2 + j] = (uint8_t)(int8_t)r;
        }
    }
}

/* ======================================================================== */
/* a4/a5: worker pool (threadpool.c:263-486, 588-767)                       */
/* ======================================================================== */

#define ORACLE_MAX_WORKERS 64 /* threadpool.c:99 */
#define SPIN_LIMIT 5000       /* threadpool.c:283, :478 */

typedef void (*pool_fn)(void* ctx, int worker, int nt);

static pthread_t g_threads[ORACLE_MAX_WORKERS];
static int g_worker_id[ORACLE_MAX_WORKERS];
static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t g_wake = PTHREAD_COND_INITIALIZER;
static pthread_cond_t g_ready_cv = PTHREAD_COND_INITIALIZER;
static int g_pool_size;
static int g_ready;
static int g_stop;
static _Atomic long g_generation;
static _Atomic long g_completed;
static _Atomic long g_sleepers;
static pool_fn g_fn;
static void* g_ctx;

static int nth_allowed_cpu(int n) {
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof(set), &set) != 0) return n;
    int count = CPU_COUNT(&set);
    if (count <= 0) return n;
    n %= count;
    for (int c = 0; c < CPU_SETSIZE; ++c)
        if (CPU_ISSET(c, &set) && n-- == 0) return c;
    return 0;
}

static void* worker_main(void* arg) {
    int id = *(int*)arg;
    /* The reference pins worker i to core i (threadpool.c:266-271); here
     * worker i goes to the i-th core this process may run on. */
    cpu_set_t set;
    CPU_ZERO(&set);
    CPU_SET(nth_allowed_cpu(id), &set);
    pthread_setaffinity_np(pthread_self(), sizeof(set), &set);

    pthread_mutex_lock(&g_mu);
    long seen = atomic_load(&g_generation);
    g_ready++;
    pthread_cond_broadcast(&g_ready_cv);
    pthread_mutex_unlock(&g_mu);

    for (;;) {
        int spins = 0;
        long gen;
        while ((gen = atomic_load_explicit(&g_generation, memory_order_acquire)) == seen) {
            if (__atomic_load_n(&g_stop, __ATOMIC_ACQUIRE)) return NULL;
            if (spins < SPIN_LIMIT) {
                _mm_pause();
                spins++;
            } else {
                pthread_mutex_lock(&g_mu);
                atomic_fetch_add(&g_sleepers, 1);
                while (atomic_load(&g_generation) == seen && !g_stop) pthread_cond_wait(&g_wake, &g_mu);
                atomic_fetch_sub(&g_sleepers, 1);
                pthread_mutex_unlock(&g_mu);
                spins = 0;
            }
        }
        if (__atomic_load_n(&g_stop, __ATOMIC_ACQUIRE)) return NULL;
        seen = gen;
        g_fn(g_ctx, id, g_pool_size);
        atomic_fetch_add_explicit(&g_completed, 1, memory_order_acq_rel);
    }
}

void oracle_threadpool_shutdown(void) {
    if (g_pool_size <= 0) return;
    pthread_mutex_lock(&g_mu);
    __atomic_store_n(&g_stop, 1, __ATOMIC_RELEASE);
    pthread_cond_broadcast(&g_wake);
    pthread_mutex_unlock(&g_mu);
    for (int i = 0; i < g_pool_size; ++i) pthread_join(g_threads[i], NULL);
    g_pool_size = 0;
}

void oracle_threadpool_init(int num_threads) {
    if (g_pool_size == num_threads && g_pool_size > 0) return; /* :341 */
    if (g_pool_size > 0) oracle_threadpool_shutdown();
    if (num_threads < 1) num_threads = 1;
    if (num_threads > ORACLE_MAX_WORKERS) num_threads = ORACLE_MAX_WORKERS;
    pthread_mutex_lock(&g_mu);
    g_stop = 0;
    g_ready = 0;
    g_pool_size = num_threads;
    pthread_mutex_unlock(&g_mu);
    for (int i = 0; i < num_threads; ++i) {
        g_worker_id[i] = i;
        pthread_create(&g_threads[i], NULL, worker_main, &g_worker_id[i]);
    }
    pthread_mutex_lock(&g_mu);
    while (g_ready < num_threads) pthread_cond_wait(&g_ready_cv, &g_mu);
    pthread_mutex_unlock(&g_mu);
}

int oracle_threadpool_get_num_threads(void) { return g_pool_size; }

/* Run fn(ctx, i, nt) on every worker and spin until all report (:469-484). */
static void pool_run(pool_fn fn, void* ctx) {
    int nt = g_pool_size;
    pthread_mutex_lock(&g_mu);
    g_fn = fn;
    g_ctx = ctx;
    atomic_store(&g_completed, 0);
    atomic_fetch_add_explicit(&g_generation, 1, memory_order_acq_rel);
    if (atomic_load(&g_sleepers) > 0) pthread_cond_broadcast(&g_wake);
    pthread_mutex_unlock(&g_mu);
    int spins = 0;
    while (atomic_load_explicit(&g_completed, memory_order_acquire) < nt) {
        if (spins < SPIN_LIMIT) {
            _mm_pause();
            spins++;
        } else {
            sched_yield();
        }
    }
}

int64_t oracle_tile_rows(int64_t M, int nt) {
    int64_t align = 16;
    int64_t tile = (M + nt - 1) / nt;
    return ((tile + align - 1) / align) * align;
}

typedef void (*rows_fn)(const void* q, const float* s, const float* x, float* y,
                        int64_t r0, int64_t r1, int64_t K);

typedef struct {
    rows_fn fn;
    const void* q;
    const float* s;
    const float* x;
    float* y;
    int64_t M, K, tile;
} rows_job;

static void rows_job_run(void* ctx, int i, int nt) {
    (void)nt;
    rows_job* j = (rows_job*)ctx;
    int64_t r0 = (int64_t)i * j->tile, r1 = r0 + j->tile;
    if (r0 > j->M) r0 = j->M;
    if (r1 > j->M) r1 = j->M;
    if (r1 > r0) j->fn(j->q, j->s, j->x, j->y, r0, r1, j->K);
}

static void dispatch_rows(rows_fn fn, const void* q, const float* s, const float* x, float* y,
                          int64_t M, int64_t K) {
    rows_job j = {fn, q, s, x, y, M, K, oracle_tile_rows(M, g_pool_size)};
    pool_run(rows_job_run, &j);
}

static void q4_avx2_rows_v(const void* q, const float* s, const float* x, float* y, int64_t r0,
                           int64_t r1, int64_t K) {
    q4_avx2_rows((const uint8_t*)q, s, x, y, r0, r1, K);
}
static void q4_avx512_rows_v(const void* q, const float* s, const float* x, float* y, int64_t r0,
                             int64_t r1, int64_t K) {
    if (oracle_has_avx512())
        q4_avx512_rows((const uint8_t*)q, s, x, y, r0, r1, K);
    else
        q4_avx512_lanes_rows((const uint8_t*)q, s, x, y, r0, r1, K);
}
static void q8_avx2_rows_v(const void* q, const float* s, const float* x, float* y, int64_t r0,
                           int64_t r1, int64_t K) {
    q8_avx2_rows((const int8_t*)q, s, x, y, r0, r1, K);
}
static void q4_0_gguf_rows_v(const void* q, const float* s, const float* x, float* y, int64_t r0,
                             int64_t r1, int64_t K) {
    (void)s;
    q4_0_gguf_avx2_rows((const uint8_t*)q, x, y, r0, r1, K);
}
static void q8_0_gguf_rows_v(const void* q, const float* s, const float* x, float* y, int64_t r0,
                             int64_t r1, int64_t K) {
    (void)s;
    q8_0_gguf_avx2_rows((const uint8_t*)q, x, y, r0, r1, K);
}

void oracle_matmul_q4_mt(const uint8_t* q, const float* s, const float* x, float* y, int64_t M,
                         int64_t K, int nt, int variant) {
    rows_fn fn = variant == 1 ? q4_avx512_rows_v : q4_avx2_rows_v;
    if (nt <= 1 || M < 32) { /* threadpool.c:399-402 */
        fn(q, s, x, y, 0, M, K);
        return;
    }
    if (g_pool_size != nt) oracle_threadpool_init(nt);
    dispatch_rows(fn, q, s, x, y, M, K);
}

void oracle_threadpool_dispatch_q8(const int8_t* q, const float* s, const float* x, float* y,
                                   int64_t M, int64_t K) {
    if (g_pool_size <= 1 || M < 32) { /* threadpool.c:596-600 */
        q8_avx2_rows(q, s, x, y, 0, M, K);
        return;
    }
    dispatch_rows(q8_avx2_rows_v, q, s, x, y, M, K);
}

void oracle_matmul_q8_mt(const int8_t* q, const float* s, const float* x, float* y, int64_t M,
                         int64_t K, int nt) {
    if (nt <= 1 || M < 32) {
        q8_avx2_rows(q, s, x, y, 0, M, K);
        return;
    }
    if (g_pool_size != nt) oracle_threadpool_init(nt);
    oracle_threadpool_dispatch_q8(q, s, x, y, M, K);
}

/* threadpool.c:101-115: the Q5 task carries the qh plane beside ql. */
typedef struct {
    const uint8_t* ql;
    const uint8_t* qh;
} q5_planes;

static void q5_avx2_rows_v(const void* q, const float* s, const float* x, float* y, int64_t r0, int64_t r1,
                           int64_t K) {
    const q5_planes* p = (const q5_planes*)q;
    q5_avx2_rows(p->ql, p->qh, s, x, y, r0, r1, K);
}

/* threadpool.c:667-748: below 32 rows or one pool thread, one call;
 * otherwise rows split into tiles of round_up(ceil(M/nt), 16) (:684-686). */
void oracle_threadpool_dispatch_q5(const uint8_t* ql, const uint8_t* qh, const float* s, const float* x, float* y,
                                   int64_t M, int64_t K) {
    if (g_pool_size <= 1 || M < 32) {
        q5_avx2_rows(ql, qh, s, x, y, 0, M, K);
        return;
    }
    q5_planes p = {ql, qh};
    dispatch_rows(q5_avx2_rows_v, &p, s, x, y, M, K);
}

/* threadpool.c:769-787. */
void oracle_matmul_q5_mt(const uint8_t* ql, const uint8_t* qh, const float* s, const float* x, float* y, int64_t M,
                         int64_t K, int nt) {
    if (nt <= 1 || M < 32) {
        q5_avx2_rows(ql, qh, s, x, y, 0, M, K);
        return;
    }
    if (g_pool_size != nt) oracle_threadpool_init(nt);
    oracle_threadpool_dispatch_q5(ql, qh, s, x, y, M, K);
}

void oracle_matmul_q4_0_gguf(const uint8_t* blocks, const float* x, float* y, int64_t M, int64_t K,
                             int nt) {
    if (nt <= 1 || M < 32) {
        q4_0_gguf_avx2_rows(blocks, x, y, 0, M, K);
        return;
    }
    if (g_pool_size != nt) oracle_threadpool_init(nt);
    dispatch_rows(q4_0_gguf_rows_v, blocks, NULL, x, y, M, K);
}

void oracle_matmul_q8_0_gguf(const uint8_t* blocks, const float* x, float* y, int64_t M, int64_t K,
                             int nt) {
    if (nt <= 1 || M < 32) {
        q8_0_gguf_avx2_rows(blocks, x, y, 0, M, K);
        return;
    }
    if (g_pool_size != nt) oracle_threadpool_init(nt);
    dispatch_rows(q8_0_gguf_rows_v, blocks, NULL, x, y, M, K);
}

static void q5_0_gguf_rows_v(const void* q, const float* s, const float* x, float* y, int64_t r0, int64_t r1,
                             int64_t K) {
    (void)s;
    q5_0_gguf_avx2_rows((const uint8_t*)q, x, y, r0, r1, K);
}

void oracle_matmul_q5_0_gguf(const uint8_t* blocks, const float* x, float* y, int64_t M, int64_t K, int nt) {
    if (nt <= 1 || M < 32) {
        q5_0_gguf_avx2_rows(blocks, x, y, 0, M, K);
        return;
    }
    if (g_pool_size != nt) oracle_threadpool_init(nt);
    dispatch_rows(q5_0_gguf_rows_v, blocks, NULL, x, y, M, K);
}

/* ======================================================================== */
/* a8: Q8_0 x Q8_0 GEMM, matmul_q4_neon.S:190-255 recipe                     */
/* ======================================================================== */

typedef struct {
    const uint8_t* w;
    const uint8_t* a;
    float* c;
    int64_t T, M, K;
} gemm_job;

static void gemm_rows(const gemm_job* g, int64_t t0, int64_t t1) {
    int64_t nb = g->K / 32;
    for (int64_t t = t0; t < t1; ++t) {
        const uint8_t* arow = g->a + t * nb * 34;
        for (int64_t j = 0; j < g->M; ++j) {
            const uint8_t* wrow = g->w + j * nb * 34;
            float acc = 0.0f;
            for (int64_t b = 0; b < nb; ++b) {
                const int8_t* qa = (const int8_t*)(arow + b * 34 + 2);
                const int8_t* qw = (const int8_t*)(wrow + b * 34 + 2);
                int32_t dot = 0;
                for (int k = 0; k < 32; ++k) dot += (int32_t)qa[k] * (int32_t)qw[k]; /* sdot */
                float sc = load_f16(wrow + b * 34) * load_f16(arow + b * 34);       /* fmul */
                acc = fmaf((float)dot, sc, acc);                                     /* scvtf, fmadd */
            }
            g->c[t * g->M + j] = acc;
        }
    }
}

static void gemm_job_run(void* ctx, int i, int nt) {
    gemm_job* g = (gemm_job*)ctx;
    int64_t per = (g->T + nt - 1) / nt;
    int64_t t0 = (int64_t)i * per, t1 = t0 + per;
    if (t0 > g->T) t0 = g->T;
    if (t1 > g->T) t1 = g->T;
    if (t1 > t0) gemm_rows(g, t0, t1);
}

void oracle_gemm_q8_0(const uint8_t* w_blocks, const uint8_t* a_blocks, float* c, int64_t T,
                      int64_t M, int64_t K, int nt) {
    gemm_job g = {w_blocks, a_blocks, c, T, M, K};
    if (nt <= 1 || T < 2) {
        gemm_rows(&g, 0, T);
        return;
    }
    if (g_pool_size != nt) oracle_threadpool_init(nt);
    pool_run(gemm_job_run, &g);
}

/* The same recipe on the split layout of asm_matmul_q8 (matmul_q8_avx2.asm:51-194):
 * int8 qs [rows][K] and fp32 scales [rows][K/32]; the scale is the fp32 product
 * w_scale * x_scale, as matmul_q4_neon.S:190-255 forms it. */
typedef struct {
    const int8_t *wq, *aq;
    const float *ws, *as;
    float* c;
    int64_t T, M, K;
} gemm_split_job;

static void gemm_split_rows(const gemm_split_job* g, int64_t t0, int64_t t1) {
    int64_t nb = g->K / 32;
    for (int64_t t = t0; t < t1; ++t) {
        for (int64_t j = 0; j < g->M; ++j) {
            float acc = 0.0f;
            for (int64_t b = 0; b < nb; ++b) {
                const int8_t* qa = g->aq + (t * nb + b) * 32;
                const int8_t* qw = g->wq + (j * nb + b) * 32;
                int32_t dot = 0;
                for (int k = 0; k < 32; ++k) dot += (int32_t)qa[k] * (int32_t)qw[k]; /* sdot */
                float sc = g->ws[j * nb + b] * g->as[t * nb + b];                    /* fmul */
                acc = fmaf((float)dot, sc, acc);                                     /* scvtf, fmadd */
            }
            g->c[t * g->M + j] = acc;
        }
    }
}

static void gemm_split_job_run(void* ctx, int i, int nt) {
    gemm_split_job* g = (gemm_split_job*)ctx;
    int64_t per = (g->T + nt - 1) / nt;
    int64_t t0 = (int64_t)i * per, t1 = t0 + per;
    if (t0 > g->T) t0 = g->T;
    if (t1 > g->T) t1 = g->T;
    if (t1 > t0) gemm_split_rows(g, t0, t1);
}

void oracle_gemm_q8_split(const int8_t* w_qs, const float* w_scales, const int8_t* a_qs, const float* a_scales,
                          float* c, int64_t T, int64_t M, int64_t K, int nt) {
    gemm_split_job g = {w_qs, a_qs, w_scales, a_scales, c, T, M, K};
    if (nt <= 1 || T < 2) {
        gemm_split_rows(&g, 0, T);
        return;
    }
    if (g_pool_size != nt) oracle_threadpool_init(nt);
    pool_run(gemm_split_job_run, &g);
}

/* ======================================================================== */
/* a9: decode-step ops                                                       */
/* ======================================================================== */

/* rmsnorm_avx2.asm:63-151. */
FMA_FN void oracle_rmsnorm(const float* x, const float* w, float* y, int64_t dim, float eps) {
    float acc[8] = {0};
    int64_t full = dim / 8;
    for (int64_t b = 0; b < full; ++b)
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(x[b * 8 + l], x[b * 8 + l], acc[l]);
    float a0 = acc[4] + acc[0], a1 = acc[5] + acc[1], a2 = acc[6] + acc[2], a3 = acc[7] + acc[3];
    float sum = (a0 + a2) + (a1 + a3);
    for (int64_t i = full * 8; i < dim; ++i) sum = fmaf(x[i], x[i], sum);
    float mean = sum / (float)dim;
    float inv = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < dim; ++i) y[i] = (x[i] * inv) * w[i];
}

/* rope_avx2.asm:52-146.  The frequency, angle and sin/cos are formed in x87
 * extended precision there; long double is the same format here. */
void oracle_rope(float* q, float* k, int64_t hd, int64_t pos, float theta) {
    float posf = (float)pos, hdf = (float)hd;
    long double l2t = log2l((long double)theta);
    for (int64_t p = 0; p < hd / 2; ++p) {
        float e = (float)(-2 * p) / hdf;
        long double freq = exp2l((long double)e * l2t);
        long double ang = freq * (long double)posf;
        float c = (float)cosl(ang), s = (float)sinl(ang);
        float q0 = q[2 * p], q1 = q[2 * p + 1];
        float a = q0 * c, b = q1 * s;
        q[2 * p] = a - b;
        a = q0 * s;
        b = q1 * c;
        q[2 * p + 1] = a + b;
        float k0 = k[2 * p], k1 = k[2 * p + 1];
        a = k0 * c;
        b = k1 * s;
        k[2 * p] = a - b;
        a = k0 * s;
        b = k1 * c;
        k[2 * p + 1] = a + b;
    }
}

/* softmax_avx2.asm:48-130 (x == y allowed). */
void oracle_softmax(const float* x, float* y, int64_t dim) {
    float mx = x[0];
    for (int64_t i = 0; i < dim; ++i) mx = x[i] > mx ? x[i] : mx;
    float sum = 0.0f;
    for (int64_t i = 0; i < dim; ++i) {
        float z = x[i] - mx;
        float e = (float)expl((long double)z);
        y[i] = e;
        sum += e;
    }
    for (int64_t i = 0; i < dim; ++i) y[i] = y[i] / sum;
}

/* swiglu_avx2.asm:45-81: gate = gate / (1 + exp(-gate)) * up, in place. */
void oracle_silu_hadamard(float* gate, const float* up, int64_t dim) {
    for (int64_t i = 0; i < dim; ++i) {
        float g = gate[i];
        float z = 0.0f - g;
        float den = (float)(1.0L + expl((long double)z));
        float r = g / den;
        gate[i] = r * up[i];
    }
}

/* attention_avx2.asm:59-218: full (non-causal) softmax(q.k^T * scale) . v. */
FMA_FN void oracle_attention(const float* q, const float* k, const float* v, float* y,
                             int64_t seq, int64_t hd, float scale) {
    float* scores = (float*)malloc((size_t)(seq > 0 ? seq : 1) * sizeof(float));
    int64_t full = hd / 8;
    for (int64_t i = 0; i < seq; ++i) {
        const float* qi = q + i * hd;
        for (int64_t j = 0; j < seq; ++j) {
            const float* kj = k + j * hd;
            float acc[8] = {0};
            for (int64_t b = 0; b < full; ++b)
                for (int l = 0; l < 8; ++l) acc[l] = fmaf(qi[b * 8 + l], kj[b * 8 + l], acc[l]);
            float a0 = acc[4] + acc[0], a1 = acc[5] + acc[1], a2 = acc[6] + acc[2], a3 = acc[7] + acc[3];
            float dot = (a0 + a2) + (a1 + a3);
            for (int64_t d = full * 8; d < hd; ++d) dot = fmaf(qi[d], kj[d], dot);
            scores[j] = dot * scale;
        }
        oracle_softmax(scores, scores, seq);
        float* yi = y + i * hd;
        for (int64_t d = 0; d < hd; ++d) yi[d] = 0.0f;
        for (int64_t j = 0; j < seq; ++j) {
            const float* vj = v + j * hd;
            for (int64_t d = 0; d < hd; ++d) yi[d] = fmaf(scores[j], vj[d], yi[d]);
        }
    }
    free(scores);
}

/* Decode attention over an fp16 cache, evaluated in float64. */
static float g_f16_table[65536];
static pthread_once_t g_f16_once = PTHREAD_ONCE_INIT;
static void f16_table_init(void) {
    for (uint32_t h = 0; h < 65536; ++h) g_f16_table[h] = oracle_f16_to_f32((uint16_t)h);
}

typedef struct {
    const float* q;
    const uint16_t* k;
    const uint16_t* v;
    float* out;
    int64_t n_heads, n_kv, hd, n_pos, stride;
} attn_job;

static void attn_heads(const attn_job* a, int64_t h0, int64_t h1) {
    double* p = (double*)malloc((size_t)(a->n_pos > 0 ? a->n_pos : 1) * sizeof(double));
    double* acc = (double*)malloc((size_t)a->hd * sizeof(double));
    double scale = 1.0 / sqrt((double)a->hd);
    int64_t group = a->n_heads / a->n_kv;
    for (int64_t h = h0; h < h1; ++h) {
        const float* qh = a->q + h * a->hd;
        int64_t kvh = h / group;
        double mx = -INFINITY;
        for (int64_t j = 0; j < a->n_pos; ++j) {
            const uint16_t* kj = a->k + j * a->stride + kvh * a->hd;
            double s = 0.0;
            for (int64_t d = 0; d < a->hd; ++d) s += (double)qh[d] * (double)g_f16_table[kj[d]];
            p[j] = s * scale;
            if (p[j] > mx) mx = p[j];
        }
        double sum = 0.0;
        for (int64_t j = 0; j < a->n_pos; ++j) {
            p[j] = exp(p[j] - mx);
            sum += p[j];
        }
        for (int64_t d = 0; d < a->hd; ++d) acc[d] = 0.0;
        for (int64_t j = 0; j < a->n_pos; ++j) {
            const uint16_t* vj = a->v + j * a->stride + kvh * a->hd;
            double w = p[j] / sum;
            for (int64_t d = 0; d < a->hd; ++d) acc[d] += w * (double)g_f16_table[vj[d]];
        }
        for (int64_t d = 0; d < a->hd; ++d) a->out[h * a->hd + d] = (float)acc[d];
    }
    free(p);
    free(acc);
}

static void attn_job_run(void* ctx, int i, int nt) {
    attn_job* a = (attn_job*)ctx;
    int64_t per = (a->n_heads + nt - 1) / nt;
    int64_t h0 = (int64_t)i * per, h1 = h0 + per;
    if (h0 > a->n_heads) h0 = a->n_heads;
    if (h1 > a->n_heads) h1 = a->n_heads;
    if (h1 > h0) attn_heads(a, h0, h1);
}

void oracle_attention_decode_f16(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                 float* out, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                 int64_t n_pos, int64_t kv_stride, int nt) {
    pthread_once(&g_f16_once, f16_table_init);
    attn_job a = {q, k_cache, v_cache, out, n_heads, n_kv_heads, head_dim, n_pos, kv_stride};
    if (nt <= 1) {
        attn_heads(&a, 0, n_heads);
        return;
    }
    if (g_pool_size != nt) oracle_threadpool_init(nt);
    pool_run(attn_job_run, &a);
}
