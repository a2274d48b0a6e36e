/*
 * oracle.h -- CPU oracle for asmllm's quantized matvec path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker and the reported
 * CPU baseline: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  No product code path calls into it.
 *
 * Every function restates the reference's algorithm in C, citing the file
 * and line of asmllm it follows (paths relative to the asmllm repository
 * root).  The reference's NASM kernels cannot be assembled in this image
 * (no nasm/yasm, and every x86 file hard-codes the Win64 ABI), so the
 * restatement keeps their arithmetic op for op: the same FMA chains, the
 * same per-block scale FMA and the same horizontal-sum order.
 *
 * Parity pinning of each function is done in tests/test_oracle.py against
 * the reference's golden recipe (tools/reference_gen.py, RandomState(42)),
 * float64 closed forms, exact special cases and a second, independently
 * written per-lane model of each SIMD kernel.
 */
#ifndef ASMLLM_ORACLE_H
#define ASMLLM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_API __attribute__((visibility("default")))

/* ---- a1/a2/a3: split-layout matvec kernels (qs + fp32 scales) ---------- */

/* matmul_q4_avx2.asm:92-262 (8-lane FMA chain, per-block scale FMA, hsum). */
ORACLE_API void oracle_matmul_q4_avx2(const uint8_t* qweights, const float* scales,
                                      const float* x, float* y, int64_t M, int64_t K);
/* Same arithmetic written as eight independent scalar lanes (no SIMD). */
ORACLE_API void oracle_matmul_q4_lanes(const uint8_t* qweights, const float* scales,
                                       const float* x, float* y, int64_t M, int64_t K);
/* matmul_q4_avx512.asm:92-254 (16-lane FMA chain).  Falls back to the
 * 16-lane scalar model when the host has no AVX-512F. */
ORACLE_API void oracle_matmul_q4_avx512(const uint8_t* qweights, const float* scales,
                                        const float* x, float* y, int64_t M, int64_t K);
ORACLE_API void oracle_matmul_q4_avx512_lanes(const uint8_t* qweights, const float* scales,
                                              const float* x, float* y, int64_t M, int64_t K);
/* matmul_q8_avx2.asm:86-169. */
ORACLE_API void oracle_matmul_q8_avx2(const int8_t* qweights, const float* scales,
                                      const float* x, float* y, int64_t M, int64_t K);
ORACLE_API void oracle_matmul_q8_lanes(const int8_t* qweights, const float* scales,
                                       const float* x, float* y, int64_t M, int64_t K);

/* matmul_q5_avx2.asm:93-210: ql nibbles + qh bit planes + fp32 scales. */
ORACLE_API void oracle_matmul_q5_avx2(const uint8_t* ql, const uint8_t* qh, const float* scales,
                                      const float* x, float* y, int64_t M, int64_t K);
ORACLE_API void oracle_matmul_q5_lanes(const uint8_t* ql, const uint8_t* qh, const float* scales,
                                       const float* x, float* y, int64_t M, int64_t K);

/* ---- a6: GGUF blocks read in place (scale widened fp16 -> fp32) --------- */

/* Q4_0 GGUF blocks (18 B: fp16 d + 16 B qs) with the a1 arithmetic; the
 * scale is widened exactly as generate.py:94-98 does. nt>1 uses the pool. */
ORACLE_API void oracle_matmul_q4_0_gguf(const uint8_t* blocks, const float* x, float* y,
                                        int64_t M, int64_t K, int nt);
/* Q8_0 GGUF blocks (34 B: fp16 d + 32 int8) with the a3 arithmetic. */
ORACLE_API void oracle_matmul_q8_0_gguf(const uint8_t* blocks, const float* x, float* y,
                                        int64_t M, int64_t K, int nt);

/* GGUF Q5_0 blocks (22 B: fp16 d, qh[4], qs[16]) with the Q5 arithmetic. */
ORACLE_API void oracle_matmul_q5_0_gguf(const uint8_t* blocks, const float* x, float* y,
                                        int64_t M, int64_t K, int nt);

/* generate.py:91-106 / :109-119: GGUF blocks -> split qs + fp32 scales. */
ORACLE_API void oracle_split_q4_0(const uint8_t* blocks, uint8_t* qs, float* scales,
                                  int64_t rows, int64_t K);
ORACLE_API void oracle_split_q8_0(const uint8_t* blocks, int8_t* qs, float* scales,
                                  int64_t rows, int64_t K);
ORACLE_API void oracle_split_q5_0(const uint8_t* blocks, uint8_t* ql, uint8_t* qh, float* scales,
                                  int64_t rows, int64_t K);
/* ops.py:16-30 / :44-53 / :67-92 applied to GGUF blocks: exact fp32 dequant. */
ORACLE_API void oracle_dequantize_q4_0(const uint8_t* blocks, float* w, int64_t rows, int64_t K);
ORACLE_API void oracle_dequantize_q8_0(const uint8_t* blocks, float* w, int64_t rows, int64_t K);
ORACLE_API void oracle_dequantize_q5_0(const uint8_t* blocks, float* w, int64_t rows, int64_t K);

/* ---- quantizers (data generation for the synthetic configs) ------------- */

/* Q4_0: d = m / -8 with m the signed element of largest magnitude, id = 1/d,
 * q = min(15, trunc(w*id + 8.5)) (round half up of w/d, +8, clamp), d stored
 * as fp16 (round to nearest even). */
ORACLE_API void oracle_quantize_q4_0(const float* w, uint8_t* blocks, int64_t rows, int64_t K);
/* Q8_0 following the reference's activation quantizer
 * (matmul_q4_neon.S:80-135): d = amax/127, inv = 127/amax (0 if amax == 0),
 * q = saturate_int8(round_half_even(x*inv)), d stored as fp16. */
ORACLE_API void oracle_quantize_q8_0(const float* w, uint8_t* blocks, int64_t rows, int64_t K);

/* ---- a4/a5: threadpool restatement (threadpool.c:263-486, 588-767) ------ */

ORACLE_API void oracle_threadpool_init(int num_threads);
ORACLE_API void oracle_threadpool_shutdown(void);
ORACLE_API int  oracle_threadpool_get_num_threads(void);
/* threadpool.c:408-410 tiling rule: round_up(ceil(M/nt), 16). */
ORACLE_API int64_t oracle_tile_rows(int64_t M, int nt);
/* threadpool.c:390-486: variant 0 = a1 (AVX2), 1 = a2 (AVX-512). */
ORACLE_API void oracle_matmul_q4_mt(const uint8_t* qweights, const float* scales,
                                    const float* x, float* y, int64_t M, int64_t K,
                                    int num_threads, int variant);
/* threadpool.c:750-767 and :588-665. */
ORACLE_API void oracle_matmul_q8_mt(const int8_t* qweights, const float* scales,
                                    const float* x, float* y, int64_t M, int64_t K,
                                    int num_threads);
/* threadpool.c:769-787 and :667-748. */
ORACLE_API void oracle_matmul_q5_mt(const uint8_t* ql, const uint8_t* qh, const float* scales,
                                    const float* x, float* y, int64_t M, int64_t K, int num_threads);
ORACLE_API void oracle_threadpool_dispatch_q5(const uint8_t* ql, const uint8_t* qh, const float* scales,
                                              const float* x, float* y, int64_t M, int64_t K);
ORACLE_API void oracle_threadpool_dispatch_q8(const int8_t* qweights, const float* scales,
                                              const float* x, float* y, int64_t M, int64_t K);

/* ---- a8: Q8_0 x Q8_0 GEMM (int32 block dot x both fp16 scales) ---------- */

/* C[t*M + j] = sum_b fma(float(idot(a[t,b], w[j,b])), d_w[j,b]*d_a[t,b], acc)
 * in block order, following matmul_q4_neon.S:190-255 (sdot, scvtf, fmul of
 * the two scales, fmadd).  nt > 1 splits over rows of C. */
ORACLE_API void oracle_gemm_q8_0(const uint8_t* w_blocks, const uint8_t* a_blocks, float* c,
                                 int64_t T, int64_t M, int64_t K, int nt);
/* The same GEMM on split operands: int8 qs [rows][K], fp32 scales [rows][K/32]
 * (scale = w_scale * a_scale in fp32, then fmaf in block order). */
ORACLE_API void oracle_gemm_q8_split(const int8_t* w_qs, const float* w_scales, const int8_t* a_qs,
                                     const float* a_scales, float* c, int64_t T, int64_t M, int64_t K, int nt);

/* ---- a9: decode-step ops -------------------------------------------------- */

ORACLE_API void oracle_rmsnorm(const float* x, const float* w, float* y, int64_t dim, float eps);
ORACLE_API void oracle_rope(float* q, float* k, int64_t head_dim, int64_t pos, float theta);
ORACLE_API void oracle_softmax(const float* x, float* y, int64_t dim);
ORACLE_API void oracle_silu_hadamard(float* gate, const float* up, int64_t dim);
ORACLE_API void oracle_attention(const float* q, const float* k, const float* v, float* y,
                                 int64_t seq_len, int64_t head_dim, float scale);
/* Single-token attention over an fp16 KV cache laid out [pos][kv_head][hd]
 * (generate.py:291-296 with the cache in fp16): scores = q.k/sqrt(hd),
 * softmax, p.V.  Heads are split over nt threads. */
ORACLE_API void oracle_attention_decode_f16(const float* q, const uint16_t* k_cache,
                                            const uint16_t* v_cache, float* out,
                                            int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                            int64_t n_pos, int64_t kv_stride, int nt);

/* fp16 helpers (round to nearest even). */
ORACLE_API uint16_t oracle_f32_to_f16(float f);
ORACLE_API float    oracle_f16_to_f32(uint16_t h);

/* Host description for logs. */
ORACLE_API int oracle_has_avx512(void);

#ifdef __cplusplus
}
#endif

#endif /* ASMLLM_ORACLE_H */
