/*
 * asmllm_hip.h -- C ABI of libasmllm.so, the MI355X (gfx950) build of asmllm's
 * quantized matvec path.
 *
 * Two groups of entry points:
 *
 *  1. Reference-named, synchronous entry points.  Same names, argument order
 *     and meaning as the symbols asmllm's ctypes callers bind (export list
 *     build_kernel.py:85-104, argtypes tests/correctness/test_runner.py:84-475,
 *     src/runtime/generate.py:221-250).  Each accepts host pointers (numpy
 *     buffers: staged through device memory) or device pointers, computes on
 *     the GPU, and returns with the result in place, as the reference's
 *     kernels do.  They return void like the reference; an error is printed
 *     to stderr, y is left untouched and asmhip_last_error() describes it.
 *
 *  2. asmhip_* device entry points: device pointers only, stream-ordered
 *     (stream NULL = HIP's default stream), no synchronization, return 0 or a
 *     negative status.  Weights stay resident in HBM in their GGUF block
 *     layout; these are the hot path.
 *
 * Block layouts (GGUF):  Q4_0 = fp16 d + 16 bytes, byte j holding weight j
 * (low nibble) and weight j+16 (high nibble), value (nibble - 8) * d;
 * Q8_0 = fp16 d + 32 int8, value q * d; Q5_0 = fp16 d + qh[4] + qs[16], qs
 * as in Q4_0 and bit j of the little-endian word qh weight j's fifth bit,
 * value ((nibble | bit << 4) - 16) * d.  Rows are [M][K/32] blocks.
 * Split layout (the reference kernels' ABI): qs [M][K/32][16 or 32] bytes
 * plus fp32 scales [M][K/32]; for Q5 ql [M][K/32][16] + qh [M][K/32][4] +
 * fp32 scales.  K must be a multiple of 32.
 */
#ifndef ASMLLM_HIP_H
#define ASMLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ASMHIP_API __attribute__((visibility("default")))

/* Status codes of the asmhip_* entry points. */
#define ASMHIP_OK 0
#define ASMHIP_ERR_INVALID_ARGUMENT (-1)
#define ASMHIP_ERR_HIP (-2)
#define ASMHIP_ERR_UNSUPPORTED (-3)
#define ASMHIP_ERR_NO_DEVICE (-4)

/* Block types, numbered as GGUF tensor types (src/runtime/generate.py:175-178). */
#define ASMHIP_Q4_0 2
#define ASMHIP_Q5_0 6
#define ASMHIP_Q8_0 8

/* Work fused into a matvec's read of x (asmhip_matmul_fused). */
#define ASMHIP_PRE_NONE 0
#define ASMHIP_PRE_RMSNORM 1 /* x <- (x * 1/sqrt(mean(x^2) + eps)) * pre_arg (the int8-MFMA stream
                                * reads x * pre_arg and scales each row total by the
                                * 1/sqrt factor: the same product, rounded in another
                                * order, within the matvec bar) */
#define ASMHIP_PRE_SWIGLU 2  /* x <- x / (1 + exp(-x)) * pre_arg             */

/* Matvec kernel selection (asmhip_set_q4_kernel): the int8-MFMA stream or the
 * fp32 VALU kernels, for Q4_0 (GGUF and split); ASMHIP_Q4_KERNEL_FP32 also
 * keeps Q5_0 and Q8_0 on the fp32 kernels.  The MFMA stream needs
 * K % 256 == 0, K <= 16384 and 16-byte aligned x (and, for split planes,
 * 16-byte aligned planes). */
#define ASMHIP_Q4_KERNEL_AUTO 0 /* int8 MFMA kernel where eligible, else fp32             */
#define ASMHIP_Q4_KERNEL_FP32 1 /* fp32 VALU kernel only                                   */
#define ASMHIP_Q4_KERNEL_MFMA 2 /* int8 MFMA kernel only (GGUF shapes it cannot take:
                                   UNSUPPORTED; split planes fall back to fp32) */

/* ---- 1. reference-named entry points ------------------------------------ */

/* src/kernels/x86_64/matmul_q4_avx2.asm:11-19, 57: y = W x, split layout. */
ASMHIP_API void asm_matmul_q4(const uint8_t* qweights, const float* scales, const float* x, float* y,
                              int64_t M, int64_t K);
/* src/kernels/x86_64/matmul_q4_avx512.asm:57 (same contract as asm_matmul_q4). */
ASMHIP_API void asm_matmul_q4_avx512(const uint8_t* qweights, const float* scales, const float* x,
                                     float* y, int64_t M, int64_t K);
/* src/kernels/x86_64/matmul_q8_avx2.asm:11-19, 51. */
ASMHIP_API void asm_matmul_q8(const int8_t* qweights, const float* scales, const float* x, float* y,
                              int64_t M, int64_t K);
/* src/kernels/x86_64/matmul_q5_avx2.asm:11-20, 52: y = W x, Q5_0 split layout
 * (ql nibbles, qh fifth-bit planes, fp32 scales). */
ASMHIP_API void asm_matmul_q5(const uint8_t* ql, const uint8_t* qh, const float* scales, const float* x,
                              float* y, int64_t M, int64_t K);
/* src/runtime/threadpool.h:49-57 / threadpool.c:390-486.  On the GPU one
 * launch covers all rows; num_threads only updates the recorded pool size
 * (threadpool.c:404-406), the result is bitwise the same for every value. */
ASMHIP_API void asm_matmul_q4_mt(const uint8_t* qweights, const float* scales, const float* x, float* y,
                                 int64_t M, int64_t K, int num_threads);
/* src/runtime/threadpool.h:59-67 / threadpool.c:750-767. */
ASMHIP_API void asm_matmul_q8_mt(const int8_t* qweights, const float* scales, const float* x, float* y,
                                 int64_t M, int64_t K, int num_threads);
/* src/runtime/threadpool.h:80-87 / threadpool.c:588-665. */
ASMHIP_API void asm_threadpool_dispatch_q8(const int8_t* qweights, const float* scales, const float* x,
                                           float* y, int64_t M, int64_t K);
/* src/runtime/threadpool.h:69-78 / threadpool.c:769-787 (num_threads as for
 * asm_matmul_q4_mt). */
ASMHIP_API void asm_matmul_q5_mt(const uint8_t* ql, const uint8_t* qh, const float* scales, const float* x,
                                 float* y, int64_t M, int64_t K, int num_threads);
/* src/runtime/threadpool.h:89-97 / threadpool.c:667-748. */
ASMHIP_API void asm_threadpool_dispatch_q5(const uint8_t* ql, const uint8_t* qh, const float* scales,
                                           const float* x, float* y, int64_t M, int64_t K);
/* src/runtime/threadpool.h:37 / threadpool.c:340-369: binds the calling
 * thread's current HIP device, creates the library stream and records the
 * pool size (clamped to [1, 64], threadpool.c:345-346). */
ASMHIP_API void asm_threadpool_init(int num_threads);
/* src/runtime/threadpool.h:42 / threadpool.c:371-382: drains and releases
 * the library stream and staging memory; pool size becomes 0. */
ASMHIP_API void asm_threadpool_shutdown(void);
/* src/runtime/threadpool.h:102 / threadpool.c:386-388. */
ASMHIP_API int asm_threadpool_get_num_threads(void);

/* Decode-step ops (build_kernel.py:85-104 export list; argtypes
 * test_runner.py:199-296; call sites generate.py:261-326). */
/* y = (x * (1/sqrt(mean(x^2) + eps))) * w   (rmsnorm_avx2.asm:63-151) */
ASMHIP_API void asm_rmsnorm(const float* x, const float* w, float* y, int64_t dim, float eps);
/* In place on one head of q and one of k: pairs (2p, 2p+1) rotated by
 * pos * theta^(-2p/head_dim)   (rope_avx2.asm:52-146) */
ASMHIP_API void asm_rope(float* q, float* k, int64_t head_dim, int64_t pos, float theta);
/* y = exp(x - max) / sum, x == y allowed   (softmax_avx2.asm:48-130) */
ASMHIP_API void asm_softmax(const float* x, float* y, int64_t dim);
/* gate = gate / (1 + exp(-gate)) * up   (swiglu_avx2.asm:45-81) */
ASMHIP_API void asm_silu_hadamard(float* gate, const float* up, int64_t dim);
/* y = softmax(q k^T * scale) v, q/k/v/y [seq_len][head_dim]
 * (attention_avx2.asm:59-218) */
ASMHIP_API void asm_attention(const float* q, const float* k, const float* v, float* y, int64_t seq_len,
                              int64_t head_dim, float scale);

/* ---- 2. device entry points (hot path) ----------------------------------- */

/* Q4_0 matvec over GGUF blocks resident in HBM: y[M] = W[M][K] x[K].  Block
 * arithmetic of matmul_q4_avx2.asm:110-178 with the GGUF scale widened
 * fp16 -> fp32 (src/runtime/generate.py:91-106). */
ASMHIP_API int asmhip_matmul_q4_0(const void* blocks, const float* x, float* y, int64_t M, int64_t K,
                                  void* stream);
/* Q8_0 matvec over GGUF blocks (matmul_q8_avx2.asm:103-155, generate.py:109-119). */
ASMHIP_API int asmhip_matmul_q8_0(const void* blocks, const float* x, float* y, int64_t M, int64_t K,
                                  void* stream);
/* Split-layout matvecs on device pointers (the asm_matmul_q4 / asm_matmul_q8
 * contract without staging or synchronization). */
ASMHIP_API int asmhip_matmul_q4_split(const uint8_t* qweights, const float* scales, const float* x,
                                      float* y, int64_t M, int64_t K, void* stream);
ASMHIP_API int asmhip_matmul_q8_split(const int8_t* qweights, const float* scales, const float* x,
                                      float* y, int64_t M, int64_t K, void* stream);
/* Q5_0 matvecs on device pointers: the asm_matmul_q5 contract
 * (matmul_q5_avx2.asm:93-210) on the split layout, and the same arithmetic
 * over 22-byte GGUF Q5_0 blocks read in place (scale widened fp16 -> fp32). */
ASMHIP_API int asmhip_matmul_q5_split(const uint8_t* ql, const uint8_t* qh, const float* scales, const float* x,
                                      float* y, int64_t M, int64_t K, void* stream);
ASMHIP_API int asmhip_matmul_q5_0(const void* blocks, const float* x, float* y, int64_t M, int64_t K,
                                  void* stream);
/* Exact fp32 dequantization of GGUF blocks into w[rows][K]
 * (tests/reference/ops.py:16-30, 44-53, 67-92). */
ASMHIP_API int asmhip_dequantize_q4_0(const void* blocks, float* w, int64_t rows, int64_t K, void* stream);
ASMHIP_API int asmhip_dequantize_q8_0(const void* blocks, float* w, int64_t rows, int64_t K, void* stream);
ASMHIP_API int asmhip_dequantize_q5_0(const void* blocks, float* w, int64_t rows, int64_t K, void* stream);

/* GGUF-block matvec with work fused around it, as forward_token sequences it
 * (generate.py:261-326): pre_op transforms x while it is read (RMSNorm with
 * weights pre_arg, or SwiGLU with x = gate and pre_arg = up), and accumulate
 * != 0 adds W x into y (the residual add) instead of overwriting y. */
ASMHIP_API int asmhip_matmul_fused(int qtype, const void* blocks, const float* x, float* y, int64_t M, int64_t K,
                                   int pre_op, const float* pre_arg, float eps, int accumulate, void* stream);
/* The FFN's gate/up matvecs and silu(gate) * up in one call (generate.py:308-313
 * computes them as two matvecs and asm_silu_hadamard, swiglu_avx2.asm:45-81):
 * blocks holds 2H rows that interleave the gate and up matrices in groups of 8
 * (rows 16g..16g+7 = gate rows 8g..8g+7, rows 16g+8..16g+15 = up rows 8g..8g+7;
 * H % 8 == 0), and h[j] = gate_j / (1 + exp(-gate_j)) * up_j, with x
 * transformed by pre_op as in asmhip_matmul_fused.  work: 2H floats of device
 * memory, written only where the int8-MFMA stream cannot take the shape (the
 * matvec then writes its 2H outputs there and a second launch combines them). */
ASMHIP_API int asmhip_matmul_swiglu(int qtype, const void* blocks, const float* x, float* h, int64_t H, int64_t K,
                                    int pre_op, const float* pre_arg, float eps, float* work, void* stream);
/* Prefill GEMM: C[T][M] = sum over blocks b of int32 dot(A[t,b], W[j,b]) * d_w[j,b] * d_a[t,b],
 * accumulated in fp32 in block order; A = T activation rows and W = M weight rows, both
 * Q8_0 blocks [rows][K/32] (quantize activations with asmhip_quantize(ASMHIP_Q8_0, ...)).
 * The reference's only quantized-activation recipe (matmul_q4_neon.S:57-143, 190-255)
 * applied to a batch; the reference itself has no GEMM. */
ASMHIP_API int asmhip_gemm_q8_0(const void* w_blocks, const void* a_blocks, float* c, int64_t T, int64_t M,
                                int64_t K, void* stream);
/* The same GEMM on operands arranged once into GEMM tiles, so that each K step of a
 * workgroup's tile is one contiguous run per operand (the kernel's LDS-direct loads
 * land it as it lies).  The tile layout is a permutation of the Q8_0 blocks: rows in
 * tiles of 128 (W) or 64 (A), tiles in order, within a tile the K steps of two
 * blocks, within a step the tile's rows, 68 bytes each (the two blocks as they lie
 * in the GGUF row); rows past the last pad the last tile.  K % 64 == 0.  Sizes:
 * asmhip_gemm_q8_0_tiled_weight_bytes(M, K), asmhip_gemm_q8_0_tiled_activation_bytes(T, K)
 * (0 for invalid shapes).  Build W once with asmhip_gemm_q8_0_tile_weights (padding
 * rows zero); build A from fp32 rows with asmhip_quantize_q8_0_tiled (the
 * asmhip_quantize Q8_0 blocks written in tile order; padding rows are not written and
 * reach only outputs that are not stored) or from Q8_0 blocks with
 * asmhip_gemm_q8_0_tile_activations.  Operands 16-byte aligned.  C is bitwise that of
 * asmhip_gemm_q8_0 on the same blocks.  No counterpart in the reference (it has no
 * GEMM). */
ASMHIP_API int64_t asmhip_gemm_q8_0_tiled_weight_bytes(int64_t M, int64_t K);
ASMHIP_API int64_t asmhip_gemm_q8_0_tiled_activation_bytes(int64_t T, int64_t K);
ASMHIP_API int asmhip_gemm_q8_0_tile_weights(const void* w_blocks, void* w_tiled, int64_t M, int64_t K,
                                             void* stream);
ASMHIP_API int asmhip_gemm_q8_0_tile_activations(const void* a_blocks, void* a_tiled, int64_t T, int64_t K,
                                                 void* stream);
ASMHIP_API int asmhip_quantize_q8_0_tiled(const float* x, void* a_tiled, int64_t T, int64_t K, void* stream);
ASMHIP_API int asmhip_gemm_q8_0_tiled(const void* w_tiled, const void* a_tiled, float* c, int64_t T, int64_t M,
                                      int64_t K, void* stream);
/* The same GEMM with W in the split layout of asm_matmul_q8 (matmul_q8_avx2.asm:51-194):
 * int8 qs planes [rows][K] (16-byte aligned) and fp32 scale planes [rows][K/32], for W (M rows)
 * and A (T rows).  The activations are int8 too: quantize the fp32 rows with
 * asmhip_quantize_q8_split (Q8_0, round to nearest even, scale amax/127 rounded to fp16).  So
 * C is NOT T calls of asm_matmul_q8, which multiplies the int8 weights by fp32 x: each
 * activation carries its quantization error, at most half its block's step d_a = amax/127
 * (|C - asm_matmul_q8(W, x)| <= sum over the row of |w| d_a / 2, about 0.4% of the row's L1
 * norm; tests/test_gemm_gpu.py measures it).  Per block the scale is the fp32 product
 * d_w * d_a (any fp32 scales), then acc = fmaf(float(dot), scale, acc) in block order: with
 * scales widened from fp16 the result is bitwise that of asmhip_gemm_q8_0 on the same blocks. */
ASMHIP_API int asmhip_gemm_q8_split(const int8_t* w_qs, const float* w_scales, const int8_t* a_qs,
                                    const float* a_scales, float* c, int64_t T, int64_t M, int64_t K, void* stream);
/* Process-wide Q4_0 GGUF kernel choice (ASMHIP_Q4_KERNEL_*). */
ASMHIP_API int asmhip_set_q4_kernel(int kernel);
ASMHIP_API int asmhip_get_q4_kernel(void);

/* fp32 rows -> GGUF blocks on the GPU: Q4_0 d = m / -8 (m the first element of
 * largest magnitude), q = min(15, trunc(w / d + 8.5)); Q8_0 d = amax / 127,
 * q = round-half-even(w * 127 / amax) saturated (matmul_q4_neon.S:80-135);
 * d stored as fp16 (round to nearest even). */
ASMHIP_API int asmhip_quantize(int qtype, const float* w, void* blocks, int64_t rows, int64_t K, void* stream);
/* Q8_0 quantization as above into the split layout: qs[rows][K] int8 (16-byte aligned) and
 * scales[rows][K/32] = the fp16 d widened to fp32 (the operands of asmhip_gemm_q8_split). */
ASMHIP_API int asmhip_quantize_q8_split(const float* w, int8_t* qs, float* scales, int64_t rows, int64_t K,
                                        void* stream);
/* Synthetic model data generated in HBM: blocks of N(0, stddev^2) weights
 * quantized as above, fp16 N(0, stddev^2) values, or a constant fill. */
ASMHIP_API int asmhip_random_blocks(int qtype, void* blocks, int64_t rows, int64_t K, uint64_t seed, float stddev,
                                    void* stream);
ASMHIP_API int asmhip_random_f16(void* out, int64_t n, uint64_t seed, float stddev, void* stream);
ASMHIP_API int asmhip_fill_f32(float* out, int64_t n, float value, void* stream);

/* Device-pointer forms of the decode-step ops.  asmhip_rope rotates
 * n_q_heads heads of q and n_k_heads heads of k; the position is *pos_dev
 * when pos_dev is not NULL (read on the GPU, so a captured graph follows it),
 * else pos. */
ASMHIP_API int asmhip_rmsnorm(const float* x, const float* w, float* y, int64_t dim, float eps, void* stream);
ASMHIP_API int asmhip_rope(float* q, float* k, int64_t n_q_heads, int64_t n_k_heads, int64_t head_dim,
                           const int* pos_dev, int64_t pos, float theta, void* stream);
ASMHIP_API int asmhip_softmax(const float* x, float* y, int64_t dim, void* stream);
ASMHIP_API int asmhip_silu_hadamard(float* gate, const float* up, int64_t dim, void* stream);
ASMHIP_API int asmhip_attention(const float* q, const float* k, const float* v, float* y, int64_t seq_len,
                                int64_t head_dim, float scale, void* stream);

/* Decode attention over an fp16 KV cache (generate.py:283-296 with the cache
 * kept on the GPU in fp16).  qkv = [q (n_heads*head_dim) | k | v
 * (n_kv_heads*head_dim each)]; caches are head-major
 * [n_kv_heads][max_ctx][head_dim] fp16.  asmhip_rope_kv_write rotates q in
 * place and writes rotated k and v at position *pos_dev.
 * asmhip_attention_decode computes, per head h (kv head h / (n_heads /
 * n_kv_heads)), softmax(q_h . k_p / sqrt(head_dim)) . v_p over positions
 * 0..*pos_dev (max_ctx <= 32768); workspace holds
 * asmhip_attention_decode_workspace() floats (calls sharing one workspace
 * must not overlap).  head_dim 48, 64 or 128. */
ASMHIP_API int asmhip_rope_kv_write(float* qkv, void* k_cache, void* v_cache, int n_heads, int n_kv_heads,
                                    int head_dim, const int* pos_dev, int max_ctx, float theta, void* stream);
ASMHIP_API int64_t asmhip_attention_decode_workspace(int n_heads, int head_dim, int max_ctx);
ASMHIP_API int asmhip_attention_decode(const float* q, const void* k_cache, const void* v_cache, float* workspace,
                                       float* out, int n_heads, int n_kv_heads, int head_dim, const int* pos_dev,
                                       int max_ctx, void* stream);
/* Both of the above fused: q and the new k rotated at *pos_dev, the
 * new k and v rows written to the caches (fp16), attention over 0..*pos_dev
 * into out; q in qkv is left unrotated (generate.py:282-296). */
ASMHIP_API int asmhip_attention_decode_rope(const float* qkv, void* k_cache, void* v_cache, float* workspace,
                                            float* out, int n_heads, int n_kv_heads, int head_dim, const int* pos_dev,
                                            int max_ctx, float theta, void* stream);
/* The RoPE angles of generate.py:282-283 (rope_avx2.asm:52-146) for every
 * position 0..max_ctx-1, formed once: table[p][2i] = cos and table[p][2i + 1]
 * = sin of pair i (head_dim / 2 pairs) at position p, max_ctx * head_dim
 * floats, the same values asmhip_rope_kv_write forms per call.
 * asmhip_attention_decode_rope_table is asmhip_attention_decode_rope with the
 * angles read from such a table (8-byte aligned) instead of formed in the
 * launch: same results, bit for bit. */
ASMHIP_API int asmhip_rope_table(float* table, int head_dim, int max_ctx, float theta, void* stream);
ASMHIP_API int asmhip_attention_decode_rope_table(const float* qkv, void* k_cache, void* v_cache, float* workspace,
                                                  float* out, int n_heads, int n_kv_heads, int head_dim,
                                                  const int* pos_dev, int max_ctx, const float* rope_table,
                                                  void* stream);
/* The decode step's attention and o projection in two launches instead of
 * three (generate.py:283-300: per-head softmax(q k^T) v, then the o matvec and
 * the residual add).  asmhip_attention_decode_partials_rope_table is
 * asmhip_attention_decode_rope_table without its merge launch: it leaves every
 * split's softmax state in `workspace` (splits of 384 positions while
 * max_ctx <= 3072, else of 512)
 * (asmhip_attention_decode_workspace() floats, 16-byte aligned).
 * asmhip_matmul_attn_output then computes y = W . attn (accumulate: y += W .
 * attn) for GGUF blocks W [M][n_heads * head_dim / 32] (qtype Q4_0 or Q8_0),
 * where attn is the merged attention output: for Q4_0 where the int8-MFMA
 * stream takes the shape (head_dim 64 or 128, n_heads * head_dim a multiple of
 * 256 and at most 8192, max_ctx <= 4096) the merge runs inside the matvec's
 * read of x; otherwise a merge launch writes attn to `work` (n_heads *
 * head_dim floats) and a matvec reads it.  Results equal the merge launch + asmhip_matmul_fused, bit for bit.
 * `workspace` and `max_ctx` must be those of the attention call. */
ASMHIP_API int asmhip_attention_decode_partials_rope_table(const float* qkv, void* k_cache, void* v_cache,
                                                           float* workspace, int n_heads, int n_kv_heads,
                                                           int head_dim, const int* pos_dev, int max_ctx,
                                                           const float* rope_table, void* stream);
ASMHIP_API int asmhip_matmul_attn_output(int qtype, const void* blocks, const float* workspace, float* work, float* y,
                                         int64_t M, int n_heads, int head_dim, int max_ctx, int accumulate,
                                         void* stream);
/* Measurement, not part of the path: reads `bytes` (< 2 GiB) of device memory
 * in one launch, every workgroup one contiguous chunk with all loads issued up
 * front, and keeps nothing; `sink` is 4 KB of device memory.  Its time is the
 * single-launch read floor a matvec over the same bytes can approach (no
 * counterpart in the reference). */
ASMHIP_API int asmhip_stream_read(const void* buf, int64_t bytes, void* sink, void* stream);
/* Measurement, not part of the path (no counterpart in the reference): the same
 * read in the launch shape of the matvec (one 1024-thread workgroup per compute
 * unit, all loads up front) with the matvec's structural pieces added by `flags`:
 * 1 = its dynamic LDS allocation of `lds` bytes (<= 160 KB), 2 = x (`xn` floats,
 * 16-byte aligned) read and a workgroup barrier before the loads, 4 = 16 floats of
 * `y` (`y_floats` floats, at least 16 per workgroup) stored per workgroup at the
 * end.  `sink` is 4 KB of device memory. */
ASMHIP_API int asmhip_stream_read_shaped(const void* buf, int64_t bytes, const float* x, int xn, float* y,
                                         int64_t y_floats, int flags, int lds, void* sink, void* stream);
/* Measurement (no counterpart in the reference): asmhip_matmul_q4_0 at its headline
 * launch shape (K = 4096, M > 2048) in an instantiation where every wave records
 * the 100 MHz real-time counter at 8 points (entry, first weight loads issued, x
 * digits ready, first unit landed, last unit landed, stream done, all waves done,
 * y written) into stamps[(workgroup * 16 + wave) * 8 + i] (device memory, at least
 * workgroups * 128 entries: min(ceil(M / 16), CUs) workgroups).  Same y. */
ASMHIP_API int asmhip_matmul_q4_0_stamped(const void* blocks, const float* x, float* y, int64_t M, int64_t K,
                                          uint64_t* stamps, int64_t stamps_len, void* stream);
/* Measurement (no counterpart in the reference): an empty kernel of `grid`
 * workgroups of `threads` threads with `lds` bytes of dynamic LDS. */
ASMHIP_API int asmhip_empty_launch(int grid, int threads, int lds, void* stream);
/* Measurement (no counterpart in the reference): `n` grid-wide barriers inside
 * one cooperative launch of one 1024-thread workgroup per compute unit, over a
 * zero-initialized device counter; *err (device) becomes nonzero if a barrier
 * does not complete within its bounded poll.  ASMHIP_ERR_UNSUPPORTED without
 * cooperative launch. */
ASMHIP_API int asmhip_grid_barrier(unsigned* counter, int n, unsigned* err, void* stream);
/* asmhip_attention_decode_rope without the workspace argument.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory (HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * split partials go to a fixed per-device scratch array of
 * asmhip_attention_decode_noalloc_max_floats() floats (4 MiB); shapes needing
 * more (n_heads * S * (head_dim + 4) floats, S = ceil(max_ctx / 384) for
 * max_ctx <= 3072, else ceil(max_ctx / 512)) are rejected with
 * ASMHIP_ERR_INVALID_ARGUMENT.  Calls that overlap on one GPU share the array and
 * race; nothing in it needs clearing between calls.  Same results, bit for bit,
 * as asmhip_attention_decode_rope.  The first call on each device looks up the
 * array's address and must be made outside stream capture (inside a capture it
 * returns ASMHIP_ERR_INVALID_ARGUMENT); later calls may be captured. */
ASMHIP_API int64_t asmhip_attention_decode_noalloc_max_floats(void);
ASMHIP_API int asmhip_attention_decode_rope_noalloc(const float* qkv, void* k_cache, void* v_cache, float* out,
                                                    int n_heads, int n_kv_heads, int head_dim, const int* pos_dev,
                                                    int max_ctx, float theta, void* stream);
/* x = row *token_dev of a Q4_0 embedding table [n_vocab][dim]
 * (generate.py:262, the table dequantized by get_tensor :169-182). */
ASMHIP_API int asmhip_embed_q4_0(const void* table, const int* token_dev, float* x, int n_vocab, int dim,
                                 void* stream);
/* The same for a Q8_0 table (generate.py:169-182 also dequantizes type 8). */
ASMHIP_API int asmhip_embed_q8_0(const void* table, const int* token_dev, float* x, int n_vocab, int dim,
                                 void* stream);
/* *token_dev = first index of max(logits) (numpy.argmax, generate.py:419-420);
 * then ++*pos_dev when pos_dev is not NULL. */
ASMHIP_API int asmhip_argmax(const float* logits, int n, int* token_dev, int* pos_dev, void* stream);
/* asmhip_argmax that also records the token: history_dev[*pos_dev] = *token_dev
 * (when 0 <= *pos_dev < history_len), then ++*pos_dev.  The generation loop of
 * generate.py:411-430 appends each greedy token on the host; here the list is
 * kept on the GPU, so a graph of several token steps returns every token, not
 * only the last. */
ASMHIP_API int asmhip_argmax_history(const float* logits, int n, int* token_dev, int* pos_dev, int* history_dev,
                                     int history_len, void* stream);

/* ---- device memory, streams, events (so a ctypes host needs no other GPU
 *      binding; the reference's buffers are numpy arrays) ----------------- */

ASMHIP_API int asmhip_device_count(void);
/* Name, compute units, peak engine clock (kHz) and memory of the current device. */
ASMHIP_API int asmhip_device_info(char* name, size_t name_len, int* compute_units, int* clock_khz,
                                  size_t* total_mem);
ASMHIP_API void* asmhip_malloc(size_t bytes);
ASMHIP_API int asmhip_free(void* ptr);
/* kind: 1 host->device, 2 device->host, 3 device->device.  Synchronous. */
ASMHIP_API int asmhip_memcpy(void* dst, const void* src, size_t bytes, int kind);
ASMHIP_API int asmhip_synchronize(void);
ASMHIP_API void* asmhip_stream_create(void);
ASMHIP_API int asmhip_stream_destroy(void* stream);
ASMHIP_API int asmhip_stream_synchronize(void* stream);
ASMHIP_API void* asmhip_event_create(void);
/* An event for timing only (hipEventDisableSystemFence): recording it does no
 * system-scope cache writeback / invalidate, so it does not perturb the work
 * that follows; waiting on it does not make device writes visible to the host. */
ASMHIP_API void* asmhip_event_create_timing(void);
ASMHIP_API int asmhip_event_destroy(void* event);
ASMHIP_API int asmhip_event_record(void* event, void* stream);
ASMHIP_API int asmhip_event_synchronize(void* event);
ASMHIP_API int asmhip_event_elapsed_ms(void* start, void* stop, float* ms);
/* Stream capture into a HIP graph: begin on a stream, enqueue work, end to
 * get an instantiated graph that asmhip_graph_launch replays on any stream. */
ASMHIP_API int asmhip_stream_begin_capture(void* stream);
ASMHIP_API int asmhip_stream_end_capture(void* stream, void** graph_exec);
ASMHIP_API int asmhip_graph_launch(void* graph_exec, void* stream);
ASMHIP_API int asmhip_graph_destroy(void* graph_exec);
/* Message for the calling thread's last failed call ("" if none). */
ASMHIP_API const char* asmhip_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* ASMLLM_HIP_H */
