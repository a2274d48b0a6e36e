// Launchers shared between the kernel translation units and the C-ABI layer.
// Every launcher validates its arguments on the host, enqueues on `stream`
// and returns a Status (0 on success); none of them synchronizes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asmhip {

enum class QuantType { Q4_0, Q8_0 };

// Work fused into a matvec: a transform applied to x while it is staged, and
// whether y is overwritten or accumulated into.
enum PreOp : int {
    kPreNone = 0,
    kPreRmsNorm = 1,  // x <- (x * 1/sqrt(mean(x^2) + eps)) * arg[k] (the MFMA stream: W (x * arg)
                      // scaled by the 1/sqrt factor per row, which needs no barrier before x's digits)
    kPreSwiGlu = 2,   // x <- x / (1 + exp(-x)) * arg[k]
    // x is the decode attention output, merged from its split partials: arg is
    // the [n_heads][attn_splits][kAttnPartStride(attn_hd)] workspace that
    // attn_decode_launch(..., out = nullptr) filled, K = n_heads * attn_hd
    // (x itself is not read).  Q4_0 int8-MFMA stream only, attn_splits <=
    // kAttnMergeMaxSplits.
    kPreAttnMerge = 3,
};

// Work fused into a matvec's write of y.  kPostSwiGlu8: the rows of W come in
// groups of 16, the first 8 gate rows and the next 8 the matching up rows, and
// y[8 g + r] = silu(row 16 g + r) * row 16 g + 8 + r (M / 2 outputs).
enum PostOp : int {
    kPostNone = 0,
    kPostSwiGlu8 = 1,
};

struct MatvecOpts {
    int pre = kPreNone;
    const float* pre_arg = nullptr;
    float eps = 0.f;
    bool accumulate = false;  // y += W x
    int post = kPostNone;
    int attn_splits = 0;      // kPreAttnMerge: splits per head and head_dim
    int attn_hd = 0;
};

// y = W x.  gguf: W is [M][K/32] GGUF blocks; otherwise W is the split qs
// array and `scales` the fp32 [M][K/32] scales.
int matvec_launch(QuantType qt, bool gguf, const void* w, const float* scales, const float* x, float* y,
                  int64_t M, int64_t K, hipStream_t stream, const MatvecOpts& opts = MatvecOpts());

// Q5_0 y = W x.  gguf: W is [M][K/32] 22-byte GGUF blocks (qh, scales unused);
// otherwise the split layout: ql = w [M][K/32][16], qh [M][K/32][4] and fp32
// scales [M][K/32].
int q5_matvec_launch(bool gguf, const void* w, const uint8_t* qh, const float* scales, const float* x, float* y,
                     int64_t M, int64_t K, hipStream_t stream);
int q5_dequant_launch(const void* blocks, float* out, int64_t rows, int64_t K, hipStream_t stream);

// Q4_0 GGUF matvec on the int8 matrix cores (matvec_launch picks it when
// q4_0_mfma_eligible holds: K % 256 == 0, K <= 16384, 16-byte aligned x).
// Process-wide choice of the Q4_0 GGUF kernel: auto (MFMA when eligible), the
// fp32 VALU kernel only, or the MFMA kernel only (ineligible shapes fail).
enum Q4Kernel : int { kQ4KernelAuto = 0, kQ4KernelFp32 = 1, kQ4KernelMfma = 2 };
int set_q4_kernel(int kernel);
int get_q4_kernel();

bool q4_0_mfma_eligible(const void* w, const float* x, const MatvecOpts& opts, int64_t M, int64_t K);
int q4_0_mfma_launch(const void* w, const float* x, float* y, int64_t M, int64_t K, hipStream_t stream,
                     const MatvecOpts& opts);
// Measurement: the headline Q4_0 launch (K = 4096, M > 2048) with every wave
// recording 8 real-time stamps (100 MHz) into stamps[(block * 16 + wave) * 8 + i].
int q4_0_mfma_stamped_launch(const void* w, const float* x, float* y, int64_t M, int64_t K, uint64_t* stamps,
                             int64_t stamps_len, hipStream_t stream);
// The same stream over 22-byte GGUF Q5_0 blocks (no fused pre-ops).
bool q5_0_mfma_eligible(const void* w, const float* x, int64_t M, int64_t K);
int q5_0_mfma_launch(const void* w, const float* x, float* y, int64_t M, int64_t K, hipStream_t stream);
// The same stream over 34-byte GGUF Q8_0 blocks.
bool q8_0_mfma_eligible(const void* w, const float* x, const MatvecOpts& opts, int64_t M, int64_t K);
int q8_0_mfma_launch(const void* w, const float* x, float* y, int64_t M, int64_t K, hipStream_t stream,
                     const MatvecOpts& opts);
// The same stream over the reference's split layout, bits = 4 (qs + fp32 scales),
// 5 (ql + qh + fp32 scales) or 8 (int8 qs + fp32 scales); K % 256 == 0, 16-byte
// aligned planes.
bool split_mfma_eligible(int bits, const void* qs, const uint8_t* qh, const float* scales, const float* x, int64_t M,
                         int64_t K);
int split_mfma_launch(int bits, const void* qs, const uint8_t* qh, const float* scales, const float* x, float* y,
                      int64_t M, int64_t K, hipStream_t stream);

// C[T][M] = A (Q8_0 blocks [T][K/32]) x W (Q8_0 blocks [M][K/32])^T, block dots
// scaled by both fp16 scales and accumulated in block order.
int gemm_q8_0_launch(const void* w, const void* a, float* c, int64_t T, int64_t M, int64_t K, hipStream_t stream);

// GEMM tile layout of Q8_0 blocks: rows in tiles of R (kGemmTileA = 64 for the
// activations, kGemmTileW = 128 for the weights), the tiles one after another,
// within a tile the K steps of two blocks, within a step the tile's rows, 68
// bytes each (the two blocks as they lie in the GGUF row).  Rows past the last
// one pad the last tile.  K % 64 == 0.
constexpr int kGemmTileA = 64;
constexpr int kGemmTileW = 128;
__host__ __device__ inline int64_t gemm_tiled_offset(int64_t row, int64_t blk, int64_t nb, int R) {
    return ((row / R * (nb / 2) + blk / 2) * R + row % R) * 68 + (blk % 2) * 34;
}
__host__ __device__ inline int64_t gemm_tiled_bytes(int64_t rows, int64_t K, int R) {
    return (rows + R - 1) / R * R * (K / 32) * 34;
}
int gemm_q8_0_tiled_launch(const void* w_tiled, const void* a_tiled, float* c, int64_t T, int64_t M, int64_t K,
                           hipStream_t stream);
int gemm_tile_blocks_launch(const void* blocks, void* tiled, int64_t rows, int64_t K, int R, hipStream_t stream);
int quantize_q8_0_tiled_launch(const float* x, void* tiled, int64_t rows, int64_t K, hipStream_t stream);
int gemm_q8_split_launch(const int8_t* wq, const float* wsc, const int8_t* aq, const float* asc, float* c, int64_t T,
                         int64_t M, int64_t K, hipStream_t stream);

// Plain streaming read of `bytes` in one launch (measurement: the single-launch
// read floor); `sink` is 4 KB of device memory the kernel practically never writes.
int stream_read_launch(const void* buf, int64_t bytes, uint32_t* sink, hipStream_t st);
// The same read in the matvec's launch shape (one 1024-thread workgroup per
// compute unit), flags: 1 the matvec's dynamic LDS (`lds` bytes), 2 x (`xn`
// floats) read and a workgroup barrier first, 4 16 floats of y stored per workgroup.
int shaped_read_launch(const void* buf, int64_t bytes, const float* x, int xn, float* y, int64_t y_floats, int flags,
                       int lds, uint32_t* sink, hipStream_t st);
// An empty kernel of the given shape (the cost of a launch that does nothing).
int empty_launch(int grid, int threads, int lds, hipStream_t st);
// n grid-wide barriers in one cooperative launch of one 1024-thread workgroup per
// compute unit; *err is set if a barrier does not complete within its poll bound.
int grid_barrier_launch(unsigned* counter, int n, unsigned* err, hipStream_t st);

// Exact fp32 dequantization of GGUF blocks, row-major [rows][K].
int dequant_launch(QuantType qt, const void* w, float* out, int64_t rows, int64_t K, hipStream_t stream);

// fp32 [rows][K] -> GGUF blocks (the rules of the host quantizers, bit for bit).
int quantize_launch(QuantType qt, const float* w, void* blocks, int64_t rows, int64_t K, hipStream_t stream);
int quantize_q8_split_launch(const float* w, int8_t* qs, float* scales, int64_t rows, int64_t K, hipStream_t stream);
// Q4_0 / Q8_0 blocks of N(0, stddev^2) weights from a counter-based generator.
int random_blocks_launch(QuantType qt, void* blocks, int64_t rows, int64_t K, uint64_t seed, float stddev,
                         hipStream_t stream);
int random_f16_launch(void* out, int64_t n, uint64_t seed, float stddev, hipStream_t stream);
int fill_f32_launch(float* out, int64_t n, float value, hipStream_t stream);

// Decode-step ops.
int rmsnorm_launch(const float* x, const float* w, float* y, int64_t dim, float eps, hipStream_t st);
int rope_launch(float* q, float* k, int64_t n_q_heads, int64_t n_k_heads, int64_t hd, const int* pos_ptr,
                int64_t pos, float theta, hipStream_t st);
int rope_kv_write_launch(float* qkv, void* k_cache, void* v_cache, int n_heads, int n_kv, int hd,
                         const int* pos_ptr, int max_ctx, float theta, hipStream_t st);
int softmax_launch(const float* x, float* y, int64_t dim, hipStream_t st);
int silu_launch(float* g, const float* u, int64_t dim, hipStream_t st);
// h[8 g + r] = silu(gu[16 g + r]) * gu[16 g + 8 + r] for j < H (H % 8 == 0):
// kPostSwiGlu8 as its own launch over a matvec's 2H outputs.
int swiglu_pairs_launch(const float* gu, float* h, int64_t H, hipStream_t st);
// h = silu(W_gate x) * (W_up x) over GGUF blocks whose 2H rows interleave gate
// and up in groups of 8 (kPostSwiGlu8), x transformed by o.pre on the way in.
// One launch where the int8-MFMA stream takes the shape; otherwise the matvec
// writes its 2H outputs to `work` and swiglu_pairs_launch combines them.
int matvec_swiglu_launch(QuantType qt, const void* w, const float* x, float* h, int64_t H, int64_t K, float* work,
                         hipStream_t st, const MatvecOpts& o);
int attention_launch(const float* q, const float* k, const float* v, float* y, int64_t seq, int64_t hd, float scale,
                     hipStream_t st);

// Decode attention over head-major fp16 caches [n_kv][max_ctx][hd], positions
// 0..*pos_ptr: attn_split_len(max_ctx)-position splits, each walked in chunks of
// kAttnRows rows per lane, then a merge launch (out != nullptr) or nothing (the
// partials are left for a matvec with kPreAttnMerge).  `part` holds
// attn_decode_workspace() floats: per head and split [m, l, -, -, acc[hd]]
// (kAttnPartStride(hd) floats).  rope = true rotates q and the new k at
// *pos_ptr and writes the new k/v rows (fp16) in the split launch.
constexpr int kAttnRows = 4;
constexpr int kAttnMaxSplits = 64;
constexpr int kAttnMergeMaxSplits = 8;  // splits a matvec merges in its x prologue
// Split length: 384 positions while that keeps the splits within what a matvec
// merges (max_ctx <= 3072), else 512 (max_ctx <= 32768).  Shorter splits put
// more workgroups on the cache stream (7B, context 2048, max_ctx 2176: 6 splits
// of 384 give split attention + o projection 14.99 us per layer, 5 of 512 15.52;
// 320 positions, 7 splits, 15.18; 256, 9 splits, 18.2).  Both are whole chunks
// for every head_dim (64 or 128 positions per chunk).
constexpr int kAttnSplitShort = 384, kAttnSplitLong = 512;
constexpr int kAttnMaxCtx = kAttnMaxSplits * kAttnSplitLong;
constexpr int attn_split_len(int max_ctx) {
    return max_ctx <= kAttnMergeMaxSplits * kAttnSplitShort ? kAttnSplitShort : kAttnSplitLong;
}
constexpr int kAttnPartStride(int hd) { return hd + 4; }
int attn_decode_splits(int max_ctx);
int64_t attn_decode_workspace(int n_heads, int hd, int max_ctx);
// rope_table (optional, with rope): [max_ctx][hd] floats from rope_table_launch,
// read instead of forming the angles in the kernel.
int attn_decode_launch(const float* qkv, void* k_cache, void* v_cache, float* part, float* out, int n_heads,
                       int n_kv, int hd, const int* pos_ptr, int max_ctx, bool rope, float theta, hipStream_t st,
                       const float* rope_table = nullptr);
// out[h][t] = the merge of the split partials `part` of head h (attn_decode_merge).
int attn_merge_launch(const float* part, float* out, int n_heads, int hd, int max_ctx, hipStream_t st);
// table[p][2i], table[p][2i + 1] = cos, sin of RoPE pair i at position p < max_ctx.
int rope_table_launch(float* table, int hd, int max_ctx, float theta, hipStream_t st);

// x = row *token of a Q4_0 or Q8_0 GGUF table [n_vocab][dim], exact.
int embed_launch(QuantType qt, const void* table, const int* token, float* x, int n_vocab, int dim, hipStream_t st);
// *token = argmax; with pos: history[*pos] = *token (when history and 0 <= *pos <
// history_len), then ++*pos.
int argmax_launch(const float* logits, int n, int* token, int* pos, hipStream_t st, int* history = nullptr,
                  int history_len = 0);

}  // namespace asmhip
