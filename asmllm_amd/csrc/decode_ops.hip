// Decode-step kernels for gfx950: the ops asmllm's forward_token sequences
// around the matvecs (src/runtime/generate.py:261-326), so a whole token
// step stays on the GPU.
//
//   rmsnorm        rmsnorm_avx2.asm:63-151       y = (x * (1/sqrt(mean(x^2) + eps))) * w
//   rope           rope_avx2.asm:52-146          interleaved pairs (2p, 2p+1), freq = theta^(-2p/hd)
//   softmax        softmax_avx2.asm:48-130       max, exp(x - max), / sum
//   silu_hadamard  swiglu_avx2.asm:45-81         gate = gate / (1 + exp(-gate)) * up
//   swiglu_pairs   the same product over gate/up values interleaved in groups of 8
//   attention      attention_avx2.asm:59-218     softmax(q k^T * scale) v, all rows (non-causal)
//
// plus the device-side pieces of the decode engine: RoPE fused with the fp16
// KV-cache write, split-K attention over the fp16 cache, embedding-row
// dequantization and greedy argmax.  The angle of RoPE is formed in double
// precision: the reference forms it in x87 extended precision, and at decode
// positions in the thousands an fp32 angle would be off by ~1e-4 rad.
#include <math.h>

#include "common.hpp"
#include "kernels.hpp"

namespace asmhip {

namespace {

constexpr int kBlock = 256;

template <int kThreads>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kThreads / kWave; ++i) t += red[i];
    return t;
}

template <int kThreads>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int i = 1; i < kThreads / kWave; ++i) t = fmaxf(t, red[i]);
    return t;
}

// ---- rmsnorm: one workgroup per vector -----------------------------------------
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       float* __restrict__ y, int dim, float eps) {
    __shared__ float red[16];
    float s = 0.f;
    for (int i = threadIdx.x; i < dim; i += 1024) s = fmaf(x[i], x[i], s);
    s = block_sum<1024>(s, red);
    const float inv = 1.0f / sqrtf(s / (float)dim + eps);
    for (int i = threadIdx.x; i < dim; i += 1024) y[i] = __fmul_rn(__fmul_rn(x[i], inv), w[i]);
}

// ---- rope: pair (2p, 2p+1) of every head of q and of k -----------------------------
__device__ __forceinline__ void rope_angle(int p, int hd, int pos, float theta, float* c, float* s) {
    const float e = (float)(-2 * p) / (float)hd;  // divss in the reference
    const double ang = pow((double)theta, (double)e) * (double)(float)pos;
    *c = (float)cos(ang);
    *s = (float)sin(ang);
}

// Two products and a sum, each rounded (mulss, mulss, subss / addss in
// rope_avx2.asm:114-145): contraction off, or the compiler fuses one product
// into an fma, and which one depends on the code around the call.
__device__ __forceinline__ void rotate(float* v, float c, float s) {
#pragma clang fp contract(off)
    const float a = v[0], b = v[1];
    v[0] = a * c - b * s;
    v[1] = a * s + b * c;
}

__global__ __launch_bounds__(kBlock) void rope_kernel(float* __restrict__ q, float* __restrict__ k, int n_q_heads,
                                                      int n_k_heads, int hd, const int* __restrict__ pos_ptr,
                                                      int pos, float theta) {
    const int half = hd >> 1;
    const int i = blockIdx.x * kBlock + threadIdx.x;
    const int total = (n_q_heads + n_k_heads) * half;
    if (i >= total) return;
    const int p = i % half, head = i / half;
    const int position = pos_ptr ? *pos_ptr : pos;
    float c, s;
    rope_angle(p, hd, position, theta, &c, &s);
    float* v = head < n_q_heads ? q + (size_t)head * hd : k + (size_t)(head - n_q_heads) * hd;
    rotate(v + 2 * p, c, s);
}

// ---- RoPE on q/k of a fused qkv vector + fp16 KV-cache write at *pos --------------
// qkv = [q (n_heads*hd) | k (n_kv*hd) | v (n_kv*hd)]; caches are head-major
// [n_kv][max_ctx][hd] fp16.  q is rotated in place.
__global__ __launch_bounds__(kBlock) void rope_kv_write_kernel(float* __restrict__ qkv, __half* __restrict__ kc,
                                                               __half* __restrict__ vc, int n_heads, int n_kv, int hd,
                                                               const int* __restrict__ pos_ptr, int max_ctx,
                                                               float theta) {
    const int half = hd >> 1;
    const int i = blockIdx.x * kBlock + threadIdx.x;
    const int n_pairs = (n_heads + n_kv) * half;
    const int pos = *pos_ptr;
    if (pos < 0 || pos >= max_ctx) return;  // the host never lets this happen; no write out of range
    if (i < n_pairs) {
        const int p = i % half, head = i / half;
        float c, s;
        rope_angle(p, hd, pos, theta, &c, &s);
        float v[2] = {qkv[(size_t)head * hd + 2 * p], qkv[(size_t)head * hd + 2 * p + 1]};
        rotate(v, c, s);
        if (head < n_heads) {
            qkv[(size_t)head * hd + 2 * p] = v[0];
            qkv[(size_t)head * hd + 2 * p + 1] = v[1];
        } else {
            const int kh = head - n_heads;
            __half* dst = kc + ((size_t)kh * max_ctx + pos) * hd + 2 * p;
            dst[0] = __float2half_rn(v[0]);
            dst[1] = __float2half_rn(v[1]);
        }
    } else if (i < n_pairs + n_kv * hd) {
        const int j = i - n_pairs, kh = j / hd, d = j % hd;
        vc[((size_t)kh * max_ctx + pos) * hd + d] = __float2half_rn(qkv[(size_t)(n_heads + n_kv) * hd + j]);
    }
}

// ---- softmax of one vector (x == y allowed) -------------------------------------------
__global__ __launch_bounds__(1024) void softmax_kernel(const float* x, float* y, int dim) {
    __shared__ float red[16];
    float m = -INFINITY;
    for (int i = threadIdx.x; i < dim; i += 1024) m = fmaxf(m, x[i]);
    m = block_max<1024>(m, red);
    float s = 0.f;
    for (int i = threadIdx.x; i < dim; i += 1024) {
        const float e = expf(x[i] - m);
        y[i] = e;
        s += e;
    }
    s = block_sum<1024>(s, red);
    for (int i = threadIdx.x; i < dim; i += 1024) y[i] = y[i] / s;
}

// ---- silu(gate) * up, in place on gate ----------------------------------------------
__device__ __forceinline__ float silu_mul(float g, float u) {
    return __fmul_rn(g / (1.0f + expf(-g)), u);
}

__global__ __launch_bounds__(kBlock) void silu_kernel(float* __restrict__ g, const float* __restrict__ u, int dim) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i < dim) g[i] = silu_mul(g[i], u[i]);
}

// gate/up rows interleaved in groups of 8: output j pairs entries 16 (j / 8) + j % 8 and + 8
__global__ __launch_bounds__(kBlock) void swiglu_pairs_kernel(const float* __restrict__ gu, float* __restrict__ h,
                                                              int H) {
    const int j = blockIdx.x * kBlock + threadIdx.x;
    if (j < H) {
        const int i = 16 * (j >> 3) + (j & 7);
        h[j] = silu_mul(gu[i], gu[i + 8]);
    }
}

// ---- reference attention: one workgroup per query row, scores in LDS ----------------
__global__ __launch_bounds__(kBlock) void attention_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ v, float* __restrict__ y,
                                                           int seq, int hd, float scale) {
    extern __shared__ float sc[];  // seq scores
    __shared__ float red[kBlock / kWave];
    const int row = blockIdx.x;
    const float* qi = q + (size_t)row * hd;
    for (int j = threadIdx.x; j < seq; j += kBlock) {
        const float* kj = k + (size_t)j * hd;
        float d = 0.f;
        for (int t = 0; t < hd; ++t) d = fmaf(qi[t], kj[t], d);
        sc[j] = d * scale;
    }
    __syncthreads();
    float m = -INFINITY;
    for (int j = threadIdx.x; j < seq; j += kBlock) m = fmaxf(m, sc[j]);
    m = block_max<kBlock>(m, red);
    float s = 0.f;
    for (int j = threadIdx.x; j < seq; j += kBlock) {
        const float e = expf(sc[j] - m);
        sc[j] = e;
        s += e;
    }
    s = block_sum<kBlock>(s, red);
    __syncthreads();
    for (int t = threadIdx.x; t < hd; t += kBlock) {
        float a = 0.f;
        for (int j = 0; j < seq; ++j) a = fmaf(sc[j], v[(size_t)j * hd + t], a);
        y[(size_t)row * hd + t] = a / s;
    }
}

// ---- decode attention over the fp16 cache: one launch per layer ----------------------
// grid (n_heads, S = ceil(max_ctx / SL)), SL = attn_split_len(max_ctx); workgroup
// (h, s) covers positions [s*SL, (s+1)*SL) of 0..pos.  Within a workgroup
// a position is read by HD/8 lanes (8 dims = 16 bytes each), so a wave covers
// 64/(HD/8) positions per row and the four waves kRowPos; a lane reads
// kAttnRows rows of k and of v per chunk (one position each), and the split is
// kChunks chunks walked with the next two chunks' loads in flight while the
// current one is scored (three register buffers).  k and v are read with nontemporal
// loads: the cache rows are read once per token.  Each lane group keeps an
// online softmax state (max m, sum l, acc[8]) over its positions; the states of
// all lane groups of the workgroup merge once through LDS; each workgroup
// writes [m, l, -, -, acc[HD]] (kAttnPartStride(HD) floats, acc 16-byte
// aligned) to `part`, and attn_decode_merge, or a matvec whose x is the
// attention output (kPreAttnMerge), combines the S partials of a head in split
// order into acc / l (attn_merge_value).
//
// ROPE != kRopeNone also does what rope_kv_write does, inside the same launch:
// q and the new k are rotated at `pos`, the new k and v are rounded to fp16 and
// written to the caches at `pos` (by the workgroup of the first query head of
// the kv group), and the lane that owns `pos` uses those fp16 values instead of
// reading the row it writes.  kRopeTheta forms the angles (rope_angle, double
// precision: about 600 fp64 instructions that every wave waits for); kRopeTable
// reads the same cos/sin values from a table that rope_table_kernel filled
// once, a load that travels with the k/v loads.
// Sum over aligned groups of N lanes (N = 8 or 16), every lane receiving its
// group's sum, with DPP adds instead of LDS permutes: quad_perm [1,0,3,2] and
// [2,3,0,1] sum the quads, row_half_mirror pairs quad 0 with 1 (2 with 3),
// row_mirror the two halves of a 16-lane row.  Each step adds two partial sums
// that are the same in every lane of a pair, so all lanes hold the same bits.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(N == 8 || N == 16, "8- or 16-lane groups");
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    if constexpr (N == 16) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
    return v;
}

// E fp16 values of one cache row slice (E = 8: one 16-byte access; E = 6: three dwords).
template <int E>
struct HalfRow {
    uint32_t w[E / 2];
    __device__ static HalfRow load(const __half* p) {
        HalfRow r;
        if constexpr (E == 8) {
            const uint4 v = *reinterpret_cast<const uint4*>(p);
            r.w[0] = v.x, r.w[1] = v.y, r.w[2] = v.z, r.w[3] = v.w;
        } else {
#pragma unroll
            for (int i = 0; i < E / 2; ++i) r.w[i] = reinterpret_cast<const uint32_t*>(p)[i];
        }
        return r;
    }
    __device__ static HalfRow zero() {
        HalfRow r;
#pragma unroll
        for (int i = 0; i < E / 2; ++i) r.w[i] = 0u;
        return r;
    }
    __device__ void store(__half* p) const {
        if constexpr (E == 8) {
            *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
            for (int i = 0; i < E / 2; ++i) reinterpret_cast<uint32_t*>(p)[i] = w[i];
        }
    }
};

constexpr uint32_t kAttnPastEnd = 0xFFFFFF00u;  // buffer offset that loads zeros

enum RopeMode : int { kRopeNone = 0, kRopeTheta = 1, kRopeTable = 2 };

template <int HD, int ROPE, int SL>
__global__ __launch_bounds__(kBlock) void attn_decode_kernel(const float* __restrict__ qkv, __half* kc, __half* vc,
                                                             float* __restrict__ part, int n_heads, int n_kv,
                                                             const int* __restrict__ pos_ptr, int max_ctx,
                                                             float theta, const float* __restrict__ rope_table) {
    constexpr int E = HD % 64 == 0 ? 8 : 6;               // fp16 elements per lane
    constexpr int kLanes = HD / E;                        // lanes per position
    static_assert(HD == E * kLanes && kWave % kLanes == 0, "head_dim 48, 64 or 128");
    constexpr int kGroups = kWave / kLanes;               // positions per wave and row
    constexpr int kRowPos = kGroups * (kBlock / kWave);   // positions per workgroup and row
    constexpr int R = kAttnRows;                          // rows per lane and chunk
    constexpr int kChunkPos = kRowPos * R;
    constexpr int kChunks = SL / kChunkPos;
    static_assert(SL % kChunkPos == 0, "split must hold whole chunks");
    constexpr int kStride = kAttnPartStride(HD);
    __shared__ float cs[HD];                 // cos, sin of pair i at 2i, 2i+1
    constexpr int kGroupsWg = kBlock / kLanes;  // lane groups (position slots) of the workgroup
    __shared__ float wst[kGroupsWg][HD + 2];

    const int h = blockIdx.x, split = blockIdx.y;
    const int group = n_heads / n_kv, kvh = h / group;
    const int pos = *pos_ptr;
    const int n_pos = (pos >= 0 && pos < max_ctx) ? pos + 1 : 0;  // an invalid position reads and writes nothing
    const int p0 = split * SL, p1 = min(p0 + SL, n_pos);
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
    const int g = lane / kLanes, c = lane % kLanes;
    const size_t head_off = (size_t)kvh * max_ctx * HD + E * c;
    // position of row r of chunk ch for this lane
    auto position = [&](int ch, int r) { return p0 + ch * kChunkPos + r * kRowPos + w * kGroups + g; };

    // q first, then the first chunk's k rows, then its v rows: loads return in
    // order, so the scores can start while v is in flight.  HD % 64 == 0:
    // branch-free buffer loads, a row outside the split (or the row at pos,
    // which this launch writes) reading zeros from past the end of the buffer.
    float qv[E];
#pragma unroll
    for (int t = 0; t < E; t += 2) {
        const float2 a = *reinterpret_cast<const float2*>(qkv + (size_t)h * HD + E * c + t);
        qv[t] = a.x, qv[t + 1] = a.y;
    }
    // cos, sin of this lane's E / 2 pairs (pair E/2 c + i at 2i, 2i + 1)
    float csl[E];
    if constexpr (ROPE == kRopeTable) {
        const float* row = rope_table + (size_t)(n_pos > 0 ? pos : 0) * HD + E * c;
#pragma unroll
        for (int t = 0; t < E; t += 2) {
            const float2 a = *reinterpret_cast<const float2*>(row + t);
            csl[t] = a.x, csl[t + 1] = a.y;
        }
    }
    // chunks in flight: the next two chunks' rows are requested before a chunk
    // is scored (three register buffers; measured at the 7B shape, 6 splits of
    // 384 positions: 7.65 us with two buffers, 7.55 with three, 7.68 with four)
    constexpr int NB = kChunks >= 3 ? 3 : kChunks;
    HalfRow<E> kr[NB][R], vr[NB][R];
    const uint32_t cache_bytes = (uint32_t)n_kv * (uint32_t)max_ctx * (uint32_t)(2 * HD);  // < 4 GB, checked at launch
    const auto kres = make_rsrc(kc, cache_bytes), vres = make_rsrc(vc, cache_bytes);
    auto issue = [&](int b, int ch) {
        uint32_t off[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int p = position(ch, r);
            const bool live = p < p1 && !(ROPE != kRopeNone && p == pos);
            off[r] = live ? 2u * (uint32_t)(head_off + (size_t)p * HD) : kAttnPastEnd;
            if constexpr (E == 8) {
                const uint4 a = buf_load_b128_nt(kres, off[r]);
                kr[b][r].w[0] = a.x, kr[b][r].w[1] = a.y, kr[b][r].w[2] = a.z, kr[b][r].w[3] = a.w;
            } else {
                kr[b][r] = live ? HalfRow<E>::load(kc + off[r] / 2) : HalfRow<E>::zero();
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (E == 8) {
                const uint4 a = buf_load_b128_nt(vres, off[r]);
                vr[b][r].w[0] = a.x, vr[b][r].w[1] = a.y, vr[b][r].w[2] = a.z, vr[b][r].w[3] = a.w;
            } else {
                vr[b][r] = off[r] != kAttnPastEnd ? HalfRow<E>::load(vc + off[r] / 2) : HalfRow<E>::zero();
            }
        }
    };
#pragma unroll
    for (int c = 0; c < NB - 1; ++c) issue(c, c);
    if constexpr (ROPE == kRopeTheta) {
        if (threadIdx.x < HD / 2 && n_pos > 0)
            rope_angle(threadIdx.x, HD, pos, theta, &cs[2 * threadIdx.x], &cs[2 * threadIdx.x + 1]);
        __syncthreads();
#pragma unroll
        for (int t = 0; t < E; ++t) csl[t] = cs[E * c + t];
    }
    // the new row: rotated k and v of kv head kvh, rounded to fp16, used by
    // the lane that owns position pos (chunk nch, row nr)
    HalfRow<E> kq = HalfRow<E>::zero(), vq = HalfRow<E>::zero();
    int nch = -1, nr = -1;
    if constexpr (ROPE != kRopeNone) {
        if (n_pos > 0) {
#pragma unroll
            for (int i = 0; i < E / 2; ++i) rotate(&qv[2 * i], csl[2 * i], csl[2 * i + 1]);
        }
        if (p0 <= pos && pos < p1) {
            const float* kn = qkv + (size_t)(n_heads + kvh) * HD + E * c;
            const float* vn = qkv + (size_t)(n_heads + n_kv + kvh) * HD + E * c;
#pragma unroll
            for (int i = 0; i < E / 2; ++i) {
                float kk[2] = {kn[2 * i], kn[2 * i + 1]};
                rotate(kk, csl[2 * i], csl[2 * i + 1]);
                kq.w[i] = (uint32_t)__half_as_ushort(__float2half_rn(kk[0])) |
                          ((uint32_t)__half_as_ushort(__float2half_rn(kk[1])) << 16);
                vq.w[i] = (uint32_t)__half_as_ushort(__float2half_rn(vn[2 * i])) |
                          ((uint32_t)__half_as_ushort(__float2half_rn(vn[2 * i + 1])) << 16);
            }
            const int rel = pos - p0, rem = rel % kRowPos;
            if (w == rem / kGroups && g == rem % kGroups) {
                nch = rel / kChunkPos;
                nr = (rel % kChunkPos) / kRowPos;
                if (h % group == 0) {
                    kq.store(kc + head_off + (size_t)pos * HD);
                    vq.store(vc + head_off + (size_t)pos * HD);
                }
            }
        }
    }
    const float scale = 1.0f / sqrtf((float)HD);
#pragma unroll
    for (int t = 0; t < E; ++t) qv[t] *= scale;

    // chunk by chunk: request the next chunk, then score this one and fold it
    // into the lane group's online softmax state
    float m = -INFINITY, l = 0.f, acc[E];
#pragma unroll
    for (int t = 0; t < E; ++t) acc[t] = 0.f;
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
        const int b = ch % NB;
        if (ch + NB - 1 < kChunks) issue((ch + NB - 1) % NB, ch + NB - 1);
        if (ch == nch) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (r == nr) kr[b][r] = kq, vr[b][r] = vq;
        }
        float sc[R];
        float mc = -INFINITY;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float d = 0.f;
#pragma unroll
            for (int t = 0; t < E / 2; ++t) {
                d = fmaf(qv[2 * t], half_lo(kr[b][r].w[t]), d);
                d = fmaf(qv[2 * t + 1], half_hi(kr[b][r].w[t]), d);
            }
            d = group_sum<kLanes>(d);
            sc[r] = position(ch, r) < p1 ? d : -INFINITY;
            mc = fmaxf(mc, sc[r]);
        }
        const float mn = fmaxf(m, mc);
        if (mn != -INFINITY) {
            const float f = __expf(m - mn);  // 0 while the state is empty
            l *= f;
#pragma unroll
            for (int t = 0; t < E; ++t) acc[t] *= f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float e = __expf(sc[r] - mn);  // 0 for positions past the split
                l += e;
#pragma unroll
                for (int t = 0; t < E / 2; ++t) {
                    acc[2 * t] = fmaf(e, half_lo(vr[b][r].w[t]), acc[2 * t]);
                    acc[2 * t + 1] = fmaf(e, half_hi(vr[b][r].w[t]), acc[2 * t + 1]);
                }
            }
            m = mn;
        }
    }
    // every lane group's softmax state to LDS (no cross-lane shuffles), then one
    // merge over all groups of the workgroup in group order; thread t < HD owns
    // dimension t of this workgroup's partial
    {
        const int gs = w * kGroups + g;
#pragma unroll
        for (int t = 0; t < E; ++t) wst[gs][2 + E * c + t] = acc[t];
        if (c == 0) wst[gs][0] = m, wst[gs][1] = l;
    }
    __syncthreads();
    float* mine = part + ((size_t)h * gridDim.y + split) * kStride;
    if (threadIdx.x < HD) {
        float M = -INFINITY;
#pragma unroll
        for (int i = 0; i < kGroupsWg; ++i) M = fmaxf(M, wst[i][0]);
        float L = 0.f, a = 0.f;
        if (M != -INFINITY) {
#pragma unroll
            for (int i = 0; i < kGroupsWg; ++i) {
                const float f = __expf(wst[i][0] - M);  // 0 for groups that saw no position
                L = fmaf(wst[i][1], f, L);
                a = fmaf(wst[i][2 + threadIdx.x], f, a);
            }
        }
        mine[4 + threadIdx.x] = a;
        if (threadIdx.x == 0) mine[0] = M, mine[1] = L;
    }
}

// Merge of the S partials of head h (blockIdx.x) in split order; thread t owns
// dimension t.  Splits past the last position hold m = -inf, l = 0.
template <int HD>
__global__ __launch_bounds__(HD) void attn_decode_merge(const float* __restrict__ part, float* __restrict__ out,
                                                        int S) {
    const int h = blockIdx.x;
    out[(size_t)h * HD + threadIdx.x] = attn_merge_value(part + (size_t)h * S * kAttnPartStride(HD), S,
                                                         kAttnPartStride(HD), threadIdx.x);
}

// ---- embedding row of a Q4_0 table -----------------------------------------------------
template <bool kQ8>
__global__ __launch_bounds__(kBlock) void embed_kernel(const uint8_t* __restrict__ table,
                                                       const int* __restrict__ token, float* __restrict__ x,
                                                       int n_vocab, int dim) {
    const int t = *token;
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= dim || t < 0 || t >= n_vocab) return;
    const int nb = dim / 32, b = i / 32, j = i % 32;
    const uint8_t* blk = table + ((size_t)t * nb + b) * (kQ8 ? 34 : 18);
    const float d = __half2float(__ushort_as_half((unsigned short)(blk[0] | (blk[1] << 8))));
    if (kQ8) {
        x[i] = (float)(int8_t)blk[2 + j] * d;
    } else {
        const int n = j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4);
        x[i] = ((float)n - 8.0f) * d;
    }
}

// ---- greedy argmax (first index of the maximum, as numpy.argmax) -------------------------
// numpy.argmax order: a NaN ranks above every number, and equal values (NaN or
// not) go to the lower index.
__device__ __forceinline__ bool argmax_better(float a, int ia, float b, int ib) {
    const bool na = a != a, nb = b != b;
    if (na || nb) return na && (!nb || ia < ib);
    return a > b || (a == b && ia < ib);
}

// VEC (n % 4 == 0, logits 16-byte aligned): 16-byte loads, 8 per thread and
// pass instead of 32 single floats; which thread sees an element does not
// change the result (ties go to the lower index).
template <bool VEC>
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ logits, int n,
                                                      int* __restrict__ token, int* __restrict__ pos,
                                                      int* __restrict__ history, int history_len) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    float v = -INFINITY;
    int idx = 0x7fffffff;  // padding: loses to every real element, -inf included
    // 32 elements per thread and pass, all loaded before any is compared (one
    // memory round per 32768 logits: a single pass for a 32000-token vocabulary)
    constexpr int kPer = 32;
    for (int base = 0; base < n; base += kPer * 1024) {
        float x[kPer];
        if constexpr (VEC) {
            // element base + 4 (k 1024 + t) + j of load k, lane j
#pragma unroll
            for (int k = 0; k < kPer / 4; ++k) {
                const int i = base + 4 * (k * 1024 + (int)threadIdx.x);
                const float4 q = i < n ? *reinterpret_cast<const float4*>(logits + i)
                                       : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
                x[4 * k] = q.x, x[4 * k + 1] = q.y, x[4 * k + 2] = q.z, x[4 * k + 3] = q.w;
            }
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int i = base + 4 * ((k >> 2) * 1024 + (int)threadIdx.x) + (k & 3);
                if (i < n && argmax_better(x[k], i, v, idx)) {
                    v = x[k];
                    idx = i;
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int i = base + k * 1024 + (int)threadIdx.x;
                x[k] = i < n ? logits[i] : -INFINITY;
            }
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int i = base + k * 1024 + (int)threadIdx.x;
                if (i < n && argmax_better(x[k], i, v, idx)) {
                    v = x[k];
                    idx = i;
                }
            }
        }
    }
    // the (value, index) order is total, so any reduction order gives the same
    // winner: within each 16-lane row through DPP, then the four rows of a wave
    // and the 16 waves in order (no LDS round trips inside a wave)
    auto take = [&](float ov, int oi) {
        if (argmax_better(ov, oi, v, idx)) {
            v = ov;
            idx = oi;
        }
    };
    auto row_reduce = [&]() {
        take(__int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kDppQuadXor1, 0xF, 0xF, false)),
             __builtin_amdgcn_update_dpp(0, idx, kDppQuadXor1, 0xF, 0xF, false));
        take(__int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kDppQuadXor2, 0xF, 0xF, false)),
             __builtin_amdgcn_update_dpp(0, idx, kDppQuadXor2, 0xF, 0xF, false));
        take(__int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kDppRowHalfMirror, 0xF, 0xF, false)),
             __builtin_amdgcn_update_dpp(0, idx, kDppRowHalfMirror, 0xF, 0xF, false));
        take(__int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kDppRowMirror, 0xF, 0xF, false)),
             __builtin_amdgcn_update_dpp(0, idx, kDppRowMirror, 0xF, 0xF, false));
    };
    row_reduce();  // every lane holds its row's winner
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    {
        const int vb = __float_as_int(v), ib = idx;
        v = __int_as_float(__builtin_amdgcn_readlane(vb, 0));
        idx = __builtin_amdgcn_readlane(ib, 0);
#pragma unroll
        for (int r = 1; r < 4; ++r)
            take(__int_as_float(__builtin_amdgcn_readlane(vb, 16 * r)), __builtin_amdgcn_readlane(ib, 16 * r));
    }
    if (lane == 0) {
        bv[w] = v;
        bi[w] = idx;
    }
    __syncthreads();
    if (w == 0) {
        v = lane < 16 ? bv[lane] : -INFINITY;
        idx = lane < 16 ? bi[lane] : 0x7fffffff;
        row_reduce();  // lanes 0-15 hold the winner of the 16 waves
    }
    if (threadIdx.x == 0) {
        const int bidx = idx;
        *token = bidx;
        if (pos) {
            // history[p] = the token chosen at position p, so that a graph of
            // several steps keeps every token, not just the last one
            const int p = *pos;
            if (history && p >= 0 && p < history_len) history[p] = bidx;
            *pos = p + 1;
        }
    }
}

}  // namespace

// The single-workgroup kernels step an int index by up to 32768 (argmax) and
// loop while it is below the length: lengths within that stride of INT32_MAX
// would overflow the index and never end the loop.
constexpr int64_t kMaxStridedLen = INT32_MAX - 65536;

int rmsnorm_launch(const float* x, const float* w, float* y, int64_t dim, float eps, hipStream_t st) {
    if (dim <= 0 || dim > kMaxStridedLen) return fail(kInvalidArgument, "rmsnorm: bad dim %lld", (long long)dim);
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, st, x, w, y, (int)dim, eps);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int rope_launch(float* q, float* k, int64_t n_q_heads, int64_t n_k_heads, int64_t hd, const int* pos_ptr,
                int64_t pos, float theta, hipStream_t st) {
    if (hd <= 0 || hd % 2 || n_q_heads < 0 || n_k_heads < 0 || pos < 0 || pos > INT32_MAX)
        return fail(kInvalidArgument, "rope: need even head_dim > 0 and pos >= 0");
    const int64_t total = (n_q_heads + n_k_heads) * (hd / 2);
    if (total == 0) return kOk;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((total + kBlock - 1) / kBlock)), dim3(kBlock), 0, st, q, k,
                       (int)n_q_heads, (int)n_k_heads, (int)hd, pos_ptr, (int)pos, theta);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int rope_kv_write_launch(float* qkv, void* k_cache, void* v_cache, int n_heads, int n_kv, int hd,
                         const int* pos_ptr, int max_ctx, float theta, hipStream_t st) {
    if (hd % 2 || n_kv <= 0 || n_heads % n_kv) return fail(kInvalidArgument, "rope_kv_write: bad head layout");
    const int total = (n_heads + n_kv) * (hd / 2) + n_kv * hd;
    hipLaunchKernelGGL(rope_kv_write_kernel, dim3((total + kBlock - 1) / kBlock), dim3(kBlock), 0, st, qkv,
                       (__half*)k_cache, (__half*)v_cache, n_heads, n_kv, hd, pos_ptr, max_ctx, theta);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int softmax_launch(const float* x, float* y, int64_t dim, hipStream_t st) {
    if (dim <= 0 || dim > kMaxStridedLen) return fail(kInvalidArgument, "softmax: bad dim");
    hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(1024), 0, st, x, y, (int)dim);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int swiglu_pairs_launch(const float* gu, float* h, int64_t H, hipStream_t st) {
    if (H <= 0 || H % 8 || H > INT32_MAX / 2) return fail(kInvalidArgument, "swiglu: need H > 0 and H %% 8 == 0");
    hipLaunchKernelGGL(swiglu_pairs_kernel, dim3((unsigned)((H + kBlock - 1) / kBlock)), dim3(kBlock), 0, st, gu, h,
                       (int)H);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int silu_launch(float* g, const float* u, int64_t dim, hipStream_t st) {
    if (dim <= 0 || dim > kMaxStridedLen) return fail(kInvalidArgument, "silu_hadamard: bad dim");
    hipLaunchKernelGGL(silu_kernel, dim3((unsigned)((dim + kBlock - 1) / kBlock)), dim3(kBlock), 0, st, g, u,
                       (int)dim);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int attention_launch(const float* q, const float* k, const float* v, float* y, int64_t seq, int64_t hd, float scale,
                     hipStream_t st) {
    if (seq <= 0 || hd <= 0) return fail(kInvalidArgument, "attention: need seq > 0 and head_dim > 0");
    if (hd > kMaxStridedLen) return fail(kInvalidArgument, "attention: head_dim %lld", (long long)hd);
    if (seq > 40000) return fail(kUnsupported, "attention: seq_len %lld exceeds the LDS score buffer", (long long)seq);
    const int rc = dynamic_lds((const void*)attention_kernel, (size_t)seq * sizeof(float));
    if (rc) return rc;
    hipLaunchKernelGGL(attention_kernel, dim3((unsigned)seq), dim3(kBlock), (size_t)seq * sizeof(float), st, q, k,
                       v, y, (int)seq, (int)hd, scale);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int attn_decode_splits(int max_ctx) {
    const int sl = attn_split_len(max_ctx);
    return (int)(((int64_t)max_ctx + sl - 1) / sl);
}

int64_t attn_decode_workspace(int n_heads, int hd, int max_ctx) {
    return (int64_t)n_heads * attn_decode_splits(max_ctx) * kAttnPartStride(hd);
}

namespace {
template <int HD, int SL>
void launch_attn_split(int mode, dim3 grid, hipStream_t st, const float* qkv, __half* kc, __half* vc, float* part,
                       int n_heads, int n_kv, const int* pos_ptr, int max_ctx, float theta, const float* rope_table) {
    if (mode == kRopeTable)
        hipLaunchKernelGGL((attn_decode_kernel<HD, kRopeTable, SL>), grid, dim3(kBlock), 0, st, qkv, kc, vc, part,
                           n_heads, n_kv, pos_ptr, max_ctx, theta, rope_table);
    else if (mode == kRopeTheta)
        hipLaunchKernelGGL((attn_decode_kernel<HD, kRopeTheta, SL>), grid, dim3(kBlock), 0, st, qkv, kc, vc, part,
                           n_heads, n_kv, pos_ptr, max_ctx, theta, rope_table);
    else
        hipLaunchKernelGGL((attn_decode_kernel<HD, kRopeNone, SL>), grid, dim3(kBlock), 0, st, qkv, kc, vc, part,
                           n_heads, n_kv, pos_ptr, max_ctx, theta, rope_table);
}

template <int HD>
void launch_attn_decode(int mode, dim3 grid, hipStream_t st, const float* qkv, __half* kc, __half* vc, float* part,
                        float* out, int n_heads, int n_kv, const int* pos_ptr, int max_ctx, float theta,
                        const float* rope_table) {
    if (attn_split_len(max_ctx) == kAttnSplitShort)
        launch_attn_split<HD, kAttnSplitShort>(mode, grid, st, qkv, kc, vc, part, n_heads, n_kv, pos_ptr, max_ctx,
                                               theta, rope_table);
    else
        launch_attn_split<HD, kAttnSplitLong>(mode, grid, st, qkv, kc, vc, part, n_heads, n_kv, pos_ptr, max_ctx,
                                              theta, rope_table);
    if (out) hipLaunchKernelGGL((attn_decode_merge<HD>), dim3(n_heads), dim3(HD), 0, st, part, out, (int)grid.y);
}
}  // namespace

int attn_decode_launch(const float* qkv, void* k_cache, void* v_cache, float* part, float* out, int n_heads,
                       int n_kv, int hd, const int* pos_ptr, int max_ctx, bool rope, float theta, hipStream_t st,
                       const float* rope_table) {
    if (n_kv <= 0 || n_heads % n_kv) return fail(kInvalidArgument, "attention: n_heads %% n_kv_heads != 0");
    if (max_ctx <= 0) return fail(kInvalidArgument, "attention: max_ctx must be > 0");
    if (max_ctx > kAttnMaxCtx)
        return fail(kUnsupported, "attention: max_ctx %d exceeds %d positions", max_ctx, kAttnMaxCtx);
    const int splits = attn_decode_splits(max_ctx);
    if ((uintptr_t)qkv % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16 || (uintptr_t)part % 16)
        return fail(kInvalidArgument, "attention: q, the caches and the workspace must be 16-byte aligned");
    if (rope_table && (uintptr_t)rope_table % 8)
        return fail(kInvalidArgument, "attention: the RoPE table must be 8-byte aligned");
    if ((int64_t)n_kv * max_ctx * hd * 2 >= (int64_t)kAttnPastEnd)
        return fail(kUnsupported, "attention: caches of 4 GB or more per layer are not supported");
    const int mode = !rope ? kRopeNone : rope_table ? kRopeTable : kRopeTheta;
    const dim3 grid(n_heads, splits);
    __half* kc = (__half*)k_cache;
    __half* vc = (__half*)v_cache;
    if (hd == 128)
        launch_attn_decode<128>(mode, grid, st, qkv, kc, vc, part, out, n_heads, n_kv, pos_ptr, max_ctx, theta,
                                rope_table);
    else if (hd == 64)
        launch_attn_decode<64>(mode, grid, st, qkv, kc, vc, part, out, n_heads, n_kv, pos_ptr, max_ctx, theta,
                               rope_table);
    else if (hd == 48)
        launch_attn_decode<48>(mode, grid, st, qkv, kc, vc, part, out, n_heads, n_kv, pos_ptr, max_ctx, theta,
                               rope_table);
    else
        return fail(kUnsupported, "attention: head_dim %d (supported: 48, 64, 128)", hd);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int attn_merge_launch(const float* part, float* out, int n_heads, int hd, int max_ctx, hipStream_t st) {
    if (n_heads <= 0 || max_ctx <= 0) return fail(kInvalidArgument, "attention merge: bad shape");
    if (max_ctx > kAttnMaxCtx)
        return fail(kUnsupported, "attention merge: max_ctx %d exceeds %d positions", max_ctx, kAttnMaxCtx);
    const int splits = attn_decode_splits(max_ctx);
    if (hd == 128)
        hipLaunchKernelGGL((attn_decode_merge<128>), dim3(n_heads), dim3(128), 0, st, part, out, splits);
    else if (hd == 64)
        hipLaunchKernelGGL((attn_decode_merge<64>), dim3(n_heads), dim3(64), 0, st, part, out, splits);
    else if (hd == 48)
        hipLaunchKernelGGL((attn_decode_merge<48>), dim3(n_heads), dim3(48), 0, st, part, out, splits);
    else
        return fail(kUnsupported, "attention merge: head_dim %d (supported: 48, 64, 128)", hd);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

// table[p][2i] = cos, table[p][2i + 1] = sin of pair i at position p (rope_angle).
__global__ __launch_bounds__(kBlock) void rope_table_kernel(float* __restrict__ table, int hd, int max_ctx,
                                                            float theta) {
    const int half = hd >> 1;
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= (int64_t)max_ctx * half) return;
    const int pair = (int)(i % half), p = (int)(i / half);
    rope_angle(pair, hd, p, theta, &table[2 * i], &table[2 * i + 1]);
}

int rope_table_launch(float* table, int hd, int max_ctx, float theta, hipStream_t st) {
    if (!table) return fail(kInvalidArgument, "rope table: null pointer");
    if (hd <= 0 || hd % 2 || max_ctx <= 0) return fail(kInvalidArgument, "rope table: bad shape");
    const int64_t n = (int64_t)max_ctx * (hd / 2);
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + kBlock - 1) / kBlock)), dim3(kBlock), 0, st, table,
                       hd, max_ctx, theta);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int embed_launch(QuantType qt, const void* table, const int* token, float* x, int n_vocab, int dim, hipStream_t st) {
    if (dim % 32) return fail(kInvalidArgument, "embedding: dim %% 32 != 0");
    const dim3 grid((dim + kBlock - 1) / kBlock);
    if (qt == QuantType::Q8_0)
        hipLaunchKernelGGL((embed_kernel<true>), grid, dim3(kBlock), 0, st, (const uint8_t*)table, token, x, n_vocab, dim);
    else
        hipLaunchKernelGGL((embed_kernel<false>), grid, dim3(kBlock), 0, st, (const uint8_t*)table, token, x, n_vocab, dim);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int argmax_launch(const float* logits, int n, int* token, int* pos, hipStream_t st, int* history, int history_len) {
    if (n <= 0) return fail(kInvalidArgument, "argmax: empty input");
    if (n > kMaxStridedLen) return fail(kInvalidArgument, "argmax: %d logits", n);
    if (history && (!pos || history_len <= 0))
        return fail(kInvalidArgument, "argmax: a token history needs the position and a length");
    if (n % 4 == 0 && (uintptr_t)logits % 16 == 0)
        hipLaunchKernelGGL(argmax_kernel<true>, dim3(1), dim3(1024), 0, st, logits, n, token, pos, history,
                           history_len);
    else
        hipLaunchKernelGGL(argmax_kernel<false>, dim3(1), dim3(1024), 0, st, logits, n, token, pos, history,
                           history_len);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

}  // namespace asmhip
