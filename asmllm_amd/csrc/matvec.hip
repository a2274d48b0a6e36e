// Q4_0 / Q8_0 / Q5_0 matrix-vector kernels for gfx950 (VALU, fp32 accumulation).
//
// y[m] = sum_b d[m,b] * sum_j (q[m,b,j] - z) * x[32b + j],  z = 8 for Q4_0 and 0 for Q8_0
//
// Replaces the reference's asm_matmul_q4 (src/kernels/x86_64/matmul_q4_avx2.asm:57-287)
// and asm_matmul_q8 (src/kernels/x86_64/matmul_q8_avx2.asm:51-194).  Two weight
// layouts are read in place:
//   * GGUF blocks: Q4_0 = fp16 d + 16 B of nibbles (18 B / 32 weights),
//                  Q8_0 = fp16 d + 32 int8       (34 B / 32 weights);
//   * the reference's split layout: qs[M][K/32][16 or 32] + fp32 scales[M][K/32].
// Byte j of a Q4 block holds weight j in its low nibble and weight j+16 in its
// high nibble (matmul_q4_avx2.asm:122-153, tests/reference/ops.py:24-28).
//
// Work mapping (one wave = 64 lanes):
//   * a lane owns one PAIR of consecutive blocks (64 columns) of a 64-pair
//     column chunk, so a wave's loads for one row cover a contiguous
//     64 x 36 B (Q4_0 GGUF) span of HBM; pairs keep GGUF rows dword-aligned;
//   * a wave walks R rows at a time through every chunk, the x values of its
//     pair sit in registers and are reused for all R rows;
//   * x is staged once per workgroup in LDS (padded 4 floats per 64 so the
//     per-lane 256 B reads are bank-conflict free); for Q4 it is stored as
//     x / 16 (exact);
//   * every weight becomes an exact float with one v_cvt_f32_i32 (SDWA byte
//     select, sign extended): a Q4 nibble n is moved to the top of its byte
//     with bit 7 flipped, which reads as the signed byte 16 (n - 8)
//     (one v_bitop3_b32 for high nibbles, a shift plus one for low nibbles),
//     and 16 (n - 8) * (x / 16) is exactly the reference's (n - 8) * x;
//     Q8 bytes are converted directly;
//   * each lane keeps one fp32 accumulator per row, reduced across the wave
//     at the end.
#include <atomic>

#include "common.hpp"
#include "kernels.hpp"

namespace asmhip {

namespace {

constexpr int kThreads = 256;  // 4 waves per workgroup
constexpr int kWavesPerBlock = kThreads / kWave;

__device__ __forceinline__ int xpad(int i) { return i + ((i >> 6) << 2); }

// Hide the masked word from the instruction combiner so that each byte is
// converted by one v_cvt_f32_ubyte{k} instead of a bfe + cvt pair.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}

__device__ __forceinline__ float sbyte(uint32_t v, int k) { return (float)(int)(int8_t)((v >> (8 * k)) & 0xFFu); }

// Low/high nibbles of bytes [k0, k1) of v are weights jb.. and jb+16.. of a
// Q4 block; xl holds x[j] / 16, xh holds x[16 + j] / 16.
template <int k0, int k1, int jb>
__device__ __forceinline__ float q4_bytes(uint32_t v, const float* xl, const float* xh, float t) {
    const uint32_t lo = opaque(((v << 4) ^ 0x80808080u) & 0xF0F0F0F0u);  // bytes 16 (n_lo - 8)
    const uint32_t hi = opaque((v ^ 0x80808080u) & 0xF0F0F0F0u);         // bytes 16 (n_hi - 8)
#pragma unroll
    for (int k = k0; k < k1; ++k) {
        t = fmaf(sbyte(lo, k), xl[jb + k - k0], t);
        t = fmaf(sbyte(hi, k), xh[jb + k - k0], t);
    }
    return t;
}

// Signed bytes [k0, k1) of v times x[jb..].
template <int k0, int k1, int jb>
__device__ __forceinline__ float q8_bytes(uint32_t v, const float* xv, float t) {
    const uint32_t u = opaque(v);
#pragma unroll
    for (int k = k0; k < k1; ++k) t = fmaf(sbyte(u, k), xv[jb + k - k0], t);
    return t;
}

// Stage x into LDS in the padded layout, transformed by the fused pre-op and
// scaled by `scale` (1/16 for Q4, exact).
__device__ __forceinline__ void stage_x(const float* __restrict__ x, float* xs, int K, float scale, int pre,
                                        const float* __restrict__ arg, float eps) {
    if (pre == kPreRmsNorm) {
        __shared__ float red[kWavesPerBlock];
        float s = 0.f;
        for (int i = threadIdx.x; i < K; i += kThreads) s = fmaf(x[i], x[i], s);
        s = wave_sum(s);
        if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x >> 6] = s;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) tot += red[w];
        const float inv = 1.0f / sqrtf(tot / (float)K + eps);
        for (int i = threadIdx.x; i < K; i += kThreads)
            xs[xpad(i)] = __fmul_rn(__fmul_rn(__fmul_rn(x[i], inv), arg[i]), scale);
    } else if (pre == kPreSwiGlu) {
        for (int i = threadIdx.x; i < K; i += kThreads) {
            const float g = x[i];
            xs[xpad(i)] = __fmul_rn(__fmul_rn(g / (1.0f + expf(-g)), arg[i]), scale);
        }
    } else {
        for (int i = threadIdx.x; i < K; i += kThreads) xs[xpad(i)] = x[i] * scale;
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Q4_0 pair kernel.  kGguf: 18-byte blocks; otherwise split qs + fp32 scales.
// ---------------------------------------------------------------------------
template <int R, bool kGguf>
__global__ __launch_bounds__(kThreads) void q4_matvec_pairs(const uint8_t* __restrict__ w,
                                                            const float* __restrict__ wscale,
                                                            const float* __restrict__ x,
                                                            float* __restrict__ y, int M, int K, int pre,
                                                            const float* __restrict__ pre_arg, float eps,
                                                            int accumulate) {
    extern __shared__ float xs[];
    stage_x(x, xs, K, 0.0625f, pre, pre_arg, eps);

    const int nb = K >> 5;
    const int np = nb >> 1;
    const uint32_t row_bytes = kGguf ? (uint32_t)nb * 18u : (uint32_t)nb * 16u;
    const auto wr = make_rsrc(w, row_bytes * (uint32_t)M);
    const auto sr = make_rsrc(wscale, kGguf ? 0u : (uint32_t)nb * 4u * (uint32_t)M);
    const int lane = threadIdx.x & (kWave - 1);
    const int nwaves = gridDim.x * kWavesPerBlock;

    for (int g = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6); g * R < M; g += nwaves) {
        const int row0 = g * R;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;

        for (int c0 = 0; c0 < np; c0 += kWave) {
            const int p = c0 + lane;
            const bool active = p < np;
            const int pc = active ? p : np - 1;

            uint32_t v[R][9];
            float dA[R], dB[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = min(row0 + r, M - 1);
                if (kGguf) {
                    const uint32_t off = (uint32_t)row * row_bytes + (uint32_t)pc * 36u;
                    const uint4 a = buf_load_b128(wr, off);
                    const uint4 b = buf_load_b128(wr, off + 16u);
                    v[r][0] = a.x; v[r][1] = a.y; v[r][2] = a.z; v[r][3] = a.w;
                    v[r][4] = b.x; v[r][5] = b.y; v[r][6] = b.z; v[r][7] = b.w;
                    v[r][8] = buf_load_b32(wr, off + 32u);
                } else {
                    const uint32_t blk = (uint32_t)row * (uint32_t)nb + 2u * (uint32_t)pc;
                    const uint4 a = buf_load_b128(wr, blk * 16u);
                    const uint4 b = buf_load_b128(wr, blk * 16u + 16u);
                    const uint2 s = buf_load_b64(sr, blk * 4u);
                    v[r][0] = a.x; v[r][1] = a.y; v[r][2] = a.z; v[r][3] = a.w;
                    v[r][4] = b.x; v[r][5] = b.y; v[r][6] = b.z; v[r][7] = b.w;
                    dA[r] = __uint_as_float(s.x);
                    dB[r] = __uint_as_float(s.y);
                }
            }

            float xr[64];
            const float4* xq = reinterpret_cast<const float4*>(xs + xpad(pc * 64));
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const float4 t = xq[q];
                xr[4 * q] = t.x; xr[4 * q + 1] = t.y; xr[4 * q + 2] = t.z; xr[4 * q + 3] = t.w;
            }

#pragma unroll
            for (int r = 0; r < R; ++r) {
                float tA = 0.f, tB = 0.f;
                if (kGguf) {
                    dA[r] = half_lo(v[r][0]);
                    dB[r] = half_hi(v[r][4]);
                    tA = q4_bytes<2, 4, 0>(v[r][0], xr, xr + 16, tA);
                    tA = q4_bytes<0, 4, 2>(v[r][1], xr, xr + 16, tA);
                    tA = q4_bytes<0, 4, 6>(v[r][2], xr, xr + 16, tA);
                    tA = q4_bytes<0, 4, 10>(v[r][3], xr, xr + 16, tA);
                    tA = q4_bytes<0, 2, 14>(v[r][4], xr, xr + 16, tA);
                    tB = q4_bytes<0, 4, 0>(v[r][5], xr + 32, xr + 48, tB);
                    tB = q4_bytes<0, 4, 4>(v[r][6], xr + 32, xr + 48, tB);
                    tB = q4_bytes<0, 4, 8>(v[r][7], xr + 32, xr + 48, tB);
                    tB = q4_bytes<0, 4, 12>(v[r][8], xr + 32, xr + 48, tB);
                } else {
                    tA = q4_bytes<0, 4, 0>(v[r][0], xr, xr + 16, tA);
                    tA = q4_bytes<0, 4, 4>(v[r][1], xr, xr + 16, tA);
                    tA = q4_bytes<0, 4, 8>(v[r][2], xr, xr + 16, tA);
                    tA = q4_bytes<0, 4, 12>(v[r][3], xr, xr + 16, tA);
                    tB = q4_bytes<0, 4, 0>(v[r][4], xr + 32, xr + 48, tB);
                    tB = q4_bytes<0, 4, 4>(v[r][5], xr + 32, xr + 48, tB);
                    tB = q4_bytes<0, 4, 8>(v[r][6], xr + 32, xr + 48, tB);
                    tB = q4_bytes<0, 4, 12>(v[r][7], xr + 32, xr + 48, tB);
                }
                float a = fmaf(dA[r], tA, acc[r]);
                a = fmaf(dB[r], tB, a);
                acc[r] = active ? a : acc[r];
            }
        }

#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = wave_sum(acc[r]);
            if (lane == r && row0 + r < M) y[row0 + r] = accumulate ? y[row0 + r] + s : s;
        }
    }
}

// ---------------------------------------------------------------------------
// Q8_0 pair kernel.  kGguf: 34-byte blocks; otherwise split qs + fp32 scales.
// ---------------------------------------------------------------------------
template <int R, bool kGguf>
__global__ __launch_bounds__(kThreads) void q8_matvec_pairs(const uint8_t* __restrict__ w,
                                                            const float* __restrict__ wscale,
                                                            const float* __restrict__ x,
                                                            float* __restrict__ y, int M, int K, int pre,
                                                            const float* __restrict__ pre_arg, float eps,
                                                            int accumulate) {
    extern __shared__ float xs[];
    stage_x(x, xs, K, 1.0f, pre, pre_arg, eps);

    const int nb = K >> 5;
    const int np = nb >> 1;
    const uint32_t row_bytes = kGguf ? (uint32_t)nb * 34u : (uint32_t)nb * 32u;
    const auto wr = make_rsrc(w, row_bytes * (uint32_t)M);
    const auto sr = make_rsrc(wscale, kGguf ? 0u : (uint32_t)nb * 4u * (uint32_t)M);
    const int lane = threadIdx.x & (kWave - 1);
    const int nwaves = gridDim.x * kWavesPerBlock;

    for (int g = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6); g * R < M; g += nwaves) {
        const int row0 = g * R;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;

        for (int c0 = 0; c0 < np; c0 += kWave) {
            const int p = c0 + lane;
            const bool active = p < np;
            const int pc = active ? p : np - 1;

            uint32_t v[R][17];
            float dA[R], dB[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = min(row0 + r, M - 1);
                if (kGguf) {
                    const uint32_t off = (uint32_t)row * row_bytes + (uint32_t)pc * 68u;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint4 a = buf_load_b128(wr, off + 16u * q);
                        v[r][4 * q] = a.x; v[r][4 * q + 1] = a.y; v[r][4 * q + 2] = a.z; v[r][4 * q + 3] = a.w;
                    }
                    v[r][16] = buf_load_b32(wr, off + 64u);
                } else {
                    const uint32_t blk = (uint32_t)row * (uint32_t)nb + 2u * (uint32_t)pc;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint4 a = buf_load_b128(wr, blk * 32u + 16u * q);
                        v[r][4 * q] = a.x; v[r][4 * q + 1] = a.y; v[r][4 * q + 2] = a.z; v[r][4 * q + 3] = a.w;
                    }
                    const uint2 s = buf_load_b64(sr, blk * 4u);
                    dA[r] = __uint_as_float(s.x);
                    dB[r] = __uint_as_float(s.y);
                }
            }

            float xr[64];
            const float4* xq = reinterpret_cast<const float4*>(xs + xpad(pc * 64));
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const float4 t = xq[q];
                xr[4 * q] = t.x; xr[4 * q + 1] = t.y; xr[4 * q + 2] = t.z; xr[4 * q + 3] = t.w;
            }

#pragma unroll
            for (int r = 0; r < R; ++r) {
                float tA = 0.f, tB = 0.f;
                if (kGguf) {
                    // v0 = [dA | q0 q1], v1..v7 = q2..q29, v8 = [q30 q31 | dB], v9..v16 = block B.
                    dA[r] = half_lo(v[r][0]);
                    dB[r] = half_hi(v[r][8]);
                    tA = q8_bytes<2, 4, 0>(v[r][0], xr, tA);
#pragma unroll
                    for (int q = 1; q < 8; ++q) tA = q8_bytes<0, 4, 0>(v[r][q], xr + 2 + 4 * (q - 1), tA);
                    tA = q8_bytes<0, 2, 30>(v[r][8], xr, tA);
#pragma unroll
                    for (int q = 0; q < 8; ++q) tB = q8_bytes<0, 4, 0>(v[r][9 + q], xr + 32 + 4 * q, tB);
                } else {
#pragma unroll
                    for (int q = 0; q < 8; ++q) tA = q8_bytes<0, 4, 0>(v[r][q], xr + 4 * q, tA);
#pragma unroll
                    for (int q = 0; q < 8; ++q) tB = q8_bytes<0, 4, 0>(v[r][8 + q], xr + 32 + 4 * q, tB);
                }
                float a = fmaf(dA[r], tA, acc[r]);
                a = fmaf(dB[r], tB, a);
                acc[r] = active ? a : acc[r];
            }
        }

#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = wave_sum(acc[r]);
            if (lane == r && row0 + r < M) y[row0 + r] = accumulate ? y[row0 + r] + s : s;
        }
    }
}

// ---------------------------------------------------------------------------
// Generic kernel: one wave per row, one block per lane, byte loads.  Covers
// what the pair kernels do not (odd K/32, rows not dword aligned, x too large
// for LDS).  Correct for every K % 32 == 0, not tuned.
// ---------------------------------------------------------------------------
template <bool kQ8, bool kGguf>
__global__ __launch_bounds__(kThreads) void matvec_generic(const uint8_t* __restrict__ w,
                                                           const float* __restrict__ wscale,
                                                           const float* __restrict__ x,
                                                           float* __restrict__ y, int M, int K, int accumulate) {
    const int nb = K >> 5;
    const int qbytes = kQ8 ? 32 : 16;
    const int64_t blk_bytes = kGguf ? qbytes + 2 : qbytes;
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (row >= M) return;
    float acc = 0.f;
    for (int b = lane; b < nb; b += kWave) {
        const int64_t blk = (int64_t)row * nb + b;
        const uint8_t* p = w + blk * blk_bytes;
        float d;
        if (kGguf) {
            d = __half2float(__ushort_as_half((unsigned short)(p[0] | (p[1] << 8))));
            p += 2;
        } else {
            d = wscale[blk];
        }
        const float* xb = x + (int64_t)b * 32;
        float t = 0.f;
        if (kQ8) {
            for (int j = 0; j < 32; ++j) t = fmaf((float)(int8_t)p[j], xb[j], t);
        } else {
            for (int j = 0; j < 16; ++j) {
                t = fmaf((float)(int)(p[j] & 15) - 8.0f, xb[j], t);
                t = fmaf((float)(int)(p[j] >> 4) - 8.0f, xb[16 + j], t);
            }
        }
        acc = fmaf(d, t, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = accumulate ? y[row] + acc : acc;
}

// ---------------------------------------------------------------------------
// Exact dequantization: one thread per block.
// ---------------------------------------------------------------------------
template <bool kQ8>
__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                                           int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nblocks) return;
    const uint8_t* p = w + i * (kQ8 ? 34 : 18);
    const float d = __half2float(__ushort_as_half((unsigned short)(p[0] | (p[1] << 8))));
    float* o = out + i * 32;
    if (kQ8) {
        for (int j = 0; j < 32; ++j) o[j] = (float)(int8_t)p[2 + j] * d;
    } else {
        for (int j = 0; j < 16; ++j) {
            o[j] = ((float)(int)(p[2 + j] & 15) - 8.0f) * d;
            o[16 + j] = ((float)(int)(p[2 + j] >> 4) - 8.0f) * d;
        }
    }
}

// ---------------------------------------------------------------------------
// Q5_0: b = nibble | (fifth bit << 4), weight (b - 16) * d
// (src/kernels/x86_64/matmul_q5_avx2.asm:93-210, tests/reference/ops.py:67-92).
// ql byte j holds weight j (low nibble) and weight j + 16 (high nibble); bit j
// of the block's little-endian 32-bit qh word is weight j's fifth bit.
//
// Each weight becomes an exact float with one sign-extending byte conversion:
// the byte ((b ^ 16) << 3), i.e. the nibble in bits 3..6 and the inverted
// fifth bit in bit 7, reads as the signed value 8 (b - 16).  x is staged as
// x / 8 (exact), so each product 8 (b - 16) * (x / 8) is exactly (b - 16) * x.
// ---------------------------------------------------------------------------

// Bits [4g, 4g + 4) of h at bit 7 of bytes 0..3 (the other bits are junk):
// with t = those bits at [7, 11), t * (1 + 2^7 + 2^14 + 2^21) puts bit j of t
// at 8j + 7; the four shifted copies of t do not overlap, so nothing carries,
// and both factors fit the 24-bit multiplier.
__device__ __forceinline__ uint32_t q5_high_bits(uint32_t h, int g) {
    const int s = 4 * g - 7;
    const uint32_t t = (s >= 0 ? (h >> s) : (h << -s)) & 0x780u;
    return __umul24(t, 0x204081u);
}

// One block: q = its four ql words, nh = ~qh word, xb = x / 8 of its 32 columns.
__device__ __forceinline__ float q5_block(const uint32_t* q, uint32_t nh, const float* xb) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = opaque(((q[i] << 3) & 0x78787878u) | (q5_high_bits(nh, i) & 0x80808080u));
        const uint32_t hi = opaque(((q[i] >> 1) & 0x78787878u) | (q5_high_bits(nh, 4 + i) & 0x80808080u));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            t = fmaf(sbyte(lo, k), xb[4 * i + k], t);
            t = fmaf(sbyte(hi, k), xb[16 + 4 * i + k], t);
        }
    }
    return t;
}

// Q5_0 pair kernel (the mapping of the Q4_0 one).  kGguf: 22-byte blocks
// (fp16 d, qh[4], qs[16]); a pair is 44 bytes, so with K/32 even every pair
// starts on a dword and block A's fields sit two bytes off the dword grid.
// Otherwise the split layout: w = ql, wh = qh, wscale = fp32 scales.
template <int R, bool kGguf>
__global__ __launch_bounds__(kThreads) void q5_matvec_pairs(const uint8_t* __restrict__ w,
                                                            const uint8_t* __restrict__ wh,
                                                            const float* __restrict__ wscale,
                                                            const float* __restrict__ x,
                                                            float* __restrict__ y, int M, int K) {
    extern __shared__ float xs[];
    stage_x(x, xs, K, 0.125f, kPreNone, nullptr, 0.f);

    const int nb = K >> 5;
    const int np = nb >> 1;
    const uint32_t row_bytes = kGguf ? (uint32_t)nb * 22u : (uint32_t)nb * 16u;
    const auto wr = make_rsrc(w, row_bytes * (uint32_t)M);
    const auto hr = make_rsrc(wh, kGguf ? 0u : (uint32_t)nb * 4u * (uint32_t)M);
    const auto sr = make_rsrc(wscale, kGguf ? 0u : (uint32_t)nb * 4u * (uint32_t)M);
    const int lane = threadIdx.x & (kWave - 1);
    const int nwaves = gridDim.x * kWavesPerBlock;

    for (int g = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6); g * R < M; g += nwaves) {
        const int row0 = g * R;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;

        for (int c0 = 0; c0 < np; c0 += kWave) {
            const int p = c0 + lane;
            const bool active = p < np;
            const int pc = active ? p : np - 1;

            uint32_t v[R][11];
            float dA[R], dB[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = min(row0 + r, M - 1);
                if (kGguf) {
                    const uint32_t off = (uint32_t)row * row_bytes + (uint32_t)pc * 44u;
                    const uint4 a = buf_load_b128(wr, off);
                    const uint4 b = buf_load_b128(wr, off + 16u);
                    const uint2 c = buf_load_b64(wr, off + 32u);
                    v[r][0] = a.x; v[r][1] = a.y; v[r][2] = a.z; v[r][3] = a.w;
                    v[r][4] = b.x; v[r][5] = b.y; v[r][6] = b.z; v[r][7] = b.w;
                    v[r][8] = c.x; v[r][9] = c.y;
                    v[r][10] = buf_load_b32(wr, off + 40u);
                } else {
                    const uint32_t blk = (uint32_t)row * (uint32_t)nb + 2u * (uint32_t)pc;
                    const uint4 a = buf_load_b128(wr, blk * 16u);
                    const uint4 b = buf_load_b128(wr, blk * 16u + 16u);
                    const uint2 h = buf_load_b64(hr, blk * 4u);
                    const uint2 sc = buf_load_b64(sr, blk * 4u);
                    v[r][0] = a.x; v[r][1] = a.y; v[r][2] = a.z; v[r][3] = a.w;
                    v[r][4] = b.x; v[r][5] = b.y; v[r][6] = b.z; v[r][7] = b.w;
                    v[r][8] = h.x; v[r][9] = h.y;
                    dA[r] = __uint_as_float(sc.x);
                    dB[r] = __uint_as_float(sc.y);
                }
            }

            float xr[64];
            const float4* xq = reinterpret_cast<const float4*>(xs + xpad(pc * 64));
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const float4 t = xq[q];
                xr[4 * q] = t.x; xr[4 * q + 1] = t.y; xr[4 * q + 2] = t.z; xr[4 * q + 3] = t.w;
            }

#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t qa[4], qb[4], ha, hb;
                if (kGguf) {
                    // bytes: [0,2) dA, [2,6) qhA, [6,22) qsA, [22,24) dB, [24,28) qhB, [28,44) qsB
                    dA[r] = half_lo(v[r][0]);
                    dB[r] = half_hi(v[r][5]);
                    ha = __builtin_amdgcn_alignbyte(v[r][1], v[r][0], 2);
#pragma unroll
                    for (int i = 0; i < 4; ++i) qa[i] = __builtin_amdgcn_alignbyte(v[r][i + 2], v[r][i + 1], 2);
                    hb = v[r][6];
#pragma unroll
                    for (int i = 0; i < 4; ++i) qb[i] = v[r][7 + i];
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        qa[i] = v[r][i];
                        qb[i] = v[r][4 + i];
                    }
                    ha = v[r][8];
                    hb = v[r][9];
                }
                const float tA = q5_block(qa, ~ha, xr);
                const float tB = q5_block(qb, ~hb, xr + 32);
                float a = fmaf(dA[r], tA, acc[r]);
                a = fmaf(dB[r], tB, a);
                acc[r] = active ? a : acc[r];
            }
        }

#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = wave_sum(acc[r]);
            if (lane == r && row0 + r < M) y[row0 + r] = s;
        }
    }
}

// Generic Q5_0 kernel: one wave per row, one block per lane, byte loads (odd
// K/32, unaligned operands, x too large for LDS).
template <bool kGguf>
__global__ __launch_bounds__(kThreads) void q5_matvec_generic(const uint8_t* __restrict__ w,
                                                              const uint8_t* __restrict__ wh,
                                                              const float* __restrict__ wscale,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ y, int M, int K) {
    const int nb = K >> 5;
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (row >= M) return;
    float acc = 0.f;
    for (int b = lane; b < nb; b += kWave) {
        const int64_t blk = (int64_t)row * nb + b;
        const uint8_t* qs;
        const uint8_t* qh;
        float d;
        if (kGguf) {
            const uint8_t* p = w + blk * 22;
            d = __half2float(__ushort_as_half((unsigned short)(p[0] | (p[1] << 8))));
            qh = p + 2;
            qs = p + 6;
        } else {
            d = wscale[blk];
            qh = wh + blk * 4;
            qs = w + blk * 16;
        }
        const uint32_t h = (uint32_t)qh[0] | ((uint32_t)qh[1] << 8) | ((uint32_t)qh[2] << 16) | ((uint32_t)qh[3] << 24);
        const float* xb = x + (int64_t)b * 32;
        float t = 0.f;
        for (int j = 0; j < 16; ++j) {
            const int lo = (qs[j] & 15) | (int)(((h >> j) & 1u) << 4);
            const int hi = (qs[j] >> 4) | (int)(((h >> (j + 16)) & 1u) << 4);
            t = fmaf((float)(lo - 16), xb[j], t);
            t = fmaf((float)(hi - 16), xb[16 + j], t);
        }
        acc = fmaf(d, t, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

// Exact dequantization of GGUF Q5_0 blocks: one thread per block.
__global__ __launch_bounds__(kThreads) void q5_dequant_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                                              int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nblocks) return;
    const uint8_t* p = w + i * 22;
    const float d = __half2float(__ushort_as_half((unsigned short)(p[0] | (p[1] << 8))));
    const uint32_t h = (uint32_t)p[2] | ((uint32_t)p[3] << 8) | ((uint32_t)p[4] << 16) | ((uint32_t)p[5] << 24);
    float* o = out + i * 32;
    for (int j = 0; j < 16; ++j) {
        const int lo = (p[6 + j] & 15) | (int)(((h >> j) & 1u) << 4);
        const int hi = (p[6 + j] >> 4) | (int)(((h >> (j + 16)) & 1u) << 4);
        o[j] = (float)(lo - 16) * d;
        o[16 + j] = (float)(hi - 16) * d;
    }
}

size_t pair_lds_bytes(int64_t K) { return (size_t)(K + K / 16) * sizeof(float); }

int pick_rows_per_wave(int64_t M, int r_max) {
    // Aim for at least ~8 waves per CU across 256 CUs before growing R.
    int r = r_max;
    while (r > 1 && (M + r - 1) / r < 2048) r >>= 1;
    return r;
}

template <int R, bool kGguf>
int launch_q4(const uint8_t* w, const float* s, const float* x, float* y, int M, int K, size_t lds,
               hipStream_t st, const MatvecOpts& o) {
    const int rc = dynamic_lds((const void*)q4_matvec_pairs<R, kGguf>, lds);
    if (rc) return rc;
    const int64_t groups = (M + R - 1) / R;
    const int blocks = (int)((groups + kWavesPerBlock - 1) / kWavesPerBlock);
    hipLaunchKernelGGL((q4_matvec_pairs<R, kGguf>), dim3(blocks), dim3(kThreads), lds, st, w, s, x, y, M, K, o.pre,
                       o.pre_arg, o.eps, (int)o.accumulate);
    return kOk;
}

template <int R, bool kGguf>
int launch_q8(const uint8_t* w, const float* s, const float* x, float* y, int M, int K, size_t lds,
               hipStream_t st, const MatvecOpts& o) {
    const int rc = dynamic_lds((const void*)q8_matvec_pairs<R, kGguf>, lds);
    if (rc) return rc;
    const int64_t groups = (M + R - 1) / R;
    const int blocks = (int)((groups + kWavesPerBlock - 1) / kWavesPerBlock);
    hipLaunchKernelGGL((q8_matvec_pairs<R, kGguf>), dim3(blocks), dim3(kThreads), lds, st, w, s, x, y, M, K, o.pre,
                       o.pre_arg, o.eps, (int)o.accumulate);
    return kOk;
}

template <int R, bool kGguf>
int launch_q5(const uint8_t* w, const uint8_t* h, const float* s, const float* x, float* y, int M, int K, size_t lds,
              hipStream_t st) {
    const int rc = dynamic_lds((const void*)q5_matvec_pairs<R, kGguf>, lds);
    if (rc) return rc;
    const int64_t groups = (M + R - 1) / R;
    const int blocks = (int)((groups + kWavesPerBlock - 1) / kWavesPerBlock);
    hipLaunchKernelGGL((q5_matvec_pairs<R, kGguf>), dim3(blocks), dim3(kThreads), lds, st, w, h, s, x, y, M, K);
    return kOk;
}

std::atomic<int> g_q4_kernel{kQ4KernelAuto};

}  // namespace

int set_q4_kernel(int kernel) {
    if (kernel < kQ4KernelAuto || kernel > kQ4KernelMfma)
        return fail(kInvalidArgument, "unknown Q4_0 matvec kernel selector %d", kernel);
    g_q4_kernel.store(kernel);
    return kOk;
}

int get_q4_kernel() { return g_q4_kernel.load(); }

int matvec_launch(QuantType qt, bool gguf, const void* w, const float* scales, const float* x, float* y,
                  int64_t M, int64_t K, hipStream_t stream, const MatvecOpts& opts) {
    if (M <= 0 || K <= 0 || (K % 32) != 0)
        return fail(kInvalidArgument, "matvec: need M > 0, K > 0 and K %% 32 == 0 (got M=%lld K=%lld)",
                    (long long)M, (long long)K);
    if (M > INT32_MAX || K > INT32_MAX) return fail(kInvalidArgument, "matvec: M and K must fit in int32");
    if (opts.pre != kPreNone && !opts.pre_arg) return fail(kInvalidArgument, "matvec: pre-op without its argument");
    if (opts.pre < kPreNone || opts.pre > kPreSwiGlu) return fail(kInvalidArgument, "matvec: unknown pre-op %d", opts.pre);
    if (opts.post != kPostNone) return fail(kInvalidArgument, "matvec: post-ops go through matvec_swiglu_launch");
    const int64_t nb = K / 32;
    const int64_t blk_bytes = qt == QuantType::Q4_0 ? (gguf ? 18 : 16) : (gguf ? 34 : 32);
    const int64_t total = M * nb * blk_bytes;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const size_t lds = pair_lds_bytes(K);
    const bool aligned = ((uintptr_t)w % 4 == 0) && (!gguf || nb % 2 == 0) && ((uintptr_t)scales % 8 == 0) &&
                         ((uintptr_t)x % 4 == 0);
    const bool pairs = nb % 2 == 0 && aligned && lds <= 160 * 1024 - 256 && total < (int64_t)UINT32_MAX;
    const int m = (int)M, k = (int)K;

    int rc = kOk;

    const int sel = g_q4_kernel.load(std::memory_order_relaxed);
    if (qt == QuantType::Q4_0 && gguf) {
        const bool mfma_ok = q4_0_mfma_eligible(w, x, opts, M, K);
        if (sel == kQ4KernelMfma && !mfma_ok)
            return fail(kUnsupported, "matvec: the MFMA Q4_0 kernel needs K %% 256 == 0, K <= 16384, "
                                      "4-byte aligned blocks and 16-byte aligned x (got M=%lld K=%lld)",
                        (long long)M, (long long)K);
        if (sel != kQ4KernelFp32 && mfma_ok) return q4_0_mfma_launch(w, x, y, M, K, stream, opts);
    }
    if (qt == QuantType::Q4_0 && !gguf && opts.pre == kPreNone && !opts.accumulate &&
        g_q4_kernel.load(std::memory_order_relaxed) != kQ4KernelFp32 &&
        split_mfma_eligible(4, w, nullptr, scales, x, M, K))
        return split_mfma_launch(4, w, nullptr, scales, x, y, M, K, stream);
    if (qt == QuantType::Q8_0 && sel != kQ4KernelFp32) {
        if (gguf && q8_0_mfma_eligible(w, x, opts, M, K)) return q8_0_mfma_launch(w, x, y, M, K, stream, opts);
        if (!gguf && opts.pre == kPreNone && !opts.accumulate && split_mfma_eligible(8, w, nullptr, scales, x, M, K))
            return split_mfma_launch(8, w, nullptr, scales, x, y, M, K, stream);
    }
    if (pairs && qt == QuantType::Q4_0) {
        const int r = pick_rows_per_wave(M, 8);
        if (gguf) {
            switch (r) {
                case 8: rc = launch_q4<8, true>(wb, scales, x, y, m, k, lds, stream, opts); break;
                case 4: rc = launch_q4<4, true>(wb, scales, x, y, m, k, lds, stream, opts); break;
                case 2: rc = launch_q4<2, true>(wb, scales, x, y, m, k, lds, stream, opts); break;
                default: rc = launch_q4<1, true>(wb, scales, x, y, m, k, lds, stream, opts); break;
            }
        } else {
            switch (r) {
                case 8: rc = launch_q4<8, false>(wb, scales, x, y, m, k, lds, stream, opts); break;
                case 4: rc = launch_q4<4, false>(wb, scales, x, y, m, k, lds, stream, opts); break;
                case 2: rc = launch_q4<2, false>(wb, scales, x, y, m, k, lds, stream, opts); break;
                default: rc = launch_q4<1, false>(wb, scales, x, y, m, k, lds, stream, opts); break;
            }
        }
    } else if (pairs) {
        const int r = pick_rows_per_wave(M, 4);
        if (gguf) {
            switch (r) {
                case 4: rc = launch_q8<4, true>(wb, scales, x, y, m, k, lds, stream, opts); break;
                case 2: rc = launch_q8<2, true>(wb, scales, x, y, m, k, lds, stream, opts); break;
                default: rc = launch_q8<1, true>(wb, scales, x, y, m, k, lds, stream, opts); break;
            }
        } else {
            switch (r) {
                case 4: rc = launch_q8<4, false>(wb, scales, x, y, m, k, lds, stream, opts); break;
                case 2: rc = launch_q8<2, false>(wb, scales, x, y, m, k, lds, stream, opts); break;
                default: rc = launch_q8<1, false>(wb, scales, x, y, m, k, lds, stream, opts); break;
            }
        }
    } else {
        if (opts.pre != kPreNone)
            return fail(kUnsupported, "matvec: fused pre-ops need K %% 64 == 0, dword-aligned rows and K <= 37000");
        const int blocks = (int)((M + kWavesPerBlock - 1) / kWavesPerBlock);
        const int acc = (int)opts.accumulate;
        if (qt == QuantType::Q4_0) {
            if (gguf)
                hipLaunchKernelGGL((matvec_generic<false, true>), dim3(blocks), dim3(kThreads), 0, stream, wb, scales, x, y, m, k, acc);
            else
                hipLaunchKernelGGL((matvec_generic<false, false>), dim3(blocks), dim3(kThreads), 0, stream, wb, scales, x, y, m, k, acc);
        } else {
            if (gguf)
                hipLaunchKernelGGL((matvec_generic<true, true>), dim3(blocks), dim3(kThreads), 0, stream, wb, scales, x, y, m, k, acc);
            else
                hipLaunchKernelGGL((matvec_generic<true, false>), dim3(blocks), dim3(kThreads), 0, stream, wb, scales, x, y, m, k, acc);
        }
    }
    if (rc) return rc;
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int dequant_launch(QuantType qt, const void* w, float* out, int64_t rows, int64_t K, hipStream_t stream) {
    if (rows <= 0 || K <= 0 || (K % 32) != 0)
        return fail(kInvalidArgument, "dequantize: need rows > 0, K > 0 and K %% 32 == 0");
    const int64_t nblocks = rows * (K / 32);
    const int64_t grid = (nblocks + kThreads - 1) / kThreads;
    if (grid > INT32_MAX) return fail(kInvalidArgument, "dequantize: tensor too large");
    if (qt == QuantType::Q4_0)
        hipLaunchKernelGGL((dequant_kernel<false>), dim3((unsigned)grid), dim3(kThreads), 0, stream,
                           static_cast<const uint8_t*>(w), out, nblocks);
    else
        hipLaunchKernelGGL((dequant_kernel<true>), dim3((unsigned)grid), dim3(kThreads), 0, stream,
                           static_cast<const uint8_t*>(w), out, nblocks);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int matvec_swiglu_launch(QuantType qt, const void* w, const float* x, float* h, int64_t H, int64_t K, float* work,
                         hipStream_t stream, const MatvecOpts& opts) {
    if (H <= 0 || H % 8 || H > INT32_MAX / 4)
        return fail(kInvalidArgument, "matvec_swiglu: need H > 0 and H %% 8 == 0 (got H=%lld)", (long long)H);
    if (opts.accumulate || opts.post != kPostNone)
        return fail(kInvalidArgument, "matvec_swiglu: the output is overwritten, no other post-op");
    if (!work) return fail(kInvalidArgument, "matvec_swiglu: null work buffer");
    MatvecOpts po = opts;
    po.post = kPostSwiGlu8;
    const int64_t M = 2 * H;
    const int sel = g_q4_kernel.load(std::memory_order_relaxed);
    if (sel != kQ4KernelFp32) {
        if (qt == QuantType::Q4_0 && q4_0_mfma_eligible(w, x, po, M, K)) return q4_0_mfma_launch(w, x, h, M, K, stream, po);
        if (qt == QuantType::Q8_0 && q8_0_mfma_eligible(w, x, po, M, K)) return q8_0_mfma_launch(w, x, h, M, K, stream, po);
    }
    // any other shape or kernel: the 2H rows to `work`, then the pairs combined
    const int rc = matvec_launch(qt, true, w, nullptr, x, work, M, K, stream, opts);
    return rc ? rc : swiglu_pairs_launch(work, h, H, stream);
}

int q5_matvec_launch(bool gguf, const void* w, const uint8_t* qh, const float* scales, const float* x, float* y,
                     int64_t M, int64_t K, hipStream_t stream) {
    if (M <= 0 || K <= 0 || (K % 32) != 0)
        return fail(kInvalidArgument, "matvec_q5: need M > 0, K > 0 and K %% 32 == 0 (got M=%lld K=%lld)",
                    (long long)M, (long long)K);
    if (M > INT32_MAX || K > INT32_MAX) return fail(kInvalidArgument, "matvec_q5: M and K must fit in int32");
    const int64_t nb = K / 32;
    const int64_t total = M * nb * (gguf ? 22 : 16);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const size_t lds = pair_lds_bytes(K);
    const bool aligned = ((uintptr_t)w % 4 == 0) && ((uintptr_t)x % 4 == 0) &&
                         (gguf || ((uintptr_t)qh % 8 == 0 && (uintptr_t)scales % 8 == 0));
    const bool pairs = nb % 2 == 0 && aligned && lds <= 160 * 1024 - 256 && total < (int64_t)UINT32_MAX;
    const int m = (int)M, k = (int)K;
    int rc = kOk;
    const int sel = g_q4_kernel.load(std::memory_order_relaxed);
    const bool mfma = sel != kQ4KernelFp32;
    if (mfma && gguf && q5_0_mfma_eligible(w, x, M, K)) return q5_0_mfma_launch(w, x, y, M, K, stream);
    if (mfma && !gguf && split_mfma_eligible(5, w, qh, scales, x, M, K))
        return split_mfma_launch(5, w, qh, scales, x, y, M, K, stream);
    if (pairs) {
        const int r = pick_rows_per_wave(M, 4);
        if (gguf) {
            switch (r) {
                case 4: rc = launch_q5<4, true>(wb, qh, scales, x, y, m, k, lds, stream); break;
                case 2: rc = launch_q5<2, true>(wb, qh, scales, x, y, m, k, lds, stream); break;
                default: rc = launch_q5<1, true>(wb, qh, scales, x, y, m, k, lds, stream); break;
            }
        } else {
            switch (r) {
                case 4: rc = launch_q5<4, false>(wb, qh, scales, x, y, m, k, lds, stream); break;
                case 2: rc = launch_q5<2, false>(wb, qh, scales, x, y, m, k, lds, stream); break;
                default: rc = launch_q5<1, false>(wb, qh, scales, x, y, m, k, lds, stream); break;
            }
        }
    } else {
        const int blocks = (int)((M + kWavesPerBlock - 1) / kWavesPerBlock);
        if (gguf)
            hipLaunchKernelGGL((q5_matvec_generic<true>), dim3(blocks), dim3(kThreads), 0, stream, wb, qh, scales, x, y, m, k);
        else
            hipLaunchKernelGGL((q5_matvec_generic<false>), dim3(blocks), dim3(kThreads), 0, stream, wb, qh, scales, x, y, m, k);
    }
    if (rc) return rc;
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int q5_dequant_launch(const void* w, float* out, int64_t rows, int64_t K, hipStream_t stream) {
    if (rows <= 0 || K <= 0 || (K % 32) != 0)
        return fail(kInvalidArgument, "dequantize: need rows > 0, K > 0 and K %% 32 == 0");
    const int64_t nblocks = rows * (K / 32);
    const int64_t grid = (nblocks + kThreads - 1) / kThreads;
    if (grid > INT32_MAX) return fail(kInvalidArgument, "dequantize: tensor too large");
    hipLaunchKernelGGL(q5_dequant_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream,
                       static_cast<const uint8_t*>(w), out, nblocks);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

}  // namespace asmhip
