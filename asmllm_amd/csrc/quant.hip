// GGUF block quantizers and synthetic-weight generators for gfx950.
//
// quantize: fp32 rows -> Q4_0 / Q8_0 blocks with the same rules, bit for bit,
// as the host quantizers (asmllm_amd/gguf.py):
//   Q4_0: d = m / -8 (m the first element of largest magnitude), id = 1/d,
//         q = min(15, trunc(w*id + 8.5)), d stored as fp16 (RNE);
//   Q8_0: d = amax / 127, inv = 127 / amax (0 if amax == 0),
//         q = saturate(rint(w*inv)) -- the reference's activation quantizer,
//         src/kernels/arm64/matmul_q4_neon.S:80-135.
// Every step is a separately rounded IEEE operation (contraction is off).
//
// random: one thread per block draws 32 N(0, stddev^2) values from a
// counter-based generator (splitmix64 of seed and element index, Box-Muller)
// and quantizes them in registers, so multi-GB synthetic models are produced
// in HBM without a host round trip.
#include "common.hpp"
#include "kernels.hpp"

namespace asmhip {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ void quant_q4_block(const float* v, uint8_t* out) {
#pragma clang fp contract(off)  // w * id and + 8.5 are two roundings, as on the host
    // (plain operators: the _rn intrinsics come from a header compiled with
    // contraction on, and their products would still fuse)
    float amax = 0.f, mx = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float a = fabsf(v[j]);
        if (a > amax) {
            amax = a;
            mx = v[j];
        }
    }
    float d = mx / -8.0f;
    // Kept opaque so that the product is not folded into an fma with a +0
    // addend on its way to fp16, which would turn d = -0 (an all-zero block)
    // into +0.
    asm volatile("" : "+v"(d));
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const unsigned short dh = __half_as_ushort(__float2half_rn(d));
    out[0] = (uint8_t)(dh & 0xFF);
    out[1] = (uint8_t)(dh >> 8);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        int q0 = (int)(v[j] * id + 8.5f);
        int q1 = (int)(v[16 + j] * id + 8.5f);
        q0 = min(q0, 15);
        q1 = min(q1, 15);
        out[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

// The Q8_0 rules for one block: the 32 quants into q, the fp16 d's bits returned.
__device__ __forceinline__ unsigned short quant_q8_values(const float* v, int8_t* q) {
#pragma clang fp contract(off)
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f;
    const float inv = amax == 0.0f ? 0.0f : 127.0f / amax;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        float r = rintf(v[j] * inv);
        r = fminf(fmaxf(r, -128.0f), 127.0f);
        q[j] = (int8_t)(int)r;
    }
    return __half_as_ushort(__float2half_rn(d));
}

__device__ __forceinline__ void quant_q8_block(const float* v, uint8_t* out) {
    int8_t q[32];
    const unsigned short dh = quant_q8_values(v, q);
    out[0] = (uint8_t)(dh & 0xFF);
    out[1] = (uint8_t)(dh >> 8);
#pragma unroll
    for (int j = 0; j < 32; ++j) out[2 + j] = (uint8_t)q[j];
}

template <bool kQ8>
__global__ __launch_bounds__(kThreads) void quantize_kernel(const float* __restrict__ w, uint8_t* __restrict__ out,
                                                            int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nblocks) return;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = w[i * 32 + j];
    if (kQ8)
        quant_q8_block(v, out + i * 34);
    else
        quant_q4_block(v, out + i * 18);
}

// The same Q8_0 blocks written in the GEMM tile layout of activations
// (gemm_tiled_offset with kGemmTileA-row tiles); padding rows are not written.
__global__ __launch_bounds__(kThreads) void quantize_q8_tiled_kernel(const float* __restrict__ w,
                                                                     uint8_t* __restrict__ out, int64_t nblocks,
                                                                     int64_t nb) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nblocks) return;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = w[i * 32 + j];
    quant_q8_block(v, out + gemm_tiled_offset(i / nb, i % nb, nb, kGemmTileA));
}

// The split layout of the same blocks: qs[i] = the 32 quants of block i
// (16-byte aligned), scales[i] = its fp16 d widened to fp32.
__global__ __launch_bounds__(kThreads) void quantize_q8_split_kernel(const float* __restrict__ w, int8_t* __restrict__ qs,
                                                                     float* __restrict__ scales, int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nblocks) return;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = w[i * 32 + j];
    union {
        int8_t b[32];
        uint4 u[2];
    } q;
    const unsigned short dh = quant_q8_values(v, q.b);
    uint4* dst = reinterpret_cast<uint4*>(qs + i * 32);
    dst[0] = q.u[0];
    dst[1] = q.u[1];
    scales[i] = __half2float(__ushort_as_half(dh));
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Two N(0,1) values for element pair `idx` of stream `seed`.
__device__ __forceinline__ void normal_pair(uint64_t seed, uint64_t idx, float* a, float* b) {
    const uint64_t r = splitmix64(seed ^ splitmix64(idx));
    const float u1 = ((float)(uint32_t)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = (float)(uint32_t)((r >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
    const float rad = sqrtf(-2.0f * logf(u1));
    float s, c;
    sincosf(6.283185307179586f * u2, &s, &c);
    *a = rad * c;
    *b = rad * s;
}

template <bool kQ8>
__global__ __launch_bounds__(kThreads) void random_blocks_kernel(uint8_t* __restrict__ out, int64_t nblocks,
                                                                 uint64_t seed, float stddev) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nblocks) return;
    float v[32];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        normal_pair(seed, (uint64_t)i * 16 + j, &v[2 * j], &v[2 * j + 1]);
        v[2 * j] *= stddev;
        v[2 * j + 1] *= stddev;
    }
    if (kQ8)
        quant_q8_block(v, out + i * 34);
    else
        quant_q4_block(v, out + i * 18);
}

__global__ __launch_bounds__(kThreads) void random_f16_kernel(__half* __restrict__ out, int64_t n, uint64_t seed,
                                                              float stddev) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (2 * i >= n) return;
    float a, b;
    normal_pair(seed, (uint64_t)i, &a, &b);
    out[2 * i] = __float2half_rn(a * stddev);
    if (2 * i + 1 < n) out[2 * i + 1] = __float2half_rn(b * stddev);
}

__global__ __launch_bounds__(kThreads) void fill_f32_kernel(float* __restrict__ out, int64_t n, float value) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) out[i] = value;
}

int64_t grid_for(int64_t n) { return (n + kThreads - 1) / kThreads; }

}  // namespace

int quantize_launch(QuantType qt, const float* w, void* blocks, int64_t rows, int64_t K, hipStream_t st) {
    if (rows <= 0 || K <= 0 || K % 32) return fail(kInvalidArgument, "quantize: need rows > 0 and K %% 32 == 0");
    const int64_t nb = rows * (K / 32);
    if (grid_for(nb) > INT32_MAX) return fail(kInvalidArgument, "quantize: tensor too large");
    if (qt == QuantType::Q4_0)
        hipLaunchKernelGGL((quantize_kernel<false>), dim3((unsigned)grid_for(nb)), dim3(kThreads), 0, st, w,
                           (uint8_t*)blocks, nb);
    else
        hipLaunchKernelGGL((quantize_kernel<true>), dim3((unsigned)grid_for(nb)), dim3(kThreads), 0, st, w,
                           (uint8_t*)blocks, nb);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int quantize_q8_split_launch(const float* w, int8_t* qs, float* scales, int64_t rows, int64_t K, hipStream_t st) {
    if (rows <= 0 || K <= 0 || K % 32) return fail(kInvalidArgument, "quantize_q8_split: need rows > 0 and K %% 32 == 0");
    if ((uintptr_t)qs % 16) return fail(kInvalidArgument, "quantize_q8_split: qs must be 16-byte aligned");
    const int64_t nb = rows * (K / 32);
    if (grid_for(nb) > INT32_MAX) return fail(kInvalidArgument, "quantize_q8_split: tensor too large");
    hipLaunchKernelGGL(quantize_q8_split_kernel, dim3((unsigned)grid_for(nb)), dim3(kThreads), 0, st, w, qs, scales, nb);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int quantize_q8_0_tiled_launch(const float* x, void* tiled, int64_t rows, int64_t K, hipStream_t st) {
    if (rows <= 0 || K <= 0 || K % 64) return fail(kInvalidArgument, "quantize_q8_0_tiled: need rows > 0 and K %% 64 == 0");
    if (!x || !tiled) return fail(kInvalidArgument, "quantize_q8_0_tiled: null pointer");
    const int64_t nb = rows * (K / 32);
    if (grid_for(nb) > INT32_MAX) return fail(kInvalidArgument, "quantize_q8_0_tiled: tensor too large");
    hipLaunchKernelGGL(quantize_q8_tiled_kernel, dim3((unsigned)grid_for(nb)), dim3(kThreads), 0, st, x,
                       (uint8_t*)tiled, nb, K / 32);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int random_blocks_launch(QuantType qt, void* blocks, int64_t rows, int64_t K, uint64_t seed, float stddev,
                         hipStream_t st) {
    if (rows <= 0 || K <= 0 || K % 32) return fail(kInvalidArgument, "random blocks: need rows > 0 and K %% 32 == 0");
    const int64_t nb = rows * (K / 32);
    if (grid_for(nb) > INT32_MAX) return fail(kInvalidArgument, "random blocks: tensor too large");
    if (qt == QuantType::Q4_0)
        hipLaunchKernelGGL((random_blocks_kernel<false>), dim3((unsigned)grid_for(nb)), dim3(kThreads), 0, st,
                           (uint8_t*)blocks, nb, seed, stddev);
    else
        hipLaunchKernelGGL((random_blocks_kernel<true>), dim3((unsigned)grid_for(nb)), dim3(kThreads), 0, st,
                           (uint8_t*)blocks, nb, seed, stddev);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int random_f16_launch(void* out, int64_t n, uint64_t seed, float stddev, hipStream_t st) {
    if (n <= 0) return fail(kInvalidArgument, "random f16: n must be > 0");
    const int64_t pairs = (n + 1) / 2;
    if (grid_for(pairs) > INT32_MAX) return fail(kInvalidArgument, "random f16: too large");
    hipLaunchKernelGGL(random_f16_kernel, dim3((unsigned)grid_for(pairs)), dim3(kThreads), 0, st, (__half*)out, n,
                       seed, stddev);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int fill_f32_launch(float* out, int64_t n, float value, hipStream_t st) {
    if (n <= 0) return fail(kInvalidArgument, "fill: n must be > 0");
    if (grid_for(n) > INT32_MAX) return fail(kInvalidArgument, "fill: too large");
    hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, st, out, n, value);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

}  // namespace asmhip
