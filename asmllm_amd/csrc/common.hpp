// Shared helpers for the gfx950 kernels and the C-ABI layer.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asmhip {

// Status codes returned by every asmhip_* entry point.
enum Status : int {
    kOk = 0,
    kInvalidArgument = -1,
    kHipError = -2,
    kUnsupported = -3,
    kNoDevice = -4,
};

// Records a formatted message as the calling thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);

// Raises `kernel`'s dynamic-LDS limit to at least `bytes` on the current
// device (launches above 64 KB need it).  Granted sizes are cached per kernel
// and device, so the hot path pays one lookup.
int dynamic_lds(const void* kernel, size_t bytes);

#define ASMHIP_TRY(expr)                                   \
    do {                                                   \
        hipError_t _e = (expr);                            \
        if (_e != hipSuccess) return ::asmhip::hip_fail(_e, #expr); \
    } while (0)

constexpr int kWave = 64;

// Buffer resource over [base, base + bytes).  Out-of-range buffer loads
// return zero instead of faulting; every kernel still keeps its offsets in
// range, the descriptor bound is a second line of defence.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    // Word 3 (0x00020000): DATA_FORMAT=32 for raw dword access on gfx9.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// Streaming variant: the nontemporal hint keeps read-once weights from
// displacing reused lines in the caches.
__device__ __forceinline__ uint4 buf_load_b128_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ uint2 buf_load_b64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
    return make_uint2(v[0], v[1]);
}

__device__ __forceinline__ uint32_t buf_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

__device__ __forceinline__ uint32_t buf_load_b32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

// Byte k of v as float (one v_cvt_f32_ubyte{k}).
template <int k>
__device__ __forceinline__ float ubyte(uint32_t v) {
    return (float)((v >> (8 * k)) & 0xFFu);
}

__device__ __forceinline__ float half_lo(uint32_t v) {
    return __half2float(__ushort_as_half((unsigned short)(v & 0xFFFFu)));
}
__device__ __forceinline__ float half_hi(uint32_t v) {
    return __half2float(__ushort_as_half((unsigned short)(v >> 16)));
}

// Sum over the 64 lanes of a wave; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// DPP controls: quad_perm [1,0,3,2] and [2,3,0,1] (lanes ^1 and ^2 within a
// quad), row_half_mirror, row_mirror.
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppRowHalfMirror = 0x141, kDppRowMirror = 0x140;

// Sum over the 64 lanes of a wave without LDS: each 16-lane row is summed
// with DPP adds (every lane of a row gets its row's sum), then the four row
// sums are added in row order, ((r0 + r1) + r2) + r3, a wave-uniform value.
__device__ __forceinline__ float wave_total_dpp(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kDppQuadXor1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kDppQuadXor2, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kDppRowHalfMirror, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kDppRowMirror, 0xF, 0xF, false));
    const int b = __float_as_int(v);
    return ((__int_as_float(__builtin_amdgcn_readlane(b, 0)) + __int_as_float(__builtin_amdgcn_readlane(b, 16))) +
            __int_as_float(__builtin_amdgcn_readlane(b, 32))) +
           __int_as_float(__builtin_amdgcn_readlane(b, 48));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Softmax merge of the S split states of one attention head, dimension t:
// state s is [m, l, -, -, acc[hd]] at ph + s * stride; the result is
// (sum_s acc_s[t] f_s) / (sum_s l_s f_s) with f_s = exp(m_s - max_s m_s), both
// sums in split order; 0 when no split saw a position (every m = -inf).
__device__ __forceinline__ float attn_merge_value(const float* ph, int S, int stride, int t) {
    float M = -INFINITY;
    for (int i = 0; i < S; ++i) M = fmaxf(M, ph[(size_t)i * stride]);
    float L = 0.f, a = 0.f;
    if (M != -INFINITY) {
        for (int i = 0; i < S; ++i) {
            const float f = __expf(ph[(size_t)i * stride] - M);
            L = fmaf(ph[(size_t)i * stride + 1], f, L);
            a = fmaf(ph[(size_t)i * stride + 4 + t], f, a);
        }
    }
    return M == -INFINITY ? 0.f : a / L;
}

// attn_merge_value for the dimensions t..t+3 and t+16..t+19 of one head (t % 4
// == 0, stride % 4 == 0, ph 16-byte aligned) over exactly S splits, bit for bit
// the same values, in two steps: load() requests every state with
// unconditional loads (so the wait before finish() counts them exactly),
// finish() forms the values once they are in.
template <int S>
struct AttnMergeQuads {
    float2 ml[S];
    float4 ac[S][2];

    __device__ __forceinline__ void load(const float* ph, int stride, int t) {
#pragma unroll
        for (int i = 0; i < S; ++i) {
            const float* e = ph + (size_t)i * stride;
            ml[i] = *reinterpret_cast<const float2*>(e);
            ac[i][0] = *reinterpret_cast<const float4*>(e + 4 + t);
            ac[i][1] = *reinterpret_cast<const float4*>(e + 20 + t);
        }
    }
    // the acc values only (the caller fills ml)
    __device__ __forceinline__ void load_acc(const float* ph, int stride, int t) {
#pragma unroll
        for (int i = 0; i < S; ++i) {
            const float* e = ph + (size_t)i * stride;
            ac[i][0] = *reinterpret_cast<const float4*>(e + 4 + t);
            ac[i][1] = *reinterpret_cast<const float4*>(e + 20 + t);
        }
    }

    __device__ __forceinline__ void finish(float4* lo, float4* hi) const {
        float M = -INFINITY;
#pragma unroll
        for (int i = 0; i < S; ++i) M = fmaxf(M, ml[i].x);
        float L = 0.f;
        float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (M != -INFINITY) {
#pragma unroll
            for (int i = 0; i < S; ++i) {
                const float f = __expf(ml[i].x - M);
                L = fmaf(ml[i].y, f, L);
                const float v[8] = {ac[i][0].x, ac[i][0].y, ac[i][0].z, ac[i][0].w,
                                    ac[i][1].x, ac[i][1].y, ac[i][1].z, ac[i][1].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) a[j] = fmaf(v[j], f, a[j]);
            }
        }
        float r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = M == -INFINITY ? 0.f : a[j] / L;
        *lo = make_float4(r[0], r[1], r[2], r[3]);
        *hi = make_float4(r[4], r[5], r[6], r[7]);
    }
};

}  // namespace asmhip
