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

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

}  // namespace asmhip
