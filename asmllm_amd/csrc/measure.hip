// Measurement kernels: a plain streaming read of a buffer in one launch, the
// same read in the shape of a matvec launch, an empty launch, and a grid-wide
// barrier inside one persistent launch.
//
// The matvec reads M (K/32) block bytes once per launch; how fast any kernel
// can read that many bytes in ONE launch on this part (launch ramp, first-load
// latency and drain included) bounds what the matvec can reach, below the HBM
// spec peak.  This kernel is that bound: every workgroup reads one contiguous
// chunk of at most 25 x 4 KB with all of its 16-byte loads issued before any
// result is used (nontemporal, the fastest read shape measured on gfx950), and
// keeps nothing.  bench.py times it at several sizes next to the matvec.
#include "common.hpp"
#include "kernels.hpp"

namespace asmhip {

namespace {

constexpr int kReadThreads = 256;
constexpr int kReadLoads = 25;  // 16-byte loads per lane: 100 KB per workgroup

__global__ __launch_bounds__(kReadThreads) void stream_read_kernel(const uint8_t* __restrict__ p, uint32_t bytes,
                                                                   uint32_t per_wg, uint32_t* __restrict__ sink) {
    const auto r = make_rsrc(p, bytes);
    const uint32_t lo = blockIdx.x * per_wg, hi = min(lo + per_wg, bytes);
    uint4 v[kReadLoads];
#pragma unroll
    for (int u = 0; u < kReadLoads; ++u) {
        const uint32_t off = lo + ((uint32_t)u * kReadThreads + threadIdx.x) * 16u;
        v[u] = buf_load_b128_nt(r, off < hi ? off : 0xFFFFFF00u);  // past the chunk: zeros, no memory access
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < kReadLoads; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x9E3779B9u) sink[blockIdx.x & 1023] = acc;  // keeps the loads; practically never stores
}

// The read above in the shape of the matvec launch (one workgroup of 1024
// threads per compute unit, every load of the chunk issued up front), with the
// matvec's structural pieces switched on one at a time by `flags`:
//   kShapeLds    the matvec's dynamic LDS allocation (`lds` bytes, untouched);
//   kShapeX      x (`xn` floats, 16-byte aligned) read first and a workgroup barrier
//                before the chunk's loads, as the matvec stages x;
//   kShapeStore  16 floats per workgroup stored at the end, as the matvec writes y.
constexpr int kShapeLds = 1, kShapeX = 2, kShapeStore = 4;
constexpr int kShapeThreads = 1024;
constexpr int kShapeLoads = 8;  // 16-byte loads per lane: 128 KB per workgroup

__global__ __launch_bounds__(kShapeThreads) void shaped_read_kernel(const uint8_t* __restrict__ p, uint32_t bytes,
                                                                    uint32_t per_wg, const float* __restrict__ x,
                                                                    int xn, float* __restrict__ y, int flags,
                                                                    uint32_t* __restrict__ sink) {
    extern __shared__ float lds_f[];
    __shared__ float red[kShapeThreads / 64];
    float xs = 0.f;
    if (flags & kShapeX) {
        for (int i = threadIdx.x * 4; i < xn; i += kShapeThreads * 4) {
            const float4 v = *reinterpret_cast<const float4*>(x + i);
            xs += v.x + v.y + v.z + v.w;
        }
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = xs;
        __syncthreads();
        xs = red[(threadIdx.x >> 6) ^ 1];
    }
    const auto r = make_rsrc(p, bytes);
    const uint32_t lo = blockIdx.x * per_wg, hi = min(lo + per_wg, bytes);
    uint4 v[kShapeLoads];
#pragma unroll
    for (int u = 0; u < kShapeLoads; ++u) {
        const uint32_t off = lo + ((uint32_t)u * kShapeThreads + threadIdx.x) * 16u;
        v[u] = buf_load_b128_nt(r, off < hi ? off : 0xFFFFFF00u);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < kShapeLoads; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if ((flags & kShapeLds) && acc == 0x9E3779B9u) lds_f[threadIdx.x] = xs;  // keeps the allocation referenced
    if (acc == 0x9E3779B9u) sink[blockIdx.x & 1023] = acc;
    if ((flags & kShapeStore) && threadIdx.x < 16) y[blockIdx.x * 16 + threadIdx.x] = xs + (float)(acc & 1u);
}

__global__ void empty_kernel(int) {}

// Grid-wide barrier: each workgroup's first thread adds to one counter (agent
// scope, coherent across the XCDs: 1, or 2^31 - (grid - 1) for workgroup 0, so
// that every barrier flips the counter's top bit once all have arrived) and
// polls it until the bit flips.  Every poll is bounded: a barrier that does not
// complete within 2^22 polls sets *err and ends the launch.
__global__ __launch_bounds__(1024) void grid_barrier_kernel(unsigned* __restrict__ counter, int n,
                                                            unsigned* __restrict__ err) {
    __shared__ unsigned ok;
    bool go = true;
    for (int b = 0; b < n && go; ++b) {
        __syncthreads();
        if (threadIdx.x == 0) {
            const unsigned add = blockIdx.x == 0 ? 0x80000000u - (gridDim.x - 1u) : 1u;
            const unsigned old = __hip_atomic_fetch_add(counter, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            unsigned polls = 0;
            while (((__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ^ old) & 0x80000000u) == 0u &&
                   ++polls < (1u << 22)) {
            }
            ok = polls < (1u << 22);
            if (!ok) atomicOr(err, 1u);
        }
        __syncthreads();
        go = ok;
    }
}

}  // namespace

int shaped_read_launch(const void* buf, int64_t bytes, const float* x, int xn, float* y, int64_t y_floats, int flags,
                       int lds, uint32_t* sink, hipStream_t st) {
    if (!buf || !sink || ((flags & kShapeX) && (!x || (uintptr_t)x % 16 || xn % 4 || xn < 0)) ||
        ((flags & kShapeStore) && !y))
        return fail(kInvalidArgument, "shaped read: bad pointer or x length");
    if (bytes <= 0 || bytes >= ((int64_t)1 << 31) || lds < 0 || lds > 160 * 1024)
        return fail(kInvalidArgument, "shaped read: need 0 < bytes < 2 GiB, 0 <= lds <= 160 KB");
    int dev = 0, cus = 0;
    ASMHIP_TRY(hipGetDevice(&dev));
    ASMHIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    if (cus <= 0) cus = 256;
    constexpr int64_t kChunk = (int64_t)kShapeLoads * kShapeThreads * 16;
    const int64_t grid = (int64_t)cus * ((bytes + (int64_t)cus * kChunk - 1) / ((int64_t)cus * kChunk));
    const uint32_t per_wg = (uint32_t)(((bytes + grid - 1) / grid + 15) / 16 * 16);
    if ((flags & kShapeStore) && y_floats < grid * 16)
        return fail(kInvalidArgument, "shaped read: y needs %lld floats (16 per workgroup)", (long long)(grid * 16));
    const size_t dyn = (flags & kShapeLds) ? (size_t)lds : 0;
    const int rc = dynamic_lds((const void*)shaped_read_kernel, dyn);
    if (rc) return rc;
    hipLaunchKernelGGL(shaped_read_kernel, dim3((unsigned)grid), dim3(kShapeThreads), dyn, st,
                       static_cast<const uint8_t*>(buf), (uint32_t)bytes, per_wg, x, xn, y, flags, sink);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int empty_launch(int grid, int threads, int lds, hipStream_t st) {
    if (grid <= 0 || threads <= 0 || threads > 1024 || lds < 0 || lds > 160 * 1024)
        return fail(kInvalidArgument, "empty launch: bad shape");
    const int rc = dynamic_lds((const void*)empty_kernel, (size_t)lds);
    if (rc) return rc;
    hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(threads), (size_t)lds, st, 0);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int grid_barrier_launch(unsigned* counter, int n, unsigned* err, hipStream_t st) {
    if (!counter || !err || n < 0) return fail(kInvalidArgument, "grid barrier: bad argument");
    int dev = 0, cus = 0, coop = 0;
    ASMHIP_TRY(hipGetDevice(&dev));
    ASMHIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    ASMHIP_TRY(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
    if (!coop || cus <= 0) return fail(kUnsupported, "grid barrier: no cooperative launch on this device");
    // one workgroup per compute unit, all resident at once (the cooperative launch fails otherwise)
    void* args[] = {&counter, &n, &err};
    ASMHIP_TRY(hipLaunchCooperativeKernel((const void*)grid_barrier_kernel, dim3(cus), dim3(1024), args, 0, st));
    return kOk;
}

int stream_read_launch(const void* buf, int64_t bytes, uint32_t* sink, hipStream_t st) {
    if (!buf || !sink) return fail(kInvalidArgument, "stream read: null pointer");
    if (bytes <= 0 || bytes >= ((int64_t)1 << 31))  // 32-bit offsets with room past the last chunk
        return fail(kInvalidArgument, "stream read: need 0 < bytes < 2 GiB (got %lld)", (long long)bytes);
    // a whole number of workgroups per compute unit, each chunk within its 25 loads per lane
    int dev = 0, cus = 0;
    ASMHIP_TRY(hipGetDevice(&dev));
    ASMHIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    if (cus <= 0) cus = 256;
    constexpr int64_t kChunk = (int64_t)kReadLoads * kReadThreads * 16;
    const int64_t grid = (int64_t)cus * ((bytes + (int64_t)cus * kChunk - 1) / ((int64_t)cus * kChunk));
    const uint32_t per_wg = (uint32_t)(((bytes + grid - 1) / grid + 15) / 16 * 16);
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)grid), dim3(kReadThreads), 0, st,
                       static_cast<const uint8_t*>(buf), (uint32_t)bytes, per_wg, sink);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

}  // namespace asmhip
