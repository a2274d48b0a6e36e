// C-ABI layer of libasmllm.so: argument checks, host/device pointer staging for
// the reference-named synchronous entry points, and the device plumbing calls.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "asmllm_hip.h"
#include "common.hpp"
#include "kernels.hpp"

namespace asmhip {

namespace {
thread_local char g_last_error[1024] = "";

constexpr int kMaxDevices = 64;
constexpr int kMaxPool = 64;  // threadpool.c:99 MAX_WORKERS

// Per-device library state used by the synchronous entry points: one stream
// (default priority) and a grow-only staging buffer for host operands.
struct DeviceState {
    hipStream_t stream = nullptr;
    void* staging = nullptr;
    size_t staging_bytes = 0;
};

std::mutex g_mu;
DeviceState g_dev[kMaxDevices];
int g_pool_size = 0;  // what asm_threadpool_init recorded
}  // namespace

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(kHipError, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

namespace {
struct LdsGrant {
    const void* kernel;
    int device;
    size_t bytes;
};
std::mutex g_lds_mu;
LdsGrant g_lds[256];
int g_lds_n = 0;
}  // namespace

int dynamic_lds(const void* kernel, size_t bytes) {
    if (bytes <= 64 * 1024) return kOk;
    int dev = 0;
    ASMHIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_lds_mu);
    int slot = -1;
    for (int i = 0; i < g_lds_n; ++i)
        if (g_lds[i].kernel == kernel && g_lds[i].device == dev) {
            if (g_lds[i].bytes >= bytes) return kOk;
            slot = i;
            break;
        }
    hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(kUnsupported, "kernel needs %zu bytes of LDS: hipFuncSetAttribute failed: %s", bytes,
                    hipGetErrorString(e));
    }
    if (slot < 0) {
        if (g_lds_n == (int)(sizeof(g_lds) / sizeof(g_lds[0]))) return kOk;  // table full: set again next time
        slot = g_lds_n++;
    }
    g_lds[slot] = {kernel, dev, bytes};
    return kOk;
}

namespace {

int current_device(int* dev) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return fail(kNoDevice, "no HIP device available");
    }
    ASMHIP_TRY(hipGetDevice(dev));
    if (*dev < 0 || *dev >= kMaxDevices) return fail(kUnsupported, "device index %d out of range", *dev);
    return kOk;
}

// Caller holds g_mu.
int ensure_state(DeviceState** out) {
    int dev = 0;
    int rc = current_device(&dev);
    if (rc) return rc;
    DeviceState& st = g_dev[dev];
    if (!st.stream) ASMHIP_TRY(hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking));
    *out = &st;
    return kOk;
}

int ensure_staging(DeviceState* st, size_t bytes) {
    if (st->staging_bytes >= bytes) return kOk;
    if (st->staging) {
        ASMHIP_TRY(hipStreamSynchronize(st->stream));
        ASMHIP_TRY(hipFree(st->staging));
        st->staging = nullptr;
        st->staging_bytes = 0;
    }
    size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    ASMHIP_TRY(hipMalloc(&st->staging, want));
    st->staging_bytes = want;
    return kOk;
}

bool is_device_pointer(const void* p) {
    if (!p) return false;
    hipPointerAttribute_t a;
    hipError_t e = hipPointerGetAttributes(&a, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

// One operand of a synchronous call: where it lives and where the kernel reads it.
struct Operand {
    const void* host;  // user pointer
    size_t bytes;
    bool in;   // uploaded before the kernel when host-resident
    bool out;  // downloaded after the kernel when host-resident
    bool on_device = false;
    void* dev = nullptr;  // device address used by the kernel
};

size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

// Places every host operand in the staging buffer and uploads the inputs.
int stage(DeviceState* st, Operand* ops, int n_ops) {
    size_t need = 0;
    for (int i = 0; i < n_ops; ++i) {
        ops[i].on_device = is_device_pointer(ops[i].host);
        if (!ops[i].on_device) need += round256(ops[i].bytes);
    }
    if (need) {
        int rc = ensure_staging(st, need);
        if (rc) return rc;
    }
    size_t off = 0;
    for (int i = 0; i < n_ops; ++i) {
        if (ops[i].on_device) {
            ops[i].dev = const_cast<void*>(ops[i].host);
            continue;
        }
        ops[i].dev = static_cast<char*>(st->staging) + off;
        off += round256(ops[i].bytes);
        if (ops[i].in)
            ASMHIP_TRY(hipMemcpyAsync(ops[i].dev, ops[i].host, ops[i].bytes, hipMemcpyHostToDevice, st->stream));
    }
    return kOk;
}

// Downloads host-resident outputs and waits for the stream.
int finish(DeviceState* st, Operand* ops, int n_ops) {
    for (int i = 0; i < n_ops; ++i)
        if (ops[i].out && !ops[i].on_device)
            ASMHIP_TRY(hipMemcpyAsync(const_cast<void*>(ops[i].host), ops[i].dev, ops[i].bytes,
                                      hipMemcpyDeviceToHost, st->stream));
    ASMHIP_TRY(hipStreamSynchronize(st->stream));
    return kOk;
}

// Synchronous call: stage the operands, enqueue `launch` on the library stream
// with their device addresses, bring the outputs back and wait.
template <class F>
int sync_call(Operand* ops, int n_ops, F&& launch) {
    for (int i = 0; i < n_ops; ++i)
        if (!ops[i].host) return fail(kInvalidArgument, "null pointer argument");
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceState* st = nullptr;
    int rc = ensure_state(&st);
    if (rc) return rc;
    rc = stage(st, ops, n_ops);
    if (rc) return rc;
    rc = launch(st->stream);
    if (rc) {
        (void)hipStreamSynchronize(st->stream);
        return rc;
    }
    return finish(st, ops, n_ops);
}

void report(int rc, const char* fn) {
    if (rc != kOk) fprintf(stderr, "[libasmllm] %s: %s\n", fn, g_last_error);
}

int sync_matvec(QuantType qt, const void* q, const float* s, const float* x, float* y, int64_t M, int64_t K) {
    if (M <= 0 || K <= 0 || K % 32 != 0)
        return fail(kInvalidArgument, "need M > 0, K > 0 and K %% 32 == 0 (got M=%lld K=%lld)", (long long)M,
                    (long long)K);
    const size_t nb = (size_t)(K / 32);
    Operand ops[4] = {
        {q, (size_t)M * nb * (qt == QuantType::Q4_0 ? 16 : 32), true, false},
        {s, (size_t)M * nb * sizeof(float), true, false},
        {x, (size_t)K * sizeof(float), true, false},
        {y, (size_t)M * sizeof(float), false, true},
    };
    return sync_call(ops, 4, [&](hipStream_t stream) {
        return matvec_launch(qt, false, ops[0].dev, static_cast<const float*>(ops[1].dev),
                             static_cast<const float*>(ops[2].dev), static_cast<float*>(ops[3].dev), M, K, stream);
    });
}

int sync_matvec_q5(const uint8_t* ql, const uint8_t* qh, const float* s, const float* x, float* y, int64_t M,
                   int64_t K) {
    if (M <= 0 || K <= 0 || K % 32 != 0)
        return fail(kInvalidArgument, "need M > 0, K > 0 and K %% 32 == 0 (got M=%lld K=%lld)", (long long)M,
                    (long long)K);
    const size_t nb = (size_t)(K / 32);
    Operand ops[5] = {
        {ql, (size_t)M * nb * 16, true, false},
        {qh, (size_t)M * nb * 4, true, false},
        {s, (size_t)M * nb * sizeof(float), true, false},
        {x, (size_t)K * sizeof(float), true, false},
        {y, (size_t)M * sizeof(float), false, true},
    };
    return sync_call(ops, 5, [&](hipStream_t stream) {
        return q5_matvec_launch(false, ops[0].dev, static_cast<const uint8_t*>(ops[1].dev),
                                static_cast<const float*>(ops[2].dev), static_cast<const float*>(ops[3].dev),
                                static_cast<float*>(ops[4].dev), M, K, stream);
    });
}

void record_pool_size(int n) {
    if (n < 1) n = 1;
    if (n > kMaxPool) n = kMaxPool;
    g_pool_size = n;
}

}  // namespace
}  // namespace asmhip

using namespace asmhip;

// ---- reference-named entry points -------------------------------------------

extern "C" void asm_matmul_q4(const uint8_t* qweights, const float* scales, const float* x, float* y, int64_t M,
                              int64_t K) {
    report(sync_matvec(QuantType::Q4_0, qweights, scales, x, y, M, K), "asm_matmul_q4");
}

extern "C" void asm_matmul_q4_avx512(const uint8_t* qweights, const float* scales, const float* x, float* y,
                                     int64_t M, int64_t K) {
    report(sync_matvec(QuantType::Q4_0, qweights, scales, x, y, M, K), "asm_matmul_q4_avx512");
}

extern "C" void asm_matmul_q8(const int8_t* qweights, const float* scales, const float* x, float* y, int64_t M,
                              int64_t K) {
    report(sync_matvec(QuantType::Q8_0, qweights, scales, x, y, M, K), "asm_matmul_q8");
}

extern "C" void asm_matmul_q5(const uint8_t* ql, const uint8_t* qh, const float* scales, const float* x, float* y,
                              int64_t M, int64_t K) {
    report(sync_matvec_q5(ql, qh, scales, x, y, M, K), "asm_matmul_q5");
}

extern "C" void asm_threadpool_init(int num_threads) {
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceState* st = nullptr;
    int rc = ensure_state(&st);
    if (rc) {
        report(rc, "asm_threadpool_init");
        return;
    }
    record_pool_size(num_threads);
}

extern "C" void asm_threadpool_shutdown(void) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_pool_size <= 0) return;  // threadpool.c:372
    int dev = 0;
    if (current_device(&dev) == kOk) {
        DeviceState& st = g_dev[dev];
        if (st.stream) {
            (void)hipStreamSynchronize(st.stream);
            (void)hipStreamDestroy(st.stream);
            st.stream = nullptr;
        }
        if (st.staging) {
            (void)hipFree(st.staging);
            st.staging = nullptr;
            st.staging_bytes = 0;
        }
    }
    g_pool_size = 0;
}

extern "C" int asm_threadpool_get_num_threads(void) {
    std::lock_guard<std::mutex> lock(g_mu);
    return g_pool_size;
}

// threadpool.c:399-406: below 32 rows or one thread the pool is not touched;
// otherwise the pool is (re)sized to num_threads.
static void mt_pool_update(int64_t M, int num_threads) {
    if (num_threads <= 1 || M < 32) return;
    bool resize;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        resize = g_pool_size != num_threads;
    }
    if (resize) asm_threadpool_init(num_threads);
}

extern "C" void asm_matmul_q4_mt(const uint8_t* qweights, const float* scales, const float* x, float* y,
                                 int64_t M, int64_t K, int num_threads) {
    mt_pool_update(M, num_threads);
    report(sync_matvec(QuantType::Q4_0, qweights, scales, x, y, M, K), "asm_matmul_q4_mt");
}

extern "C" void asm_matmul_q8_mt(const int8_t* qweights, const float* scales, const float* x, float* y,
                                 int64_t M, int64_t K, int num_threads) {
    mt_pool_update(M, num_threads);
    report(sync_matvec(QuantType::Q8_0, qweights, scales, x, y, M, K), "asm_matmul_q8_mt");
}

extern "C" void asm_threadpool_dispatch_q8(const int8_t* qweights, const float* scales, const float* x, float* y,
                                           int64_t M, int64_t K) {
    report(sync_matvec(QuantType::Q8_0, qweights, scales, x, y, M, K), "asm_threadpool_dispatch_q8");
}

extern "C" void asm_matmul_q5_mt(const uint8_t* ql, const uint8_t* qh, const float* scales, const float* x, float* y,
                                 int64_t M, int64_t K, int num_threads) {
    mt_pool_update(M, num_threads);
    report(sync_matvec_q5(ql, qh, scales, x, y, M, K), "asm_matmul_q5_mt");
}

extern "C" void asm_threadpool_dispatch_q5(const uint8_t* ql, const uint8_t* qh, const float* scales, const float* x,
                                           float* y, int64_t M, int64_t K) {
    report(sync_matvec_q5(ql, qh, scales, x, y, M, K), "asm_threadpool_dispatch_q5");
}

// rmsnorm_avx2.asm:63-151: y = (x * (1/sqrt(mean(x^2) + eps))) * w.
extern "C" void asm_rmsnorm(const float* x, const float* w, float* y, int64_t dim, float eps) {
    if (dim <= 0) return report(fail(kInvalidArgument, "dim must be > 0"), "asm_rmsnorm");
    const size_t b = (size_t)dim * sizeof(float);
    Operand ops[3] = {{x, b, true, false}, {w, b, true, false}, {y, b, false, true}};
    report(sync_call(ops, 3,
                     [&](hipStream_t st) {
                         return rmsnorm_launch((const float*)ops[0].dev, (const float*)ops[1].dev,
                                               (float*)ops[2].dev, dim, eps, st);
                     }),
           "asm_rmsnorm");
}

// rope_avx2.asm:52-146: one head of q and one of k, rotated in place.
extern "C" void asm_rope(float* q, float* k, int64_t head_dim, int64_t pos, float theta) {
    if (head_dim <= 0) return report(fail(kInvalidArgument, "head_dim must be > 0"), "asm_rope");
    const size_t b = (size_t)head_dim * sizeof(float);
    Operand ops[2] = {{q, b, true, true}, {k, b, true, true}};
    report(sync_call(ops, 2,
                     [&](hipStream_t st) {
                         return rope_launch((float*)ops[0].dev, (float*)ops[1].dev, 1, 1, head_dim, nullptr, pos,
                                            theta, st);
                     }),
           "asm_rope");
}

// softmax_avx2.asm:48-130; x == y allowed.
extern "C" void asm_softmax(const float* x, float* y, int64_t dim) {
    if (dim <= 0) return report(fail(kInvalidArgument, "dim must be > 0"), "asm_softmax");
    const size_t b = (size_t)dim * sizeof(float);
    if (x == y) {
        Operand ops[1] = {{y, b, true, true}};
        return report(sync_call(ops, 1,
                                [&](hipStream_t st) {
                                    return softmax_launch((const float*)ops[0].dev, (float*)ops[0].dev, dim, st);
                                }),
                      "asm_softmax");
    }
    Operand ops[2] = {{x, b, true, false}, {y, b, false, true}};
    report(sync_call(ops, 2,
                     [&](hipStream_t st) {
                         return softmax_launch((const float*)ops[0].dev, (float*)ops[1].dev, dim, st);
                     }),
           "asm_softmax");
}

// swiglu_avx2.asm:45-81: gate = gate / (1 + exp(-gate)) * up, in place.
extern "C" void asm_silu_hadamard(float* gate, const float* up, int64_t dim) {
    if (dim <= 0) return report(fail(kInvalidArgument, "dim must be > 0"), "asm_silu_hadamard");
    const size_t b = (size_t)dim * sizeof(float);
    Operand ops[2] = {{gate, b, true, true}, {up, b, true, false}};
    report(sync_call(ops, 2,
                     [&](hipStream_t st) {
                         return silu_launch((float*)ops[0].dev, (const float*)ops[1].dev, dim, st);
                     }),
           "asm_silu_hadamard");
}

// attention_avx2.asm:59-218: y = softmax(q k^T * scale) v over [seq][head_dim] rows.
extern "C" void asm_attention(const float* q, const float* k, const float* v, float* y, int64_t seq_len,
                              int64_t head_dim, float scale) {
    if (seq_len <= 0 || head_dim <= 0)
        return report(fail(kInvalidArgument, "need seq_len > 0 and head_dim > 0"), "asm_attention");
    const size_t b = (size_t)seq_len * head_dim * sizeof(float);
    Operand ops[4] = {{q, b, true, false}, {k, b, true, false}, {v, b, true, false}, {y, b, false, true}};
    report(sync_call(ops, 4,
                     [&](hipStream_t st) {
                         return attention_launch((const float*)ops[0].dev, (const float*)ops[1].dev,
                                                 (const float*)ops[2].dev, (float*)ops[3].dev, seq_len, head_dim,
                                                 scale, st);
                     }),
           "asm_attention");
}

// ---- device entry points -------------------------------------------------------

static int check_ptrs(const void* a, const void* b, const void* c) {
    if (!a || !b || !c) return fail(kInvalidArgument, "null pointer argument");
    return kOk;
}

extern "C" int asmhip_matmul_q4_0(const void* blocks, const float* x, float* y, int64_t M, int64_t K, void* stream) {
    int rc = check_ptrs(blocks, x, y);
    return rc ? rc : matvec_launch(QuantType::Q4_0, true, blocks, nullptr, x, y, M, K, (hipStream_t)stream);
}

extern "C" int asmhip_matmul_q8_0(const void* blocks, const float* x, float* y, int64_t M, int64_t K, void* stream) {
    int rc = check_ptrs(blocks, x, y);
    return rc ? rc : matvec_launch(QuantType::Q8_0, true, blocks, nullptr, x, y, M, K, (hipStream_t)stream);
}

extern "C" int asmhip_matmul_q4_split(const uint8_t* qweights, const float* scales, const float* x, float* y,
                                      int64_t M, int64_t K, void* stream) {
    int rc = check_ptrs(qweights, x, y);
    if (!rc && !scales) rc = fail(kInvalidArgument, "null scales");
    return rc ? rc : matvec_launch(QuantType::Q4_0, false, qweights, scales, x, y, M, K, (hipStream_t)stream);
}

extern "C" int asmhip_matmul_q8_split(const int8_t* qweights, const float* scales, const float* x, float* y,
                                      int64_t M, int64_t K, void* stream) {
    int rc = check_ptrs(qweights, x, y);
    if (!rc && !scales) rc = fail(kInvalidArgument, "null scales");
    return rc ? rc : matvec_launch(QuantType::Q8_0, false, qweights, scales, x, y, M, K, (hipStream_t)stream);
}

extern "C" int asmhip_matmul_q5_split(const uint8_t* ql, const uint8_t* qh, const float* scales, const float* x,
                                      float* y, int64_t M, int64_t K, void* stream) {
    int rc = check_ptrs(ql, x, y);
    if (!rc && (!qh || !scales)) rc = fail(kInvalidArgument, "null qh or scales");
    return rc ? rc : q5_matvec_launch(false, ql, qh, scales, x, y, M, K, (hipStream_t)stream);
}

extern "C" int asmhip_matmul_q5_0(const void* blocks, const float* x, float* y, int64_t M, int64_t K, void* stream) {
    int rc = check_ptrs(blocks, x, y);
    return rc ? rc : q5_matvec_launch(true, blocks, nullptr, nullptr, x, y, M, K, (hipStream_t)stream);
}

extern "C" int asmhip_dequantize_q5_0(const void* blocks, float* w, int64_t rows, int64_t K, void* stream) {
    if (!blocks || !w) return fail(kInvalidArgument, "null pointer argument");
    return q5_dequant_launch(blocks, w, rows, K, (hipStream_t)stream);
}

extern "C" int asmhip_dequantize_q4_0(const void* blocks, float* w, int64_t rows, int64_t K, void* stream) {
    if (!blocks || !w) return fail(kInvalidArgument, "null pointer argument");
    return dequant_launch(QuantType::Q4_0, blocks, w, rows, K, (hipStream_t)stream);
}

extern "C" int asmhip_dequantize_q8_0(const void* blocks, float* w, int64_t rows, int64_t K, void* stream) {
    if (!blocks || !w) return fail(kInvalidArgument, "null pointer argument");
    return dequant_launch(QuantType::Q8_0, blocks, w, rows, K, (hipStream_t)stream);
}

static int quant_type(int qtype, QuantType* qt) {
    if (qtype == ASMHIP_Q4_0) *qt = QuantType::Q4_0;
    else if (qtype == ASMHIP_Q8_0) *qt = QuantType::Q8_0;
    else return fail(kInvalidArgument, "unknown quantization type %d", qtype);
    return kOk;
}

extern "C" int asmhip_matmul_fused(int qtype, const void* blocks, const float* x, float* y, int64_t M, int64_t K,
                                   int pre_op, const float* pre_arg, float eps, int accumulate, void* stream) {
    QuantType qt;
    int rc = check_ptrs(blocks, x, y);
    if (!rc) rc = quant_type(qtype, &qt);
    if (rc) return rc;
    MatvecOpts o;
    o.pre = pre_op;
    o.pre_arg = pre_arg;
    o.eps = eps;
    o.accumulate = accumulate != 0;
    return matvec_launch(qt, true, blocks, nullptr, x, y, M, K, (hipStream_t)stream, o);
}

extern "C" int asmhip_matmul_swiglu(int qtype, const void* blocks, const float* x, float* h, int64_t H, int64_t K,
                                    int pre_op, const float* pre_arg, float eps, float* work, void* stream) {
    QuantType qt;
    int rc = check_ptrs(blocks, x, h);
    if (!rc) rc = quant_type(qtype, &qt);
    if (rc) return rc;
    MatvecOpts o;
    o.pre = pre_op;
    o.pre_arg = pre_arg;
    o.eps = eps;
    if (o.pre != kPreNone && !o.pre_arg) return fail(kInvalidArgument, "matvec_swiglu: pre-op without its argument");
    if (o.pre < kPreNone || o.pre > kPreSwiGlu) return fail(kInvalidArgument, "matvec_swiglu: unknown pre-op %d", o.pre);
    return matvec_swiglu_launch(qt, blocks, x, h, H, K, work, (hipStream_t)stream, o);
}

extern "C" int asmhip_gemm_q8_0(const void* w_blocks, const void* a_blocks, float* c, int64_t T, int64_t M,
                                int64_t K, void* stream) {
    int rc = check_ptrs(w_blocks, a_blocks, c);
    return rc ? rc : gemm_q8_0_launch(w_blocks, a_blocks, c, T, M, K, (hipStream_t)stream);
}

extern "C" int64_t asmhip_gemm_q8_0_tiled_weight_bytes(int64_t M, int64_t K) {
    return M > 0 && K > 0 && K % 64 == 0 ? gemm_tiled_bytes(M, K, kGemmTileW) : 0;
}

extern "C" int64_t asmhip_gemm_q8_0_tiled_activation_bytes(int64_t T, int64_t K) {
    return T > 0 && K > 0 && K % 64 == 0 ? gemm_tiled_bytes(T, K, kGemmTileA) : 0;
}

extern "C" int asmhip_gemm_q8_0_tile_weights(const void* w_blocks, void* w_tiled, int64_t M, int64_t K,
                                             void* stream) {
    return gemm_tile_blocks_launch(w_blocks, w_tiled, M, K, kGemmTileW, (hipStream_t)stream);
}

extern "C" int asmhip_gemm_q8_0_tile_activations(const void* a_blocks, void* a_tiled, int64_t T, int64_t K,
                                                 void* stream) {
    return gemm_tile_blocks_launch(a_blocks, a_tiled, T, K, kGemmTileA, (hipStream_t)stream);
}

extern "C" int asmhip_quantize_q8_0_tiled(const float* x, void* a_tiled, int64_t T, int64_t K, void* stream) {
    return quantize_q8_0_tiled_launch(x, a_tiled, T, K, (hipStream_t)stream);
}

extern "C" int asmhip_gemm_q8_0_tiled(const void* w_tiled, const void* a_tiled, float* c, int64_t T, int64_t M,
                                      int64_t K, void* stream) {
    return gemm_q8_0_tiled_launch(w_tiled, a_tiled, c, T, M, K, (hipStream_t)stream);
}

extern "C" int asmhip_gemm_q8_split(const int8_t* w_qs, const float* w_scales, const int8_t* a_qs,
                                    const float* a_scales, float* c, int64_t T, int64_t M, int64_t K, void* stream) {
    int rc = check_ptrs(w_qs, a_qs, c);
    if (!rc && (!w_scales || !a_scales)) rc = fail(kInvalidArgument, "null scales");
    return rc ? rc : gemm_q8_split_launch(w_qs, w_scales, a_qs, a_scales, c, T, M, K, (hipStream_t)stream);
}

extern "C" int asmhip_set_q4_kernel(int kernel) { return set_q4_kernel(kernel); }
extern "C" int asmhip_get_q4_kernel(void) { return get_q4_kernel(); }

extern "C" int asmhip_quantize(int qtype, const float* w, void* blocks, int64_t rows, int64_t K, void* stream) {
    QuantType qt;
    if (!w || !blocks) return fail(kInvalidArgument, "null pointer argument");
    int rc = quant_type(qtype, &qt);
    return rc ? rc : quantize_launch(qt, w, blocks, rows, K, (hipStream_t)stream);
}

extern "C" int asmhip_quantize_q8_split(const float* w, int8_t* qs, float* scales, int64_t rows, int64_t K,
                                        void* stream) {
    int rc = check_ptrs(w, qs, scales);
    return rc ? rc : quantize_q8_split_launch(w, qs, scales, rows, K, (hipStream_t)stream);
}

extern "C" int asmhip_random_blocks(int qtype, void* blocks, int64_t rows, int64_t K, uint64_t seed, float stddev,
                                    void* stream) {
    QuantType qt;
    if (!blocks) return fail(kInvalidArgument, "null pointer argument");
    int rc = quant_type(qtype, &qt);
    return rc ? rc : random_blocks_launch(qt, blocks, rows, K, seed, stddev, (hipStream_t)stream);
}

extern "C" int asmhip_random_f16(void* out, int64_t n, uint64_t seed, float stddev, void* stream) {
    if (!out) return fail(kInvalidArgument, "null pointer argument");
    return random_f16_launch(out, n, seed, stddev, (hipStream_t)stream);
}

extern "C" int asmhip_fill_f32(float* out, int64_t n, float value, void* stream) {
    if (!out) return fail(kInvalidArgument, "null pointer argument");
    return fill_f32_launch(out, n, value, (hipStream_t)stream);
}

extern "C" int asmhip_rmsnorm(const float* x, const float* w, float* y, int64_t dim, float eps, void* stream) {
    int rc = check_ptrs(x, w, y);
    return rc ? rc : rmsnorm_launch(x, w, y, dim, eps, (hipStream_t)stream);
}

extern "C" int asmhip_rope(float* q, float* k, int64_t n_q_heads, int64_t n_k_heads, int64_t head_dim,
                           const int* pos_dev, int64_t pos, float theta, void* stream) {
    if ((n_q_heads && !q) || (n_k_heads && !k)) return fail(kInvalidArgument, "null pointer argument");
    return rope_launch(q, k, n_q_heads, n_k_heads, head_dim, pos_dev, pos, theta, (hipStream_t)stream);
}

extern "C" int asmhip_softmax(const float* x, float* y, int64_t dim, void* stream) {
    if (!x || !y) return fail(kInvalidArgument, "null pointer argument");
    return softmax_launch(x, y, dim, (hipStream_t)stream);
}

extern "C" int asmhip_silu_hadamard(float* gate, const float* up, int64_t dim, void* stream) {
    if (!gate || !up) return fail(kInvalidArgument, "null pointer argument");
    return silu_launch(gate, up, dim, (hipStream_t)stream);
}

extern "C" int asmhip_attention(const float* q, const float* k, const float* v, float* y, int64_t seq_len,
                                int64_t head_dim, float scale, void* stream) {
    if (!q || !k || !v || !y) return fail(kInvalidArgument, "null pointer argument");
    return attention_launch(q, k, v, y, seq_len, head_dim, scale, (hipStream_t)stream);
}

extern "C" int asmhip_rope_kv_write(float* qkv, void* k_cache, void* v_cache, int n_heads, int n_kv_heads,
                                    int head_dim, const int* pos_dev, int max_ctx, float theta, void* stream) {
    if (!qkv || !k_cache || !v_cache || !pos_dev) return fail(kInvalidArgument, "null pointer argument");
    if (n_heads <= 0 || head_dim <= 0 || max_ctx <= 0) return fail(kInvalidArgument, "bad attention shape");
    return rope_kv_write_launch(qkv, k_cache, v_cache, n_heads, n_kv_heads, head_dim, pos_dev, max_ctx, theta,
                                (hipStream_t)stream);
}

extern "C" int64_t asmhip_attention_decode_workspace(int n_heads, int head_dim, int max_ctx) {
    if (n_heads <= 0 || head_dim <= 0 || max_ctx <= 0) return 0;
    return attn_decode_workspace(n_heads, head_dim, max_ctx);
}

extern "C" int asmhip_attention_decode(const float* q, const void* k_cache, const void* v_cache, float* workspace,
                                       float* out, int n_heads, int n_kv_heads, int head_dim, const int* pos_dev,
                                       int max_ctx, void* stream) {
    if (!q || !k_cache || !v_cache || !workspace || !out || !pos_dev)
        return fail(kInvalidArgument, "null pointer argument");
    if (n_heads <= 0 || max_ctx <= 0) return fail(kInvalidArgument, "bad attention shape");
    return attn_decode_launch(q, const_cast<void*>(k_cache), const_cast<void*>(v_cache), workspace, out, n_heads,
                              n_kv_heads, head_dim, pos_dev, max_ctx, false, 0.f, (hipStream_t)stream);
}

extern "C" int asmhip_attention_decode_rope(const float* qkv, void* k_cache, void* v_cache, float* workspace,
                                            float* out, int n_heads, int n_kv_heads, int head_dim, const int* pos_dev,
                                            int max_ctx, float theta, void* stream) {
    if (!qkv || !k_cache || !v_cache || !workspace || !out || !pos_dev)
        return fail(kInvalidArgument, "null pointer argument");
    if (n_heads <= 0 || max_ctx <= 0 || head_dim % 2) return fail(kInvalidArgument, "bad attention shape");
    return attn_decode_launch(qkv, k_cache, v_cache, workspace, out, n_heads, n_kv_heads, head_dim, pos_dev, max_ctx,
                              true, theta, (hipStream_t)stream);
}

extern "C" int asmhip_rope_table(float* table, int head_dim, int max_ctx, float theta, void* stream) {
    return rope_table_launch(table, head_dim, max_ctx, theta, (hipStream_t)stream);
}

extern "C" int asmhip_attention_decode_rope_table(const float* qkv, void* k_cache, void* v_cache, float* workspace,
                                                  float* out, int n_heads, int n_kv_heads, int head_dim,
                                                  const int* pos_dev, int max_ctx, const float* rope_table,
                                                  void* stream) {
    if (!qkv || !k_cache || !v_cache || !workspace || !out || !pos_dev || !rope_table)
        return fail(kInvalidArgument, "null pointer argument");
    if (n_heads <= 0 || max_ctx <= 0 || head_dim % 2) return fail(kInvalidArgument, "bad attention shape");
    return attn_decode_launch(qkv, k_cache, v_cache, workspace, out, n_heads, n_kv_heads, head_dim, pos_dev, max_ctx,
                              true, 0.f, (hipStream_t)stream, rope_table);
}

extern "C" int asmhip_attention_decode_partials_rope_table(const float* qkv, void* k_cache, void* v_cache,
                                                           float* workspace, int n_heads, int n_kv_heads,
                                                           int head_dim, const int* pos_dev, int max_ctx,
                                                           const float* rope_table, void* stream) {
    if (!qkv || !k_cache || !v_cache || !workspace || !pos_dev || !rope_table)
        return fail(kInvalidArgument, "null pointer argument");
    if (n_heads <= 0 || max_ctx <= 0 || head_dim % 2) return fail(kInvalidArgument, "bad attention shape");
    return attn_decode_launch(qkv, k_cache, v_cache, workspace, nullptr, n_heads, n_kv_heads, head_dim, pos_dev,
                              max_ctx, true, 0.f, (hipStream_t)stream, rope_table);
}

extern "C" int asmhip_matmul_attn_output(int qtype, const void* blocks, const float* workspace, float* work, float* y,
                                         int64_t M, int n_heads, int head_dim, int max_ctx, int accumulate,
                                         void* stream) {
    QuantType qt;
    int rc = check_ptrs(blocks, workspace, y);
    if (!rc && !work) rc = fail(kInvalidArgument, "null pointer argument");
    if (!rc) rc = quant_type(qtype, &qt);
    if (rc) return rc;
    if (n_heads <= 0 || head_dim <= 0 || max_ctx <= 0) return fail(kInvalidArgument, "bad attention shape");
    if (max_ctx > kAttnMaxCtx)
        return fail(kUnsupported, "attention output: max_ctx %d exceeds %d positions", max_ctx, kAttnMaxCtx);
    const int splits = attn_decode_splits(max_ctx);
    const int64_t K = (int64_t)n_heads * head_dim;
    const hipStream_t st = (hipStream_t)stream;
    MatvecOpts o;
    o.pre = kPreAttnMerge;
    o.pre_arg = workspace;
    o.accumulate = accumulate != 0;
    o.attn_splits = splits;
    o.attn_hd = head_dim;
    // one launch where the int8-MFMA stream takes the shape: the merge is its x prologue
    if (get_q4_kernel() != kQ4KernelFp32) {
        if (qt == QuantType::Q4_0 && q4_0_mfma_eligible(blocks, workspace, o, M, K))
            return q4_0_mfma_launch(blocks, workspace, y, M, K, st, o);
        if (qt == QuantType::Q8_0 && q8_0_mfma_eligible(blocks, workspace, o, M, K))
            return q8_0_mfma_launch(blocks, workspace, y, M, K, st, o);
    }
    // otherwise the merge launch into `work`, then the matvec over it
    rc = attn_merge_launch(workspace, work, n_heads, head_dim, max_ctx, st);
    if (rc) return rc;
    MatvecOpts p;
    p.accumulate = o.accumulate;
    return matvec_launch(qt, true, blocks, nullptr, work, y, M, K, st, p);
}

// ---- decode attention without a caller workspace -----------------------------------------
//
// For callers that cannot allocate (graph capture, tight serving loops): the
// split partials live in `scratch`, a fixed array in every device's copy of the
// library, instead of a workspace argument.  Its device address differs per GPU
// and is only known through hipGetSymbolAddress (host code must never pass the
// array's own name to a kernel), so it is looked up once per device, with that
// device current, on the first call there.  The split kernel writes every
// split's partial (empty splits included) before the merge reads them, so
// nothing needs clearing between calls; calls that overlap on one GPU share the
// array and race.
namespace {
constexpr int64_t kNoAllocScratchFloats = 1 << 20;  // 4 MiB: n_heads * splits * (head_dim + 4)
__device__ __align__(256) float scratch[kNoAllocScratchFloats];
float* g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(float** out, hipStream_t st) {
    int dev = 0;
    const int rc = current_device(&dev);
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch_ptr[dev]) {
        // the address is looked up on the first call on each device; that lookup is
        // not a stream operation, so it is kept out of stream capture
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        ASMHIP_TRY(hipStreamIsCapturing(st, &cs));
        if (cs != hipStreamCaptureStatusNone)
            return fail(kInvalidArgument,
                        "attention without a workspace: the first call on a device must be made outside stream "
                        "capture (it looks up the device's scratch address); make one call before capturing");
        void* p = nullptr;
        ASMHIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(kHipError, "hipGetSymbolAddress returned no address for the attention scratch");
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return kOk;
}
}  // namespace

extern "C" int asmhip_stream_read(const void* buf, int64_t bytes, void* sink, void* stream) {
    return stream_read_launch(buf, bytes, static_cast<uint32_t*>(sink), (hipStream_t)stream);
}

extern "C" int asmhip_stream_read_shaped(const void* buf, int64_t bytes, const float* x, int xn, float* y,
                                         int64_t y_floats, int flags, int lds, void* sink, void* stream) {
    return shaped_read_launch(buf, bytes, x, xn, y, y_floats, flags, lds, static_cast<uint32_t*>(sink),
                              (hipStream_t)stream);
}

extern "C" int asmhip_matmul_q4_0_stamped(const void* blocks, const float* x, float* y, int64_t M, int64_t K,
                                          uint64_t* stamps, int64_t stamps_len, void* stream) {
    if (!blocks || !x || !y) return fail(kInvalidArgument, "null pointer argument");
    return q4_0_mfma_stamped_launch(blocks, x, y, M, K, stamps, stamps_len, (hipStream_t)stream);
}

extern "C" int asmhip_empty_launch(int grid, int threads, int lds, void* stream) {
    return empty_launch(grid, threads, lds, (hipStream_t)stream);
}

extern "C" int asmhip_grid_barrier(unsigned* counter, int n, unsigned* err, void* stream) {
    return grid_barrier_launch(counter, n, err, (hipStream_t)stream);
}

extern "C" int64_t asmhip_attention_decode_noalloc_max_floats(void) { return kNoAllocScratchFloats; }

extern "C" int asmhip_attention_decode_rope_noalloc(const float* qkv, void* k_cache, void* v_cache, float* out,
                                                    int n_heads, int n_kv_heads, int head_dim, const int* pos_dev,
                                                    int max_ctx, float theta, void* stream) {
    if (!qkv || !k_cache || !v_cache || !out || !pos_dev) return fail(kInvalidArgument, "null pointer argument");
    if (n_heads <= 0 || head_dim <= 0 || max_ctx <= 0 || head_dim % 2)
        return fail(kInvalidArgument, "bad attention shape");
    const int64_t need = attn_decode_workspace(n_heads, head_dim, max_ctx);
    if (need > kNoAllocScratchFloats)
        return fail(kInvalidArgument,
                    "attention without a workspace: n_heads %d x %d splits x (head_dim %d + 4) = %lld floats "
                    "exceeds the %lld-float scratch; pass a workspace to asmhip_attention_decode_rope",
                    n_heads, attn_decode_splits(max_ctx), head_dim, (long long)need,
                    (long long)kNoAllocScratchFloats);
    float* part = nullptr;
    const int rc = scratch_for_current_device(&part, (hipStream_t)stream);
    if (rc) return rc;
    return attn_decode_launch(qkv, k_cache, v_cache, part, out, n_heads, n_kv_heads, head_dim, pos_dev, max_ctx,
                              true, theta, (hipStream_t)stream);
}

extern "C" int asmhip_embed_q4_0(const void* table, const int* token_dev, float* x, int n_vocab, int dim,
                                 void* stream) {
    if (!table || !token_dev || !x) return fail(kInvalidArgument, "null pointer argument");
    if (n_vocab <= 0 || dim <= 0) return fail(kInvalidArgument, "bad embedding shape");
    return embed_launch(QuantType::Q4_0, table, token_dev, x, n_vocab, dim, (hipStream_t)stream);
}

extern "C" int asmhip_embed_q8_0(const void* table, const int* token_dev, float* x, int n_vocab, int dim,
                                 void* stream) {
    if (!table || !token_dev || !x) return fail(kInvalidArgument, "null pointer argument");
    if (n_vocab <= 0 || dim <= 0) return fail(kInvalidArgument, "bad embedding shape");
    return embed_launch(QuantType::Q8_0, table, token_dev, x, n_vocab, dim, (hipStream_t)stream);
}

extern "C" int asmhip_argmax(const float* logits, int n, int* token_dev, int* pos_dev, void* stream) {
    if (!logits || !token_dev) return fail(kInvalidArgument, "null pointer argument");
    return argmax_launch(logits, n, token_dev, pos_dev, (hipStream_t)stream);
}

extern "C" int asmhip_argmax_history(const float* logits, int n, int* token_dev, int* pos_dev, int* history_dev,
                                     int history_len, void* stream) {
    if (!logits || !token_dev || !pos_dev || !history_dev) return fail(kInvalidArgument, "null pointer argument");
    return argmax_launch(logits, n, token_dev, pos_dev, (hipStream_t)stream, history_dev, history_len);
}

// ---- plumbing --------------------------------------------------------------------

extern "C" int asmhip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

extern "C" int asmhip_device_info(char* name, size_t name_len, int* compute_units, int* clock_khz,
                                  size_t* total_mem) {
    int dev = 0;
    int rc = current_device(&dev);
    if (rc) return rc;
    hipDeviceProp_t p;
    ASMHIP_TRY(hipGetDeviceProperties(&p, dev));
    if (name && name_len) {
        snprintf(name, name_len, "%s", p.gcnArchName);
    }
    if (compute_units) *compute_units = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    if (total_mem) *total_mem = p.totalGlobalMem;
    return kOk;
}

extern "C" void* asmhip_malloc(size_t bytes) {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        hip_fail(e, "hipMalloc");
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}

extern "C" int asmhip_free(void* ptr) {
    if (!ptr) return kOk;
    ASMHIP_TRY(hipFree(ptr));
    return kOk;
}

extern "C" int asmhip_memcpy(void* dst, const void* src, size_t bytes, int kind) {
    hipMemcpyKind k;
    switch (kind) {
        case 1: k = hipMemcpyHostToDevice; break;
        case 2: k = hipMemcpyDeviceToHost; break;
        case 3: k = hipMemcpyDeviceToDevice; break;
        default: return fail(kInvalidArgument, "memcpy kind %d (use 1 h2d, 2 d2h, 3 d2d)", kind);
    }
    if (!bytes) return kOk;
    if (!dst || !src) return fail(kInvalidArgument, "null pointer argument");
    ASMHIP_TRY(hipMemcpy(dst, src, bytes, k));
    return kOk;
}

extern "C" int asmhip_synchronize(void) {
    ASMHIP_TRY(hipDeviceSynchronize());
    return kOk;
}

extern "C" void* asmhip_stream_create(void) {
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) {
        hip_fail(e, "hipStreamCreateWithFlags");
        return nullptr;
    }
    return (void*)s;
}

extern "C" int asmhip_stream_destroy(void* stream) {
    if (!stream) return kOk;
    ASMHIP_TRY(hipStreamDestroy((hipStream_t)stream));
    return kOk;
}

extern "C" int asmhip_stream_synchronize(void* stream) {
    ASMHIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return kOk;
}

extern "C" void* asmhip_event_create(void) {
    hipEvent_t e = nullptr;
    hipError_t r = hipEventCreate(&e);
    if (r != hipSuccess) {
        hip_fail(r, "hipEventCreate");
        return nullptr;
    }
    return (void*)e;
}

extern "C" void* asmhip_event_create_timing(void) {
    hipEvent_t e = nullptr;
    hipError_t r = hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
    if (r != hipSuccess) {
        hip_fail(r, "hipEventCreateWithFlags");
        return nullptr;
    }
    return (void*)e;
}

extern "C" int asmhip_event_destroy(void* event) {
    if (!event) return kOk;
    ASMHIP_TRY(hipEventDestroy((hipEvent_t)event));
    return kOk;
}

extern "C" int asmhip_event_record(void* event, void* stream) {
    if (!event) return fail(kInvalidArgument, "null event");
    ASMHIP_TRY(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
    return kOk;
}

extern "C" int asmhip_event_synchronize(void* event) {
    if (!event) return fail(kInvalidArgument, "null event");
    ASMHIP_TRY(hipEventSynchronize((hipEvent_t)event));
    return kOk;
}

extern "C" int asmhip_event_elapsed_ms(void* start, void* stop, float* ms) {
    if (!start || !stop || !ms) return fail(kInvalidArgument, "null argument");
    ASMHIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return kOk;
}

extern "C" int asmhip_stream_begin_capture(void* stream) {
    if (!stream) return fail(kInvalidArgument, "capture needs a created stream, not the default stream");
    ASMHIP_TRY(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
    return kOk;
}

extern "C" int asmhip_stream_end_capture(void* stream, void** graph_exec) {
    if (!stream || !graph_exec) return fail(kInvalidArgument, "null argument");
    hipGraph_t graph = nullptr;
    ASMHIP_TRY(hipStreamEndCapture((hipStream_t)stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    *graph_exec = (void*)exec;
    return kOk;
}

extern "C" int asmhip_graph_launch(void* graph_exec, void* stream) {
    if (!graph_exec) return fail(kInvalidArgument, "null graph");
    ASMHIP_TRY(hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream));
    return kOk;
}

extern "C" int asmhip_graph_destroy(void* graph_exec) {
    if (!graph_exec) return kOk;
    ASMHIP_TRY(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
    return kOk;
}

extern "C" const char* asmhip_last_error(void) { return g_last_error; }
