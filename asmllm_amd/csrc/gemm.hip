// Q8_0 x Q8_0 prefill GEMM on the matrix cores of gfx950.
//
// C[t][j] = sum_b (sum_k a[t,b,k] w[j,b,k]) * (d_w[j,b] * d_a[t,b])
//
// A is T rows of activations and W is M rows of weights, both GGUF Q8_0 blocks
// (fp16 d + 32 int8); C is fp32 [T][M].  The semantics are those of the
// reference's quantized-activation recipe (int32 block dot, scvtf, product of
// the two scales, fmadd: src/kernels/arm64/matmul_q4_neon.S:190-255), applied
// block by block in order.
//
// Per 32x32 output tile and block, two matrix instructions and two VALU ones:
//   v_mfma_i32_32x32x32_i8   the exact int32 block dots;
//   v_mfma_f32_32x32x2_f32   the outer product d_a (x) d_w of the block scales
//                            (K = 2 with the second slice zero), which lands in
//                            the same lane/register layout as the dots;
//   v_cvt_f32_i32 + v_fma    acc += float(dot) * scale, in block order.
// The scale product on the matrix pipe keeps the VALU at two instructions per
// output and block (the bound of this GEMM: every output needs its own scale
// in every block).
//
// Work mapping: a workgroup of 4 waves computes a 64 (T) x 128 (M) tile; wave
// (wt, wm) owns rows 32 wt.. and columns 64 wm.. (two 32x32 tiles).  K goes in
// steps of 4 blocks: the workgroup stages the step's 64 + 128 block rows in LDS
// with qs realigned to 32-byte rows (padded to 144 bytes: conflict-free 16-byte
// operand reads) and scales widened to fp32, double-buffered, the next step's
// global loads in flight during the current step's MFMAs.
#include "common.hpp"
#include "kernels.hpp"

namespace asmhip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kTT = 64;            // T rows per workgroup
constexpr int kTM = 128;           // M columns per workgroup
constexpr int kKB = 4;             // blocks per K step
constexpr int kPitch = kKB * 32 + 16;  // LDS bytes per staged row of qs
constexpr int kThreadsG = 256;
constexpr int kStageBlocks = (kTT + kTM) * kKB;            // 768
constexpr int kPerThread = kStageBlocks / kThreadsG;       // 3
constexpr uint32_t kPastEnd = 0xFFFFFF00u;
// LDS of one stage: qs of A and W rows, then their fp32 scales
constexpr int kStageBytes = (kTT + kTM) * kPitch + (kTT + kTM) * kKB * 4;

static_assert(kStageBlocks % kThreadsG == 0, "staging splits evenly");

struct Staged {
    uint32_t dw[9];  // dwords covering the 32 qs bytes (the ninth: its low half only)
    uint32_t d16;    // the fp16 scale
};

__global__ __launch_bounds__(kThreadsG) void gemm_q8_0_kernel(const uint8_t* __restrict__ w,
                                                              const uint8_t* __restrict__ a,
                                                              float* __restrict__ c, int T, int M, int K) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int nb = K >> 5;
    const uint32_t row_bytes = (uint32_t)nb * 34u;
    const int t0 = blockIdx.y * kTT, j0 = blockIdx.x * kTM;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wt = wave >> 1, wm = wave & 1;
    const auto ar = make_rsrc(a, row_bytes * (uint32_t)T);
    const auto wr = make_rsrc(w, row_bytes * (uint32_t)M);

    // this thread's staged blocks: index ib = tid + 256 i; A blocks first
    auto fetch = [&](Staged* st, int kb0) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int ib = (int)threadIdx.x + kThreadsG * i;
            const bool is_a = ib < kTT * kKB;
            const int local = is_a ? ib : ib - kTT * kKB;
            const int row = local / kKB, blk = local - row * kKB;
            const int grow = (is_a ? t0 : j0) + row;
            const bool live = kb0 + blk < nb;  // rows past T / M fall beyond the buffer
            const uint32_t addr = (uint32_t)grow * row_bytes + (uint32_t)(kb0 + blk) * 34u;
            const uint32_t q = addr + 2u;  // first qs byte
            const uint32_t p = live ? (q & ~3u) : kPastEnd;
            const auto r = is_a ? ar : wr;
#pragma unroll
            for (int k = 0; k < 8; ++k) st[i].dw[k] = buf_load_b32(r, p + 4u * k);
            // the last two qs bytes when the block starts on a dword: a full dword
            // would reach past the block (and past the buffer for the last block)
            st[i].dw[8] = buf_load_u16(r, p + 32u);
            st[i].d16 = buf_load_u16(r, live ? addr : kPastEnd);
        }
    };
    auto park = [&](const Staged* st, uint8_t* stage, int kb0) {
        uint8_t* qs_base = stage;
        float* sc_base = reinterpret_cast<float*>(stage + (kTT + kTM) * kPitch);
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int ib = (int)threadIdx.x + kThreadsG * i;
            const bool is_a = ib < kTT * kKB;
            const int local = is_a ? ib : ib - kTT * kKB;
            const int row = local / kKB, blk = local - row * kKB;
            const int srow = (is_a ? 0 : kTT) + row;
            const int grow = (is_a ? t0 : j0) + row;
            const uint32_t q = (uint32_t)grow * row_bytes + (uint32_t)(kb0 + blk) * 34u + 2u;
            const uint32_t sh = q & 3u;  // 0 or 2
            uint32_t o[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = __builtin_amdgcn_alignbyte(st[i].dw[k + 1], st[i].dw[k], sh);
            uint4* dst = reinterpret_cast<uint4*>(qs_base + srow * kPitch + blk * 32);
            dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
            dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
            sc_base[srow * kKB + blk] = __half2float(__ushort_as_half((unsigned short)st[i].d16));
        }
    };

    const int m = lane & 31, g = lane >> 5;
    v16f acc[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[nt][i] = 0.f;

    const int nsteps = (nb + kKB - 1) / kKB;
    Staged st[kPerThread];
    fetch(st, 0);
    for (int s = 0; s < nsteps; ++s) {
        uint8_t* stage = lds + (s & 1) * kStageBytes;
        park(st, stage, s * kKB);
        __syncthreads();
        if (s + 1 < nsteps) fetch(st, (s + 1) * kKB);
        const uint8_t* qs_base = stage;
        const float* sc_base = reinterpret_cast<const float*>(stage + (kTT + kTM) * kPitch);
        const int arow = 32 * wt + m;
#pragma unroll 1
        for (int blk = 0; blk < kKB; ++blk) {
            const v4i av = *reinterpret_cast<const v4i*>(qs_base + arow * kPitch + blk * 32 + 16 * g);
            const float da = g == 0 ? sc_base[arow * kKB + blk] : 0.f;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int wrow = kTT + 64 * wm + 32 * nt + m;
                const v4i bv = *reinterpret_cast<const v4i*>(qs_base + wrow * kPitch + blk * 32 + 16 * g);
                const float dw = g == 0 ? sc_base[wrow * kKB + blk] : 0.f;
                const v16i zi = {};
                const v16f zf = {};
                const v16i dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zi, 0, 0, 0);
                const v16f sc = __builtin_amdgcn_mfma_f32_32x32x2f32(da, dw, zf, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[nt][i] = fmaf((float)dot[i], sc[i], acc[nt][i]);
            }
        }
    }

    // lane l, register i holds row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32 of a 32x32 tile
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int col = j0 + 64 * wm + 32 * nt + m;
        if (col >= M) continue;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = t0 + 32 * wt + 8 * (i / 4) + 4 * g + i % 4;
            if (row < T) c[(size_t)row * M + col] = acc[nt][i];
        }
    }
}

}  // namespace

int gemm_q8_0_launch(const void* w, const void* a, float* c, int64_t T, int64_t M, int64_t K, hipStream_t st) {
    if (T <= 0 || M <= 0 || K <= 0 || K % 32)
        return fail(kInvalidArgument, "gemm: need T, M, K > 0 and K %% 32 == 0 (got T=%lld M=%lld K=%lld)",
                    (long long)T, (long long)M, (long long)K);
    const int64_t row_bytes = K / 32 * 34;
    if ((T + kTT) * row_bytes >= (int64_t)kPastEnd || (M + kTM) * row_bytes >= (int64_t)kPastEnd)
        return fail(kInvalidArgument, "gemm: operands above 4 GB are not supported");
    if ((uintptr_t)w % 4 || (uintptr_t)a % 4) return fail(kInvalidArgument, "gemm: blocks must be 4-byte aligned");
    const dim3 grid((unsigned)((M + kTM - 1) / kTM), (unsigned)((T + kTT - 1) / kTT));
    if (grid.y > 65535) return fail(kInvalidArgument, "gemm: T too large");
    const size_t lds = 2 * (size_t)kStageBytes;
    const int rc = dynamic_lds((const void*)gemm_q8_0_kernel, lds);
    if (rc) return rc;
    hipLaunchKernelGGL(gemm_q8_0_kernel, grid, dim3(kThreadsG), lds, st, static_cast<const uint8_t*>(w),
                       static_cast<const uint8_t*>(a), c, (int)T, (int)M, (int)K);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

}  // namespace asmhip
