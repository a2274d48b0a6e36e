// Q8_0 x Q8_0 prefill GEMM on the matrix cores of gfx950.
//
// C[t][j] = sum_b (sum_k a[t,b,k] w[j,b,k]) * (d_w[j,b] * d_a[t,b])
//
// A is T rows of activations and W is M rows of weights, both GGUF Q8_0 blocks
// (fp16 d + 32 int8); C is fp32 [T][M].  The semantics are those of the
// reference's quantized-activation recipe (int32 block dot, scvtf, product of
// the two scales, fmadd: src/kernels/arm64/matmul_q4_neon.S:190-255), applied
// block by block in order; the result is bitwise that of the CPU oracle.
//
// Per 32x32 output tile and block, two matrix instructions and two VALU ones:
//   v_mfma_i32_32x32x32_i8   the exact int32 block dots;
//   v_mfma_f32_32x32x8_f16   the outer product of the raw fp16 block scales
//                            (each placed in both lane halves: 2 d_a d_w,
//                            exact in fp32), in the same lane/register layout
//                            as the dots;
//   v_cvt_f32_i32 + v_fma    acc += float(dot) * 2 d_a d_w, in block order;
// the result is halved (exactly) at the store.  The scale product on the
// matrix pipe keeps the VALU at two instructions per output and block, the
// bound of this GEMM: every output needs its own scale in every block.
//
// Work mapping: a workgroup computes a 64 (T) x 128 (M) tile, as 8 waves of
// one 32x32 tile on the coalesced path below (4 waves of two on the general
// path: wave (wt, wm) owns rows 32 wt.. and columns 64 wm..).
// Fast path (K % 64 == 0): K goes in steps of two blocks; a row's step is 68
// contiguous bytes, fetched as the 16-byte aligned 80-byte window around them
// with 16-byte loads by consecutive lanes and parked raw in LDS (two stages side
// by side in each row, row stride an odd number of dwords: conflict-free operand
// reads), with the next two steps' loads in flight.  Other K: blocks are staged
// one by one with qs realigned on the way into LDS.
// gemm_q8_split takes the split operands of asm_matmul_q8 (int8 qs planes and
// fp32 scale planes) with the same tiling; see its comment.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace asmhip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr int kTT = 64;            // T rows per workgroup
constexpr int kTM = 128;           // M columns per workgroup
constexpr int kThreadsG = 256;
constexpr uint32_t kPastEnd = 0xFFFFFF00u;

// Geometry of a K step of KB blocks.
template <int KB>
struct Step {
    static constexpr int kPitch = KB * 32 + 16;                                   // LDS bytes per staged row of qs
    static constexpr int kBlocks = (kTT + kTM) * KB;                              // blocks staged per step
    static constexpr int kPerThread = (kBlocks + kThreadsG - 1) / kThreadsG;
    static constexpr int kBytes = (kTT + kTM) * kPitch + (kTT + kTM) * KB * 4;    // qs rows, then fp32 scales
};

struct Staged {
    uint32_t dw[9];  // dwords covering the 32 qs bytes (the ninth: its low half only)
    uint32_t d16;    // the fp16 scale
};

template <int KB, bool kPipe>
__global__ __launch_bounds__(kThreadsG) void gemm_q8_0_kernel(const uint8_t* __restrict__ w,
                                                              const uint8_t* __restrict__ a,
                                                              float* __restrict__ c, int T, int M, int K) {
    using S = Step<KB>;
    constexpr int kKB = KB, kPitch = S::kPitch, kPerThread = S::kPerThread, kStageBytes = S::kBytes;
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
            if (ib >= S::kBlocks) break;  // wave-uniform
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
            if (ib >= S::kBlocks) break;
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
        // block blk, column tile nt: exact int32 dots and the scale outer product
        auto issue = [&](int blk, v16i* dot, v16f* scl) {
            const v4i av = *reinterpret_cast<const v4i*>(qs_base + arow * kPitch + blk * 32 + 16 * g);
            const float da = g == 0 ? sc_base[arow * kKB + blk] : 0.f;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int wrow = kTT + 64 * wm + 32 * nt + m;
                const v4i bv = *reinterpret_cast<const v4i*>(qs_base + wrow * kPitch + blk * 32 + 16 * g);
                const float dw = g == 0 ? sc_base[wrow * kKB + blk] : 0.f;
                const v16i zi = {};
                const v16f zf = {};
                dot[nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zi, 0, 0, 0);
                scl[nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(da, dw, zf, 0, 0, 0);
            }
        };
        auto retire = [&](const v16i* dot, const v16f* scl) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[nt][i] = fmaf((float)dot[nt][i], scl[nt][i], acc[nt][i]);
        };
        if (kPipe) {
            // block b+1's matrix work is issued before block b's epilogue
            v16i dot[2][2];
            v16f scl[2][2];
            issue(0, dot[0], scl[0]);
#pragma unroll
            for (int blk = 1; blk < kKB; ++blk) {
                issue(blk, dot[blk & 1], scl[blk & 1]);
                __builtin_amdgcn_sched_barrier(0);
                retire(dot[(blk - 1) & 1], scl[(blk - 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
            retire(dot[(kKB - 1) & 1], scl[(kKB - 1) & 1]);
        } else {
#pragma unroll 1
            for (int blk = 0; blk < kKB; ++blk) {
                v16i dot[2];
                v16f scl[2];
                issue(blk, dot, scl);
                retire(dot, scl);
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

// ---------------------------------------------------------------------------
// Coalesced variant (K % 64 == 0): a step's K chunk of a row is KB * 34
// contiguous bytes, fetched with aligned 16-byte loads by consecutive lanes and
// parked raw in LDS; a row's two stages sit side by side and rows are an odd
// number of dwords apart (lanes of a 32-row operand read land in distinct
// banks).  The even block's qs start 2 bytes past a dword and are read in
// another order of k (raw_qs).
// ---------------------------------------------------------------------------
template <int KB, int NTH, int TT, int TM>
struct RawStep {
    static constexpr int kChunk = KB * 34;                        // bytes of a row's K chunk
    static constexpr int kPieces = (kChunk + 12 + 15) / 16;       // 16-byte loads per row (the chunk starts
                                                                  // up to 12 bytes into its aligned window)
    static constexpr int kStageOff = kPieces * 16;                // stage 1 of a row follows stage 0
    static constexpr int kRowStride = ((2 * kStageOff / 4) | 1) * 4;  // odd number of dwords
    static constexpr int kRows = TT + TM;
    static constexpr int kTotal = kRows * kPieces;
    static constexpr int kPerThread = (kTotal + NTH - 1) / NTH;
    static constexpr int kBytes = kRows * kRowStride + 2 * kStageOff;  // + a dead slot's landing place
};

// 16 qs bytes of block BLK (of a dword-aligned pair) for lane group g.  The odd
// block's qs are dword aligned.  The even block's start 2 bytes past a dword,
// after its scale: lane group g reads the pair's aligned dwords 4g..4g+3, and
// group 0 (selector 0x07060100; group 1 passes 0x07060504, the identity) puts
// q30 and q31, the low half of dword 8, in place of the scale's two bytes.  The
// 32 qs then sit in another order of k than the block's, the same order for A
// and W, so the int32 dot is unchanged.
template <int BLK>
__device__ __forceinline__ v4i raw_qs(const uint8_t* row, int g, uint32_t sel) {
    if constexpr (BLK == 1) {
        const uint32_t* d = reinterpret_cast<const uint32_t*>(row + 36 + 16 * g);
        return v4i{(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
    } else {
        const uint32_t* d = reinterpret_cast<const uint32_t*>(row + 16 * g);
        const uint32_t tail = *reinterpret_cast<const uint32_t*>(row + 32);
        return v4i{(int)__builtin_amdgcn_perm(d[0], tail, sel), (int)d[1], (int)d[2], (int)d[3]};
    }
}

// A 32x32x8 f16 MFMA operand holding the block's raw fp16 scale in its first
// half (the 16-bit LDS read zero-extends): with the scale in both lane halves
// of A and B, D = 2 d_a d_w exactly.
template <int BLK>
__device__ __forceinline__ v4h raw_scale(const uint8_t* row) {
    typedef uint32_t v2u __attribute__((ext_vector_type(2)));
    uint32_t d = *reinterpret_cast<const uint16_t*>(row + 34 * BLK);
    asm("" : "+v"(d));  // an opaque dword: the pair is built without masking the high half again
    return __builtin_bit_cast(v4h, (v2u){d, 0u});
}

// A workgroup computes a TT x TM tile with (TT / 32) x (TM / (32 WT)) waves,
// each of WT 32x32 tiles side by side (WT = 1: one tile a wave, twice the waves
// of WT = 2 to hide each wave's MFMA -> epilogue latency).  Two K steps of
// loads in flight per thread.  The loop body is written once for each step of
// a four-step cycle (stage s % 2, window shift 4 (s % 4) bytes), so every LDS
// address is a per-lane base plus a constant.  The register budget is held to
// six waves per SIMD (80 VGPRs).
template <int KB, int WT, int TT, int TM>
__global__ __launch_bounds__(TT * TM / (16 * WT)) __attribute__((amdgpu_waves_per_eu(6))) void gemm_q8_0_coalesced(const uint8_t* __restrict__ w,
                                                               const uint8_t* __restrict__ a,
                                                               float* __restrict__ c, int T, int M, int K,
                                                               int tiles_t, int n_tiles) {
    constexpr int MW = TM / (32 * WT), NTH = (TT / 32) * MW * 64;  // waves along M; threads
    using S = RawStep<KB, NTH, TT, TM>;
    static_assert(TT * S::kPieces % 64 == 0 && NTH % 64 == 0, "every wave's load slot is all A or all W");
    static_assert(KB == 2, "a step's window shift 4 (s % 4) holds for 68-byte steps");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    // XCD-aware tile order: workgroup ids are dealt round-robin to the 8 XCDs,
    // so id -> (xcd = id % 8, j = id / 8) -> tile xcd * chunk + j gives each XCD
    // a run of consecutive tiles, T fastest: the T tiles sharing a weight tile
    // meet in one L2.  The grid is padded to a multiple of 8; extra ids exit.
    const int chunk = (int)gridDim.x >> 3;
    const int tile = ((int)blockIdx.x & 7) * chunk + ((int)blockIdx.x >> 3);
    if (tile >= n_tiles) return;
    const int nb = K >> 5;
    const uint32_t row_bytes = (uint32_t)nb * 34u;
    const uint32_t a_bytes = row_bytes * (uint32_t)T, w_bytes = row_bytes * (uint32_t)M;
    const int t0 = (tile % tiles_t) * TT, j0 = (tile / tiles_t) * TM;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wt = wave / MW, wm = wave % MW;

    // piece q = (staged row q / kPieces, 16-byte piece q % kPieces); A rows first.
    // Slots past the last piece load from past the buffer (zeros, no access) and
    // park in the stage's spare dwords.
    uint32_t goff[S::kPerThread], loff[S::kPerThread];
    bool is_a[S::kPerThread];
#pragma unroll
    for (int i = 0; i < S::kPerThread; ++i) {
        const int q = (int)threadIdx.x + NTH * i;
        const bool live = q < S::kTotal;
        const int qq = live ? q : 0;
        const int r = qq / S::kPieces, k = qq - r * S::kPieces;
        is_a[i] = r < TT;
        const int grow = is_a[i] ? t0 + r : j0 + (r - TT);
        goff[i] = live ? (uint32_t)grow * row_bytes + 16u * (uint32_t)k : kPastEnd;
        loff[i] = live ? (uint32_t)(r * S::kRowStride + 16 * k) : (uint32_t)(S::kRows * S::kRowStride);
    }
    uint4 pre[2][S::kPerThread];  // two steps of loads in flight
    // A's pieces end at piece TT kPieces, a multiple of 64, and NTH is a multiple
    // of 64, so every wave's slot i is all A or all W: the choice of buffer is
    // wave-uniform (made scalar here; a per-lane choice of descriptor would turn
    // every load into a waterfall loop).
    bool a_wave[S::kPerThread];
#pragma unroll
    for (int i = 0; i < S::kPerThread; ++i) a_wave[i] = __builtin_amdgcn_readfirstlane((int)is_a[i]) != 0;
    // Step s of a row is the 16-byte aligned window of 80 bytes holding its 68
    // (kb0 * 34 rounded down to 16: the window starts 4 (s % 4) bytes early), so
    // every 16-byte load is aligned.  The window's offset goes into the
    // descriptors (base advanced, size cut by the same amount): the per-slot
    // offsets stay fixed, and the range check still ends at each buffer's last
    // byte (a window that runs past it reads zeros for the dwords beyond).
    auto fetch = [&](uint4* dst, int kb0) {
        const uint32_t kofs = ((uint32_t)kb0 * 34u) & ~15u;
        const auto ar = make_rsrc(a + kofs, a_bytes - kofs);
        const auto wr = make_rsrc(w + kofs, w_bytes - kofs);
#pragma unroll
        for (int i = 0; i < S::kPerThread; ++i) dst[i] = buf_load_b128(a_wave[i] ? ar : wr, goff[i]);
    };
    auto park = [&](const uint4* src, uint8_t* stage) {
#pragma unroll
        for (int i = 0; i < S::kPerThread; ++i) {
            uint32_t* d = reinterpret_cast<uint32_t*>(stage + loff[i]);  // 4-byte aligned
            d[0] = src[i].x;
            d[1] = src[i].y;
            d[2] = src[i].z;
            d[3] = src[i].w;
        }
    };

    const int m = lane & 31, g = lane >> 5;
    const uint32_t sel = g ? 0x07060504u : 0x07060100u;
    v16f acc[WT];
#pragma unroll
    for (int nt = 0; nt < WT; ++nt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[nt][i] = 0.f;

    const int nsteps = nb / KB;
    fetch(pre[0], 0);
    fetch(pre[1], min(1, nsteps - 1) * KB);
    // step s parks in stage s % 2 of every row; its data start 4 (s % 4) bytes
    // into the stage.  Both stages of a row sit side by side, so one base
    // address per row serves both with offsets the LDS instructions carry.
    auto step = [&](auto s4_c, int s) {
        constexpr int S4 = decltype(s4_c)::value;
        uint8_t* stage = lds + (S4 & 1) * S::kStageOff;
        park(pre[S4 & 1], stage);
        __syncthreads();
        // unconditional, so the loop body stays one basic block: the last two
        // steps load the last step again, into registers that are never parked
        fetch(pre[S4 & 1], min(s + 2, nsteps - 1) * KB);
        const uint8_t* arow = stage + (32 * wt + m) * S::kRowStride + 4 * S4;
        const uint8_t* wrow = stage + (TT + 32 * WT * wm + m) * S::kRowStride + 4 * S4;
        // block BLK (0 or 1) of the dword-aligned pair at byte 68 bp: operands,
        // then the matrix instructions back to back, then the epilogue
        auto block = [&](auto blk_c, int bp) {
            constexpr int BLK = decltype(blk_c)::value;
            const uint8_t* ar_ = arow + 68 * bp;
            const v4i av = raw_qs<BLK>(ar_, g, sel);
            const v4h da = raw_scale<BLK>(ar_);
            v4i bv[WT];
            v4h dw[WT];
#pragma unroll
            for (int nt = 0; nt < WT; ++nt) {
                const uint8_t* w_ = wrow + 32 * nt * S::kRowStride + 68 * bp;
                bv[nt] = raw_qs<BLK>(w_, g, sel);
                dw[nt] = raw_scale<BLK>(w_);
            }
            __builtin_amdgcn_sched_barrier(0);
            const v16i zi = {};
            const v16f zf = {};
            v16i dd[WT];
            v16f ss[WT];
#pragma unroll
            for (int nt = 0; nt < WT; ++nt) {
                dd[nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv[nt], zi, 0, 0, 0);
                ss[nt] = __builtin_amdgcn_mfma_f32_32x32x8f16(da, dw[nt], zf, 0, 0, 0);  // 2 d_a d_w
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int nt = 0; nt < WT; ++nt)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[nt][i] = fmaf((float)dd[nt][i], ss[nt][i], acc[nt][i]);
        };
#pragma unroll
        for (int bp = 0; bp < KB / 2; ++bp) {
            block(std::integral_constant<int, 0>{}, bp);
            block(std::integral_constant<int, 1>{}, bp);
        }
    };
    int s = 0;
    for (; s + 3 < nsteps; s += 4) {
        step(std::integral_constant<int, 0>{}, s);
        step(std::integral_constant<int, 1>{}, s + 1);
        step(std::integral_constant<int, 2>{}, s + 2);
        step(std::integral_constant<int, 3>{}, s + 3);
    }
    if (s < nsteps) step(std::integral_constant<int, 0>{}, s);
    if (s + 1 < nsteps) step(std::integral_constant<int, 1>{}, s + 1);
    if (s + 2 < nsteps) step(std::integral_constant<int, 2>{}, s + 2);

#pragma unroll
    for (int nt = 0; nt < WT; ++nt) {
        const int col = j0 + 32 * WT * wm + 32 * nt + m;
        if (col >= M) continue;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = t0 + 32 * wt + 8 * (i / 4) + 4 * g + i % 4;
            if (row < T) c[(size_t)row * M + col] = 0.5f * acc[nt][i];  // the scales entered doubled
        }
    }
}


// ---------------------------------------------------------------------------
// Tiled variant: the operands in the GEMM tile layout (gemm_tiled_offset), so a
// workgroup's K step is one contiguous run per operand: TT rows x 68 bytes of A
// and TM rows x 68 bytes of W.  Each wave's 16-byte buffer loads write LDS
// themselves (buffer_load_dwordx4 ... lds: lane i lands at M0 + 16 i), so a
// run lands as it lies: rows 68 bytes (17 dwords, odd) apart, conflict-free
// operand reads, no staging registers and no LDS write instructions.  Three
// stages, two steps in flight.  The compiler cannot tell the stages apart for
// its own LDS-DMA wait bookkeeping (it would wait for every load in flight
// before each LDS read), so the loads are issued from inline asm and each step
// waits by count for its own loads only (s_waitcnt vmcnt), then a bare barrier.
// ---------------------------------------------------------------------------
template <int TT, int TM>
struct DmaStep {
    static constexpr int kARegion = (TT * 68 + 1023) / 1024 * 1024;  // A rows, padded to whole 1 KB loads
    static constexpr int kWRegion = (TM * 68 + 1023) / 1024 * 1024;
    static constexpr int kLoads = (kARegion + kWRegion) / 1024;      // wave-wide 1 KB loads per step
    static constexpr int kALoads = kARegion / 1024;
    static constexpr int kStage = kARegion + kWRegion + 1024;         // + the landing place of padding loads
};

// The dwords of a raw buffer descriptor (base, stride 0, size; word 3 as
// make_rsrc), for use as an asm operand.
__device__ __forceinline__ v4i raw_rsrc(const void* base, uint32_t bytes) {
    const uint64_t p = (uint64_t)base;
    return v4i{(int)(uint32_t)p, (int)(uint32_t)((p >> 32) & 0xFFFFu), (int)bytes, 0x00020000};
}

template <int TT, int TM>
__global__ __launch_bounds__(TT * TM / 16) __attribute__((amdgpu_waves_per_eu(6))) void gemm_q8_0_tiled(
    const uint8_t* __restrict__ w, const uint8_t* __restrict__ a, float* __restrict__ c, int T, int M, int K,
    int tiles_t, int n_tiles) {
    constexpr int MW = TM / 32, NW = (TT / 32) * MW;  // waves along M; waves
    using S = DmaStep<TT, TM>;
    constexpr int kPerWave = (S::kLoads + NW - 1) / NW;  // loads each wave issues per step (padding ones too)
    __shared__ __attribute__((aligned(1024))) uint8_t st0[S::kStage];
    __shared__ __attribute__((aligned(1024))) uint8_t st1[S::kStage];
    __shared__ __attribute__((aligned(1024))) uint8_t st2[S::kStage];
    // XCD-aware tile order, as gemm_q8_0_coalesced
    const int chunk = (int)gridDim.x >> 3;
    const int tile = ((int)blockIdx.x & 7) * chunk + ((int)blockIdx.x >> 3);
    if (tile >= n_tiles) return;
    const int nsteps = K >> 6;
    const int tt = tile % tiles_t, tm = tile / tiles_t;
    const int t0 = tt * TT, j0 = tm * TM;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wt = wave / MW, wm = wave % MW;
    const uint8_t* abase = a + (size_t)tt * nsteps * (TT * 68);
    const uint8_t* wbase = w + (size_t)tm * nsteps * (TM * 68);
    // Step s into stage ST: load j = wave + NW u of the step's 1 KB loads, A's
    // first; loads past the last one read past the buffer (zeros, no access)
    // into the stage's spare kilobyte, so every wave issues kPerWave.
    auto fetch = [&](auto stage_c, int s) {
        constexpr int ST = decltype(stage_c)::value;
        uint8_t* stage = ST == 0 ? st0 : ST == 1 ? st1 : st2;
        const v4i ar = raw_rsrc(abase + (size_t)s * (TT * 68), TT * 68);
        const v4i wr = raw_rsrc(wbase + (size_t)s * (TM * 68), TM * 68);
#pragma unroll
        for (int u = 0; u < kPerWave; ++u) {
            const int j = wave + NW * u;  // wave-uniform
            const bool is_a = j < S::kALoads, pad = j >= S::kLoads;
            const int jj = is_a ? j : j - S::kALoads;
            uint8_t* dst = stage + (pad ? S::kARegion + S::kWRegion : is_a ? 1024 * jj : S::kARegion + 1024 * jj);
            const uint32_t off = pad ? kPastEnd : (uint32_t)(1024 * jj + 16 * lane);
            const uint32_t m0 = (uint32_t)(size_t)(__attribute__((address_space(3))) void*)dst;
            const v4i rs = is_a ? ar : wr;
            // M0 is the only LDS-DMA operand the builtin would set; this kernel has
            // no other M0 user (no compiler-issued LDS DMA, no movrel indexing), so
            // clobbering it here, which clang warns of in general, is safe
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
            asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(off), "s"(m0), "s"(rs)
                         : "memory", "m0");
#pragma clang diagnostic pop
        }
    };
    const int m = lane & 31, g = lane >> 5;
    const uint32_t sel = g ? 0x07060504u : 0x07060100u;
    v16f acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    fetch(std::integral_constant<int, 0>{}, 0);
    fetch(std::integral_constant<int, 1>{}, min(1, nsteps - 1));
    auto step = [&](auto stage_c, int s) {
        constexpr int ST = decltype(stage_c)::value;
        const uint8_t* stage = ST == 0 ? st0 : ST == 1 ? st1 : st2;
        // this wave's loads of step s have landed once at most those of step
        // s + 1 are outstanding (vmcnt <= kPerWave; expcnt, lgkmcnt not waited)
        __builtin_amdgcn_s_waitcnt(0xF70 | kPerWave);
        __builtin_amdgcn_s_barrier();
        // stage (s + 2) % 3 was read by step s - 1, which every wave finished
        // before the barrier; past the end the last step is loaded again
        fetch(std::integral_constant<int, (ST + 2) % 3>{}, min(s + 2, nsteps - 1));
        const uint8_t* arow = stage + (32 * wt + m) * 68;
        const uint8_t* wrow = stage + S::kARegion + (32 * wm + m) * 68;
        auto block = [&](auto blk_c) {
            constexpr int BLK = decltype(blk_c)::value;
            const v4i av = raw_qs<BLK>(arow, g, sel);
            const v4h da = raw_scale<BLK>(arow);
            const v4i bv = raw_qs<BLK>(wrow, g, sel);
            const v4h dw = raw_scale<BLK>(wrow);
            __builtin_amdgcn_sched_barrier(0);
            const v16i zi = {};
            const v16f zf = {};
            const v16i dd = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zi, 0, 0, 0);
            const v16f ss = __builtin_amdgcn_mfma_f32_32x32x8f16(da, dw, zf, 0, 0, 0);  // 2 d_a d_w
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = fmaf((float)dd[i], ss[i], acc[i]);
        };
        block(std::integral_constant<int, 0>{});
        block(std::integral_constant<int, 1>{});
    };
    int s = 0;
    for (; s + 2 < nsteps; s += 3) {
        step(std::integral_constant<int, 0>{}, s);
        step(std::integral_constant<int, 1>{}, s + 1);
        step(std::integral_constant<int, 2>{}, s + 2);
    }
    if (s < nsteps) step(std::integral_constant<int, 0>{}, s);
    if (s + 1 < nsteps) step(std::integral_constant<int, 1>{}, s + 1);
    __builtin_amdgcn_s_waitcnt(0xF70);  // no wave ends with loads into LDS in flight
    const int col = j0 + 32 * wm + m;
    if (col < M) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = t0 + 32 * wt + 8 * (i / 4) + 4 * g + i % 4;
            if (row < T) c[(size_t)row * M + col] = 0.5f * acc[i];  // the scales entered doubled
        }
    }
}

// GGUF Q8_0 rows -> the GEMM tile layout: one thread per (tile, step, row)
// run of 68 bytes (17 dwords); rows past the last one are zero.
__global__ __launch_bounds__(256) void gemm_tile_blocks_kernel(const uint32_t* __restrict__ src,
                                                               uint32_t* __restrict__ dst, int64_t rows,
                                                               int64_t padded_rows, int nb, int R) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // run index in tiled order
    const int64_t nsteps = nb / 2;
    if (i >= padded_rows * nsteps) return;
    const int64_t row_in = i % R, step = (i / R) % nsteps, tile = i / (R * nsteps);
    const int64_t row = tile * R + row_in;
    uint32_t* d = dst + i * 17;
    if (row < rows) {
        const uint32_t* s = src + (row * nb * 34 + step * 68) / 4;  // nb even: dword aligned
#pragma unroll
        for (int k = 0; k < 17; ++k) d[k] = s[k];
    } else {
#pragma unroll
        for (int k = 0; k < 17; ++k) d[k] = 0u;
    }
}

// ---------------------------------------------------------------------------
// Split-layout variant: int8 qs planes [rows][K] and fp32 scale planes
// [rows][K/32], the operand layout of the reference's asm_matmul_q8
// (matmul_q8_avx2.asm:51-194: qweights int8[M][K/32][32], scales f32[M][K/32]).
// A K step of two blocks is 64 contiguous qs bytes and 8 scale bytes per row.
// qs rows are parked at an 80-byte pitch (five 16-byte units; the counters
// still show bank conflicts on 35% of LDS-active cycles), so an operand is one
// aligned ds_read_b128 with no realignment.  The
// scale product d_a d_w comes from v_mfma_f32_32x32x2_f32 with the scales in
// k = 0 and zeros in k = 1: one fp32 product per output, rounded once, as the
// CPU's fmul, for any fp32 scales.  The k = 1 lanes read their zeros from a
// zero-filled copy of the scale area, so no per-block select is needed.
// ---------------------------------------------------------------------------
constexpr int kSplitThreads = 512;                              // 8 waves of one 32x32 tile
constexpr int kSplitPitch = 80;                                 // qs bytes per staged row (64 used)
constexpr int kSplitRows = kTT + kTM;                           // A rows, then W rows
constexpr int kSplitScOff = kSplitRows * kSplitPitch;           // scales [g][row][2 blocks], g = 1 zeros
constexpr int kSplitScHalf = kSplitRows * 2 * 4;
constexpr int kSplitStage = kSplitScOff + 2 * kSplitScHalf;

__global__ __launch_bounds__(kSplitThreads) void gemm_q8_split(const int8_t* __restrict__ wq,
                                                               const float* __restrict__ wsc,
                                                               const int8_t* __restrict__ aq,
                                                               const float* __restrict__ asc,
                                                               float* __restrict__ c, int T, int M, int K,
                                                               int tiles_t, int n_tiles) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    // XCD-aware tile order, as in gemm_q8_0_coalesced
    const int chunk = (int)gridDim.x >> 3;
    const int tile = ((int)blockIdx.x & 7) * chunk + ((int)blockIdx.x >> 3);
    if (tile >= n_tiles) return;
    const int nb = K >> 5;
    const int t0 = (tile % tiles_t) * kTT, j0 = (tile / tiles_t) * kTM;
    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wt = wave >> 2, wm = wave & 3;
    const auto aqr = make_rsrc(aq, (uint32_t)T * (uint32_t)K);
    const auto wqr = make_rsrc(wq, (uint32_t)M * (uint32_t)K);
    const auto asr = make_rsrc(asc, (uint32_t)T * (uint32_t)nb * 4u);
    const auto wsr = make_rsrc(wsc, (uint32_t)M * (uint32_t)nb * 4u);

    // Staging roles (wave-uniform): piece q = (staged row q / 4, 16-byte piece
    // q % 4) of the step's 768 qs pieces.  Slot 0: piece tid (waves 0-3: A
    // rows, waves 4-7: W rows 0-63); slot 1 (waves 0-3): piece 512 + tid (W rows
    // 64-127); waves 4-6 also fetch the 8 scale bytes of staged row tid - 256.
    const bool two_qs = wave < 4, has_sc = wave >= 4 && wave < 7;
    const bool sc_a = wave == 4;
    const int r0 = tid >> 2, r1 = 128 + (tid >> 2), k4 = tid & 3;
    const int rs = tid - 256;  // staged row of this thread's scales (waves 4-6)
    auto grow_of = [&](int r) { return r < kTT ? t0 + r : j0 + (r - kTT); };
    auto row_live = [&](int r) { return r < kTT ? t0 + r < T : j0 + (r - kTT) < M; };
    const uint32_t q0 = row_live(r0) ? (uint32_t)grow_of(r0) * (uint32_t)K + 16u * k4 : kPastEnd;
    const uint32_t q1 = two_qs && row_live(r1) ? (uint32_t)grow_of(r1) * (uint32_t)K + 16u * k4 : kPastEnd;
    const uint32_t s0 = has_sc && row_live(rs) ? (uint32_t)grow_of(rs) * (uint32_t)nb * 4u : kPastEnd;
    // a K step past the last block (K % 64 == 32): its second block's pieces load zeros
    const bool hi_piece = k4 >= 2;

    uint4 p0, p1;
    uint2 ps;
    auto fetch = [&](int kb0) {
        const bool pair = kb0 + 1 < nb;  // wave-uniform
        const uint32_t kq = (uint32_t)kb0 * 32u;
        const uint32_t o0 = q0 == kPastEnd || (hi_piece && !pair) ? kPastEnd : q0 + kq;
        p0 = buf_load_b128(two_qs ? aqr : wqr, o0);
        if (two_qs) {
            const uint32_t o1 = q1 == kPastEnd || (hi_piece && !pair) ? kPastEnd : q1 + kq;
            p1 = buf_load_b128(wqr, o1);
        }
        if (has_sc) {
            const uint32_t os = s0 == kPastEnd ? kPastEnd : s0 + (uint32_t)kb0 * 4u;
            if (pair)
                ps = buf_load_b64(sc_a ? asr : wsr, os);
            else
                ps = make_uint2(buf_load_b32(sc_a ? asr : wsr, os), 0u);
        }
    };
    auto park = [&](uint8_t* stage) {
        *reinterpret_cast<uint4*>(stage + r0 * kSplitPitch + 16 * k4) = p0;
        if (two_qs) *reinterpret_cast<uint4*>(stage + r1 * kSplitPitch + 16 * k4) = p1;
        if (has_sc) *reinterpret_cast<uint2*>(stage + kSplitScOff + rs * 8) = ps;
    };
    // the k = 1 half of both stages' scale areas: zeros, written once
    for (int i = tid; i < 2 * kSplitScHalf / 4; i += kSplitThreads) {
        const int st = i / (kSplitScHalf / 4), e = i - st * (kSplitScHalf / 4);
        reinterpret_cast<float*>(lds + st * kSplitStage + kSplitScOff + kSplitScHalf)[e] = 0.f;
    }

    const int m = lane & 31, g = lane >> 5;
    const int arow = 32 * wt + m, wrow = kTT + 32 * wm + m;
    const int a_qs = arow * kSplitPitch + 16 * g, w_qs = wrow * kSplitPitch + 16 * g;
    const int a_sc = kSplitScOff + g * kSplitScHalf + arow * 8, w_sc = kSplitScOff + g * kSplitScHalf + wrow * 8;
    v16f acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;

    const int nsteps = (nb + 1) >> 1;
    fetch(0);
    for (int s = 0; s < nsteps; ++s) {
        uint8_t* stage = lds + (s & 1) * kSplitStage;
        park(stage);
        __syncthreads();
        if (s + 1 < nsteps) fetch(2 * (s + 1));
        const bool pair = 2 * s + 1 < nb;  // false only in the last step of an odd block count
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            if (blk == 1 && !pair) break;  // no block: nothing is added (not even a zero)
            const v4i av = *reinterpret_cast<const v4i*>(stage + a_qs + 32 * blk);
            const v4i bv = *reinterpret_cast<const v4i*>(stage + w_qs + 32 * blk);
            const float da = *reinterpret_cast<const float*>(stage + a_sc + 4 * blk);
            const float dw = *reinterpret_cast<const float*>(stage + w_sc + 4 * blk);
            __builtin_amdgcn_sched_barrier(0);
            const v16i zi = {};
            const v16f zf = {};
            const v16i dd = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zi, 0, 0, 0);
            const v16f ss = __builtin_amdgcn_mfma_f32_32x32x2f32(da, dw, zf, 0, 0, 0);  // d_a d_w
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = fmaf((float)dd[i], ss[i], acc[i]);
        }
    }

    const int col = j0 + 32 * wm + m;
    if (col < M) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = t0 + 32 * wt + 8 * (i / 4) + 4 * g + i % 4;
            if (row < T) c[(size_t)row * M + col] = acc[i];
        }
    }
}

// Two blocks per staged K step, two steps of loads in flight per thread, at
// 80 VGPRs: six waves per SIMD, so three 8-wave workgroups share a compute unit.
// Deeper rings and 4- or 8-block steps cost occupancy on MI355X, and so did
// issuing both blocks' matrix instructions before either epilogue (194 VGPRs
// with two tiles a wave).  Workgroup tiles of 128 x 96 (12 waves) and 64 x 192
// measured slower than 64 x 128 at 512 x 11008 x 4096 (101.8 and 87.6 us
// against 85.2).
constexpr int kGemmKB = 2;  // blocks per staged K step (even)
constexpr int kCoTT = 64;   // T rows per workgroup tile of the coalesced kernel
constexpr int kCoTM = 128;  // M columns per workgroup tile of the coalesced kernel
constexpr int kGemmWT = 1;  // 32-column tiles per wave: 8 waves of one tile (4 of two measured 4% slower)

}  // namespace

int gemm_q8_0_launch(const void* w, const void* a, float* c, int64_t T, int64_t M, int64_t K, hipStream_t st) {
    if (T <= 0 || M <= 0 || K <= 0 || K % 32)
        return fail(kInvalidArgument, "gemm: need T, M, K > 0 and K %% 32 == 0 (got T=%lld M=%lld K=%lld)",
                    (long long)T, (long long)M, (long long)K);
    const int64_t row_bytes = K / 32 * 34;
    if ((T + 128) * row_bytes >= (int64_t)kPastEnd || (M + 256) * row_bytes >= (int64_t)kPastEnd)
        return fail(kInvalidArgument, "gemm: operands above 4 GB are not supported");
    if ((uintptr_t)w % 4 || (uintptr_t)a % 4) return fail(kInvalidArgument, "gemm: blocks must be 4-byte aligned");
    const dim3 grid((unsigned)((M + kTM - 1) / kTM), (unsigned)((T + kTT - 1) / kTT));
    if (grid.y > 65535) return fail(kInvalidArgument, "gemm: T too large");
    if ((K / 32) % kGemmKB == 0) {
        const int tiles_t = (int)((T + kCoTT - 1) / kCoTT), n_tiles = tiles_t * (int)((M + kCoTM - 1) / kCoTM);
        const unsigned padded = (unsigned)((n_tiles + 7) / 8 * 8);
        constexpr int kThreads = kCoTT * kCoTM / (16 * kGemmWT);
        const size_t lds = (size_t)RawStep<kGemmKB, kThreads, kCoTT, kCoTM>::kBytes;
        const auto kern = gemm_q8_0_coalesced<kGemmKB, kGemmWT, kCoTT, kCoTM>;
        const int rc = dynamic_lds((const void*)kern, lds);
        if (rc) return rc;
        hipLaunchKernelGGL(kern, dim3(padded), dim3(kThreads), lds, st,
                           static_cast<const uint8_t*>(w), static_cast<const uint8_t*>(a), c, (int)T, (int)M, (int)K,
                           tiles_t, n_tiles);
    } else {
        // any K % 32 == 0: blocks staged one by one, qs realigned on the way into LDS
        constexpr int kKB = 4;
        const size_t lds = 2 * (size_t)Step<kKB>::kBytes;
        const int rc = dynamic_lds((const void*)gemm_q8_0_kernel<kKB, false>, lds);
        if (rc) return rc;
        hipLaunchKernelGGL((gemm_q8_0_kernel<kKB, false>), grid, dim3(kThreadsG), lds, st,
                           static_cast<const uint8_t*>(w), static_cast<const uint8_t*>(a), c, (int)T, (int)M, (int)K);
    }
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int gemm_q8_split_launch(const int8_t* wq, const float* wsc, const int8_t* aq, const float* asc, float* c, int64_t T,
                         int64_t M, int64_t K, hipStream_t st) {
    if (T <= 0 || M <= 0 || K <= 0 || K % 32)
        return fail(kInvalidArgument, "gemm_split: need T, M, K > 0 and K %% 32 == 0 (got T=%lld M=%lld K=%lld)",
                    (long long)T, (long long)M, (long long)K);
    if ((T + kTT) * K >= (int64_t)kPastEnd || (M + kTM) * K >= (int64_t)kPastEnd)
        return fail(kInvalidArgument, "gemm_split: operands above 4 GB are not supported");
    if ((uintptr_t)wq % 16 || (uintptr_t)aq % 16 || (uintptr_t)wsc % 4 || (uintptr_t)asc % 4)
        return fail(kInvalidArgument, "gemm_split: qs planes must be 16-byte aligned, scales 4-byte aligned");
    const int64_t tiles_t = (T + kTT - 1) / kTT, n_tiles = tiles_t * ((M + kTM - 1) / kTM);
    if (n_tiles > (1 << 24)) return fail(kInvalidArgument, "gemm_split: T x M too large");
    const unsigned padded = (unsigned)((n_tiles + 7) / 8 * 8);
    const size_t lds = 2 * (size_t)kSplitStage;
    const int rc = dynamic_lds((const void*)gemm_q8_split, lds);
    if (rc) return rc;
    hipLaunchKernelGGL(gemm_q8_split, dim3(padded), dim3(kSplitThreads), lds, st, wq, wsc, aq, asc, c, (int)T, (int)M,
                       (int)K, (int)tiles_t, (int)n_tiles);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int gemm_q8_0_tiled_launch(const void* w_tiled, const void* a_tiled, float* c, int64_t T, int64_t M, int64_t K,
                           hipStream_t st) {
    if (T <= 0 || M <= 0 || K <= 0 || K % 64)
        return fail(kInvalidArgument, "gemm_tiled: need T, M, K > 0 and K %% 64 == 0 (got T=%lld M=%lld K=%lld)",
                    (long long)T, (long long)M, (long long)K);
    if (!w_tiled || !a_tiled || !c) return fail(kInvalidArgument, "gemm_tiled: null pointer");
    if ((uintptr_t)w_tiled % 16 || (uintptr_t)a_tiled % 16)
        return fail(kInvalidArgument, "gemm_tiled: operands must be 16-byte aligned");
    const int64_t tiles_t = (T + kGemmTileA - 1) / kGemmTileA, n_tiles = tiles_t * ((M + kGemmTileW - 1) / kGemmTileW);
    if (n_tiles > (1 << 24)) return fail(kInvalidArgument, "gemm_tiled: T x M too large");
    const unsigned padded = (unsigned)((n_tiles + 7) / 8 * 8);
    hipLaunchKernelGGL((gemm_q8_0_tiled<kGemmTileA, kGemmTileW>), dim3(padded), dim3(kGemmTileA * kGemmTileW / 16), 0, st,
                       static_cast<const uint8_t*>(w_tiled), static_cast<const uint8_t*>(a_tiled), c, (int)T, (int)M,
                       (int)K, (int)tiles_t, (int)n_tiles);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

int gemm_tile_blocks_launch(const void* blocks, void* tiled, int64_t rows, int64_t K, int R, hipStream_t st) {
    if (rows <= 0 || K <= 0 || K % 64) return fail(kInvalidArgument, "gemm tiling: need rows > 0 and K %% 64 == 0");
    if (!blocks || !tiled || (uintptr_t)blocks % 4 || (uintptr_t)tiled % 4)
        return fail(kInvalidArgument, "gemm tiling: null or unaligned buffer");
    const int64_t padded = (rows + R - 1) / R * R, runs = padded * (K / 64);
    if ((runs + 255) / 256 > INT32_MAX) return fail(kInvalidArgument, "gemm tiling: tensor too large");
    hipLaunchKernelGGL(gemm_tile_blocks_kernel, dim3((unsigned)((runs + 255) / 256)), dim3(256), 0, st,
                       static_cast<const uint32_t*>(blocks), static_cast<uint32_t*>(tiled), rows, padded,
                       (int)(K / 32), R);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

}  // namespace asmhip
