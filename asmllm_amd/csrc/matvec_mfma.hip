// Q4_0 GGUF matvec on the int8 matrix cores of gfx950.
//
// y[m] = sum_b d[m,b] * sum_j (n[m,b,j] - 8) * x[32b + j]
// (the reference's asm_matmul_q4, src/kernels/x86_64/matmul_q4_avx2.asm:57-287,
// over GGUF blocks read in place).
//
// One v_mfma_i32_16x16x32_i8 per (16 rows, one 32-weight block):
//   B operand  lane (n, g): qs dword g of row n's block as signed bytes
//              16 (q - 8): low nibbles (weights 4g..4g+3) and high nibbles
//              (weights 16+4g..16+4g+3), two bit operations each, exact;
//   A operand  lane (m, g): the same 8 positions of x in two fixed-point levels
//              relative to 2^e > the block's largest |x|:
//                X1 = trunc(x 2^(30-e)),  X2 = trunc((x 2^(30-e) - X1) 2^30),
//              each split into four signed base-256 digits: rows 0-3 hold X1,
//              rows 4-7 hold X2 (rows 8-15 repeat rows 0-7);
//   D          lane n of group g (g = 0, 1) holds row n's four exact int32
//              digit dots of level g+1: value = 2^24 D0 + 2^16 D1 + 2^8 D2 + D3
//              = sum_j X_j 16 (q_j - 8).  Level 1 accumulates in lanes 0-15 and
//              level 2 in lanes 16-31 with the same scale 2^(e-34) d; the two
//              are joined with a 2^-30 weight at the end.
// Per weight, x is exact to 2^-60 of its block's largest |x| (truncation); the
// remaining error is fp32 rounding of per-block values, so a row stays within
// ~1e-7 of sum |w| |x| of an fp32 evaluation unless x spans more than 2^56
// inside one 32-block.  Every instruction above runs once per MFMA whichever
// level a lane holds, so the second level costs only x preparation and LDS.
//
// Work mapping: a workgroup of 4 waves owns 16 rows; the waves take K in
// 16-block chunks round robin.  A wave streams a chunk (16 rows x 288 bytes)
// with coalesced 16-byte buffer loads, two chunks in flight, parks it in LDS
// and reads the MFMA operands back.  x is digitized once per workgroup into
// LDS; its loads are issued before the weight loads (loads retire in order),
// so the digit work waits on x only and overlaps the weight stream.
#include "common.hpp"
#include "kernels.hpp"

namespace asmhip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreadsM = kWaves * kWave;
constexpr int kCB = 16;                      // blocks per chunk
constexpr int kPitch = 304;                  // LDS bytes per staged row: 16 x 18 = 288 used, 16-aligned
constexpr int kWBuf = 16 * kPitch;           // LDS bytes per wave
constexpr int kXBlk = 256;                   // LDS bytes of x digits per block: [g][level*4+digit][8]
constexpr int kPieces = 16 * kCB * 18 / 16;  // 16-byte pieces per chunk (288)
constexpr int kMaxBlocks = 512;              // K <= 16384

static_assert(kPieces <= 5 * kWave, "a chunk is five 16-byte loads per lane");

__device__ __forceinline__ long pack_q4(uint32_t q) {
    const uint32_t lo = ((q << 4) ^ 0x80808080u) & 0xF0F0F0F0u;  // bytes 16 (n_lo - 8)
    const uint32_t hi = (q ^ 0x80808080u) & 0xF0F0F0F0u;         // bytes 16 (n_hi - 8)
    return (long)(((uint64_t)hi << 32) | lo);
}

// X (|X| < 2^30) -> word whose four bytes, read as int8, are digits s0..s3
// with X = s0 + 2^8 s1 + 2^16 s2 + 2^24 s3.  Adding 128 to each of the three
// low digit positions and flipping their sign bits recentres [0, 255] on
// [-128, 127]; the carries land in the top byte, which stays within [-65, 64].
__device__ __forceinline__ uint32_t digit_word(int X) {
    return ((uint32_t)X + 0x808080u) ^ 0x808080u;
}

// Y[t] holds digits s0..s3 of element t; out[k] gathers digit k of the four
// elements (element t in byte t).
__device__ __forceinline__ void transpose_digits(const uint32_t* Y, uint32_t* out) {
    const uint32_t lo01 = __builtin_amdgcn_perm(Y[1], Y[0], 0x05010400u);
    const uint32_t hi01 = __builtin_amdgcn_perm(Y[1], Y[0], 0x07030602u);
    const uint32_t lo23 = __builtin_amdgcn_perm(Y[3], Y[2], 0x05010400u);
    const uint32_t hi23 = __builtin_amdgcn_perm(Y[3], Y[2], 0x07030602u);
    out[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
    out[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
    out[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
    out[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

__device__ __forceinline__ float block_value(v4i d) {
    const int hi = d[0] * 256 + d[1];  // |d| < 2^19: exact in int32
    const int lo = d[2] * 256 + d[3];
    return fmaf((float)hi, 65536.0f, (float)lo);
}

template <int XQ>
__global__ __launch_bounds__(kThreadsM) void q4_0_mfma_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                              float* __restrict__ y, int M, int K, int pre,
                                                              const float* __restrict__ pre_arg, float eps,
                                                              int accumulate) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float red[kWaves];
    const int nb = K >> 5;
    const int nch = (nb + kCB - 1) / kCB;
    const uint32_t row_bytes = (uint32_t)nb * 18u;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
    const int row0 = blockIdx.x * 16;
    const auto wr = make_rsrc(w, row_bytes * (uint32_t)M);
    uint8_t* wbuf = lds + wave * kWBuf;
    uint8_t* xdig = lds + kWaves * kWBuf;
    float* xscale = reinterpret_cast<float*>(xdig + nb * kXBlk);
    float* part = xscale + nb;

    // 1) x (and the pre-op argument) first.
    const int nq = nb * 8;
    float4 xv[XQ], av[XQ];
#pragma unroll
    for (int i = 0; i < XQ; ++i) {
        const int qi = min((int)threadIdx.x + kThreadsM * i, nq - 1);
        xv[i] = *reinterpret_cast<const float4*>(x + 4 * qi);
        if (pre != kPreNone) av[i] = *reinterpret_cast<const float4*>(pre_arg + 4 * qi);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2) this wave's first two chunks (chunk index and row clamped; every load issued).
    uint4 b0[5], b1[5];
    auto load_chunk = [&](uint4* buf, int c) {
        c = min(c, nch - 1);
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int q = min(lane + kWave * i, kPieces - 1);
            const int n = q / 18, p = q - n * 18;
            const int row = min(row0 + n, M - 1);
            buf[i] = buf_load_b128(wr, (uint32_t)row * row_bytes + (uint32_t)c * (kCB * 18) + 16u * p);
        }
    };
    int c = wave;
    load_chunk(b0, c);
    load_chunk(b1, c + kWaves);
    __builtin_amdgcn_sched_barrier(0);

    // 3) fused pre-op on x, then digits.
    if (pre == kPreRmsNorm) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < XQ; ++i)
            if ((int)threadIdx.x + kThreadsM * i < nq) {
                ss = fmaf(xv[i].x, xv[i].x, ss);
                ss = fmaf(xv[i].y, xv[i].y, ss);
                ss = fmaf(xv[i].z, xv[i].z, ss);
                ss = fmaf(xv[i].w, xv[i].w, ss);
            }
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = 1.0f / sqrtf(tot / (float)K + eps);
#pragma unroll
        for (int i = 0; i < XQ; ++i) {
            xv[i].x = __fmul_rn(__fmul_rn(xv[i].x, inv), av[i].x);
            xv[i].y = __fmul_rn(__fmul_rn(xv[i].y, inv), av[i].y);
            xv[i].z = __fmul_rn(__fmul_rn(xv[i].z, inv), av[i].z);
            xv[i].w = __fmul_rn(__fmul_rn(xv[i].w, inv), av[i].w);
        }
    } else if (pre == kPreSwiGlu) {
#pragma unroll
        for (int i = 0; i < XQ; ++i) {
            xv[i].x = __fmul_rn(xv[i].x / (1.0f + expf(-xv[i].x)), av[i].x);
            xv[i].y = __fmul_rn(xv[i].y / (1.0f + expf(-xv[i].y)), av[i].y);
            xv[i].z = __fmul_rn(xv[i].z / (1.0f + expf(-xv[i].z)), av[i].z);
            xv[i].w = __fmul_rn(xv[i].w / (1.0f + expf(-xv[i].w)), av[i].w);
        }
    }
#pragma unroll
    for (int i = 0; i < XQ; ++i) {
        const int qi = (int)threadIdx.x + kThreadsM * i;
        const float4 v = xv[i];
        // the 8 quads of a block sit in 8 consecutive lanes
        float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        mx = fmaxf(mx, __shfl_xor(mx, 1, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 2, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 4, kWave));
        int e;
        frexpf(mx, &e);  // mx < 2^e (e = 0 for mx = 0)
        e = max(e, -60);
        const float sc = ldexpf(1.0f, 30 - e);
        const float f[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};  // exact: power-of-two scaling, |f| < 2^30
        uint32_t Y1[4], Y2[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float tr = truncf(f[t]);
            Y1[t] = digit_word((int)tr);
            Y2[t] = digit_word((int)((f[t] - tr) * 1073741824.0f));  // fraction exact; 2^30
        }
        uint32_t d1[4], d2[4];
        transpose_digits(Y1, d1);
        transpose_digits(Y2, d2);
        if (qi < nq) {
            // quad qq holds x[4qq .. 4qq+3] of block b: k-group qq & 3, half qq >> 2
            const int b = qi >> 3, qq = qi & 7;
            uint8_t* base = xdig + b * kXBlk + (qq & 3) * 64 + (qq >> 2) * 4;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                *reinterpret_cast<uint32_t*>(base + 8 * k) = d1[3 - k];       // rows 0-3: X1, top digit first
                *reinterpret_cast<uint32_t*>(base + 32 + 8 * k) = d2[3 - k];  // rows 4-7: X2
            }
            if (qq == 0) xscale[b] = ldexpf(1.0f, e - 34);  // 2^(e-30) for X1, 1/16 for the weight bytes
        }
    }
    __syncthreads();

    // 4) MFMA over this wave's chunks.
    const int n = lane & 15, g = lane >> 4;
    const int aoff = g * 64 + (n & 7) * 8;
    const uint8_t* rowd = wbuf + n * kPitch;  // row n's staged blocks (scales at 18 j)
    const uint8_t* rowp = rowd + 4 * g;       // this lane's qs dword
    float acc = 0.f;
    auto compute = [&](const uint4* buf, int cc) {
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int q = lane + kWave * i;
            if (q < kPieces) {
                const int r = q / 18, p = q - r * 18;
                *reinterpret_cast<uint4*>(wbuf + r * kPitch + 16 * p) = buf[i];
            }
        }
        __builtin_amdgcn_wave_barrier();
        const int nbk = min(kCB, nb - cc * kCB);  // even: nb % 8 == 0
        const v4i z = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < kCB; j += 2) {
            if (j < nbk) {
                // blocks j (bytes 18j..) and j+1 (bytes 18j+18..) of row n
                const uint32_t w0 = *reinterpret_cast<const uint32_t*>(rowp + 18 * j);
                const uint32_t w1 = *reinterpret_cast<const uint32_t*>(rowp + 18 * j + 4);
                const uint32_t w5 = *reinterpret_cast<const uint32_t*>(rowp + 18 * j + 20);
                // fp16 scales of blocks j (low half) and j+1 (high half), the same for every lane group
                const uint32_t sA = *reinterpret_cast<const uint32_t*>(rowd + 18 * j);
                const uint32_t sB = *reinterpret_cast<const uint32_t*>(rowd + 18 * j + 16);
                const int jb = cc * kCB + j;
                const long aA = *reinterpret_cast<const long*>(xdig + jb * kXBlk + aoff);
                const long aB = *reinterpret_cast<const long*>(xdig + (jb + 1) * kXBlk + aoff);
                const v4i dA = __builtin_amdgcn_mfma_i32_16x16x32_i8(aA, pack_q4(__builtin_amdgcn_alignbyte(w1, w0, 2)),
                                                                     z, 0, 0, 0);
                const v4i dB = __builtin_amdgcn_mfma_i32_16x16x32_i8(aB, pack_q4(w5), z, 0, 0, 0);
                acc = fmaf(block_value(dA) * xscale[jb], half_lo(sA), acc);
                acc = fmaf(block_value(dB) * xscale[jb + 1], half_hi(sB), acc);
            }
        }
        __builtin_amdgcn_wave_barrier();
    };
    while (c < nch) {
        compute(b0, c);
        const int c2 = c + kWaves;
        if (c2 < nch) {
            if (c2 + kWaves < nch) load_chunk(b0, c2 + kWaves);
            compute(b1, c2);
            if (c2 + 2 * kWaves < nch) load_chunk(b1, c2 + 2 * kWaves);
        }
        c = c2 + kWaves;
    }

    // 5) combine the waves' partial sums in a fixed order.
    const float acc2 = __shfl_down(acc, 16, kWave);  // level 2 of row n
    if (g == 0) part[wave * 16 + n] = fmaf(acc2, 9.313225746154785e-10f, acc);  // 2^-30
    __syncthreads();
    if (wave == 0 && lane < 16 && row0 + lane < M) {
        const float s = (part[lane] + part[16 + lane]) + (part[32 + lane] + part[48 + lane]);
        y[row0 + lane] = accumulate ? y[row0 + lane] + s : s;
    }
}

template <int XQ>
int launch_xq(const uint8_t* w, const float* x, float* y, int M, int K, size_t lds, hipStream_t st,
              const MatvecOpts& o) {
    const int rc = dynamic_lds((const void*)q4_0_mfma_kernel<XQ>, lds);
    if (rc) return rc;
    hipLaunchKernelGGL((q4_0_mfma_kernel<XQ>), dim3((M + 15) / 16), dim3(kThreadsM), lds, st, w, x, y, M, K, o.pre,
                       o.pre_arg, o.eps, (int)o.accumulate);
    return kOk;
}

size_t mfma_lds_bytes(int nb) { return (size_t)kWaves * kWBuf + (size_t)nb * (kXBlk + 4) + kWaves * 16 * 4; }

}  // namespace

bool q4_0_mfma_eligible(const void* w, const float* x, const MatvecOpts& o, int64_t M, int64_t K) {
    const int64_t nb = K / 32;
    return K % 256 == 0 && nb >= 8 && nb <= kMaxBlocks && M >= 1 && M * nb * 18 < (int64_t)UINT32_MAX &&
           (uintptr_t)w % 4 == 0 && (uintptr_t)x % 16 == 0 &&
           (o.pre == kPreNone || (uintptr_t)o.pre_arg % 16 == 0);
}

int q4_0_mfma_launch(const void* w, const float* x, float* y, int64_t M, int64_t K, hipStream_t st,
                     const MatvecOpts& o) {
    const int nb = (int)(K / 32);
    const int xq = (nb * 8 + kThreadsM - 1) / kThreadsM;  // quads of x per thread
    const size_t lds = mfma_lds_bytes(nb);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const int m = (int)M, k = (int)K;
    int rc;
    if (xq <= 4)
        rc = launch_xq<4>(wb, x, y, m, k, lds, st, o);
    else if (xq <= 8)
        rc = launch_xq<8>(wb, x, y, m, k, lds, st, o);
    else if (xq <= 12)
        rc = launch_xq<12>(wb, x, y, m, k, lds, st, o);
    else
        rc = launch_xq<16>(wb, x, y, m, k, lds, st, o);
    if (rc) return rc;
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

}  // namespace asmhip
