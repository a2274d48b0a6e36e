// Quantized matvec on the int8 matrix cores of gfx950.
//
// y[m] = sum_b d[m,b] * sum_j w[m,b,j] * x[32b + j], with w = n - 8 (Q4_0),
// (n | bit << 4) - 16 (Q5_0) or q (Q8_0): the reference's asm_matmul_q4 /
// asm_matmul_q5 / asm_matmul_q8 (src/kernels/x86_64/matmul_q4_avx2.asm:57-287,
// matmul_q5_avx2.asm:52-238, matmul_q8_avx2.asm:51-194), over GGUF blocks read
// in place or over the reference's split qs / qh / fp32-scale planes.  The
// block format is a template parameter (Fmt / Unit below); the description
// that follows uses Q4_0, the other formats differ only in how a lane builds
// its weight bytes and in the x scale.
//
// One v_mfma_i32_16x16x64_i8 per (16 rows, block pair 2p, 2p+1):
//   B operand  lane (n, G), n the weight row, G the k-group: groups 0-1 take
//              block 2p, groups 2-3 block 2p+1; group G covers qs bytes
//              8h..8h+7 (h = G & 1) of row n's block as signed bytes
//              16 (q - 8): low nibbles (weights 8h..8h+7) and high nibbles
//              (weights 16+8h..16+8h+7), two bit operations per dword, exact;
//   A operand  the same 16 positions of x in two fixed-point levels relative to
//              2^e > the block's largest |x|:
//                X1 = trunc(x 2^(30-e)),  X2 = trunc((x 2^(30-e) - X1) 2^30),
//              each split into four signed base-256 digits: rows 0-3 hold X1 and
//              rows 4-7 X2 of block 2p (in groups 0-1, zero in groups 2-3),
//              rows 8-15 the same for block 2p+1 (in groups 2-3);
//   D          lanes 0-15 / 16-31 hold row n's four exact int32 digit dots of
//              level 1 / 2 of block 2p, lanes 32-47 / 48-63 those of block 2p+1:
//              value = 2^24 D0 + 2^16 D1 + 2^8 D2 + D3 = sum_j X_j 16 (q_j - 8),
//              scaled by 2^(e-34) d of the lane's block; every lane's epilogue is
//              useful, and the four lane groups of a row are joined at the end
//              of a tile (level 2 with a 2^-30 weight).
// Per weight, x is exact to 2^-60 of its block's largest |x| (truncation); the
// remaining error is fp32 rounding of per-block values, so a row stays within
// ~1e-7 of sum |w| |x| of an fp32 evaluation unless x spans more than 2^56
// inside one 32-block.  Every instruction above runs once per MFMA whichever
// level or block a lane holds, so the second level costs only x preparation.
//
// Work mapping (persistent stream): one workgroup of NW waves per compute
// unit.  Workgroup b owns the 16-row tiles b, b + G, b + 2G, ... (G = grid
// size; small Q8_0 / split-layout matvecs use 8-row tiles, the upper 8 MFMA
// rows zero); a tile's K is cut into 8-block units (16 rows x 144 bytes), and wave w
// takes units w, w + NW, ... of every tile in turn, so each wave walks one long
// sequence of units.  D units of loads stay in flight per wave (coalesced
// 16-byte buffer loads; past the end of the sequence the offset is pushed
// beyond the buffer, which returns zeros without touching memory).  A unit is
// parked in the wave's LDS slot (rows at a 152-byte pitch, so the operand
// reads are free of bank conflicts) and its MFMA operands are read back.  x is
// digitized once per workgroup into LDS while the first loads are in flight.
// When every wave takes the same units of every tile (K = 4096 with 16 waves:
// unit w), a wave loads its A operands and block scales into registers once
// and reuses them for every tile, which takes the x reads out of the per-unit
// LDS traffic.  Each wave keeps its per-tile partial sums in LDS; after the
// stream the workgroup adds the NW partials of every row in a fixed order
// (kPostSwiGlu8: a tile's 8 gate and 8 up rows leave as 8 silu(gate) * up).
// The main loop has no workgroup barrier.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace asmhip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kUnitBlocks = 8;                     // blocks per unit

// Block formats the stream reads in place.  A unit is 16 rows x 8 blocks; each
// row's slice is parked in LDS at a padded pitch (pitches chosen so that the
// operand reads of the 16 rows fall on 16 distinct banks).
enum BlockFmt : int {
    kFmtQ4_0 = 0, kFmtQ5_0 = 1, kFmtQ4Split = 2, kFmtQ5Split = 3, kFmtQ8_0 = 4, kFmtQ8Split = 5
};
template <int QT>
struct Fmt;
template <>
struct Fmt<kFmtQ4_0> {
    static constexpr int kBlockBytes = 18;   // fp16 d, qs[16]
    static constexpr int kQsBytes = 16;
    static constexpr int kRowPitch = 152;    // 38 dwords (a 144-byte pitch pairs rows n and n + 8)
    static constexpr int kXScaleShift = 34;  // weight bytes hold 16 (n - 8): x scale 2^(e - 30) / 16
};
template <>
struct Fmt<kFmtQ5_0> {
    static constexpr int kBlockBytes = 22;   // fp16 d, qh[4], qs[16]
    static constexpr int kQsBytes = 16;
    static constexpr int kRowPitch = 184;    // 46 dwords
    static constexpr int kXScaleShift = 33;  // weight bytes hold 8 (b - 16): x scale 2^(e - 30) / 8
};
template <>
struct Fmt<kFmtQ8_0> {
    static constexpr int kBlockBytes = 34;   // fp16 d, qs[32] (int8)
    static constexpr int kQsBytes = 32;
    static constexpr int kRowPitch = 280;    // 70 dwords
    static constexpr int kXScaleShift = 30;  // weight bytes are the int8 values themselves
};
// The reference's split layout: a qs plane [M][K/32][16 or 32], for Q5 a qh plane
// [M][K/32][4], and an fp32 scale plane [M][K/32].  A unit row is parked as
// [qs slice | qh 32 B | scales 32 B].
template <>
struct Fmt<kFmtQ4Split> {
    static constexpr int kBlockBytes = 20;   // per block over the planes: 16 qs + 4 scale bytes
    static constexpr int kQsBytes = 16;
    static constexpr int kRowPitch = 168;    // 42 dwords
    static constexpr int kXScaleShift = 34;
};
template <>
struct Fmt<kFmtQ5Split> {
    static constexpr int kBlockBytes = 24;   // 16 qs + 4 qh + 4 scale bytes
    static constexpr int kQsBytes = 16;
    static constexpr int kRowPitch = 200;    // 50 dwords
    static constexpr int kXScaleShift = 33;
};
template <>
struct Fmt<kFmtQ8Split> {
    static constexpr int kBlockBytes = 36;   // 32 qs + 4 scale bytes
    static constexpr int kQsBytes = 32;
    static constexpr int kRowPitch = 296;    // 74 dwords
    static constexpr int kXScaleShift = 30;
};
template <int QT>
struct Unit {
    static constexpr bool kSplit = QT == kFmtQ4Split || QT == kFmtQ5Split || QT == kFmtQ8Split;
    static constexpr bool kQ5 = QT == kFmtQ5_0 || QT == kFmtQ5Split;
    static constexpr bool kQ8 = QT == kFmtQ8_0 || QT == kFmtQ8Split;
    static constexpr int kBB = Fmt<QT>::kBlockBytes;
    static constexpr int kQsPerBlock = Fmt<QT>::kQsBytes;
    // main plane (GGUF records, or the split qs plane): bytes per block, per row slice, pieces
    static constexpr int kMainPerBlock = kSplit ? kQsPerBlock : kBB;
    static constexpr int kMainRow = kUnitBlocks * kMainPerBlock;  // 144 / 176 / 272 / 128 / 128 / 256
    static constexpr int kCols = kMainRow / 16;                    // 16-byte pieces per row slice
    static constexpr int kMainPieces = 16 * kCols;
    static constexpr int kQhOff = kMainRow;                        // split: row offsets of the qh / scale slices
    static constexpr int kScOff = kMainRow + (kQ5 && kSplit ? 32 : 0);
    static constexpr int kPieces = kMainPieces + (kSplit ? (kQ5 ? 64 : 32) : 0);
    static constexpr int kLoads = (kPieces + 63) / 64;             // 16-byte loads per lane: 3 (Q4, Q5) or 5 (Q8)
    static constexpr int kPitch = Fmt<QT>::kRowPitch;
    static constexpr int kSlotBytes = 16 * kPitch;                 // LDS slot per wave
    static_assert(kMainRow % 16 == 0 && (!kSplit || kMainPieces % 64 == 0), "piece layout");
    static_assert(kPitch >= kScOff + (kSplit ? 32 : 0) && kPitch % 8 == 0, "row pitch");
};
constexpr int kXStride = 272;                      // LDS bytes of x digits per block: [half][level*4+digit][16] + 16 pad
                                                   // (16-byte rows for the 16-byte A operands)
                                                   // (the pad staggers blocks across banks: conflict-free 8-byte writes)
constexpr int kMaxBlocks = 512;                    // K <= 16384
constexpr int kMaxTilesPerGroup = 8;
constexpr uint32_t kPastEnd = 0xFFFFFF00u;         // buffer offset that loads zeros

// LDS offset, within the wave's slot, of piece q of a unit: pieces
// [0, kMainPieces) are row q / kCols, bytes 16 (q % kCols) of the row's main
// slice; for split layouts the next 32 (Q5) are the rows' qh slices and the
// last 32 the scale slices (row i / 2, half i % 2).
template <int QT>
__device__ __forceinline__ int piece_lds(int q) {
    using U = Unit<QT>;
    if (!U::kSplit || q < U::kMainPieces) {
        const int r = q / U::kCols, c = q - U::kCols * r;
        return r * U::kPitch + 16 * c;
    }
    const int i = q - U::kMainPieces;
    if (U::kQ5 && i < 32) return (i >> 1) * U::kPitch + U::kQhOff + 16 * (i & 1);
    const int j = U::kQ5 ? i - 32 : i;
    return (j >> 1) * U::kPitch + U::kScOff + 16 * (j & 1);
}

template <int QT>
__device__ __forceinline__ void park_piece(uint8_t* wbuf, int q, uint4 v) {
    uint2* dst = reinterpret_cast<uint2*>(wbuf + piece_lds<QT>(q));
    dst[0] = make_uint2(v.x, v.y);
    dst[1] = make_uint2(v.z, v.w);
}

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

// One v_mfma_i32_16x16x64_i8 per block pair (2p, 2p + 1) of 16 staged rows.
// Lane (n, G): n = lane & 15 is the weight row (B column), G = lane >> 4 the
// k-group.  Groups 0-1 carry block 2p, groups 2-3 block 2p + 1; group G covers
// positions 8h..8h+7 and 16+8h..16+8h+7 of its block (h = G & 1).  A rows 0-7
// hold block 2p's x digits (levels 1, 2) in groups 0-1 and zeros in groups
// 2-3; rows 8-15 the reverse for block 2p + 1.  So D lanes 0-15 / 16-31 hold
// the level 1 / level 2 digit dots of block 2p and lanes 32-47 / 48-63 those
// of block 2p + 1: every lane's epilogue is useful work.
struct PairLane {
    int bp;        // 0: this lane's block is the even one of the pair, 1: the odd one
    int h;         // which 8 positions of each half of the block: 8h..8h+7, 16+8h..16+8h+7
    int qoff;      // byte offset (dword aligned) of the lane's qs bytes within the pair
    uint32_t sh;   // alignbyte shift: 2 where the block's fields sit two bytes off the dword grid
    int hoff;      // Q5_0: byte offset (dword aligned) of the block's qh word
    int doff;      // byte offset of the dword holding the block's fp16 scale
    uint32_t dsh;  // shift of that scale inside the dword
};

template <int QT>
__device__ __forceinline__ PairLane pair_lane(int lane) {
    constexpr int BB = Fmt<QT>::kBlockBytes;
    const int G = lane >> 4, bp = G >> 1, h = G & 1;
    if constexpr (Unit<QT>::kSplit) {  // offsets within pair 0; pairs step 2 kQsBytes / 8 / 8 bytes
        PairLane pl;
        pl.bp = bp;
        pl.h = h;
        pl.qoff = Fmt<QT>::kQsBytes * bp + 8 * h;
        pl.sh = 0u;
        pl.hoff = Unit<QT>::kQhOff + 4 * bp;
        pl.doff = Unit<QT>::kScOff + 4 * bp;
        pl.dsh = 0u;
        return pl;
    }
    const int o = BB * bp;                  // the block's first byte within the pair
    const int qs = o + (BB - Fmt<QT>::kQsBytes) + 8 * h;   // the lane's first qs byte
    PairLane pl;
    pl.bp = bp;
    pl.h = h;
    pl.qoff = qs & ~3;
    pl.sh = (uint32_t)(qs & 3);
    pl.hoff = (o + 2) & ~3;                 // qh at byte 2 of a Q5_0 block (same shift as qs)
    pl.doff = o & ~3;
    pl.dsh = 8u * (uint32_t)(o & 3);
    return pl;
}

// Q5_0 weight bytes 8 (b - 16) of four positions: the nibbles v (already at
// bits 3..6 of each byte) with the inverted fifth bits nh[pos0 .. pos0+3] at
// bit 7.  ((t << 7) * (1 + 2^7 + 2^14 + 2^21) puts bit j of the 4-bit t at
// 8j + 7; the shifted copies do not overlap and both factors fit 24 bits.)
__device__ __forceinline__ uint32_t q5_bytes(uint32_t nib3, uint32_t nh, int pos0) {
    const uint32_t t = __builtin_amdgcn_ubfe(nh, (uint32_t)pos0, 4u) << 7;
    return (nib3 & 0x78787878u) | (__umul24(t, 0x204081u) & 0x80808080u);
}

// Row n's dot with x over NB staged blocks (NB even), given the lane's A
// operands aq[p] and block x-scales xs[p] (of the lane's block of pair p):
// every weight operand is read from LDS first, then the MFMAs issue back to
// back, then the per-pair epilogues.
template <int NB, int QT>
__device__ __forceinline__ float chunk_dot_x(const uint8_t* rowd, const PairLane& pl, const v4i* aq,
                                             const float* xs, float acc) {
    using U = Unit<QT>;
    constexpr int NP = NB / 2;
    // pair strides: GGUF blocks are interleaved records; split planes step 2 kQsBytes (qs), 8 (qh, scales)
    constexpr int PQ = U::kSplit ? 2 * U::kQsPerBlock : 2 * Fmt<QT>::kBlockBytes;
    constexpr int PH = U::kSplit ? 8 : PQ;
    v4i bq[NP];
    uint32_t sc[NP];
    // 8 bytes of the lane's block at byte offset off of the pair (dword aligned base, shift pl.sh)
    auto read8 = [&](const uint8_t* b, uint32_t* lo, uint32_t* hi) {
        if constexpr (U::kSplit) {
            *lo = *reinterpret_cast<const uint32_t*>(b);
            *hi = *reinterpret_cast<const uint32_t*>(b + 4);
        } else {
            const uint32_t w0 = *reinterpret_cast<const uint32_t*>(b);
            const uint32_t w1 = *reinterpret_cast<const uint32_t*>(b + 4);
            const uint32_t w2 = *reinterpret_cast<const uint32_t*>(b + 8);
            *lo = __builtin_amdgcn_alignbyte(w1, w0, pl.sh);
            *hi = __builtin_amdgcn_alignbyte(w2, w1, pl.sh);
        }
    };
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const uint8_t* pq = rowd + PQ * p + pl.qoff;
        uint32_t qa, qb;  // qs bytes 8h..8h+3 and 8h+4..8h+7 of the lane's block
        read8(pq, &qa, &qb);
        if constexpr (U::kQ8) {
            uint32_t qc, qd;  // int8 weights at positions 16+8h..16+8h+7
            read8(pq + 16, &qc, &qd);
            bq[p] = (v4i){(int)qa, (int)qb, (int)qc, (int)qd};
        } else if constexpr (!U::kQ5) {
            const long la = pack_q4(qa), lb = pack_q4(qb);  // (lo | hi << 32) of each dword
            bq[p] = (v4i){(int)(uint32_t)la, (int)(uint32_t)lb, (int)(uint32_t)(la >> 32), (int)(uint32_t)(lb >> 32)};
        } else {
            const uint8_t* ph = rowd + PH * p + pl.hoff;
            uint32_t hq;
            if constexpr (U::kSplit) {
                hq = *reinterpret_cast<const uint32_t*>(ph);
            } else {
                const uint32_t h0 = *reinterpret_cast<const uint32_t*>(ph);
                const uint32_t h1 = *reinterpret_cast<const uint32_t*>(ph + 4);
                hq = __builtin_amdgcn_alignbyte(h1, h0, pl.sh);
            }
            const uint32_t nh = ~hq;
            const int b0 = 8 * pl.h;
            bq[p] = (v4i){(int)q5_bytes(qa << 3, nh, b0), (int)q5_bytes(qb << 3, nh, b0 + 4),
                          (int)q5_bytes(qa >> 1, nh, 16 + b0), (int)q5_bytes(qb >> 1, nh, 20 + b0)};
        }
        sc[p] = *reinterpret_cast<const uint32_t*>(rowd + PH * p + pl.doff) >> pl.dsh;
    }
    const v4i z = {0, 0, 0, 0};
    v4i d[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) d[p] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aq[p], bq[p], z, 0, 0, 0);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        // GGUF: fp16 scale (converted inside the FMA); split: the fp32 scale itself
        const float dw = U::kSplit ? __uint_as_float(sc[p]) : half_lo(sc[p]);
        acc = fmaf(block_value(d[p]) * xs[p], dw, acc);
    }
    return acc;
}

// Byte offset of this lane's A operand inside a block pair's digits; -1 where
// the operand is zero (rows 0-7 in groups 2-3, rows 8-15 in groups 0-1).
__device__ __forceinline__ int a_offset(int lane) {
    const int n = lane & 15, G = lane >> 4;
    if ((n < 8) != (G < 2)) return -1;
    return (G >> 1) * kXStride + (G & 1) * 128 + (n & 7) * 16;
}

// The same with the A operands read from the x digits in LDS.
template <int NB, int QT>
__device__ __forceinline__ float chunk_dot(const uint8_t* rowd, const PairLane& pl, const uint8_t* xu, int aoff,
                                           const float* xsu, float acc) {
    constexpr int NP = NB / 2;
    v4i aq[NP];
    float xs[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        aq[p] = aoff >= 0 ? *reinterpret_cast<const v4i*>(xu + 2 * p * kXStride + aoff) : (v4i){0, 0, 0, 0};
        xs[p] = xsu[2 * p + pl.bp];
    }
    return chunk_dot_x<NB, QT>(rowd, pl, aq, xs, acc);
}

// Row n's total from the lanes of a finished tile: level 1 + level 2 * 2^-30
// over the even and odd blocks (valid in lanes 0-15).
__device__ __forceinline__ float tile_total(float acc) {
    acc += __shfl_down(acc, 32, 64);                                        // + odd blocks
    return fmaf(__shfl_down(acc, 16, 64), 9.313225746154785e-10f, acc);     // + 2^-30 level 2
}

// PW > 0: every wave streams exactly PW units of each tile (K = 256 NW PW), so
// its x operands are the same for every tile and stay in registers; PW = 0:
// any K, operands read from LDS per unit.  AMS > 0: x is the decode attention
// output, merged in this launch from the AMS split states per head in pre_arg
// (kPreAttnMerge: heads of pre_hd dimensions, pre_hd % 32 == 0, one x item per
// thread); the states are requested before the weight stream, as x is, with a
// fixed number of loads per wave so the wait for them does not also wait for
// the weights.  RP (accumulate launches): each workgroup's rows of y are read
// right after the first weight loads are issued, so y += W x does not wait for
// a read of y after the stream.
// Argument order: what the prologue reads before the first weight loads comes
// first (the leading kernel-argument dwords arrive preloaded in SGPRs; a later
// one would cost a kernel-argument load in front of the weight stream).
// ST (measurement only): every wave records the 100 MHz real-time counter at
// kStampCount points of its life into stamps[(block * NW + wave) * kStampCount + i].
// XW (PW = 0, no merge): a wave takes the same units of every tile, so it
// digitizes only its own units' x and starts its stream behind a wave barrier,
// not a workgroup one; with the RMSNorm pre-op the waves' sums of squares meet
// after the stream.  SKIPX (the Q4_0 RMSNorm launches at K = 4096): waves
// holding no x item load nothing, where the plain instantiation's load the last
// item again (measured: each form is the faster one for its own launches).
constexpr int kStampCount = 8;
template <int QT, int XQ, int NW, int D, int PW, int AMS, bool NTW, int TH, bool RP, bool ST = false, bool XW = false,
          bool SKIPX = false>
__global__ __launch_bounds__(NW * 64) void gguf_mfma_stream(const uint8_t* __restrict__ w,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ pre_arg,
                                                            const uint8_t* __restrict__ wh,
                                                            const float* __restrict__ wsc, int M, int K, int pre,
                                                            float* __restrict__ y, float eps, int accumulate,
                                                            int post, int pre_hd, uint64_t* __restrict__ stamps) {
    // stamps: 0 entry, 1 first weight loads issued, 2 x digits ready (after the
    // barrier), 3 first unit landed, 4 last unit landed, 5 stream done, 6 all
    // waves done (after the barrier), 7 y stored and its writes complete
    uint64_t stv[ST ? kStampCount : 1];
    auto mark = [&](int i) {
        if constexpr (ST) stv[i] = __builtin_amdgcn_s_memrealtime();
    };
    mark(0);
    using U = Unit<QT>;
    constexpr int kThreads = NW * 64;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float red[NW];
    const int nb = K >> 5;
    const int nu = nb / kUnitBlocks;  // units per tile
    // main plane bytes per row (GGUF records, or the split qs plane); split qh / scale planes 4 per block
    const uint32_t row_bytes = (uint32_t)nb * (uint32_t)U::kMainPerBlock;
    const uint32_t row_bytes4 = (uint32_t)nb * 4u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int G = gridDim.x;
    // tiles of TH rows (16, or 8 for small Q8_0 and split-layout matvecs); MFMA
    // rows TH..15 of a tile load zeros and are not written
    static_assert(TH == 16 || TH == 8, "tile height");
    const int n_tiles = (M + TH - 1) >> (TH == 16 ? 4 : 3);
    const int per_w = wave < nu ? (nu - wave + NW - 1) / NW : 0;  // this wave's units per tile
    int my_tiles = 0, L = 0;  // this workgroup's tiles, the length of this wave's stream (set at step 2)
    const auto wr = make_rsrc(w, row_bytes * (uint32_t)M);
    const auto hr = make_rsrc(U::kQ5 && U::kSplit ? wh : w, U::kQ5 && U::kSplit ? row_bytes4 * (uint32_t)M : 0u);
    const auto sr = make_rsrc(U::kSplit ? (const void*)wsc : (const void*)w, U::kSplit ? row_bytes4 * (uint32_t)M : 0u);
    uint8_t* wbuf = lds + wave * U::kSlotBytes;
    uint8_t* xdig = lds + NW * U::kSlotBytes;
    float* xscale = reinterpret_cast<float*>(xdig + nb * kXStride);
    float* part = xscale + nb;  // [my_tiles][NW][16]

    // This lane's 16-byte pieces of a unit: piece q = lane + 64 k (see piece_lds).
    // Main-plane pieces past the unit (GGUF tails) are clamped to its last piece
    // and not parked; rows past M fall beyond the buffer and load zeros, and so
    // do the pieces of rows TH..15 (plive false).
    uint32_t poff[U::kLoads];
    bool plive[U::kLoads];
#pragma unroll
    for (int k = 0; k < U::kLoads; ++k) {
        const int q = lane + 64 * k;
        if (!U::kSplit || q < U::kMainPieces) {
            const int qc = min(q, U::kMainPieces - 1);
            poff[k] = (uint32_t)(qc / U::kCols) * row_bytes + 16u * (uint32_t)(qc % U::kCols);
            plive[k] = TH == 16 || qc / U::kCols < TH;
        } else {
            const int i = (q - U::kMainPieces) & 31;  // row i / 2, half i % 2 of a qh or scale slice
            poff[k] = (uint32_t)(i >> 1) * row_bytes4 + 16u * (uint32_t)(i & 1);
            plive[k] = TH == 16 || (i >> 1) < TH;
        }
    }
    // unit s of the stream -> (tile slot i, unit u)
    auto load_unit = [&](uint4* buf, int s) {
        const int i = s / max(per_w, 1);
        const int u = wave + NW * (s - i * per_w);
        const uint32_t row0 = (uint32_t)(((int)blockIdx.x + G * i) * TH);
        const uint32_t base = s < L ? row0 * row_bytes + (uint32_t)u * (uint32_t)U::kMainRow : kPastEnd;
        const uint32_t base4 = s < L ? row0 * row_bytes4 + (uint32_t)u * 32u : kPastEnd;
#pragma unroll
        for (int k = 0; k < U::kLoads; ++k) {
            if (!U::kSplit || 64 * k + 63 < U::kMainPieces) {  // the whole load is main plane
                const uint32_t o = s < L && plive[k] ? base + poff[k] : kPastEnd;
                buf[k] = NTW ? buf_load_b128_nt(wr, o) : buf_load_b128(wr, o);
            } else {  // split tail: qh (Q5, lanes 0-31) and scale slices; no piece for the rest
                const int q = lane + 64 * k - U::kMainPieces;
                const uint32_t o = s < L && plive[k] ? base4 + poff[k] : kPastEnd;
                if (U::kQ5 && q < 32)
                    buf[k] = buf_load_b128(hr, o);
                else if (q < (U::kQ5 ? 64 : 32))
                    buf[k] = buf_load_b128(sr, o);
                else
                    buf[k] = make_uint4(0, 0, 0, 0);
            }
        }
    };

    // 1) x (and the pre-op argument) first.  Item it = (block it / 4, k-group
    // g = it % 4): x[32b + 4g .. +3] and x[32b + 16 + 4g .. +3], the 8 positions
    // of one A-operand lane.
    const int ni = nb * 4;
    float4 xv[XQ][2], av[XQ][2];
    constexpr bool AM = AMS > 0;
    AttnMergeQuads<AM ? AMS : 1> am;
    float2 sml[AM ? 4 : 1][AM ? AMS : 1];  // head_dim 128: the (m, l) of the wave's 4 heads, per split
    // waves holding x items (a wave-uniform test: in a wave past the last item
    // no load is issued, in the others every lane loads)
    const bool am_items = wave * 64 < ni;
    if constexpr (AM) {
        static_assert(XQ == 1, "the attention merge takes one x item per thread");
        const int it = min((int)threadIdx.x, ni - 1);
        const int off = 32 * (it >> 2) + 4 * (it & 3);  // positions off.. and off + 16.. of one head
        const int hh = off / pre_hd;
        const float* ph = pre_arg + (size_t)hh * AMS * (pre_hd + 4);
        if (am_items && pre_hd == 128) {
            // head_dim 128: a wave's 64 items are 4 heads of 16 lanes.  The acc
            // values are requested per lane; each split's (m, l) of the four heads
            // comes through wave-uniform scalar loads, picked per 16-lane group
            // only after the weights are requested (64-lane loads of (m, l), 16
            // lanes on each address, cost ~0.8 us a launch at 6 splits).
            am.load_acc(ph, 128 + 4, off - hh * 128);
            const int nh = ni >> 4, h0 = wave * 4;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < AMS; ++i)
                    sml[j][i] = *reinterpret_cast<const float2*>(
                        pre_arg + ((size_t)min(h0 + j, nh - 1) * AMS + i) * (128 + 4));
        } else if (am_items) {
            am.load(ph, pre_hd + 4, off - hh * pre_hd);
        }
    } else if constexpr (XW) {
        static_assert(AMS == 0 && PW == 0, "x per wave: the any-K stream, no merge");
        // only the items of this wave's own units (the same units in every tile):
        // round i holds units 2i (lanes 0-31) and 2i + 1 (lanes 32-63) of the wave
#pragma unroll
        for (int i = 0; i < XQ; ++i) {
            const int j = 2 * i + (lane >> 5);
            const int it = (j < per_w ? wave + NW * j : wave) * 32 + (lane & 31);
            const int off = 32 * (it >> 2) + 4 * (it & 3);
            xv[i][0] = *reinterpret_cast<const float4*>(x + off);
            xv[i][1] = *reinterpret_cast<const float4*>(x + off + 16);
            if (pre != kPreNone) {
                av[i][0] = *reinterpret_cast<const float4*>(pre_arg + off);
                av[i][1] = *reinterpret_cast<const float4*>(pre_arg + off + 16);
            }
        }
    } else if constexpr (SKIPX) {
        // (the RMSNorm launches' instantiation) a wave whose items of this round
        // are all past the last one loads nothing (wave-uniform); in the other
        // instantiations its lanes load the last item again
#pragma unroll
        for (int i = 0; i < XQ; ++i) {
            xv[i][0] = xv[i][1] = av[i][0] = av[i][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (pre != kPreNone && kThreads * i + 64 * wave >= ni) continue;
            const int it = min((int)threadIdx.x + kThreads * i, ni - 1);
            const int off = 32 * (it >> 2) + 4 * (it & 3);
            xv[i][0] = *reinterpret_cast<const float4*>(x + off);
            xv[i][1] = *reinterpret_cast<const float4*>(x + off + 16);
            if (pre != kPreNone) {
                av[i][0] = *reinterpret_cast<const float4*>(pre_arg + off);
                av[i][1] = *reinterpret_cast<const float4*>(pre_arg + off + 16);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < XQ; ++i) {
            const int it = min((int)threadIdx.x + kThreads * i, ni - 1);
            const int off = 32 * (it >> 2) + 4 * (it & 3);
            xv[i][0] = *reinterpret_cast<const float4*>(x + off);
            xv[i][1] = *reinterpret_cast<const float4*>(x + off + 16);
            if (pre != kPreNone) {
                av[i][0] = *reinterpret_cast<const float4*>(pre_arg + off);
                av[i][1] = *reinterpret_cast<const float4*>(pre_arg + off + 16);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2) the first D units of this wave's stream.  With one unit in flight and
    // plain loads, unit 0 (tile blockIdx.x: the grid never exceeds the tiles;
    // unit = wave) is requested before the tile count is divided out of the grid
    // size (measured: 11008x4096 6.87 -> 6.77 us, split layouts 0.25-0.35 us less;
    // the nontemporal instantiations (Q8_0, Q4_0 up to 2048 rows) measured
    // 0.05-0.15 us slower that way and keep the division first).
    uint4 buf[D][U::kLoads];
    if constexpr (D == 1 && !NTW) {
        const bool v0 = wave < nu;
        const uint32_t base = v0 ? (uint32_t)blockIdx.x * TH * row_bytes + (uint32_t)wave * (uint32_t)U::kMainRow
                                 : kPastEnd;
        const uint32_t base4 = v0 ? (uint32_t)blockIdx.x * TH * row_bytes4 + (uint32_t)wave * 32u : kPastEnd;
#pragma unroll
        for (int k = 0; k < U::kLoads; ++k) {
            if (!U::kSplit || 64 * k + 63 < U::kMainPieces) {
                const uint32_t o = v0 && plive[k] ? base + poff[k] : kPastEnd;
                buf[0][k] = buf_load_b128(wr, o);
            } else {  // split tail: qh (Q5, lanes 0-31) and scale slices, as load_unit
                const int q = lane + 64 * k - U::kMainPieces;
                const uint32_t o = v0 && plive[k] ? base4 + poff[k] : kPastEnd;
                if (U::kQ5 && q < 32)
                    buf[0][k] = buf_load_b128(hr, o);
                else if (q < (U::kQ5 ? 64 : 32))
                    buf[0][k] = buf_load_b128(sr, o);
                else
                    buf[0][k] = make_uint4(0, 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        my_tiles = (n_tiles - (int)blockIdx.x + G - 1) / G;
        L = my_tiles * per_w;
    } else {
        my_tiles = (n_tiles - (int)blockIdx.x + G - 1) / G;
        L = my_tiles * per_w;
#pragma unroll
        for (int d = 0; d < D; ++d) load_unit(buf[d], d);
    }
    __builtin_amdgcn_sched_barrier(0);
    mark(1);
    // the residual rows this thread adds to (one row at most: my_tiles * 16 <= the threads)
    float resid = 0.f;
    if constexpr (RP) {
        static_assert(kMaxTilesPerGroup * 16 <= kThreads, "one stored row per thread");
        const int i = (int)threadIdx.x >> 4, r = (int)threadIdx.x & 15;
        const int row = ((int)blockIdx.x + G * i) * TH + r;
        if ((int)threadIdx.x < my_tiles * 16 && r < TH && row < M) resid = y[row];
    }

    // 3) fused pre-op on x, then digits; partial sums start at zero.
    // partial sums start at zero where some wave streams no unit of a tile
    // (fewer units per tile than waves); otherwise every entry is written
    if (nu < NW)
        for (int i = threadIdx.x; i < my_tiles * NW * 16; i += kThreads) part[i] = 0.f;
    if constexpr (AM) {
        if (am_items && pre_hd == 128) {
            // branch-free pick of head lane >> 4 of the four: bitwise selects on the
            // bit patterns (exact for every value, -inf included)
            const uint32_t b16 = 0u - (uint32_t)((lane >> 4) & 1), b32 = 0u - (uint32_t)((lane >> 5) & 1);
            auto pick = [&](float f0, float f1, float f2, float f3) {
                const uint32_t lo = (b16 & __float_as_uint(f1)) | (~b16 & __float_as_uint(f0));
                const uint32_t hi = (b16 & __float_as_uint(f3)) | (~b16 & __float_as_uint(f2));
                return __uint_as_float((b32 & hi) | (~b32 & lo));
            };
#pragma unroll
            for (int i = 0; i < AMS; ++i)
                am.ml[i] = make_float2(pick(sml[0][i].x, sml[1][i].x, sml[2][i].x, sml[3][i].x),
                                       pick(sml[0][i].y, sml[1][i].y, sml[2][i].y, sml[3][i].y));
        }
        if (am_items) am.finish(&xv[0][0], &xv[0][1]);
        else xv[0][0] = xv[0][1] = make_float4(0.f, 0.f, 0.f, 0.f);  // no item: no digit writes below
    } else if (pre == kPreRmsNorm) {
        // RMSNorm without a barrier before the digits: y = W (inv (x * g)) =
        // inv (W (x * g)), so x * g is digitized now and every row total is
        // scaled by inv = 1 / sqrt(mean(x^2) + eps) from the waves' sums of
        // squares (XW: the waves' units cover every block of x exactly once)
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < XQ; ++i)
            if (XW ? 2 * i + (lane >> 5) < per_w : (int)threadIdx.x + kThreads * i < ni) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    ss = fmaf(xv[i][h].x, xv[i][h].x, ss);
                    ss = fmaf(xv[i][h].y, xv[i][h].y, ss);
                    ss = fmaf(xv[i][h].z, xv[i][h].z, ss);
                    ss = fmaf(xv[i][h].w, xv[i][h].w, ss);
                }
            }
        ss = wave_total_dpp(ss);
        if (lane == 0) red[wave] = ss;
#pragma unroll
        for (int i = 0; i < XQ; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                xv[i][h].x = __fmul_rn(xv[i][h].x, av[i][h].x);
                xv[i][h].y = __fmul_rn(xv[i][h].y, av[i][h].y);
                xv[i][h].z = __fmul_rn(xv[i][h].z, av[i][h].z);
                xv[i][h].w = __fmul_rn(xv[i][h].w, av[i][h].w);
            }
    } else if (pre == kPreSwiGlu) {
#pragma unroll
        for (int i = 0; i < XQ; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                xv[i][h].x = __fmul_rn(xv[i][h].x / (1.0f + expf(-xv[i][h].x)), av[i][h].x);
                xv[i][h].y = __fmul_rn(xv[i][h].y / (1.0f + expf(-xv[i][h].y)), av[i][h].y);
                xv[i][h].z = __fmul_rn(xv[i][h].z / (1.0f + expf(-xv[i][h].z)), av[i][h].z);
                xv[i][h].w = __fmul_rn(xv[i][h].w / (1.0f + expf(-xv[i][h].w)), av[i][h].w);
            }
    }
#pragma unroll
    for (int i = 0; i < XQ; ++i) {
        // a wave whose items of this round are all past the last one skips the
        // round (wave-uniform), leaving its SIMD to the waves that have items
        if (XW ? 2 * i >= per_w : kThreads * i + 64 * wave >= ni) break;
        const int jw = 2 * i + (lane >> 5);  // XW: this lane's unit of the wave
        const int it = XW ? (jw < per_w ? wave + NW * jw : wave) * 32 + (lane & 31) : (int)threadIdx.x + kThreads * i;
        const float v[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                            xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
        // the 4 items of a block sit in 4 consecutive lanes.  The block maximum
        // is taken over the bit patterns of |x|: NaN and infinities sort above
        // every finite value, so a block holding one gets a NaN scale below and
        // the rows it touches come out NaN (no extra reduction for the check).
        uint32_t mb = 0u;
#pragma unroll
        for (int t = 0; t < 8; ++t) mb = max(mb, __float_as_uint(v[t]) & 0x7FFFFFFFu);
        // quad max through DPP (lanes ^1, ^2): no LDS round trip on the way to the digits
        mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, kDppQuadXor1, 0xF, 0xF, false));
        mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, kDppQuadXor2, 0xF, 0xF, false));
        const bool finite = mb < 0x7F800000u;
        const float mx = __uint_as_float(finite ? mb : 0u);
        int e;
        frexpf(mx, &e);  // mx < 2^e (e = 0 for mx = 0)
        e = max(e, -60);
        const float sc = ldexpf(1.0f, 30 - e);
        uint32_t Y1[8], Y2[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float f = v[t] * sc;  // exact: power-of-two scaling, |f| < 2^30
            const float tr = truncf(f);
            Y1[t] = digit_word((int)tr);
            Y2[t] = digit_word((int)((f - tr) * 1073741824.0f));  // fraction exact; 2^30
        }
        uint32_t d1l[4], d1h[4], d2l[4], d2h[4];
        transpose_digits(Y1, d1l);
        transpose_digits(Y1 + 4, d1h);
        transpose_digits(Y2, d2l);
        transpose_digits(Y2 + 4, d2h);
        if (XW ? jw < per_w : it < ni) {
            // digit row r (0-3 X1, 4-7 X2, top digit first) of half hh = g / 2 of block b:
            // 16 bytes at hh * 128 + 16 r; positions 4g..4g+3 go to bytes 4 (g & 1) ..,
            // positions 16+4g..16+4g+3 to bytes 8 + 4 (g & 1) ..
            const int b = it >> 2, g = it & 3;
            uint32_t* base = reinterpret_cast<uint32_t*>(xdig + b * kXStride + (g >> 1) * 128) + (g & 1);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                base[4 * k] = d1l[3 - k];
                base[4 * k + 2] = d1h[3 - k];
                base[4 * (4 + k)] = d2l[3 - k];
                base[4 * (4 + k) + 2] = d2h[3 - k];
            }
            if (g == 0)  // 2^(e-30) for X1, / 16 or 8 for the weight bytes
                xscale[b] = finite ? ldexpf(1.0f, e - Fmt<QT>::kXScaleShift) : __builtin_nanf("");
        }
    }
    // XW: a wave reads only the digits it wrote (its own units' blocks), and
    // LDS operations of one wave complete in order: no workgroup barrier, each
    // wave starts its stream as soon as its own digits are in
    if constexpr (XW)
        __builtin_amdgcn_wave_barrier();
    else
        __syncthreads();
    mark(2);
    // RMSNorm: every wave's sum of squares is in red[] once x's digits are
    // (the barrier above), so the scale is formed now, while the first units
    // are in flight, instead of after the stream (XW, with no barrier here:
    // after the barrier that ends the stream)
    float inv = 1.f;
    auto rms_scale = [&]() {
        float tot = 0.f;
#pragma unroll
        for (int k = 0; k < NW; ++k) tot += red[k];
        return 1.0f / sqrtf(tot / (float)K + eps);
    };
    if (!XW && !AM && pre == kPreRmsNorm) inv = rms_scale();

    // 4) the stream: stage unit s, multiply, refill its buffer with unit s + D.
    constexpr int kPairs = kUnitBlocks / 2;
    const int n = lane & 15;
    const int aoff = a_offset(lane);
    const PairLane pl = pair_lane<QT>(lane);
    const uint8_t* rowd = wbuf + n * U::kPitch;      // row n's staged blocks
    float acc = 0.f;
    if constexpr (PW > 0) {
        static_assert(D % PW == 0 || PW % D == 0, "the load ring and the tile's units align");
        v4i aq[PW][kPairs];
        float xsr[PW][kPairs];
#pragma unroll
        for (int j = 0; j < PW; ++j)
#pragma unroll
            for (int p = 0; p < kPairs; ++p) {
                const int blk = (wave + NW * j) * kUnitBlocks + 2 * p;
                aq[j][p] = aoff >= 0 ? *reinterpret_cast<const v4i*>(xdig + blk * kXStride + aoff) : (v4i){0, 0, 0, 0};
                xsr[j][p] = xscale[blk + pl.bp];
            }
        // whole rounds of max(D, PW) units: units past the stream's end were
        // loaded as zeros and only their partial-sum writes are skipped
        constexpr int R = D > PW ? D : PW;
        for (int s0 = 0; s0 < L; s0 += R) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int s = s0 + r, j = r % PW, d = r % D;
#pragma unroll
                for (int k = 0; k < U::kLoads; ++k) {
                    const int q = lane + 64 * k;
                    if (q < U::kPieces) park_piece<QT>(wbuf, q, buf[d][k]);
                }
                __builtin_amdgcn_wave_barrier();
                if constexpr (ST) {
                    if (s == 0) mark(3);
                    if (s == L - 1) mark(4);
                }
                // the unit is parked: refill its registers before the compute,
                // so the next unit's latency overlaps this unit's MFMAs
                load_unit(buf[d], s + D);
                __builtin_amdgcn_sched_barrier(0);
                acc = chunk_dot_x<kUnitBlocks, QT>(rowd, pl, aq[j], xsr[j], acc);
                __builtin_amdgcn_wave_barrier();
                if (j == PW - 1) {  // last unit of tile s / PW
                    const float t = tile_total(acc);
                    if (lane < 16 && s < L) part[((s / PW) * NW + wave) * 16 + n] = t;
                    acc = 0.f;
                }
            }
        }
    } else
    for (int s0 = 0; s0 < L; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int s = s0 + d;
            if (s < L) {
#pragma unroll
                for (int k = 0; k < U::kLoads; ++k) {
                    const int q = lane + 64 * k;
                    if (q < U::kPieces) park_piece<QT>(wbuf, q, buf[d][k]);
                }
                __builtin_amdgcn_wave_barrier();
                load_unit(buf[d], s + D);
                __builtin_amdgcn_sched_barrier(0);
                const int i = s / per_w;
                const int u = wave + NW * (s - i * per_w);
                acc = chunk_dot<kUnitBlocks, QT>(rowd, pl, xdig + u * kUnitBlocks * kXStride, aoff,
                                             xscale + u * kUnitBlocks, acc);
                __builtin_amdgcn_wave_barrier();
                if (s - i * per_w == per_w - 1) {  // last unit of tile slot i
                    const float t = tile_total(acc);
                    if (lane < 16) part[(i * NW + wave) * 16 + n] = t;
                    acc = 0.f;
                }
            }
        }
    }
    mark(5);
    __syncthreads();
    mark(6);
    if (XW && pre == kPreRmsNorm) inv = rms_scale();  // XW: red[] is complete only here

    // 5) add the waves' partial sums of every row in a fixed order (RMSNorm:
    // then scale the total by inv).
    if (post == kPostSwiGlu8) {
        // a tile is 8 gate rows and their 8 up rows (M % 16 == 0, TH = 16): y[8 tile + r] = silu(gate) * up
        for (int idx = threadIdx.x; idx < my_tiles * 8; idx += kThreads) {
            const int i = idx >> 3, r = idx & 7;
            const int tile = (int)blockIdx.x + G * i;
            float gs = 0.f, us = 0.f;
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                gs += part[(i * NW + k) * 16 + r];
                us += part[(i * NW + k) * 16 + 8 + r];
            }
            gs = __fmul_rn(gs, inv);
            us = __fmul_rn(us, inv);
            y[tile * 8 + r] = __fmul_rn(gs / (1.0f + expf(-gs)), us);
        }
        return;
    }
    for (int idx = threadIdx.x; idx < my_tiles * 16; idx += kThreads) {
        const int i = idx >> 4, r = idx & 15;
        const int row = ((int)blockIdx.x + G * i) * TH + r;
        if (r < TH && row < M) {
            float sum = 0.f;
#pragma unroll
            for (int k = 0; k < NW; ++k) sum += part[(i * NW + k) * 16 + r];
            sum = __fmul_rn(sum, inv);
            y[row] = RP ? resid + sum : accumulate ? y[row] + sum : sum;
        }
    }
    if constexpr (ST) {
        __builtin_amdgcn_s_waitcnt(0);  // the y stores complete
        mark(7);
        if (lane == 0)
            for (int i = 0; i < kStampCount; ++i) stamps[((size_t)blockIdx.x * NW + wave) * kStampCount + i] = stv[i];
    }
}

// Launch shapes.  The wide shape runs 16 waves with one unit of loads in
// flight each (4 waves per SIMD interleave the per-unit LDS -> MFMA ->
// epilogue chains); where its LDS does not fit (K above ~14K), 8 waves with
// two units in flight each.  Both keep one 16-row tile of loads in flight per
// CU: deeper streams (3-6 units per wave) measured slower on MI355X, the
// extra requests queueing in the memory system (and delaying x) without
// raising throughput.
constexpr int kWideWaves = 16, kWideDepth = 1;
constexpr int kNarrowWaves = 8, kNarrowDepth = 2;
constexpr size_t kLdsBudget = 160 * 1024 - 256;

// The weight planes of one launch: GGUF blocks in w, or the split qs / qh / scale planes.
struct Planes {
    const uint8_t* w;
    const uint8_t* wh;
    const float* wsc;
};

template <int QT, int XQ, int NW, int D, int PW, int AMS, bool NTW, int TH, bool RP, bool XW = false,
          bool SKIPX = false>
int launch_rp(const Planes& pw, const float* x, float* y, int M, int K, int grid, size_t lds, hipStream_t st,
              const MatvecOpts& o) {
    // Q4_0 with RMSNorm at K = 4096 (the decode step's q/k/v, gate/up and lm-head):
    // the instantiation whose waves past the last x item load nothing.  Measured
    // per instantiation, in back-to-back launches: RMSNorm 4096x4096 5.07 -> 4.64 us,
    // 6144x4096 5.85 -> 5.61; the same code in the plain launches' instantiation
    // made those 0.5-0.8 us slower (4096x4096 4.17 -> 4.97), so they keep theirs.
    if constexpr (QT == kFmtQ4_0 && PW == 1 && AMS == 0 && !XW && !SKIPX && !NTW)
        if (o.pre == kPreRmsNorm) return launch_rp<QT, XQ, NW, D, PW, AMS, NTW, TH, RP, false, true>(pw, x, y, M, K, grid,
                                                                                                     lds, st, o);
    const void* fn = (const void*)gguf_mfma_stream<QT, XQ, NW, D, PW, AMS, NTW, TH, RP, false, XW, SKIPX>;
    const int rc = dynamic_lds(fn, lds);
    if (rc) return rc;
    hipLaunchKernelGGL((gguf_mfma_stream<QT, XQ, NW, D, PW, AMS, NTW, TH, RP, false, XW, SKIPX>), dim3(grid),
                       dim3(NW * 64), lds, st,
                       pw.w, x, o.pre_arg, pw.wh, pw.wsc, M, K, o.pre, y, o.eps, (int)o.accumulate, o.post,
                       o.attn_hd, nullptr);
    return kOk;
}

// Q4_0 accumulate launches whose waves stream several units per tile (PW = 0:
// K != 4096, the decode engine's down projection) take the kernel that reads
// its residual rows early (4096x11008 / 4096x14336: 9.38 -> 9.20 us); with one
// unit per wave (K = 4096) the early read measured slower (4.68 -> 4.93 us) and
// the rows are read after the stream.
template <int QT, int XQ, int NW, int D, int PW, int AMS = 0, bool NTW = false, int TH = 16>
int launch_xq(const Planes& pw, const float* x, float* y, int M, int K, int grid, size_t lds, hipStream_t st,
              const MatvecOpts& o) {
    if constexpr (QT == kFmtQ4_0 && PW == 0)
        if (o.accumulate) return launch_rp<QT, XQ, NW, D, PW, AMS, NTW, TH, true>(pw, x, y, M, K, grid, lds, st, o);
    return launch_rp<QT, XQ, NW, D, PW, AMS, NTW, TH, false>(pw, x, y, M, K, grid, lds, st, o);
}

// Q4_0, any K other than 4096 at 16 waves, no pre-op or the RMSNorm, no
// post-op, every wave with a unit of every tile and at most 4: each wave
// digitizes only its own units' x (XW), with no workgroup barrier before the
// stream.  Rounds of two units per wave.
template <int NW, int D>
int launch_xw(const Planes& pw, const float* x, float* y, int M, int K, int grid, size_t lds, hipStream_t st,
              const MatvecOpts& o) {
    const int nu = K / 32 / kUnitBlocks;
    const int rounds = ((nu + NW - 1) / NW + 1) / 2;
    if (o.accumulate)
        return rounds <= 1 ? launch_rp<kFmtQ4_0, 1, NW, D, 0, 0, false, 16, true, true>(pw, x, y, M, K, grid, lds, st, o)
                           : launch_rp<kFmtQ4_0, 2, NW, D, 0, 0, false, 16, true, true>(pw, x, y, M, K, grid, lds, st, o);
    return rounds <= 1 ? launch_rp<kFmtQ4_0, 1, NW, D, 0, 0, false, 16, false, true>(pw, x, y, M, K, grid, lds, st, o)
                       : launch_rp<kFmtQ4_0, 2, NW, D, 0, 0, false, 16, false, true>(pw, x, y, M, K, grid, lds, st, o);
}

// x items (8 positions) per thread -> the matching instantiation
template <int QT, int NW, int D>
int launch_nw(const Planes& pw, const float* x, float* y, int M, int K, int grid, size_t lds, hipStream_t st,
              const MatvecOpts& o) {
    const int nb = K / 32;
    if constexpr (QT == kFmtQ4_0 && NW == kWideWaves) {
        const int nu = nb / kUnitBlocks;
        if ((o.pre == kPreNone || o.pre == kPreRmsNorm) && o.post == kPostNone && nu >= NW && (nu + NW - 1) / NW <= 4)
            return launch_xw<NW, D>(pw, x, y, M, K, grid, lds, st, o);
    }
    const int xq = (nb * 4 + NW * 64 - 1) / (NW * 64);
    if (xq <= 1) return launch_xq<QT, 1, NW, D, 0>(pw, x, y, M, K, grid, lds, st, o);
    if constexpr (NW >= 16) {  // nb <= 512: at most 2 items per thread
        return launch_xq<QT, 2, NW, D, 0>(pw, x, y, M, K, grid, lds, st, o);
    } else {
        if (xq <= 2) return launch_xq<QT, 2, NW, D, 0>(pw, x, y, M, K, grid, lds, st, o);
        return launch_xq<QT, 4, NW, D, 0>(pw, x, y, M, K, grid, lds, st, o);  // NW >= 8: at most 4 items per thread
    }
}

// Workgroup layout of one launch: grid size, tiles per workgroup, waves, LDS bytes.
struct StreamShape {
    int grid, tiles_per_group, waves;
    size_t lds;
};

int compute_units();

size_t stream_lds(int slot_bytes, int nw, int nb, int tiles_per_group) {
    return (size_t)nw * slot_bytes + (size_t)nb * (kXStride + 4) + (size_t)tiles_per_group * nw * 16 * sizeof(float);
}

// Workgroup layout for tiles of th rows (16; 8 for small Q8_0 and split-layout matvecs, see mfma_launch).
StreamShape stream_shape(int slot_bytes, int64_t M, int64_t K, int th = 16) {
    const int nb = (int)(K / 32);
    const int cus = compute_units();
    StreamShape sh;
    const int n_tiles = (int)((M + th - 1) / th);
    sh.grid = std::max(std::min(n_tiles, cus), (n_tiles + kMaxTilesPerGroup - 1) / kMaxTilesPerGroup);
    sh.tiles_per_group = (n_tiles + sh.grid - 1) / sh.grid;
    sh.waves = kWideWaves;
    sh.lds = stream_lds(slot_bytes, kWideWaves, nb, sh.tiles_per_group);
    if (sh.lds > kLdsBudget) {
        sh.waves = kNarrowWaves;
        sh.lds = stream_lds(slot_bytes, kNarrowWaves, nb, sh.tiles_per_group);
    }
    return sh;
}

int compute_units() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 256;
    }
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        cus[dev] = n;
    }
    return cus[dev];
}

template <int QT>
bool mfma_eligible(const Planes& pw, const float* x, const MatvecOpts& o, int64_t M, int64_t K) {
    using U = Unit<QT>;
    const int64_t nb = K / 32;
    const int64_t plane = (M + 16) * nb * U::kMainPerBlock;  // largest plane, with the last tile's padding
    bool aligned = (uintptr_t)pw.w % 4 == 0;
    if (U::kSplit) aligned = (uintptr_t)pw.w % 16 == 0 && (uintptr_t)pw.wsc % 16 == 0 && (!U::kQ5 || (uintptr_t)pw.wh % 16 == 0);
    if (o.pre == kPreAttnMerge) {  // one x item per thread of the 16-wave shape, heads of whole 32-blocks
        const StreamShape sh = stream_shape(U::kSlotBytes, M, K);
        if (QT != kFmtQ4_0 || o.post != kPostNone || sh.waves != kWideWaves || nb * 4 > kWideWaves * 64 ||
            o.attn_hd <= 0 || o.attn_hd % 32 || K % o.attn_hd || o.attn_splits < 1 ||
            o.attn_splits > kAttnMergeMaxSplits)
            return false;
    }
    return K % 256 == 0 && nb >= kUnitBlocks && nb <= kMaxBlocks && M >= 1 && M <= INT32_MAX - 16 &&
           plane < (int64_t)kPastEnd && aligned && (uintptr_t)x % 16 == 0 &&
           (o.pre == kPreNone || (uintptr_t)o.pre_arg % 16 == 0) &&
           (o.post == kPostNone || (M % 16 == 0 && !o.accumulate && !U::kSplit)) &&
           stream_shape(U::kSlotBytes, M, K).lds <= kLdsBudget;
}

// The attention-merge stream for the split count of the launch (1..kAttnMergeMaxSplits).
template <int QT, int PW>
int launch_merge(const Planes& pw, const float* x, float* y, int m, int k, const StreamShape& sh, hipStream_t st,
                 const MatvecOpts& o) {
    switch (o.attn_splits) {
        case 1: return launch_xq<QT, 1, kWideWaves, kWideDepth, PW, 1>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
        case 2: return launch_xq<QT, 1, kWideWaves, kWideDepth, PW, 2>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
        case 3: return launch_xq<QT, 1, kWideWaves, kWideDepth, PW, 3>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
        case 4: return launch_xq<QT, 1, kWideWaves, kWideDepth, PW, 4>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
        case 5: return launch_xq<QT, 1, kWideWaves, kWideDepth, PW, 5>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
        case 6: return launch_xq<QT, 1, kWideWaves, kWideDepth, PW, 6>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
        case 7: return launch_xq<QT, 1, kWideWaves, kWideDepth, PW, 7>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
        case 8: return launch_xq<QT, 1, kWideWaves, kWideDepth, PW, 8>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
        default: return fail(kUnsupported, "attention merge stream: %d splits", o.attn_splits);
    }
}

template <int QT>
int mfma_launch(const Planes& pw, const float* x, float* y, int64_t M, int64_t K, hipStream_t st,
                const MatvecOpts& o) {
    const int nb = (int)(K / 32);
    const StreamShape sh = stream_shape(Unit<QT>::kSlotBytes, M, K);
    const int m = (int)M, k = (int)K;
    int rc;
    if constexpr (QT == kFmtQ4_0) {
        if (o.pre == kPreAttnMerge) {  // eligibility fixed the 16-wave shape with one x item per thread
            rc = nb / kUnitBlocks == kWideWaves ? launch_merge<QT, 1>(pw, x, y, m, k, sh, st, o)
                                                : launch_merge<QT, 0>(pw, x, y, m, k, sh, st, o);
            if (rc) return rc;
            ASMHIP_TRY(hipGetLastError());
            return kOk;
        }
    }
    if (sh.waves == kWideWaves && nb / kUnitBlocks == kWideWaves) {
        // K = 4096: one unit per wave and tile, the wave's x operands in registers;
        // nontemporal weight loads for Q4_0 with at most 128 tiles (M <= 2048;
        // measured: 1024x4096 4.29 -> 3.95 us, no gain from 4096 rows up) and for
        // Q8_0 (4096x4096 6.37 -> 6.18 us, 11008x4096 11.3 -> 11.0 us)
        constexpr bool kNtFormat = QT == kFmtQ4_0 || QT == kFmtQ8_0;
        // Q8_0 and the split layouts with at most one 8-row tile per CU (M <= 2048
        // on 256 CUs) run 8-row tiles: twice the workgroups, half the bytes each
        // (measured at 32 / 1024 / 2048 rows: Q8_0 4.82 -> 4.32, 5.23 -> 4.79,
        // 5.54 -> 5.22 us; Q8 split 4.86 -> 4.57, 5.35 -> 4.96, 5.94 -> 5.66;
        // Q4 / Q5 split 0.05-0.15 us less).  GGUF Q4_0 and Q5_0 lost 0.05-0.2 us
        // at 8 rows, and 4- to 1-row tiles lost for every format.
        constexpr bool kEightRowFormat =
            QT == kFmtQ8_0 || QT == kFmtQ8Split || QT == kFmtQ5Split || QT == kFmtQ4Split;
        if constexpr (kEightRowFormat) {
            const StreamShape s8 = stream_shape(Unit<QT>::kSlotBytes, M, K, 8);
            if (o.post == kPostNone && (M + 7) / 8 <= compute_units() && s8.waves == kWideWaves) {
                rc = launch_xq<QT, 1, kWideWaves, kWideDepth, 1, 0, kNtFormat, 8>(pw, x, y, m, k, s8.grid, s8.lds, st,
                                                                                  o);
                if (rc) return rc;
                ASMHIP_TRY(hipGetLastError());
                return kOk;
            }
        }
        if (kNtFormat && (QT == kFmtQ8_0 || (M + 15) / 16 <= 128))
            rc = launch_xq<QT, 1, kWideWaves, kWideDepth, 1, 0, kNtFormat>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
        else
            rc = launch_xq<QT, 1, kWideWaves, kWideDepth, 1>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
    } else if (sh.waves == kWideWaves)
        rc = launch_nw<QT, kWideWaves, kWideDepth>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
    else
        rc = launch_nw<QT, kNarrowWaves, kNarrowDepth>(pw, x, y, m, k, sh.grid, sh.lds, st, o);
    if (rc) return rc;
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

}  // namespace

bool q4_0_mfma_eligible(const void* w, const float* x, const MatvecOpts& o, int64_t M, int64_t K) {
    return mfma_eligible<kFmtQ4_0>(Planes{static_cast<const uint8_t*>(w), nullptr, nullptr}, x, o, M, K);
}

int q4_0_mfma_launch(const void* w, const float* x, float* y, int64_t M, int64_t K, hipStream_t st,
                     const MatvecOpts& o) {
    return mfma_launch<kFmtQ4_0>(Planes{static_cast<const uint8_t*>(w), nullptr, nullptr}, x, y, M, K, st, o);
}

int q4_0_mfma_stamped_launch(const void* w, const float* x, float* y, int64_t M, int64_t K, uint64_t* stamps,
                             int64_t stamps_len, hipStream_t st) {
    using U = Unit<kFmtQ4_0>;
    const Planes pw{static_cast<const uint8_t*>(w), nullptr, nullptr};
    const MatvecOpts o;
    const StreamShape sh = stream_shape(U::kSlotBytes, M, K);
    // the headline launch shape only: K = 4096, 16 waves with their x operands in
    // registers, 16-row tiles, plain loads (M > 2048)
    if (!mfma_eligible<kFmtQ4_0>(pw, x, o, M, K) || K != 16 * 256 || sh.waves != kWideWaves || (M + 15) / 16 <= 128)
        return fail(kUnsupported, "stamped matvec: only Q4_0 K = 4096, M > 2048 (the headline launch shape)");
    if (!stamps || stamps_len < (int64_t)sh.grid * kWideWaves * kStampCount)
        return fail(kInvalidArgument, "stamped matvec: stamps needs %lld entries",
                    (long long)sh.grid * kWideWaves * kStampCount);
    const void* fn = (const void*)gguf_mfma_stream<kFmtQ4_0, 1, kWideWaves, kWideDepth, 1, 0, false, 16, false, true>;
    const int rc = dynamic_lds(fn, sh.lds);
    if (rc) return rc;
    hipLaunchKernelGGL((gguf_mfma_stream<kFmtQ4_0, 1, kWideWaves, kWideDepth, 1, 0, false, 16, false, true>),
                       dim3(sh.grid), dim3(kWideWaves * 64), sh.lds, st, pw.w, x, o.pre_arg, pw.wh, pw.wsc, (int)M,
                       (int)K, o.pre, y, o.eps, 0, o.post, o.attn_hd, stamps);
    ASMHIP_TRY(hipGetLastError());
    return kOk;
}

bool q5_0_mfma_eligible(const void* w, const float* x, int64_t M, int64_t K) {
    return mfma_eligible<kFmtQ5_0>(Planes{static_cast<const uint8_t*>(w), nullptr, nullptr}, x, MatvecOpts(), M, K);
}

int q5_0_mfma_launch(const void* w, const float* x, float* y, int64_t M, int64_t K, hipStream_t st) {
    return mfma_launch<kFmtQ5_0>(Planes{static_cast<const uint8_t*>(w), nullptr, nullptr}, x, y, M, K, st,
                                 MatvecOpts());
}

bool q8_0_mfma_eligible(const void* w, const float* x, const MatvecOpts& o, int64_t M, int64_t K) {
    return mfma_eligible<kFmtQ8_0>(Planes{static_cast<const uint8_t*>(w), nullptr, nullptr}, x, o, M, K);
}

int q8_0_mfma_launch(const void* w, const float* x, float* y, int64_t M, int64_t K, hipStream_t st,
                     const MatvecOpts& o) {
    return mfma_launch<kFmtQ8_0>(Planes{static_cast<const uint8_t*>(w), nullptr, nullptr}, x, y, M, K, st, o);
}

bool split_mfma_eligible(int bits, const void* qs, const uint8_t* qh, const float* scales, const float* x, int64_t M,
                         int64_t K) {
    const Planes pw{static_cast<const uint8_t*>(qs), qh, scales};
    const MatvecOpts o;
    switch (bits) {
        case 4: return mfma_eligible<kFmtQ4Split>(pw, x, o, M, K);
        case 5: return mfma_eligible<kFmtQ5Split>(pw, x, o, M, K);
        case 8: return mfma_eligible<kFmtQ8Split>(pw, x, o, M, K);
        default: return false;
    }
}

int split_mfma_launch(int bits, const void* qs, const uint8_t* qh, const float* scales, const float* x, float* y,
                      int64_t M, int64_t K, hipStream_t st) {
    const Planes pw{static_cast<const uint8_t*>(qs), qh, scales};
    const MatvecOpts o;
    switch (bits) {
        case 4: return mfma_launch<kFmtQ4Split>(pw, x, y, M, K, st, o);
        case 5: return mfma_launch<kFmtQ5Split>(pw, x, y, M, K, st, o);
        case 8: return mfma_launch<kFmtQ8Split>(pw, x, y, M, K, st, o);
        default: return fail(kInvalidArgument, "split matvec: %d-bit planes", bits);
    }
}

}  // namespace asmhip
