// tc_prefill.hip -- prefill GEMM out[m][n] = W[n] . x[m] for Q4_K, Q5_K,
// Q6_K, Q8_0, IQ3_XXS, IQ3_S and IQ2_S weights on the int8 matrix cores
// (v_mfma_i32_32x32x32_i8). The weights of a tile are converted once per
// token tile of up to 128 tokens, in the registers of the lanes that feed
// them to the MFMA.
//
// Replaces the reference prefill GEMM (int8Gemm, GemmDispatch.cu:595-698 and
// its stream-K kernel GemmKernels.cuh:3707-4030) with the CPU reference's
// numerics: the activations are quantized by the bit-exact quantizers (Q8_K
// for Q4_K and the IQ types, the 32-wide Q8_0 rule for Q8_0), every integer dot
// product of a weight block with an activation block is exact, and only the
// scale combination runs in fp32.
//
// Decomposition. A workgroup has 8 waves (two per SIMD). Per 256-wide
// superblock of K, the tile's activations (int8 values and their scale data)
// and raw weight blocks are loaded straight into LDS (no registers, whole
// cache lines per wave instruction), double-buffered. Each lane then reads
// the bytes of its weight row and k-half, converts them into its MFMA B
// operand, and runs the MFMAs against activation fragments read from LDS.
//  * Q4_K: wave w owns 32 weight rows and every token of the tile (256 rows
//    per workgroup), so no weight is converted twice for one tile.
//  * Q8_0: 128 rows per workgroup, waves w and w + 4 share rows and take one
//    half of the tile's tokens each (the Q8_0 weight blocks take 272 bytes of
//    LDS per row and superblock); from 257 tokens 256 rows as Q4_K, with one
//    weight region in LDS instead of two (as Q6_K at 128-token tiles: each
//    wave reads its rows' raw bytes into registers, then a barrier, then the
//    next superblock's weight loads).
//  * Q5_K, Q6_K: as Q4_K (256 rows); their 128-token tiles keep one weight
//    region in LDS.
//  * IQ3_XXS, IQ3_S: as Q4_K (256 rows); the sign-applied codebook is built
//    in LDS once per workgroup.
//  * IQ2_S: as Q4_K (256 rows); its codebook (8-byte entries) in LDS, the
//    signs applied in registers.
//
// Q4_K (reference dequantizeQ4_KBlock, GGMLDequantize.hpp:436-477): a weight
// of sub-block s is w = d*sc_s*q - dmin*m_s with q in 0..15 and sc_s, m_s in
// 0..63. With sc_s = 8*h_s + l_s (h_s, l_s in 0..7) the products h_s*q and
// l_s*q fit int8, so the hi chain (8 MFMAs) and the lo chain (8 more) give
// C = sum_s sc_s * (q . x)_s exactly as 8*hi + lo. The min term Mn = sum_s
// m_s * S_s (S_s the sum of the 32 activations of sub-block s) is one bf16
// MFMA: the quantizer writes S_s as two exact bf16 pieces 128*(S_s >> 7) and
// S_s & 127, the weights give m_s (6 bits) against each, and every product
// and partial sum is an integer below 2^24, so the fp32 result is Mn exactly.
// Per superblock and output, in fp32: acc += d8 * (d*C - dmin*Mn).
//
// Q8_0 (reference matMulVecBatchQ8_0_Q8K_AVX2, SIMDMatMulVecAVX2.cpp:4239-4383):
// one MFMA per 32-block gives the exact integer I; the scale dw * d8 of every
// output of the block comes from one bf16 MFMA as an outer product of their
// exact bf16 pieces (dw = h + l, d8 = h + m + l, 6 exact products summed in
// fp32), so the fp32 combination acc += I * (dw*d8) is two VALU operations
// per output (a convert and an fma) instead of three.
//
// MFMA operands: lane l feeds row (l & 31) and k-group (l >> 5) of A and of B
// (any fixed pairing of k positions works, as both operands use it). A =
// activations (row = token), B = weights (column = weight row), so a lane's
// 16 results share one weight row (its scales are lane constants) and cover
// tokens 8*(r/4) + 4*(l >> 5) + (r % 4).
//
// Work split: the (tile, superblock) units, tiles ordered row block fastest,
// are divided evenly over one workgroup per CU (stream-K); workgroup ranges
// are numbered so that the workgroups of one XCD (dispatched round robin over
// the 8 XCDs) hold one contiguous range and share one token tile's activations
// in their L2. A tile split over a few workgroups is summed by the last of
// them to finish its part, in workgroup order (deterministic); the others
// leave their partial tiles in memory (system-scope stores) and count their
// arrival on the tile's counter. Tiles split over more workgroups are summed
// by k_pf_fixup, a second launch, in the same order. A workgroup's range falls
// into one segment per tile; each segment's last superblock iteration stages
// the next segment's first superblock.
#include <type_traits>

#include "tc_kernels.hpp"

namespace tc {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));

constexpr uint32_t PW = 8;  // waves per workgroup (two per SIMD)

// Per weight type: rows per workgroup tile, waves per row group (waves that
// share rows and split the tokens), unit bytes, and the activation scale
// data per token and superblock (Q4_K: 16 bf16 pieces of the 32-wide sums +
// the fp32 d; Q8_0: 8 blocks x 4 bf16 pieces).
template <int TYPE>
struct PfType;
template <>
struct PfType<kQ4_K> {
    static constexpr uint32_t PR = 256, TSPLIT = 1, UB = 144, XB = 32;
};
// Q5_K: as Q4_K, 176-byte units; at 128-token tiles one weight region in
// LDS (two stages of 256 such rows would not fit).
template <>
struct PfType<kQ5_K> {
    static constexpr uint32_t PR = 256, TSPLIT = 1, UB = 176, XB = 32;
};
template <>
struct PfType<kQ8_0> {
    static constexpr uint32_t PR = 128, TSPLIT = 2, UB = 272, XB = 64;
};
// Q8_0 from 257 tokens: 256 rows per workgroup (each wave 32 rows x 128
// tokens, so a weight is converted once per 4 token blocks instead of 2),
// with one weight region in LDS (see pf_shared_w). An id of this file only.
constexpr int kQ8W = 108;
template <>
struct PfType<kQ8W> {
    static constexpr uint32_t PR = 256, TSPLIT = 1, UB = 272, XB = 64;
};
// Q6_K: the 210-byte unit (2-byte aligned) in the 224-byte window from its
// 4-byte-aligned start (14 chunks, loaded as 15 at a 240-byte row stride:
// conflict-free 16-byte reads); at most 64 tokens per tile (256 such rows
// would not fit LDS twice with 128-token stages).
template <>
struct PfType<kQ6_K> {
    static constexpr uint32_t PR = 256, TSPLIT = 1, UB = 240, XB = 0;
};
// IQ3_XXS: a row's 98-byte unit is 2-byte aligned; LDS holds the 100-byte
// window from its 4-byte-aligned start down: 6 chunks at a 112-byte row
// stride (conflict-free 16-byte reads) and the last dword in TAIL.
template <>
struct PfType<kIQ3_XXS> {
    static constexpr uint32_t PR = 256, TSPLIT = 1, UB = 112, XB = 0;
};
// IQ3_S: the 110-byte unit (2-byte aligned) in the 112-byte window from its
// 4-byte-aligned start (7 chunks; the last ends at most 2 bytes past the
// unit, inside the dword-rounded range).
template <>
struct PfType<kIQ3_S> {
    static constexpr uint32_t PR = 256, TSPLIT = 1, UB = 112, XB = 0;
};
// IQ2_S: the 82-byte unit (2-byte aligned) in the 84-byte window from its
// 4-byte-aligned start (6 chunks at a 112-byte row stride, slot 6 unused).
template <>
struct PfType<kIQ2_S> {
    static constexpr uint32_t PR = 256, TSPLIT = 1, UB = 112, XB = 0;
};
// Codebook types: IQ3_XXS / IQ3_S the sign-applied grid (entries x 16 sign
// nibbles x 4 bytes), IQ2_S its 1024 8-byte entries as they are.
__host__ __device__ constexpr uint32_t pf_grid_bytes(int type) {
    return type == kIQ3_XXS ? 256 * 16 * 4 : type == kIQ3_S ? 512 * 16 * 4 : type == kIQ2_S ? 1024 * 8 : 0;
}

// One LDS buffer: [TT][256] activation values (16-byte chunk c of token t at
// slot c ^ (t & 15)), [TT][XB] scale data, the Q8_K types' [max(TT, 64)]
// fp32 d, [PR][UB] raw weight blocks. IQ3_XXS's signed grid (256 x 16
// words, one copy per workgroup, at offset 0 so that a lookup's address is
// its index times 4), then the two buffers.
// Q6_K at 128-token tiles keeps one weight region (WS, after the two
// buffers): each wave reads its rows' raw bytes into registers first, and the
// next superblock's weights are loaded only after a barrier that follows
// those reads (the activations stay double-buffered).
template <int TYPE, int NT>
constexpr bool pf_shared_w() { return ((TYPE == kQ5_K || TYPE == kQ6_K) && NT == 4) || TYPE == kQ8W; }
template <int TYPE, int NT>
struct PLds {
    using T = PfType<TYPE>;
    static constexpr bool SW = pf_shared_w<TYPE, NT>();
    static constexpr uint32_t TT = 32 * NT;
    static constexpr uint32_t GRID = 0;  // IQ3_XXS's signed grid (before the two buffers)
    static constexpr uint32_t BUF0 = pf_grid_bytes(TYPE);
    static constexpr uint32_t QS = 0;
    static constexpr uint32_t XS = TT * 256;
    static constexpr uint32_t D8 = XS + TT * T::XB;
    static constexpr uint32_t W = D8 + (TYPE != kQ8_0 && TYPE != kQ8W ? (TT < 64 ? 64 : TT) * 4 : 0);
    static constexpr uint32_t TAIL = W + (SW ? 0 : T::PR * T::UB);
    static constexpr uint32_t bytes = TAIL + (TYPE == kIQ3_XXS ? T::PR * 4 : 0);
    static constexpr uint32_t WS = BUF0 + 2 * bytes;  // the shared weight region (SW)
    static constexpr uint32_t FLAG = WS + (SW ? T::PR * T::UB : 0);  // a split tile's arrival count
    static constexpr uint32_t total = FLAG + 16;
};

struct PfArgs {
    const uint8_t *W;
    const int8_t *qs;   // block-major [nblk][M][256]
    const float *d8;    // Q4_K: [nblk][M]
    const int8_t *xs;   // Q4_K sum pieces [nblk][M][32 B]; Q8_0 d pieces [nblk][M][64 B]
    float *out;         // [M][N]
    float *ws;          // partial tiles [G][2][TT][PR]
    uint32_t *ctr;      // per tile: contributors arrived (zero before the launch, zero after it)
    uint32_t fused;     // split tiles summed by their last contributor (else by k_pf_fixup)
    uint32_t M, N, K;
    uint32_t row_bytes, nblk;
    uint32_t ntm, ntn, ntiles;  // token tiles, row blocks, tiles
    uint32_t G;                 // workgroups
    // Grouped (MoE) mode: token tile i covers rows [mt[3i], mt[3i+1]) of the
    // expert-sorted activations and uses expert mt[3i+2]'s matrix at W +
    // expert * wstride; the tile count is read from *ntm_dev (written on the
    // device by the router).
    const uint32_t *mt;
    const uint32_t *ntm_dev;
    uint64_t wstride;
    // Grouped mode with two matrices of one shape (MoE gate and up): the
    // tiles of W2 / out2 follow those of W / out in one launch.
    const uint8_t *W2;
    float *out2;
};

// A tile's token rows [m0, mend), weight matrix and output.
struct PfTile {
    uint32_t m0, mend, n0;
    const uint8_t *W;
    float *out;
};
template <bool GRP>
__device__ __forceinline__ PfTile pf_tile(const PfArgs &a, uint32_t tile, uint32_t TT, uint32_t PR) {
    PfTile t;
    if constexpr (GRP) {
        const uint32_t nt1 = *a.ntm_dev * a.ntn;  // tiles of one matrix
        const bool second = a.W2 != nullptr && tile >= nt1;
        if (second) tile -= nt1;
        const uint32_t tn = tile % a.ntn, tm = tile / a.ntn;
        t.n0 = tn * PR;
        // (wave-uniform: readfirstlane keeps them, and the load descriptors
        // built from them, in scalar registers)
        t.m0 = __builtin_amdgcn_readfirstlane(a.mt[3 * tm]);
        t.mend = __builtin_amdgcn_readfirstlane(a.mt[3 * tm + 1]);
        t.W = (second ? a.W2 : a.W) + uint64_t(__builtin_amdgcn_readfirstlane(a.mt[3 * tm + 2])) * a.wstride;
        t.out = second ? a.out2 : a.out;
    } else {
        const uint32_t tn = tile % a.ntn, tm = tile / a.ntn;
        t.n0 = tn * PR;
        t.m0 = tm * TT;
        t.mend = a.M;
        t.W = a.W;
        t.out = a.out;
    }
    return t;
}
template <bool GRP>
__device__ __forceinline__ uint32_t pf_ntiles(const PfArgs &a) {
    if constexpr (GRP)
        return *a.ntm_dev * a.ntn * (a.W2 != nullptr ? 2u : 1u);
    else
        return a.ntiles;
}

__device__ __forceinline__ v16i mfma(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v16f mfma_bf16(v4i a, v4i b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0,
                                                  0, 0);
}
__device__ __forceinline__ u4 lds4(const unsigned char *p) { return *reinterpret_cast<const u4 *>(p); }
__device__ __forceinline__ uint32_t lds1(const unsigned char *p) { return *reinterpret_cast<const uint32_t *>(p); }
__device__ __forceinline__ v4i as_v4i(u4 v) { return __builtin_bit_cast(v4i, v); }

// The lane's activation chunk 2s + g of sub-block s (s < 8) for its token of
// the first token block (chunks XOR-swizzled by token): one address per
// sub-block, formed once per superblock; token block t lies 8192*t bytes on,
// which the LDS reads take as an immediate offset.
// (32-bit byte offsets into the workgroup's LDS array)
struct ASet {
    const unsigned char *lds;
    uint32_t o[8];
};
__device__ __forceinline__ ASet aset(const unsigned char *lds, uint32_t row0, uint32_t j, uint32_t g) {
    ASet a;
    a.lds = lds;
#pragma unroll
    for (int s = 0; s < 8; ++s) a.o[s] = row0 + 16 * ((2 * s + g) ^ (j & 15));
    return a;
}

// Bytewise products of four values (each <= 15) with one multiplier <= 7
// held in both 16-bit halves of m: no product exceeds a byte, so the 16-bit
// multiplies carry nothing into the neighbouring byte.
__device__ __forceinline__ int pkmul(uint32_t q, uint32_t m) {
    return __builtin_bit_cast(int, __builtin_bit_cast(us2, q) * __builtin_bit_cast(us2, m));
}
// Byte k of w into bytes 0 and 2 (the other bytes zero).
__device__ __forceinline__ uint32_t bcast16(uint32_t w, uint32_t k) {
    return __builtin_amdgcn_perm(0u, w, 0x0c000c00u | (k << 16) | k);
}

// ---- Q4_K: B operands of one superblock ------------------------------------

// The 16-byte header and, for k-half g, bytes 16g..16g+15 of each 32-byte
// quant group of this lane's weight row, from the tile's blocks in LDS (row
// stride 144 bytes: the 16-byte reads of 16 consecutive rows fall on
// distinct banks).
struct Q4Raw {
    u4 h, q[4];
};
__device__ __forceinline__ void q4_read(Q4Raw &r, const unsigned char *blk, uint32_t g) {
    r.h = lds4(blk);
#pragma unroll
    for (int p = 0; p < 4; ++p) r.q[p] = lds4(blk + 16 + 32 * p + 16 * g);
}

// Digit planes of sc*q per sub-block, the mins and the row scales.
struct Q4Frag {
    v4i bh[8], bl[8];
    v4i mb;  // the 8 mins as bf16 (both k-halves: against the high and the low pieces)
    float d, dm;
};

// bf16 of the small integers in bytes 2i and 2i + 1 of w (exact: <= 8 bits).
__device__ __forceinline__ int bf16_pair(uint32_t w, int i) {
    const float f0 = float((w >> (16 * i)) & 0xFFu), f1 = float((w >> (16 * i + 8)) & 0xFFu);
    return int(__builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0), 0x07060302u));
}

// One 32-token block (activation row arow, this k-half's sum pieces at dgp,
// token scales at d8) against this wave's converted weights: the MFMAs (the
// hi and lo chains as two independent accumulators, activation fragments
// read one sub-block ahead, the bf16 min term mid-chain) leave hi in ch, lo
// in cl and Mn in mn; q4_combine is the fp32 combination acc += d8 * (d*C -
// dmin*Mn) with C = 8*hi + lo. A wave issues in order, so VALU work placed
// after a whole chain would wait for it: a block's MFMAs are interleaved in
// program order with VALU work that does not depend on them, the weights'
// conversion for a superblock's first block (k_convert_chain) and the
// previous block's combination for the others (k_chain_combine).
__device__ __forceinline__ void q4_combine(const float *d8, const Q4Frag &f, const v16i &c, const v16f &mn,
                                           float (&acc)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 dv = *reinterpret_cast<const float4 *>(d8 + 8 * q);
        const float dd[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 4 * q + e;
            acc[r] = fmaf(dd[e], fmaf(f.d, float(c[r]), -f.dm * mn[r]), acc[r]);
        }
    }
}

// ---- Q5_K: B operands of one superblock ------------------------------------
// Reference dequantizeQ5_KBlock (GGMLDequantize.hpp:392-402): the Q4_K
// header and nibbles plus a fifth bit per weight, bit s of qh[i] for element
// i of sub-block s; w = d*sc_s*q - dmin*m_s with q = nibble + 16 b (0..31).
// e = sc_s q <= 1953 as digits e = 128 hi + lo (hi <= 15, lo <= 127): the
// same two MFMA chains as Q4_K, C = 128*hi + lo, and the same min term.
using Q5Frag = Q4Frag;
struct Q5Raw : Q4Raw {
    u4 qh;
};
__device__ __forceinline__ void q5_read(Q5Raw &r, const unsigned char *blk, uint32_t g) {
    r.h = lds4(blk);
    r.qh = lds4(blk + 16 + 16 * g);
#pragma unroll
    for (int p = 0; p < 4; ++p) r.q[p] = lds4(blk + 48 + 32 * p + 16 * g);
}
// ---- Q4_K / Q5_K: MFMA chains interleaved with VALU work ------------------
// (q4_combine describes the split.) One step of sub-block s: the hi and lo
// MFMAs, for Q5_K the bit-plane MFMA into the hi chain.
template <bool Q5, typename F>
__device__ __forceinline__ void k_step(const v4i &a, const F &f, int s, v16i &ch, v16i &cl) {
    ch = mfma(a, f.bh[s], ch);
    cl = mfma(a, f.bl[s], cl);
}
// Q5_K digits of e = sc * q for four values q (bytes, <= 31) and sc <= 63
// held in both 16-bit halves of m: hi = e >> 7, lo = e & 127, in byte order.
__device__ __forceinline__ void q5_digits(uint32_t q, uint32_t m, int &hi, int &lo) {
    const uint32_t ee = uint32_t(pkmul(q & 0x00FF00FFu, m)), eo = uint32_t(pkmul((q >> 8) & 0x00FF00FFu, m));
    lo = int(__builtin_amdgcn_perm(eo & 0x007F007Fu, ee & 0x007F007Fu, 0x06020400u));
    hi = int(__builtin_amdgcn_perm((eo >> 7) & 0x001F001Fu, (ee >> 7) & 0x001F001Fu, 0x06020400u));
}

// The conversion of this wave's weights with the first token block's MFMAs,
// in slices: after the MFMAs of sub-block s, the planes of sub-block s + 2.
// The 6-bit scales and mins of the 8 sub-blocks as bytes (reference
// get_scale_min_k4, GGMLDequantize.hpp:436-447); sc = 8h + l with h, l in
// 0..7, so h*q and l*q (q <= 15) are the bytewise products of pkmul; Q5_K's
// bit plane is 2*sc*b (<= 126).
template <bool Q5, typename R, typename F>
__device__ __forceinline__ void k_convert_chain(const R &r, F &f, const ASet &as, uint32_t toff, const unsigned char *dgp,
                                                uint32_t j, uint32_t g, v16i &ch, v16i &cl, v16f &mn) {
    const u4 h = r.h;
    const uint32_t scl = h.y & 0x3F3F3F3Fu, mnl = h.z & 0x3F3F3F3Fu;
    const uint32_t sch = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t mnh = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    const uint32_t hw[2] = {(scl >> 3) & 0x07070707u, (sch >> 3) & 0x07070707u};
    const uint32_t lw[2] = {scl & 0x07070707u, sch & 0x07070707u};
    f.d = h2f(h.x & 0xFFFFu);
    f.dm = h2f(h.x >> 16);
    f.mb = v4i{bf16_pair(mnl, 0), bf16_pair(mnl, 1), bf16_pair(mnh, 0), bf16_pair(mnh, 1)};
    auto conv = [&](int sb) __attribute__((always_inline)) {
        const uint32_t mh = bcast16(hw[sb >> 2], sb & 3), ml = bcast16(lw[sb >> 2], sb & 3);
        const u4 qv = r.q[sb >> 1];
        const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
        if constexpr (!Q5) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t nib = (sb & 1) ? (q[k] >> 4) & 0x0F0F0F0Fu : q[k] & 0x0F0F0F0Fu;
                f.bh[sb][k] = pkmul(nib, mh);
                f.bl[sb][k] = pkmul(nib, ml);
            }
        } else {
            const uint32_t msc = bcast16(sb < 4 ? scl : sch, sb & 3);  // sc_s in both 16-bit halves
            const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t nib = (sb & 1) ? (q[k] >> 4) & 0x0F0F0F0Fu : q[k] & 0x0F0F0F0Fu;
                int hi, lo;
                q5_digits(nib | (((qh[k] >> sb) & 0x01010101u) << 4), msc, hi, lo);
                f.bh[sb][k] = hi;
                f.bl[sb][k] = lo;
            }
        }
    };
    auto aread = [&](int s) __attribute__((always_inline)) { return as_v4i(lds4(as.lds + (as.o[s] + toff))); };
    const v4i dgv = as_v4i(lds4(dgp));
    v4i af[2];
    af[0] = aread(0);
    conv(0);
    conv(1);
    ch = v16i{};
    cl = v16i{};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        if (s + 1 < 8) af[(s + 1) & 1] = aread(s + 1);
        k_step<Q5>(af[s & 1], f, s, ch, cl);
        if (s == 3) mn = mfma_bf16(dgv, f.mb, v16f{});
        if (s + 2 < 8) conv(s + 2);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Block t + 1's MFMAs with block t's combination (as q4_combine) in slices:
// after the MFMAs of sub-block s, the combination of outputs 2s and 2s + 1.
template <bool Q5, typename F>
__device__ __forceinline__ void k_chain_combine(const ASet &as, uint32_t toff, const unsigned char *dgp, const F &f,
                                                uint32_t j, uint32_t g, v16i &ch, v16i &cl, v16f &mn,
                                                const float *d8, const v16i &c, const v16f &mnp, float (&acc)[16]) {
    auto aread = [&](int s) __attribute__((always_inline)) { return as_v4i(lds4(as.lds + (as.o[s] + toff))); };
    const v4i dgv = as_v4i(lds4(dgp));
    float4 dv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) dv[q] = *reinterpret_cast<const float4 *>(d8 + 8 * q);
    v4i af[2];
    af[0] = aread(0);
    ch = v16i{};
    cl = v16i{};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        if (s + 1 < 8) af[(s + 1) & 1] = aread(s + 1);
        k_step<Q5>(af[s & 1], f, s, ch, cl);
        if (s == 3) mn = mfma_bf16(dgv, f.mb, v16f{});
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int r = 2 * s + e;
            const float4 dq = dv[r >> 2];
            const float dd = (r & 3) == 0 ? dq.x : (r & 3) == 1 ? dq.y : (r & 3) == 2 ? dq.z : dq.w;
            acc[r] = fmaf(dd, fmaf(f.d, float(c[r]), -f.dm * mnp[r]), acc[r]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// ---- Q6_K: B operands of one superblock ------------------------------------
// Reference dequantizeQ6_KBlock (GGMLDequantize.hpp:503-527): per 128-element
// half n, element l + 32k (l < 32, k < 4) has q = nibble k / 2 of
// ql[64n + l + 32 (k % 2)] with bits 2k, 2k + 1 of qh[32n + l] above it, and
// scale sc[8n + l / 16 + 2k] (int8); w = d * sc * (q - 32). The lane's k-half
// g of 32-block s = 4n + k is l = 16g .. 16g + 15: 16 values under one scale.
// e = sc * (q - 32) (|e| <= 4096) as signed digits e = 128 hi + lo (hi in
// -32..31, lo in 0..127), so the hi chain, a shift by 7 and the lo chain on
// top give C = sum_s e . x exactly; acc += d8 * (d * C).
struct Q6Frag {
    v4i bh[8], bl[8];
    float d;
};
typedef short s16x2 __attribute__((ext_vector_type(2)));

// 16 unit bytes from offset o (a multiple of 16) of the lane's 2-byte-aligned
// unit at byte sh (0 or 2) of its LDS window: the 16-byte chunk and the next
// dword, realigned; *next receives that dword.
__device__ __forceinline__ u4 q6_read16(const unsigned char *win, uint32_t o, uint32_t sh, uint32_t *next = nullptr) {
    const u4 c = lds4(win + o);
    const uint32_t n = lds1(win + o + 16);
    if (next) *next = n;
    return u4{__builtin_amdgcn_alignbyte(c.y, c.x, sh), __builtin_amdgcn_alignbyte(c.z, c.y, sh),
              __builtin_amdgcn_alignbyte(c.w, c.z, sh), __builtin_amdgcn_alignbyte(n, c.w, sh)};
}

// Signed byte digits of e = sc * (q - 32) for the four values of q (bytes,
// 0..63): 16-bit products of the even and the odd bytes, hi = e >> 7
// (arithmetic), lo = e & 127, packed back in byte order.
__device__ __forceinline__ void q6_digits(uint32_t q, s16x2 sc2, s16x2 m32sc, uint32_t &hi, uint32_t &lo) {
    const s16x2 ee = __builtin_bit_cast(s16x2, q & 0x00FF00FFu) * sc2 + m32sc;
    const s16x2 eo = __builtin_bit_cast(s16x2, (q >> 8) & 0x00FF00FFu) * sc2 + m32sc;
    const s16x2 he = ee >> s16x2{7, 7}, ho = eo >> s16x2{7, 7};
    lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, eo) & 0x007F007Fu,
                               __builtin_bit_cast(uint32_t, ee) & 0x007F007Fu, 0x06020400u);
    hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, ho), __builtin_bit_cast(uint32_t, he), 0x06020400u);
}

struct Q6Raw {
    u4 ql[4], qh[2], sc;  // ql[2n + (k % 2)], qh[n]
    uint32_t dw;          // the dword after the scales (d)
};
__device__ __forceinline__ void q6_read(Q6Raw &r, const unsigned char *win, uint32_t sh, uint32_t g) {
#pragma unroll
    for (int i = 0; i < 4; ++i) r.ql[i] = q6_read16(win, 64 * (i >> 1) + 32 * (i & 1) + 16 * g, sh);
#pragma unroll
    for (int n = 0; n < 2; ++n) r.qh[n] = q6_read16(win, 128 + 32 * n + 16 * g, sh);
    r.sc = q6_read16(win, 192, sh, &r.dw);
}
// The planes of 32-block s into f.
__device__ __forceinline__ void q6_conv(const Q6Raw &r, uint32_t g, int s, Q6Frag &f) {
    const int n = s >> 2, k = s & 3;
    const u4 qlv = r.ql[2 * n + (k & 1)], qhv = r.qh[n];
    const uint32_t ql[4] = {qlv.x, qlv.y, qlv.z, qlv.w}, qh[4] = {qhv.x, qhv.y, qhv.z, qhv.w};
    const uint32_t scw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
    // the lane's scale byte 8n + 2k + g: in dword 2n + k / 2, byte 2 (k % 2) + g
    const short sc = short(int8_t(__builtin_amdgcn_ubfe(scw[2 * n + (k >> 1)], 8 * (2 * (k & 1) + g), 8)));
    const s16x2 sc2 = {sc, sc}, m32sc = {short(-32 * sc), short(-32 * sc)};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t nib = (k >> 1) ? (ql[i] >> 4) & 0x0F0F0F0Fu : ql[i] & 0x0F0F0F0Fu;
        const uint32_t q = nib | (((qh[i] >> (2 * k)) & 0x03030303u) << 4);
        uint32_t hi, lo;
        q6_digits(q, sc2, m32sc, hi, lo);
        f.bh[s][i] = int(hi);
        f.bl[s][i] = int(lo);
    }
}

// The conversion with the first token block's MFMAs (after the MFMA pair of
// block s, the planes of block s + 2), then each further block's MFMAs with
// the previous block's combination (as for Q4_K).
// conv(s): the planes of 32-block s into f.bh[s], f.bl[s]
template <typename Conv>
__device__ __forceinline__ void dig_convert_chain(Conv &&conv, Q6Frag &f, const ASet &as, uint32_t toff, v16i &ch,
                                                  v16i &cl) {
    auto aread = [&](int s) __attribute__((always_inline)) { return as_v4i(lds4(as.lds + (as.o[s] + toff))); };
    v4i af[2];
    af[0] = aread(0);
    conv(0);
    conv(1);
    ch = v16i{};
    cl = v16i{};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        if (s + 1 < 8) af[(s + 1) & 1] = aread(s + 1);
        ch = mfma(af[s & 1], f.bh[s], ch);
        cl = mfma(af[s & 1], f.bl[s], cl);
        if (s + 2 < 8) conv(s + 2);
        __builtin_amdgcn_sched_barrier(0);
    }
}
__device__ __forceinline__ void q6_chain_combine(const ASet &as, uint32_t toff, const Q6Frag &f, uint32_t g,
                                                 v16i &ch, v16i &cl, const float *d8, const v16i &c,
                                                 float (&acc)[16]) {
    auto aread = [&](int s) __attribute__((always_inline)) { return as_v4i(lds4(as.lds + (as.o[s] + toff))); };
    float4 dv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) dv[q] = *reinterpret_cast<const float4 *>(d8 + 8 * q);
    v4i af[2];
    af[0] = aread(0);
    ch = v16i{};
    cl = v16i{};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        if (s + 1 < 8) af[(s + 1) & 1] = aread(s + 1);
        ch = mfma(af[s & 1], f.bh[s], ch);
        cl = mfma(af[s & 1], f.bl[s], cl);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int rr = 2 * s + e;
            const float4 dq = dv[rr >> 2];
            const float dd = (rr & 3) == 0 ? dq.x : (rr & 3) == 1 ? dq.y : (rr & 3) == 2 ? dq.z : dq.w;
            acc[rr] = fmaf(dd, f.d * float(c[rr]), acc[rr]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}
__device__ __forceinline__ void q6_combine(const float *d8, const Q6Frag &f, const v16i &c, float (&acc)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 dv = *reinterpret_cast<const float4 *>(d8 + 8 * q);
        const float dd[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[4 * q + e] = fmaf(dd[e], f.d * float(c[4 * q + e]), acc[4 * q + e]);
    }
}

// ---- IQ2_S: B operands of one superblock -----------------------------------
// Reference dequantizeIQ2_SBlock and its fused block dot
// (GGMLDequantize.hpp:1215-1242, :2028-2057): group l (8 weights) of 32-block
// ib has the 8 magnitudes (8, 25 or 43) of codebook entry qs[4ib + l] | bits
// 2l, 2l+1 of qh[ib] << 8, negated by the bits of signs[4ib + l], times
// 2ls + 1 with ls nibble l / 2 of scales[ib]; the row is scaled by d/8. The
// lane's k-half g of 32-block s is groups 2g and 2g + 1: one scale k. With the
// signs applied bytewise and the sign bit flipped, q = w + 128 (85..171), so
// e = k*q - 128k (|e| <= 1333) takes Q6_K's signed digits, C = 128 hi + lo,
// acc += d8 * ((d/8) * C).
struct I2Raw {
    uint32_t qs[8], sg[8];  // the lane's index and sign byte pairs per 32-block
    uint32_t qh[2], sc[2];  // qh[0..7], scales[0..7]
    uint32_t d;
};
__device__ __forceinline__ void i2_read(I2Raw &r, const unsigned char *win, uint32_t sh, uint32_t g) {
    const uint16_t *u = reinterpret_cast<const uint16_t *>(win + sh);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        r.qs[s] = u[1 + 2 * s + g];
        r.sg[s] = u[17 + 2 * s + g];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        r.qh[i] = uint32_t(u[33 + 2 * i]) | (uint32_t(u[34 + 2 * i]) << 16);
        r.sc[i] = uint32_t(u[37 + 2 * i]) | (uint32_t(u[38 + 2 * i]) << 16);
    }
    r.d = u[0];
}
__device__ __forceinline__ void i2_conv(const I2Raw &r, const unsigned char *grid, uint32_t g, int s, Q6Frag &f) {
    const uint32_t qhb = __builtin_amdgcn_ubfe(r.qh[s >> 2], 8 * (s & 3) + 4 * g, 4);  // bits of groups 2g, 2g + 1
    const short k = short(2 * __builtin_amdgcn_ubfe(r.sc[s >> 2], 8 * (s & 3) + 4 * g, 4) + 1);
    const s16x2 k2 = {k, k}, off = {short(-128 * k), short(-128 * k)};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t idx = __builtin_amdgcn_ubfe(r.qs[s], 8 * h, 8) | (((qhb >> (2 * h)) & 3u) << 8);
        const uint2 gv = *reinterpret_cast<const uint2 *>(grid + 8 * idx);
        const uint32_t sb = __builtin_amdgcn_ubfe(r.sg[s], 8 * h, 8);
        const uint32_t m1 = spread_sign4(sb & 15u), m2 = spread_sign4(sb >> 4);
        const uint32_t q0 = ((gv.x ^ m1) + (m1 & 0x01010101u)) ^ 0x80808080u;
        const uint32_t q1 = ((gv.y ^ m2) + (m2 & 0x01010101u)) ^ 0x80808080u;
        uint32_t hi, lo;
        q6_digits(q0, k2, off, hi, lo);
        f.bh[s][2 * h] = int(hi);
        f.bl[s][2 * h] = int(lo);
        q6_digits(q1, k2, off, hi, lo);
        f.bh[s][2 * h + 1] = int(hi);
        f.bl[s][2 * h + 1] = int(lo);
    }
}

__constant__ uint64_t c_pf_iq2s_grid[1024] = {
#include "iq2s_grid.inc"
};

// ---- Q8_0: B operands of one superblock ------------------------------------

// The 8 blocks of this lane's row (34-byte blocks, so 2-byte aligned; read
// as the 16-byte chunks that hold them, conflict-free at the 272-byte row
// stride): the 16 values of k-half g of each block as one B operand, and each block's
// scale as bf16 pieces dw = h + l (l exact: dw has 11 significant bits) laid
// out against the activation pieces of a block pair, [h8 m8 l8 0] of the
// even block then of the odd one, in both k-halves: k-half 0 holds h against
// this block's pieces, k-half 1 holds l, and the other block's slots are zero.
struct Q8Frag {
    v4i bw[8], bp[8];
};

__device__ __forceinline__ void q8_convert(const unsigned char *row, uint32_t g, Q8Frag &f) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        // the 16 values start at byte 34k + 2 + 16g: in the 16-byte chunks
        // cs + g and cs + g + 1 (cs = (34k + 2) / 16) at shift sh
        const int sb = 34 * k + 2, cs = sb / 16, sh = sb % 16;  // constants once unrolled
        const unsigned char *cp = row + 16 * (cs + g);
        uint32_t v[8] = {};
        const u4 lo = lds4(cp);
        v[0] = lo.x, v[1] = lo.y, v[2] = lo.z, v[3] = lo.w;
        if (sh != 0) {
            const u4 hi = lds4(cp + 16);
            v[4] = hi.x, v[5] = hi.y, v[6] = hi.z, v[7] = hi.w;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            f.bw[k][i] = sh % 4 == 0 ? int(v[sh / 4 + i])
                                     : int(__builtin_amdgcn_alignbyte(v[sh / 4 + i + 1], v[sh / 4 + i], sh % 4));
        const uint32_t dword = lds1(row + ((34 * k) & ~3u));
        const uint32_t dbits = (k & 1) ? dword >> 16 : dword & 0xFFFFu;
        const float d = h2f(dbits);
        const uint32_t hb = __builtin_bit_cast(uint32_t, d) & 0xFFFF0000u;
        const uint32_t lb = __builtin_bit_cast(uint32_t, d - __builtin_bit_cast(float, hb));
        const uint32_t h16 = hb >> 16, l16 = lb >> 16;
        const int p0 = int(g == 0 ? h16 | hb : l16 | (l16 << 16)), p1 = int(g == 0 ? h16 : l16);
        f.bp[k] = (k & 1) ? v4i{0, 0, p0, p1} : v4i{p0, p1, 0, 0};
    }
}

// One 32-token block (the token's activation pieces at prow, those of blocks
// 2c, 2c + 1 at prow + 256 c): per 32-wide weight block k, the exact integer
// product I (int8 MFMA) and the scales dw*d8 of its 32x32 outputs (bf16
// MFMA), then acc += I * scale. Block k + 1's MFMAs are issued before block
// k's fp32 combination, so that the matrix core works while the VALU does.
__device__ __forceinline__ void q8_block(const ASet &as, uint32_t toff, const unsigned char *prow, const Q8Frag &f,
                                         uint32_t j, uint32_t g, float (&acc)[16]) {
    auto aread = [&](int k) __attribute__((always_inline)) { return as_v4i(lds4(as.lds + (as.o[k] + toff))); };
    auto pread = [&](int c) __attribute__((always_inline)) { return as_v4i(lds4(prow + 256 * c)); };
    v4i af[3], pp[2];
    af[0] = aread(0);
    af[1] = aread(1);
    pp[0] = pread(0);
    v16i I[2];
    v16f S[2];
    I[0] = mfma(af[0], f.bw[0], v16i{});
    S[0] = mfma_bf16(pp[0], f.bp[0], v16f{});
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        if (k + 2 < 8) af[(k + 2) % 3] = aread(k + 2);
        if (k + 1 < 8 && ((k + 1) & 1) == 0) pp[((k + 1) >> 1) & 1] = pread((k + 1) >> 1);
        if (k + 1 < 8) {
            I[(k + 1) & 1] = mfma(af[(k + 1) % 3], f.bw[k + 1], v16i{});
            S[(k + 1) & 1] = mfma_bf16(pp[((k + 1) >> 1) & 1], f.bp[k + 1], v16f{});
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = fmaf(float(I[k & 1][r]), S[k & 1][r], acc[r]);
        __builtin_amdgcn_sched_barrier(0);
    }
}


// ---- IQ3_XXS: B operands of one superblock ---------------------------------
// Reference dequantizeIQ3_XXSBlock (GGMLDequantize.hpp:1135-1161) and the
// fused dot (:2064-2097): per 32-block ib, 8 grid indices (qs, 4 weights
// each), and aux = 4 7-bit sign indices (sign byte = idx | parity(idx) << 7)
// and the scale ls in bits 28-31; a weight is d * (0.5 + ls) * 0.5 * grid
// byte * sign, i.e. (d / 4) * (2 ls + 1) * signed grid byte. The signed
// grid bytes (|w| <= 62) are the int8 B operand as they are, so one MFMA per
// 32-block gives the exact integer I_ib; isum = sum_ib (2 ls + 1) I_ib by
// 24-bit integer multiply-adds (|I| < 2^18), then acc += (d / 4) * d8 * isum.

__constant__ uint32_t c_pf_iq3_grid[256] = {
#include "iq3xxs_grid.inc"
};

struct I3Frag {
    v4i bw[8];  // the signed grid bytes of k-half g of each 32-block
    int sc[8];  // 2 ls + 1
    float d;    // d / 4
};

// This lane's row: the 100-byte window (its unit at byte sh of it) in the
// row's LDS chunks, its bytes 96-99 in tail. Fields are read as 2-byte
// halves (the unit is 2-byte aligned). sgrid: the signed grid in LDS, entry
// 16 i + n = grid word i with the signs of nibble n applied bytewise.
__device__ __forceinline__ void i3_convert(const unsigned char *row, const unsigned char *tail, uint32_t sh,
                                           const uint32_t *sgrid, uint32_t g, I3Frag &f) {
    auto h16 = [&](uint32_t x) __attribute__((always_inline)) {  // window bytes x, x + 1 (x even, < 96)
        return uint32_t(*reinterpret_cast<const uint16_t *>(row + x));
    };
    f.d = 0.25f * h2f(h16(sh));
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        const uint32_t qo = sh + 2 + 8 * ib + 4 * g, ao = sh + 66 + 4 * ib;
        const uint32_t qsw = h16(qo) | (h16(qo + 2) << 16);
        uint32_t aux;
        if (ib < 7) {
            aux = h16(ao) | (h16(ao + 2) << 16);
        } else {  // window bytes sh + 94 .. sh + 97: the last ones in tail
            const uint32_t t = *reinterpret_cast<const uint32_t *>(tail);
            aux = sh ? t : __builtin_amdgcn_alignbyte(t, h16(94) << 16, 2);
        }
        f.sc[ib] = 2 * int(aux >> 28) + 1;
        uint32_t e[4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {  // sign group l = 2g + u: 8 weights, grid indices bytes 2u, 2u + 1 of qsw
            const uint32_t s7 = __builtin_amdgcn_ubfe(aux, 14 * g + 7 * u, 7);
            const uint32_t s8 = s7 | ((__builtin_popcount(s7) & 1u) << 7);
            e[2 * u] = sgrid[(__builtin_amdgcn_ubfe(qsw, 16 * u, 8) << 4) | (s8 & 15u)];
            e[2 * u + 1] = sgrid[(__builtin_amdgcn_ubfe(qsw, 16 * u + 8, 8) << 4) | (s8 >> 4)];
        }
        f.bw[ib] = v4i{int(e[0]), int(e[1]), int(e[2]), int(e[3])};
    }
}


// ---- IQ3_S: B operands of one superblock ------------------------------------
// Reference dequantizeIQ3_SBlock (GGMLDequantize.hpp:1164-1212) and the
// fused dot (:2102-2145): per 32-block ib, 8 grid indices (qs bytes, bit 8
// from qh[ib]) into the 512-word codebook (magnitudes <= 15), 32 sign bits
// (signs[4 ib .. 4 ib + 3], one per weight) and the scale 2 ls + 1 (ls the
// nibble ib % 2 of scales[ib / 2]); value = d * d8 * isum as for IQ3_XXS
// (no 1/4 factor).

__constant__ uint32_t c_pf_iq3s_grid[512] = {
#include "iq3s_grid.inc"
};

// This lane's row: the 112-byte window (its unit at byte sh) in the row's
// LDS chunks; fields read as 2-byte halves.
__device__ __forceinline__ void is3_convert(const unsigned char *row, uint32_t sh, const uint32_t *sgrid, uint32_t g,
                                            I3Frag &f) {
    auto h16 = [&](uint32_t x) __attribute__((always_inline)) {  // window bytes x, x + 1 (x even)
        return uint32_t(*reinterpret_cast<const uint16_t *>(row + x));
    };
    f.d = h2f(h16(sh));
    const uint32_t scw = h16(sh + 106) | (h16(sh + 108) << 16);  // the 8 scale nibbles
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        const uint32_t qo = sh + 2 + 8 * ib + 4 * g;
        const uint32_t qsw = h16(qo) | (h16(qo + 2) << 16);             // indices 4g .. 4g + 3 (low 8 bits)
        const uint32_t qhb = h16(sh + 66 + (ib & ~1)) >> (8 * (ib & 1)); // qh[ib] (bits 8 of the 8 indices)
        const uint32_t sgn = h16(sh + 74 + 4 * ib + 2 * g);            // sign bytes of groups 2g, 2g + 1
        f.sc[ib] = 2 * int((scw >> (4 * ib)) & 15u) + 1;
        uint32_t e[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {  // word k: index 4g + k, sign nibble k % 2 of group 2g + k / 2
            const uint32_t idx = __builtin_amdgcn_ubfe(qsw, 8 * k, 8) | (__builtin_amdgcn_ubfe(qhb, 4 * g + k, 1) << 8);
            const uint32_t nib = __builtin_amdgcn_ubfe(sgn, 4 * k, 4);
            e[k] = sgrid[(idx << 4) | nib];
        }
        f.bw[ib] = v4i{int(e[0]), int(e[1]), int(e[2]), int(e[3])};
    }
}

// P (1 or 2) 32-token blocks (activation rows arow[t], token scales d8[t]):
// per 32-block the MFMAs of all P token blocks first, then their integer
// multiply-adds (so that no multiply-add waits for the MFMA issued just
// before it).
template <int P>
__device__ __forceinline__ void i3_blocks(const ASet &as, uint32_t toff, const float *const (&d8)[P], const I3Frag &f,
                                          float (&acc)[P][16]) {
    int is[P][16];
#pragma unroll
    for (int t = 0; t < P; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) is[t][r] = 0;
    auto aread = [&](int ib, int t) __attribute__((always_inline)) {
        return as_v4i(lds4(as.lds + (as.o[ib] + toff + 8192u * t)));
    };
    // Activation fragments two 32-blocks ahead, and block ib + 1's MFMAs
    // issued before block ib's multiply-adds (the matrix core works while
    // the VALU does); the scheduling barriers keep that order (the scheduler
    // otherwise reads each fragment right before its MFMA and runs each
    // block's multiply-adds right after its own MFMA).
    v4i af[3][P];
    v16i I[2][P];
#pragma unroll
    for (int t = 0; t < P; ++t) {
        af[0][t] = aread(0, t);
        af[1][t] = aread(1, t);
    }
#pragma unroll
    for (int t = 0; t < P; ++t) I[0][t] = mfma(af[0][t], f.bw[0], v16i{});
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        if (ib + 2 < 8)
#pragma unroll
            for (int t = 0; t < P; ++t) af[(ib + 2) % 3][t] = aread(ib + 2, t);
        if (ib + 1 < 8)
#pragma unroll
            for (int t = 0; t < P; ++t) I[(ib + 1) & 1][t] = mfma(af[(ib + 1) % 3][t], f.bw[ib + 1], v16i{});
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < P; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                is[t][r] = __mul24(f.sc[ib], I[ib & 1][t][r]) + is[t][r];  // v_mad_i32_i24
                // kept as one multiply-add per 32-block: the compiler would
                // otherwise reassociate the chain into multiplies and 3-way adds
                asm("" : "+v"(is[t][r]));
            }
        __builtin_amdgcn_sched_barrier(0);
    }
    float4 dv[P][4];
#pragma unroll
    for (int t = 0; t < P; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) dv[t][q] = *reinterpret_cast<const float4 *>(d8[t] + 8 * q);
#pragma unroll
    for (int t = 0; t < P; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float dd[4] = {dv[t][q].x, dv[t][q].y, dv[t][q].z, dv[t][q].w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc[t][4 * q + e] = fmaf(dd[e] * f.d, float(is[t][4 * q + e]), acc[t][4 * q + e]);
        }
}

// The lane's index recomputed where it is used (v_mbcnt on an opaque zero):
// a value the compiler cannot hoist, so that no register holds the lane
// across the kernel's loops (held, it was spilled, and the reload's wait also
// waited for the stage loads just issued).
__device__ __forceinline__ uint32_t lane_now() {
    uint32_t z = 0;
    asm volatile("" : "+s"(z));
    return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, z));
}

// ---- loads into LDS ---------------------------------------------------------

// Direct-to-LDS buffer loads (no registers, no LDS stores): lane l's 16 (or
// 4) bytes land at lds_dst + 16 l (4 l). Inline, so that the compiler, which
// cannot tell which LDS bytes these write, does not wait for them before the
// wave's other LDS reads; the kernel waits (vmcnt) before its barrier. m0 (the
// LDS destination) is restored afterwards: the compiler may hold a value there.
__device__ __forceinline__ void lds_load16(uint32_t lds_dst, v4i rs, uint32_t voff) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(__builtin_amdgcn_readfirstlane(lds_dst)), "v"(voff), "s"(rs), "s"(0u)
                 : "memory");
}
__device__ __forceinline__ void lds_load4(uint32_t lds_dst, v4i rs, uint32_t voff) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dword %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(__builtin_amdgcn_readfirstlane(lds_dst)), "v"(voff), "s"(rs), "s"(0u)
                 : "memory");
}

__device__ __forceinline__ v4i rs4(const void *p, uint32_t bytes) {
    const uint64_t base = reinterpret_cast<uint64_t>(p);
    return v4i{int(uint32_t(base)), int(uint32_t(base >> 32) & 0xFFFF), int(bytes), 0x00020000};
}
__device__ __forceinline__ uint32_t lds_addr(const unsigned char *p) {
    return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)(p)));
}

// Wave instruction k of N (k = w, w + PW, ...) -- the loads of one stage are
// spread over the waves.
// Waves 0-3 issue all of a stage's loads: the second wave on each SIMD
// (w + 4) runs behind the first (the hardware favours the older wave), and
// measured 2-8% faster with no loads to issue (the first waves otherwise wait
// for it at the barrier).
constexpr uint32_t LW = 4;
template <uint32_t N, typename F>
__device__ __forceinline__ void each_inst(uint32_t w, F &&f) {
    if (w >= LW) return;
#pragma unroll
    for (uint32_t i = 0; i < (N + LW - 1) / LW; ++i) {
        const uint32_t k = w + LW * i;
        if (N % LW == 0 || k < N) f(k);
    }
}

// Superblock b of the tile into one LDS buffer: activation values (1 KB per
// wave instruction = 4 tokens, XOR-swizzled chunks), their scale data, and the
// weight blocks of rows n0 .. n0 + PR - 1 ([row][UB]; a wave instruction
// covers 64 consecutive 16-byte chunks, so its loads fall on consecutive
// rows: whole cache lines). Tokens past M read other tokens' bytes or zeros
// and rows past N lie outside the descriptor (zeros); neither is stored.
template <int TYPE, int NT>
__device__ __forceinline__ void stage(const PfArgs &a, const uint8_t *W, uint32_t m0, uint32_t n0, uint32_t b,
                                      unsigned char *buf, uint32_t w, unsigned char *wbuf) {
    using L = PLds<TYPE, NT>;
    using T = PfType<TYPE>;
    constexpr uint32_t TT = L::TT;
    const uint32_t base = lds_addr(buf), wbase = lds_addr(wbuf);
    const uint32_t tb = b * a.M + m0;  // first token record of the tile in this superblock
    const uint32_t ln = lane_now();  // per-call lane arithmetic (not hoisted into held registers)
    const v4i rq = rs4(a.qs, a.M * a.K);
    each_inst<TT / 4>(w, [&](uint32_t k) {
        const uint32_t t = 4 * k + ln / 16;
        lds_load16(base + L::QS + 1024 * k, rq, (tb + t) * 256 + 16 * ((ln & 15) ^ (t & 15)));
    });
    const v4i rx = rs4(a.xs, a.M * a.nblk * T::XB);
    if constexpr (TYPE != kQ8_0 && TYPE != kQ8W) {
        if constexpr (T::XB != 0)
            each_inst<TT / 32>(w, [&](uint32_t k) {
                lds_load16(base + L::XS + 1024 * k, rx, (tb + 32 * k) * T::XB + 16 * ln);
            });
        const v4i rd = rs4(a.d8, a.M * a.nblk * 4);
        each_inst<(TT + 63) / 64>(w, [&](uint32_t k) { lds_load4(base + L::D8 + 256 * k, rd, (tb + 64 * k + ln) * 4); });
    } else {
        // chunk-major per 16 tokens: slot 16c + t of group k holds chunk c
        // (blocks 2c, 2c + 1) of token 16k + t, so that the 32 tokens' reads
        // of one block fall on distinct banks
        each_inst<TT * T::XB / 1024>(w, [&](uint32_t k) {
            lds_load16(base + L::XS + 1024 * k, rx, (tb + 16 * k + (ln & 15)) * T::XB + 16 * (ln >> 4));
        });
    }
    constexpr uint32_t CPR = T::UB / 16;  // 16-byte chunks per row
    // the weight range rounded up to whole dwords: the range check zeroes a
    // dword that is only partly in range, and the 2-byte-aligned IQ3_XXS
    // units end 2 bytes into one when their count is odd (the dword stays in
    // the same 4 KB page as the matrix's last byte)
    const v4i rw = rs4(W, (a.N * a.row_bytes + 3) & ~3u);
    each_inst<T::PR * CPR / 64>(w, [&](uint32_t k) {
        const uint32_t c = 64 * k + ln, r = c / CPR, p = c - CPR * r;
        if constexpr (TYPE == kIQ3_XXS)  // the window from the unit's 4-byte-aligned start (slot 6: unused)
            lds_load16(wbase + 1024 * k, rw, (((n0 + r) * a.row_bytes + b * 98) & ~3u) + 16 * min(p, 5u));
        else if constexpr (TYPE == kIQ3_S)
            lds_load16(wbase + 1024 * k, rw, (((n0 + r) * a.row_bytes + b * 110) & ~3u) + 16 * p);
        else if constexpr (TYPE == kIQ2_S)  // (slot 6: unused)
            lds_load16(wbase + 1024 * k, rw, (((n0 + r) * a.row_bytes + b * 82) & ~3u) + 16 * min(p, 5u));
        else if constexpr (TYPE == kQ6_K)  // (slot 14: unused)
            lds_load16(wbase + 1024 * k, rw, (((n0 + r) * a.row_bytes + b * 210) & ~3u) + 16 * min(p, 13u));
        else
            lds_load16(wbase + 1024 * k, rw, (n0 + r) * a.row_bytes + b * T::UB + 16 * p);
    });
    if constexpr (TYPE == kIQ3_XXS)  // the window's 25th dword (ends at most 2 bytes past the unit)
        each_inst<T::PR / 64>(w, [&](uint32_t k) {
            lds_load4(base + L::TAIL + 256 * k, rw, (((n0 + 64 * k + ln) * a.row_bytes + b * 98) & ~3u) + 96);
        });
}

__host__ __device__ inline uint32_t sk_begin(uint32_t units, uint32_t grid, uint32_t v) {
    return uint32_t(uint64_t(units) * v / grid);
}
// Range number of workgroup `bid`: the workgroups of one XCD take
// consecutive ranges (bid % 8 is the XCD under round-robin dispatch).
__device__ __forceinline__ uint32_t sk_logical(uint32_t bid, uint32_t G) {
    return (G & 7) ? bid : (bid & 7) * (G >> 3) + (bid >> 3);
}

template <int TYPE, int NT, bool GRP>
__global__ __launch_bounds__(64 * PW) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_prefill(PfArgs a) {
    extern __shared__ __align__(16) unsigned char lds[];
    using L = PLds<TYPE, NT>;
    using T = PfType<TYPE>;
    constexpr uint32_t TT = L::TT, PR = T::PR;
    constexpr uint32_t RG = PW / T::TSPLIT;       // row groups of 32
    constexpr int NB = NT / int(T::TSPLIT);       // 32-token blocks per wave
    static_assert(NB >= 1, "at least one token block per wave");
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t rg = w % RG, tg = w / RG;      // row group, token group
    // the two stage buffers by parity (ph: the one holding the superblock
    // being computed; a running count, as segments hand their last stage on)
    auto buf = [&](uint32_t p) __attribute__((always_inline)) { return lds + L::BUF0 + (p & 1) * L::bytes; };
    auto wbuf = [&](uint32_t p) __attribute__((always_inline)) { return L::SW ? lds + L::WS : buf(p) + L::W; };

    if constexpr (TYPE == kIQ2_S) {
        uint2 *gr = reinterpret_cast<uint2 *>(lds + L::GRID);
        for (uint32_t e = tid; e < 1024; e += 64 * PW) {
            const uint64_t v = c_pf_iq2s_grid[e];
            gr[e] = make_uint2(uint32_t(v), uint32_t(v >> 32));
        }
    } else if constexpr (pf_grid_bytes(TYPE) != 0) {
        // the signed grid: entry 16 i + n = grid word i with the signs of
        // nibble n applied bytewise (grid bytes are nonzero: no carries)
        uint32_t *sg = reinterpret_cast<uint32_t *>(lds + L::GRID);
        for (uint32_t e = tid; e < pf_grid_bytes(TYPE) / 4; e += 64 * PW) {
            const uint32_t m = spread_sign4(e & 15u);
            const uint32_t gw = TYPE == kIQ3_XXS ? c_pf_iq3_grid[e >> 4] : c_pf_iq3s_grid[e >> 4];
            sg[e] = (gw ^ m) + (m & 0x01010101u);
        }
        // first read after the superblock loop's barrier
    }
    const uint32_t v = sk_logical(blockIdx.x, a.G);
    const uint32_t units = pf_ntiles<GRP>(a) * a.nblk;
    const uint32_t ub = sk_begin(units, a.G, v), ue = sk_begin(units, a.G, v + 1);
    uint32_t ph = 0;
    if (ub < ue) {
        const uint32_t tile = ub / a.nblk;
        const PfTile t0 = pf_tile<GRP>(a, tile, TT, PR);
        stage<TYPE, NT>(a, t0.W, t0.m0, t0.n0, ub - tile * a.nblk, buf(ph), w, wbuf(ph));
    }
    for (uint32_t u = ub; u < ue;) {
        const uint32_t tile = u / a.nblk;
        const uint32_t b0 = u - tile * a.nblk;
        const uint32_t b1 = min(a.nblk, b0 + (ue - u));
        const bool whole = b0 == 0 && b1 == a.nblk;
        float *const part = whole ? nullptr : a.ws + (size_t(v) * 2 + (u == ub ? 0 : 1)) * (TT * PR);
        u += b1 - b0;
        // The lane's row and k-half, recomputed per segment: the opaque copy
        // keeps the compiler from hoisting the address arithmetic of the
        // final stores out of the segment loop into registers held throughout.
        const uint32_t ln = lane_now();
        const uint32_t j = ln & 31, g = ln >> 5;
        const PfTile tg_ = pf_tile<GRP>(a, tile, TT, PR);
        const uint32_t n0 = tg_.n0, m0 = tg_.m0;
        const uint32_t rl = 32 * rg + j;  // the lane's row in the tile

        float acc[NB][16];
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;

        // The segment's first superblock is staged already (before the loop,
        // or by the previous segment's last iteration); the last iteration
        // stages the next segment's first, so that its loads overlap this
        // segment's final MFMAs and epilogue (M = 128: 1-7% faster; MoE
        // grouped launches 4-5%).
        const uint32_t ntile = u / a.nblk;  // (u < ue: the next segment's tile, starting at superblock 0)
        auto stage_next = [&](uint32_t b) __attribute__((always_inline)) {
            if (b + 1 < b1) {
                stage<TYPE, NT>(a, tg_.W, m0, n0, b + 1, buf(ph + 1), w, wbuf(ph + 1));
            } else if (u < ue) {
                const PfTile nt_ = pf_tile<GRP>(a, ntile, TT, PR);
                stage<TYPE, NT>(a, nt_.W, nt_.m0, nt_.n0, 0, buf(ph + 1), w, wbuf(ph + 1));
            }
        };
        // Per superblock: its loads are waited for, the next superblock's
        // issued into the other LDS buffer, this lane's weights converted,
        // then the MFMAs.
        for (uint32_t b = b0; b < b1; ++b) {
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            __syncthreads();
            // (SW: after this superblock's raw weight reads, below)
            if constexpr (!L::SW) stage_next(b);
            const unsigned char *bb = buf(ph);
            const unsigned char *wb = wbuf(ph);
            // this lane's activation addresses of the wave's first token block
            const ASet as = aset(lds, uint32_t(bb - lds) + L::QS + (32 * tg * NB + j) * 256, j, g);
            if constexpr (TYPE == kQ4_K || TYPE == kQ5_K) {
                constexpr bool Q5 = TYPE == kQ5_K;
                using Frag = std::conditional_t<Q5, Q5Frag, Q4Frag>;
                Frag f;
                // token block t + 1's MFMAs issued before block t's fp32
                // combination: the matrix core works while the VALU does
                auto d8_t = [&](int t) __attribute__((always_inline)) {
                    return reinterpret_cast<const float *>(bb + L::D8) + 32 * (tg * NB + t) + 4 * g;
                };
                // (C = 8*hi + lo formed once block t + 1's MFMAs are done,
                // so that only C and Mn of block t stay live across them)
                v16i c[2], ch, cl;
                v16f mn[2];
                __builtin_amdgcn_sched_barrier(0);
                {
                    std::conditional_t<Q5, Q5Raw, Q4Raw> rr;
                    // (the row's offset recomputed here: held across the
                    // segment, it was spilled)
                    const unsigned char *wrow = wb + (32 * rg + (lane_now() & 31)) * T::UB;
                    if constexpr (Q5)
                        q5_read(rr, wrow, g);
                    else
                        q4_read(rr, wrow, g);
                    if constexpr (L::SW) {
                        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): every raw read done
                        __syncthreads();
                        stage_next(b);
                    }
                    const uint32_t tok = 32 * tg * NB + j;
                    k_convert_chain<Q5>(rr, f, as, 0u, bb + L::XS + tok * T::XB + 16 * g, j, g, ch, cl, mn[0]);
                }
                constexpr int CSH = Q5 ? 7 : 3;  // C = 128*hi + lo (Q5_K), 8*hi + lo (Q4_K)
#pragma unroll
                for (int r = 0; r < 16; ++r) c[0][r] = (ch[r] << CSH) + cl[r];
#pragma unroll
                for (int t = 0; t < NB; ++t) {
                    if (t + 1 < NB) {
                        const uint32_t tok = 32 * (tg * NB + t + 1) + j;
                        k_chain_combine<Q5>(as, 8192u * (t + 1), bb + L::XS + tok * T::XB + 16 * g, f, j, g, ch, cl,
                                            mn[(t + 1) & 1], d8_t(t), c[t & 1], mn[t & 1], acc[t]);
                    } else {
                        q4_combine(d8_t(t), f, c[t & 1], mn[t & 1], acc[t]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    if (t + 1 < NB) {
#pragma unroll
                        for (int r = 0; r < 16; ++r) c[(t + 1) & 1][r] = (ch[r] << CSH) + cl[r];
                    }
                }
            } else if constexpr (TYPE == kQ6_K || TYPE == kIQ2_S) {
                Q6Frag f;
                auto d8_t = [&](int t) __attribute__((always_inline)) {
                    return reinterpret_cast<const float *>(bb + L::D8) + 32 * (tg * NB + t) + 4 * g;
                };
                v16i c[2], ch, cl;
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (TYPE == kQ6_K) {
                    const uint32_t sh = ((n0 + rl) * a.row_bytes + b * 210) & 3u;
                    Q6Raw rr;
                    q6_read(rr, wb + rl * T::UB, sh, g);
                    if constexpr (L::SW) {
                        // every wave's raw reads done, then the next
                        // superblock's loads (into the one weight region)
                        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                        __syncthreads();
                        stage_next(b);
                    }
                    dig_convert_chain([&](int s) __attribute__((always_inline)) { q6_conv(rr, g, s, f); }, f, as, 0u,
                                      ch, cl);
                    f.d = h2f(sh ? rr.dw >> 16 : rr.dw & 0xFFFFu);
                } else {
                    static_assert(!L::SW, "IQ2_S: two weight stages");
                    const uint32_t sh = ((n0 + rl) * a.row_bytes + b * 82) & 3u;
                    I2Raw rr;
                    i2_read(rr, wb + rl * T::UB, sh, g);
                    const unsigned char *grid = lds + L::GRID;
                    dig_convert_chain([&](int s) __attribute__((always_inline)) { i2_conv(rr, grid, g, s, f); }, f,
                                      as, 0u, ch, cl);
                    f.d = 0.125f * h2f(rr.d);  // (a power of two: exact)
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) c[0][r] = (ch[r] << 7) + cl[r];
#pragma unroll
                for (int t = 0; t < NB; ++t) {
                    if (t + 1 < NB) {
                        q6_chain_combine(as, 8192u * (t + 1), f, g, ch, cl, d8_t(t), c[t & 1], acc[t]);
                    } else {
                        q6_combine(d8_t(t), f, c[t & 1], acc[t]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    if (t + 1 < NB) {
#pragma unroll
                        for (int r = 0; r < 16; ++r) c[(t + 1) & 1][r] = (ch[r] << 7) + cl[r];
                    }
                }
            } else if constexpr (TYPE == kIQ3_XXS || TYPE == kIQ3_S) {
                I3Frag f;
                if constexpr (TYPE == kIQ3_XXS)
                    i3_convert(wb + rl * T::UB, bb + L::TAIL + 4 * rl, ((n0 + rl) * a.row_bytes + b * 98) & 3u,
                               reinterpret_cast<const uint32_t *>(lds + L::GRID), g, f);
                else
                    is3_convert(wb + rl * T::UB, ((n0 + rl) * a.row_bytes + b * 110) & 3u,
                                reinterpret_cast<const uint32_t *>(lds + L::GRID), g, f);
                constexpr int P = NB >= 2 ? 2 : 1;
                static_assert(NB % P == 0, "token blocks in pairs");
#pragma unroll
                for (int t = 0; t < NB; t += P) {
                    __builtin_amdgcn_sched_barrier(0);
                    const float *dp[P];
#pragma unroll
                    for (int i = 0; i < P; ++i)
                        dp[i] = reinterpret_cast<const float *>(bb + L::D8) + 32 * (tg * NB + t + i) + 4 * g;
                    i3_blocks<P>(as, 8192u * t, dp, f, reinterpret_cast<float(&)[P][16]>(acc[t]));
                }
            } else {
                Q8Frag f;
                q8_convert(wb + rl * T::UB, g, f);
                if constexpr (L::SW) {
                    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): every raw read done
                    __syncthreads();
                    stage_next(b);
                }
#pragma unroll
                for (int t = 0; t < NB; ++t) {
                    __builtin_amdgcn_sched_barrier(0);
                    const uint32_t tok = 32 * (tg * NB + t) + j;
                    q8_block(as, 8192u * t, bb + L::XS + 1024 * (tok >> 4) + 16 * (tok & 15), f, j, g, acc[t]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            ph ^= 1;
        }

        // lane: row n0 + rl, tokens m0 + 32 (tg NB + t) + 8q + 4g + e
        const uint32_t n = n0 + rl;
        if (part == nullptr) {
#pragma unroll
            for (int t = 0; t < NB; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t ml = 32 * (tg * NB + t) + 8 * q + 4 * g + e, m = m0 + ml;
                        if (m < tg_.mend && n < a.N) tg_.out[size_t(m) * a.N + n] = acc[t][4 * q + e];
                    }
            continue;
        }
        if (!a.fused) {
#pragma unroll
            for (int t = 0; t < NB; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        part[(32 * (tg * NB + t) + 8 * q + 4 * g + e) * PR + rl] = acc[t][4 * q + e];
            continue;
        }
        // A split tile: publish this segment's partial (system-scope stores
        // go through to memory, where other XCDs' loads find them), then
        // count the arrival. The last of the tile's contributors to arrive
        // sums the partials in range order and writes the tile; nobody waits
        // for anybody. (The stores of one instruction cover two whole 128-byte
        // lines of the [token][row] partial; 16-byte stores of a [row][token]
        // layout, partial lines each, measured slower.)
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t ml = 32 * (tg * NB + t) + 8 * q + 4 * g + e;
                    __hip_atomic_store(part + ml * PR + rl, acc[t][4 * q + e], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
                }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // this thread's partial is in memory
        __syncthreads();
        // contributors: the nonempty ranges from vf (holding the tile's first
        // unit) to vl (its last); grouped launches size the grid for the
        // largest tile count, so some ranges may be empty there
        const uint32_t t0 = tile * a.nblk, t1 = t0 + a.nblk;
        uint32_t vf = v;
        while (vf > 0 && sk_begin(units, a.G, vf) > t0) --vf;
        uint32_t vl = v;
        while (vl + 1 < a.G && sk_begin(units, a.G, vl + 1) < t1) ++vl;
        auto live = [&](uint32_t c) __attribute__((always_inline)) {
            return !GRP || sk_begin(units, a.G, c) != sk_begin(units, a.G, c + 1);
        };
        uint32_t ncontrib = 0, other = v;
        for (uint32_t c = vf; c <= vl; ++c)
            if (live(c)) {
                ++ncontrib;
                if (c != v) other = c;
            }
        uint32_t *const flag = reinterpret_cast<uint32_t *>(lds + L::FLAG);
        if (tid == 0)
            *flag = __builtin_amdgcn_atomic_inc32(a.ctr + tile, ncontrib - 1, __ATOMIC_RELAXED, "");
        __syncthreads();
        const bool last = *flag == ncontrib - 1;  // the counter wrapped back to 0
        if (!last) continue;
        const uint32_t first_slot = sk_begin(units, a.G, vf) < t0 ? 1u : 0u;  // vf's second segment
        // this lane's partial of contributor c, into p
        auto ld = [&](uint32_t c, float (&p)[NB][16]) __attribute__((always_inline)) {
            const float *src = a.ws + (size_t(c) * 2 + (c == vf ? first_slot : 0u)) * (TT * PR);
            uint32_t lo = 4 * g * PR + rl;  // this lane's offset, recomputed per contributor
            asm volatile("" : "+v"(lo));
#pragma unroll
            for (int t = 0; t < NB; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        p[t][4 * q + e] = __hip_atomic_load(src + (32 * (tg * NB + t) + 8 * q + e) * PR + lo,
                                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        };
        if (ncontrib == 2) {
            // own + other in either order: the same bits
            float p[NB][16];
            ld(other, p);
#pragma unroll
            for (int t = 0; t < NB; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[t][r] += p[t][r];
        } else {
            // every contributor's partial from memory in range order (this
            // workgroup's too: it is there already, and acc's registers then
            // hold the sum)
            for (uint32_t c = vf; c <= vl; ++c) {
                if (!live(c)) continue;
                float p[NB][16];
                ld(c, p);
#pragma unroll
                for (int t = 0; t < NB; ++t)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[t][r] = c == vf ? p[t][r] : acc[t][r] + p[t][r];
            }
        }
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t ml = 32 * (tg * NB + t) + 8 * q + 4 * g + e, m = m0 + ml;
                    if (m < tg_.mend && n < a.N) tg_.out[size_t(m) * a.N + n] = acc[t][4 * q + e];
                }
    }
}

// Tiles split over many workgroups (launches with more than kFusedMax
// contributors per tile): out = the partial segments summed in workgroup
// (range) order. A split tile is summed by kFixSlices(TT, PR)
// workgroups, each a slice of kFixNI float4 per thread; group j takes the
// tile holding range boundary j + 1 when that boundary splits it and is the
// first to do so. A thread issues the loads of up to kFixC contributors
// before adding them (in order), so that a CU has many partial lines in flight.
constexpr uint32_t kFixNI = 2;
// contributors whose loads are issued before they are added (Q4_K 5120x17408
// M = 128: 50.0 -> 48.3 us with 16 instead of 4; 8 in between)
constexpr uint32_t kFixC = 16;
__host__ __device__ constexpr uint32_t kFixSlices(uint32_t TT, uint32_t PR) { return TT * PR / 4 / (256 * kFixNI); }
template <uint32_t TT, uint32_t PR, bool GRP>
__global__ __launch_bounds__(256) void k_pf_fixup(PfArgs a) {
    constexpr uint32_t NS = kFixSlices(TT, PR);
    static_assert(NS * 256 * kFixNI * 4 == TT * PR, "a fixup slice is a whole number of 256-thread rounds");
    const uint32_t ntiles = pf_ntiles<GRP>(a);
    const uint32_t units = ntiles * a.nblk, G = a.G;
    const uint32_t slice = blockIdx.x % NS;
    const uint32_t wb = blockIdx.x / NS + 1, ubd = sk_begin(units, G, wb);
    const uint32_t tile = ubd / a.nblk;
    if (ubd % a.nblk == 0 || sk_begin(units, G, wb - 1) > tile * a.nblk) return;
    if (tile >= ntiles) return;
    const uint32_t t0 = tile * a.nblk, t1 = t0 + a.nblk;
    // contributors: the nonempty ranges from vf (the one holding t0) to vl
    // (the one holding t1 - 1); grouped launches size the grid for the
    // largest tile count, so some ranges may be empty there
    uint32_t vf = uint32_t(uint64_t(t0) * G / units);
    while (vf + 1 < G && sk_begin(units, G, vf + 1) <= t0) ++vf;
    while (vf > 0 && sk_begin(units, G, vf) > t0) --vf;
    uint32_t vl = vf;
    while (vl + 1 < G && sk_begin(units, G, vl + 1) < t1) ++vl;
    const uint32_t first_slot = sk_begin(units, G, vf) < t0 ? 1u : 0u;  // vf's second segment
    const PfTile tg_ = pf_tile<GRP>(a, tile, TT, PR);
    const uint32_t n0 = tg_.n0, m0 = tg_.m0;
    const uint32_t e0 = slice * (256 * kFixNI) + threadIdx.x;  // float4 index of item k: e0 + 256 k
    float4 s[kFixNI];
#pragma unroll
    for (uint32_t k = 0; k < kFixNI; ++k) s[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t v = vf; v <= vl; v += kFixC) {
        float4 p[kFixC][kFixNI];
        bool live[kFixC];
#pragma unroll
        for (uint32_t c = 0; c < kFixC; ++c) {
            const uint32_t vc = v + c;
            live[c] = vc <= vl && (!GRP || sk_begin(units, G, vc) != sk_begin(units, G, vc + 1));
            if (live[c]) {
                const float4 *src = reinterpret_cast<const float4 *>(
                    a.ws + (size_t(vc) * 2 + (vc == vf ? first_slot : 0u)) * (TT * PR));
#pragma unroll
                for (uint32_t k = 0; k < kFixNI; ++k) p[c][k] = src[e0 + 256 * k];
            }
        }
#pragma unroll
        for (uint32_t c = 0; c < kFixC; ++c) {
            if (live[c]) {
#pragma unroll
                for (uint32_t k = 0; k < kFixNI; ++k) {
                    s[k].x += p[c][k].x;
                    s[k].y += p[c][k].y;
                    s[k].z += p[c][k].z;
                    s[k].w += p[c][k].w;
                }
            }
        }
    }
#pragma unroll
    for (uint32_t k = 0; k < kFixNI; ++k) {
        const uint32_t i = e0 + 256 * k;
        const uint32_t ml = (4 * i) / PR, nl = (4 * i) % PR;
        const uint32_t m = m0 + ml, n = n0 + nl;
        if (m >= tg_.mend) continue;
        float *o = tg_.out + size_t(m) * a.N + n;
        const float sv[4] = {s[k].x, s[k].y, s[k].z, s[k].w};
        if (n + 3 < a.N && (a.N & 3) == 0) {
            *reinterpret_cast<float4 *>(o) = s[k];
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n + e < a.N) o[e] = sv[e];
        }
    }
}

// Token-tile width from M (the reference picks its tile from seqLen too,
// GemmDispatch.cu:634-643): the smallest of 32, 64, 128 tokens that holds M,
// else 128 (Q8_0: 64 or 128, as its waves split the tile's tokens in two).
int pf_nt(int type, uint32_t M) {
    static_assert(PLds<kIQ3_XXS, 4>::total <= 160 * 1024 && PLds<kIQ3_S, 4>::total <= 160 * 1024 &&
                      PLds<kQ5_K, 4>::total <= 160 * 1024 && PLds<kQ6_K, 2>::total <= 160 * 1024 &&
                      PLds<kQ6_K, 4>::total <= 160 * 1024 &&
                      PLds<kQ4_K, 4>::total <= 160 * 1024 &&
                      PLds<kQ8_0, 4>::total <= 160 * 1024 && PLds<kQ8W, 4>::total <= 160 * 1024 &&
                      PLds<kIQ2_S, 4>::total <= 160 * 1024,
                  "LDS of one workgroup");
    const int nt = M <= 32 ? 1 : M <= 64 ? 2 : 4;
    return type == kQ8_0 ? std::max(nt, 2) : nt;
}
uint32_t pf_rows(int type) { return type == kQ8_0 ? PfType<kQ8_0>::PR : PfType<kQ4_K>::PR; }  // the others: 256

// Split tiles are summed inside the main kernel, by their last contributor,
// when no tile has more than kFusedMax contributors: that workgroup reads the
// others' partial tiles alone (one CU's bandwidth, at the end of the launch),
// which beats a fixup launch for 2-3 partials and loses to it for more
// (measured: Q4_K 17408x5120, M=512 (2 per tile) 120 -> 115 us; M=128 (5
// per tile) 47 -> 56 us).
constexpr uint32_t kFusedMax = 3;
bool pf_fused(uint64_t units, uint32_t G, uint32_t nblk, uint32_t fmax) {
    const uint64_t len = units / G;  // shortest range
    if (len == 0) return false;
    return (nblk - 1 + len - 1) / len + 1 <= fmax;
}

struct PfGeom {
    int nt;
    bool wide;   // Q8_0: the 256-row geometry (kQ8W)
    bool fused;  // split tiles summed inside the kernel (else by the fixup launch)
    uint32_t tt, pr, ntm, ntn, ntiles, G;
};
// The wide Q8_0 geometry from this many tokens on (at 128: 65 against 58 us,
// its 4-token-block tiles split over 5 workgroups each and needing the fixup
// launch; from 512 on faster: M = 2048 586 -> 525 us).
constexpr uint32_t kQ8WideMinM = 256;
PfGeom pf_geom_nt(int type, int nt, uint32_t M, uint32_t N, uint32_t K, int num_cu) {
    PfGeom g;
    g.nt = nt;
    g.wide = type == kQ8_0 && nt == 4 && M > kQ8WideMinM;
    g.tt = 32u * g.nt;
    g.pr = g.wide ? PfType<kQ8W>::PR : pf_rows(type);
    g.ntm = (M + g.tt - 1) / g.tt;
    g.ntn = (N + g.pr - 1) / g.pr;
    g.ntiles = g.ntm * g.ntn;
    const uint64_t units = uint64_t(g.ntiles) * (K / 256);
    // one workgroup per CU, each with at least 2 superblocks of work
    g.G = uint32_t(std::max<uint64_t>(1, std::min<uint64_t>(uint64_t(num_cu), units / 2)));
    g.fused = pf_fused(units, g.G, K / 256, kFusedMax);
    // Where the tiles do not fuse at one workgroup per CU, a grid of c
    // workgroups per tile (c <= kFusedMax, still >= 90% of the CUs) splits
    // every tile exactly c ways, so that the splits are summed in the kernel
    // and the fixup launch goes (5120x17408 at M = 512, 80 tiles on 240
    // workgroups: Q4_K 108.9 -> 106.4 us, Q8_0 158.5 -> 154.1).
    if (!g.fused && g.ntiles <= uint32_t(num_cu)) {
        const uint32_t c = uint32_t(num_cu) / g.ntiles;
        if (c >= 1 && c <= kFusedMax && uint64_t(g.ntiles) * c * 10 >= uint64_t(num_cu) * 9 &&
            units / (uint64_t(g.ntiles) * c) >= 2) {
            g.G = g.ntiles * c;
            g.fused = true;
        }
    }
    return g;
}
// 64-token tiles instead of 128 where that lets the split tiles be summed
// inside the kernel (at most kFusedMax contributors) and 128 would not: the
// weights are converted twice as often, but the fixup launch goes (Q4_K
// 17408x5120, M = 128: 52.2 -> 49.7 us; where neither or both fuse, 128-token
// tiles measured as fast or faster). Only up to kNt2MaxM tokens: the fixup
// launch costs the same at any M while the doubled conversion grows with it.
constexpr uint32_t kNt2MaxM = 256;
// Up to kNt2MaxM tokens, the types whose weight conversion costs most per
// superblock (all but Q4_K and Q8_0) keep their 128-token tiles where the
// tiles' split has at most 6 contributors, summed in the kernel (18944x3584,
// M = 128: Q5_K 50.9 -> 48.2 us, Q6_K 51.1 -> 47.0, IQ3_XXS 49.5 -> 47.5,
// IQ2_S 55.5 -> 47.5; Q4_K at 17408x5120 measured 45.3 -> 55.9 that way). The
// 64-token fallback keeps the limit of 3 (with 6 it took 3584x18944 at M = 256
// from 72 to 90 us).
constexpr uint32_t kFusedMaxKeep = 6;
PfGeom pf_geom(int type, uint32_t M, uint32_t N, uint32_t K, int num_cu) {
    PfGeom g = pf_geom_nt(type, pf_nt(type, M), M, N, K, num_cu);
    if (g.nt != 4 || M > kNt2MaxM || type == kQ8_0 || g.fused) return g;
    if (type != kQ4_K && pf_fused(uint64_t(g.ntiles) * (K / 256), g.G, K / 256, kFusedMaxKeep)) {
        g.fused = true;
        return g;
    }
    const PfGeom h = pf_geom_nt(type, 2, M, N, K, num_cu);
    return h.fused ? h : g;
}

template <int TYPE, int NT, bool GRP = false>
hipError_t pf_launch(const PfArgs &a, hipStream_t st) {
    using L = PLds<TYPE, NT>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_prefill<TYPE, NT, GRP>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, L::total);
    if (attr != hipSuccess) return attr;
    k_prefill<TYPE, NT, GRP><<<dim3{a.G, 1u, 1u}, 64 * PW, L::total, st>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.fused || a.G == 1) return e;
    const uint32_t units = a.ntiles * a.nblk;
    bool split = false;
    for (uint32_t v = 1; v < a.G && !split; ++v) split = sk_begin(units, a.G, v) % a.nblk != 0;
    if (!split) return hipSuccess;
    k_pf_fixup<L::TT, PfType<TYPE>::PR, GRP>
        <<<dim3{(a.G - 1) * kFixSlices(L::TT, PfType<TYPE>::PR), 1u, 1u}, 256, 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace

bool prefill_type(int type) {
    return type == kQ4_K || type == kQ5_K || type == kQ6_K || type == kQ8_0 || type == kIQ3_XXS || type == kIQ3_S ||
           type == kIQ2_S;
}

// Workspace: the per-tile arrival counters (256-byte rounded), then the
// partial tiles, two per workgroup.
namespace {
size_t ctr_bytes(uint64_t ntiles) { return (ntiles * 4 + 255) & ~uint64_t(255); }
}  // namespace
uint32_t prefill_counter_words(int type, uint32_t M, uint32_t N, uint32_t K, int num_cu) {
    return prefill_type(type) ? pf_geom(type, M, N, K, num_cu).ntiles : 0;
}
size_t prefill_workspace_bytes(int type, uint32_t M, uint32_t N, uint32_t K, int num_cu) {
    if (!prefill_type(type)) return 0;
    const PfGeom g = pf_geom(type, M, N, K, num_cu);
    return ctr_bytes(g.ntiles) + size_t(g.G) * 2 * g.tt * g.pr * 4;
}

hipError_t launch_prefill(int type, const void *W, const ActView &act, float *out, uint32_t M, uint32_t N,
                          uint32_t K, int num_cu, void *workspace, hipStream_t st) {
    if (!prefill_type(type) || M == 0 || N == 0 || K == 0 || K % 256 || workspace == nullptr ||
        ((type == kQ4_K || type == kQ5_K || type == kQ8_0) && act.dg == nullptr))
        return hipErrorInvalidValue;
    if (uint64_t(M) * K >= (uint64_t(1) << 32) || uint64_t(N) * (K / 256) * unit_bytes(type) >= (uint64_t(1) << 32))
        return hipErrorInvalidValue;
    const PfGeom g = pf_geom(type, M, N, K, num_cu);
    PfArgs a{};
    a.W = static_cast<const uint8_t *>(W);
    a.qs = act.qs;
    a.d8 = act.d;
    a.xs = act.dg;
    a.out = out;
    a.ctr = static_cast<uint32_t *>(workspace);
    a.ws = reinterpret_cast<float *>(static_cast<char *>(workspace) + ctr_bytes(g.ntiles));
    a.M = M;
    a.N = N;
    a.K = K;
    a.nblk = K / 256;
    a.row_bytes = a.nblk * unit_bytes(type);
    a.ntm = g.ntm;
    a.ntn = g.ntn;
    a.ntiles = g.ntiles;
    a.G = g.G;
    a.fused = g.fused ? 1u : 0u;
    if (type == kQ8_0) {
        if (g.wide) return pf_launch<kQ8W, 4>(a, st);
        return g.nt == 2 ? pf_launch<kQ8_0, 2>(a, st) : pf_launch<kQ8_0, 4>(a, st);
    }
    if (type == kIQ3_XXS) {
        switch (g.nt) {
            case 1: return pf_launch<kIQ3_XXS, 1>(a, st);
            case 2: return pf_launch<kIQ3_XXS, 2>(a, st);
            default: return pf_launch<kIQ3_XXS, 4>(a, st);
        }
    }
    if (type == kQ5_K) {
        switch (g.nt) {
            case 1: return pf_launch<kQ5_K, 1>(a, st);
            case 2: return pf_launch<kQ5_K, 2>(a, st);
            default: return pf_launch<kQ5_K, 4>(a, st);
        }
    }
    if (type == kQ6_K) {
        switch (g.nt) {
            case 1: return pf_launch<kQ6_K, 1>(a, st);
            case 2: return pf_launch<kQ6_K, 2>(a, st);
            default: return pf_launch<kQ6_K, 4>(a, st);
        }
    }
    if (type == kIQ2_S) {
        switch (g.nt) {
            case 1: return pf_launch<kIQ2_S, 1>(a, st);
            case 2: return pf_launch<kIQ2_S, 2>(a, st);
            default: return pf_launch<kIQ2_S, 4>(a, st);
        }
    }
    if (type == kIQ3_S) {
        switch (g.nt) {
            case 1: return pf_launch<kIQ3_S, 1>(a, st);
            case 2: return pf_launch<kIQ3_S, 2>(a, st);
            default: return pf_launch<kIQ3_S, 4>(a, st);
        }
    }
    switch (g.nt) {
        case 1: return pf_launch<kQ4_K, 1>(a, st);
        case 2: return pf_launch<kQ4_K, 2>(a, st);
        default: return pf_launch<kQ4_K, 4>(a, st);
    }
}

// Grouped (MoE) mode: token-tile width from the average rows per expert.
int pf_grouped_nt(uint32_t rows_total, uint32_t n_experts) {
    const uint32_t avg = (rows_total + n_experts - 1) / n_experts;
    // (128-row tiles from 49 rows per expert on: 1024 tokens x top-8 over 128
    // experts, 64 rows each, 255 -> 249 us with them against 64-row tiles)
    return avg <= 32 ? 1 : avg <= 48 ? 2 : 4;
}
uint32_t prefill_grouped_tile(uint32_t rows_total, uint32_t n_experts) {
    return 32u * pf_grouped_nt(rows_total, n_experts);
}
namespace {
uint32_t pf_grouped_grid(uint32_t ntm_max, uint32_t N, uint32_t K, int num_cu, uint32_t mats) {
    const uint64_t units = uint64_t(mats) * ntm_max * ((N + PfType<kQ4_K>::PR - 1) / PfType<kQ4_K>::PR) * (K / 256);
    return uint32_t(std::max<uint64_t>(1, std::min<uint64_t>(uint64_t(num_cu), units / 2)));
}
}  // namespace
uint32_t prefill_grouped_counter_words(uint32_t ntm_max, uint32_t N, uint32_t mats) {
    return mats * ntm_max * ((N + PfType<kQ4_K>::PR - 1) / PfType<kQ4_K>::PR);
}
size_t prefill_grouped_workspace_bytes(uint32_t tile, uint32_t ntm_max, uint32_t N, uint32_t K, int num_cu,
                                       uint32_t mats) {
    return size_t(pf_grouped_grid(ntm_max, N, K, num_cu, mats)) * 2 * tile * PfType<kQ4_K>::PR * 4;
}

hipError_t launch_prefill_grouped(const void *W, uint64_t wstride, const ActView &act, float *out,
                                  uint32_t rows_total, uint32_t N, uint32_t K, const uint32_t *mt, const uint32_t *ntm,
                                  uint32_t ntm_max, uint32_t tile, int num_cu, uint32_t *ctr, void *workspace,
                                  hipStream_t st, const void *W2, float *out2) {
    if (rows_total == 0 || N == 0 || K == 0 || K % 256 || ntm_max == 0 || workspace == nullptr || ctr == nullptr ||
        act.dg == nullptr)
        return hipErrorInvalidValue;
    const uint32_t ntn = (N + PfType<kQ4_K>::PR - 1) / PfType<kQ4_K>::PR;
    if (uint64_t(rows_total) * K >= (uint64_t(1) << 32) || uint64_t(N) * (K / 256) * 144 >= (uint64_t(1) << 32) ||
        uint64_t(ntm_max) * ntn * (K / 256) * 2 >= (uint64_t(1) << 32) || (W2 == nullptr) != (out2 == nullptr))
        return hipErrorInvalidValue;
    PfArgs a{};
    a.W = static_cast<const uint8_t *>(W);
    a.qs = act.qs;
    a.d8 = act.d;
    a.xs = act.dg;
    a.out = out;
    a.ctr = ctr;
    a.fused = 1;  // the tile count is known on the device only
    a.ws = static_cast<float *>(workspace);
    a.M = rows_total;
    a.N = N;
    a.K = K;
    a.nblk = K / 256;
    a.row_bytes = a.nblk * 144;
    a.ntn = ntn;
    a.mt = mt;
    a.ntm_dev = ntm;
    a.wstride = wstride;
    a.W2 = static_cast<const uint8_t *>(W2);
    a.out2 = out2;
    a.G = pf_grouped_grid(ntm_max, N, K, num_cu, W2 != nullptr ? 2u : 1u);
    switch (tile) {
        case 32: return pf_launch<kQ4_K, 1, true>(a, st);
        case 64: return pf_launch<kQ4_K, 2, true>(a, st);
        case 128: return pf_launch<kQ4_K, 4, true>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace tc
