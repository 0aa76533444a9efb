// tc_gemm.hip -- prefill GEMM: out[m][n] = W[n] . x[m] for M tokens against raw
// GGUF weight rows of IQ2_S, on the int8 matrix cores
// (v_mfma_i32_32x32x32_i8). (Q4_K, Q5_K, Q6_K, Q8_0, IQ3_XXS and IQ3_S run the
// register-conversion kernel of tc_prefill.hip.)
//
// Replaces the reference prefill GEMM (int8Gemm, GemmDispatch.cu:595-698) with
// the CPU reference's numerics: the activations are quantized by the same
// bit-exact Q8_K quantizer as the mat-vec path, every integer dot product of
// a weight block with an activation block is exact, and only the final
// per-block scale combination runs in fp32.
//
// Decomposition. One workgroup owns a tile of 64 weight rows x 128 tokens and
// walks K one 256-element superblock at a time; the (tile, superblock) units
// are spread evenly over one workgroup per CU (stream-K, partial tiles summed
// by k_gemm_fixup). The activations arrive block-major (256-column block b of
// token m at b*M + m), so one superblock of a token tile is one contiguous
// 32 KB run. The kernel runs 12 waves: 4 producers (weight loads two
// superblocks ahead, conversion into one half of a double-buffered LDS) and 8
// consumers (the activation plane loaded straight into LDS, MFMAs on the
// other half).
//
// Every weight of a superblock becomes an exact signed integer e
// ((2ls+1)*(+-grid value)) written to two int8 planes,
// e = 128*hi + lo, so that one MFMA chain over the hi plane, a shift by 7 and
// the lo chain on top give sum_s e . x exactly. Per superblock and output:
// acc += d8 * d * main.
//
// MFMA operands: lane l feeds row (l & 31) and the 16 bytes of k-group
// (l >> 5) of both A (weights) and B (activations), so each product pairs the
// same k positions of both; the 32x32 int32 result holds row
// 8*(r/4) + 4*(l>>5) + (r%4) and column (l & 31) in register r.
#include "tc_kernels.hpp"

namespace tc {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int GT = 256;       // producer threads per workgroup
constexpr int GN = 64;        // weight rows per workgroup tile
constexpr int GM = 128;       // tokens per workgroup tile
constexpr int PL = 272;       // LDS weight-plane row stride (256 + 16: conflict-free b128 reads)

// Codebook bytes the converter reads from LDS (past the two stage buffers).
__host__ __device__ constexpr uint32_t grid_bytes(int t) {
    return t == kIQ2_S ? 1024 * 8 : 0;
}

// One stage buffer (bytes).
struct GLds {
    static constexpr uint32_t A0 = 0;                  // hi digit plane [GN][PL]
    static constexpr uint32_t A1 = A0 + GN * PL;       // lo digit plane [GN][PL]
    static constexpr uint32_t AS = A1 + GN * PL;       // row d [GN] (IQ2_S: d/8)
    // activation int8 [GM][256]: 16-byte chunk j of token t at slot
    // j ^ (t & 15) (written by direct-to-LDS loads)
    static constexpr uint32_t BP = 256;
    static constexpr uint32_t B = AS + GN * 4;
    static constexpr uint32_t BD = B + GM * BP;        // Q8_K d [GM]
    static constexpr uint32_t bytes = BD + GM * 4;
};

struct GemmArgs {
    const uint8_t *W;
    const int8_t *qs;       // activations [M][K]
    const float *d8;        // [M][K/256] (Q8_K)
    float *out;             // [M][N]
    uint32_t M, N, K;
    uint32_t row_bytes;     // bytes per weight row
    uint32_t ntm;           // token tiles
    uint32_t nblk;          // superblocks per row
    uint32_t ntiles;        // output tiles
    uint32_t skg;           // stream-K workgroups
    float *ws;              // stream-K partial tiles [grid][2][GM][GN]
};

__device__ __forceinline__ u4 lds4(const unsigned char *p) { return *reinterpret_cast<const u4 *>(p); }
__device__ __forceinline__ v4i as_v4i(u4 v) { return __builtin_bit_cast(v4i, v); }

template <int TYPE>
struct GPrefetch {
    // the bytes of the two 32-chunks 2qq, 2qq+1 (4-byte-aligned words,
    // realigned on conversion)
    uint32_t ex[9];
    uint32_t sh;           // the block's byte offset mod 4
    float d8;              // Q8_K d (128 tokens)
};

// Buffer descriptors over the operands and this thread's fixed per-lane
// offsets; superblock b only moves the scalar offsets. Rows past N and tokens
// past M fall outside the descriptors and load zeros (never stored).
struct GSrc {
    __amdgpu_buffer_rsrc_t w, d;
    uint32_t vw, vd;   // per-lane offsets
    uint32_t qq;       // the thread's quarter
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t grsrc(const void *p, uint64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), short(0), int(uint32_t(bytes)), 0x00020000);
}

template <int TYPE>
__device__ __forceinline__ GSrc gemm_src(const GemmArgs &a, uint32_t n0, uint32_t m0, uint32_t tid) {
    GSrc g;
    // whole dwords: the range check zeroes a dword that is only partly in
    // range, and 2-byte-aligned units end 2 bytes into
    // one when their count is odd (it stays in the page of the last byte)
    g.w = grsrc(a.W, (uint64_t(a.N) * a.row_bytes + 3) & ~uint64_t(3));
    g.d = grsrc(a.d8, uint64_t(a.M) * (a.K / 256) * 4);
    g.vw = (n0 + tid / 4) * a.row_bytes;
    g.qq = tid & 3;
    g.vd = (m0 + (tid & 127)) * 4;
    return g;
}

template <int TYPE>
__device__ __forceinline__ void gemm_prefetch(const GemmArgs &a, const GSrc &g, uint32_t b, GPrefetch<TYPE> &p) {
    constexpr uint32_t UB = unit_bytes(TYPE);
    static_assert(TYPE == kIQ2_S, "IQ2_S only");
    {
        // 2-byte-aligned blocks; each piece from its 4-byte-aligned address
        // down, the block start's offset mod 4 in sh
        const uint32_t blk = g.vw + b * UB;
        p.sh = blk & 3;
        const uint32_t al = blk & ~3u;
        auto w32 = [&](uint32_t off) __attribute__((always_inline)) {
            return __builtin_amdgcn_raw_buffer_load_b32(g.w, (blk + off) & ~3u, 0, 0);
        };
        const uint32_t qq = g.qq;
        p.ex[0] = w32(2 + 8 * qq);        // qs (grid low bytes)
        p.ex[1] = w32(2 + 8 * qq + 4);
        p.ex[2] = w32(2 + 8 * qq + 8);
        p.ex[3] = w32(34 + 8 * qq);       // signs
        p.ex[4] = w32(34 + 8 * qq + 4);
        p.ex[5] = w32(34 + 8 * qq + 8);
        p.ex[7] = w32(66 + 2 * qq);       // qh bytes 2qq, 2qq+1
        p.ex[8] = w32(74 + 2 * qq);       // scale bytes 2qq, 2qq+1
        p.ex[6] = __builtin_amdgcn_raw_buffer_load_b32(g.w, al, 0, 0);  // d
    }
    p.d8 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(g.d, g.vd, b * a.M * 4, 0));
}

typedef short s16x2 __attribute__((ext_vector_type(2)));

// Signed byte digits of e = k * v for four values packed in a word (16-bit
// lanes: v at bytes 0 and 2 of `even`, bytes 1 and 3 of the original at bytes 0
// and 2 of `odd`), |e| <= 4096: hi = e >> 7 (arithmetic) and lo = e & 127 as
// bytes in the original order, so that e = 128*hi + lo exactly.
__device__ __forceinline__ void digits_s16(s16x2 ve, s16x2 vo, short k, uint32_t &hi, uint32_t &lo) {
    const s16x2 kk = {k, k};
    const s16x2 ee = ve * kk, eo = vo * kk;
    const s16x2 he = ee >> s16x2{7, 7}, ho = eo >> s16x2{7, 7};
    const uint32_t le = __builtin_bit_cast(uint32_t, ee) & 0x007F007Fu, lo_ = __builtin_bit_cast(uint32_t, eo) & 0x007F007Fu;
    lo = __builtin_amdgcn_perm(lo_, le, 0x06020400u);
    hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, ho), __builtin_bit_cast(uint32_t, he), 0x06020400u);
}

// Four signed bytes per word (signed grid values) -> digits of k * v.
__device__ __forceinline__ void digits_i8(uint32_t v, int k, uint32_t &hi, uint32_t &lo) {
    // sign extension per 16-bit lane: (b ^ 0x80) - 0x80
    const s16x2 ve = __builtin_bit_cast(s16x2, (v & 0x00FF00FFu) ^ 0x00800080u) - s16x2{128, 128};
    const s16x2 vo = __builtin_bit_cast(s16x2, ((v >> 8) & 0x00FF00FFu) ^ 0x00800080u) - s16x2{128, 128};
    digits_s16(ve, vo, short(k), hi, lo);
}

__device__ __forceinline__ uint32_t realign(uint32_t hi, uint32_t lo, uint32_t sh) {
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
}

// IQ2_S weights of this thread (row tid/4, 32-chunks ib = 2qq + c) -> the
// digit planes and d/8 (the row scale 0.125 of the reference's fused path,
// include/GGMLDequantize.hpp:2148-2159, is a power of two: exact on d). Group
// l (8 weights) of chunk ib: the 8 magnitudes of codebook entry qs[4ib + l]
// with bits 8-9 from bits 2l, 2l+1 of qh[ib], negated by the bits of
// signs[4ib + l], times 2ls+1 with ls nibble l/2 of scales[ib]
// (GGMLDequantize.hpp:1215-1242, :2028-2057).
__device__ __forceinline__ void iq2s_convert(const GPrefetch<kIQ2_S> &p, unsigned char *lds, const uint32_t *grid,
                                             uint32_t tid) {
    using L = GLds;
    const uint32_t r = tid / 4, qq = tid & 3;
    const uint32_t s8b = (p.sh + 2) & 3;  // qs at 2 + 8qq and signs at 34 + 8qq: the same offset mod 4
    const uint32_t qs[2] = {realign(p.ex[1], p.ex[0], s8b), realign(p.ex[2], p.ex[1], s8b)};
    const uint32_t sg[2] = {realign(p.ex[4], p.ex[3], s8b), realign(p.ex[5], p.ex[4], s8b)};
    const uint32_t qh2 = p.ex[7] >> (8 * ((p.sh + 66 + 2 * qq) & 3));
    const uint32_t sc2 = p.ex[8] >> (8 * ((p.sh + 74 + 2 * qq) & 3));
    const uint32_t dh = p.sh ? (p.ex[6] >> 16) : (p.ex[6] & 0xFFFFu);
    unsigned char *a0 = lds + L::A0 + r * PL, *a1 = lds + L::A1 + r * PL;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const uint32_t qh = (qh2 >> (8 * c)) & 0xFFu, scb = (sc2 >> (8 * c)) & 0xFFu;
        uint32_t hi[8], lo[8];
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const int k = 2 * int((scb >> (4 * (l >> 1))) & 15u) + 1;
            const uint32_t idx = ((qs[c] >> (8 * l)) & 0xFFu) | (((qh >> (2 * l)) & 3u) << 8);
            const uint32_t s8 = (sg[c] >> (8 * l)) & 0xFFu;
            const uint32_t m1 = spread_sign4(s8 & 15u), m2 = spread_sign4(s8 >> 4);
            digits_i8((grid[2 * idx] ^ m1) + (m1 & 0x01010101u), k, hi[2 * l], lo[2 * l]);
            digits_i8((grid[2 * idx + 1] ^ m2) + (m2 & 0x01010101u), k, hi[2 * l + 1], lo[2 * l + 1]);
        }
        const uint32_t k0 = 64 * qq + 32 * c;
        *reinterpret_cast<u4 *>(a0 + k0) = u4{hi[0], hi[1], hi[2], hi[3]};
        *reinterpret_cast<u4 *>(a0 + k0 + 16) = u4{hi[4], hi[5], hi[6], hi[7]};
        *reinterpret_cast<u4 *>(a1 + k0) = u4{lo[0], lo[1], lo[2], lo[3]};
        *reinterpret_cast<u4 *>(a1 + k0 + 16) = u4{lo[4], lo[5], lo[6], lo[7]};
    }
    reinterpret_cast<float *>(lds + L::AS)[r] = 0.125f * h2f(dh);
}

__constant__ uint64_t c_iq2s_grid[1024] = {
#include "iq2s_grid.inc"
};

// Staged registers -> LDS: the weights converted to the digit planes
// straight from registers, and the activation scales.
template <int TYPE>
__device__ __forceinline__ void gemm_stage(const GPrefetch<TYPE> &p, unsigned char *lds, uint32_t tid,
                                           const uint32_t *grid = nullptr) {
    using L = GLds;
    iq2s_convert(p, lds, grid, tid);
    reinterpret_cast<float *>(lds + L::BD)[tid & (GM - 1)] = p.d8;  // threads tid and tid+128 hold the same d
}

__device__ __forceinline__ v16i mfma(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// The activation plane of superblock b of this tile straight into LDS
// (buffer loads with the LDS destination: no registers, no LDS stores). Each
// wave instruction fills 1 KB = 4 token rows; lane l writes slot l%16 of
// token 4k + l/16 and so reads chunk (l%16) ^ (t%16) of its 256 bytes. Tokens past M read the next
// superblock's bytes (their outputs are never stored); past the buffer, zeros.
template <int TYPE, int CW>
__device__ __forceinline__ void dig_act_to_lds(const GemmArgs &a, uint32_t m0, uint32_t b, unsigned char *ldsb,
                                               uint32_t w, uint32_t lane) {
    using L = GLds;
    typedef int v4i32 __attribute__((ext_vector_type(4)));
    const uint64_t base = reinterpret_cast<uint64_t>(a.qs);
    const v4i32 rs = {int(uint32_t(base)), int(uint32_t(base >> 32) & 0xFFFF), int(a.M * a.K), 0x00020000};
    // wave w, instruction i fills 1 KB block k = CW*i + w: tokens 4k..4k+3
    const uint32_t t0 = (4 * w + lane / 16) & 15;  // = t % 16 (CW*4*i is a multiple of 16)
    const uint32_t voff = (m0 + 4 * w + lane / 16) * 256 + 16 * ((lane & 15) ^ t0);
    const uint32_t dst =
        uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)(ldsb + L::B))) + 1024 * w;
    // Inline so that the compiler, which cannot tell which LDS bytes these
    // loads write, does not wait for them before this wave's next LDS reads
    // (of the other buffer); the caller waits (vmcnt) before the barrier.
#pragma unroll
    for (uint32_t i = 0; i < 32 / CW; ++i)
    {
        // m0 (the LDS destination) is restored afterwards: the compiler
        // treats it as reserved and may hold its own value there.
        uint32_t saved;
        asm volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(dst + 1024 * CW * i), "v"(voff), "s"(rs), "s"(b * a.M * 256 + i * 1024 * CW)
            : "memory");
    }
}

// One superblock of a consumer wave's 32-row x (32 NTT)-token Q4_K tile from
// the LDS planes at `lds` (MFMA chains and the fp32 combination into acc).
// tok0: the wave's first token row in the tile.
template <int TYPE, int NTT>
__device__ __forceinline__ void dig_consume(const unsigned char *lds, uint32_t wn, uint32_t tok0, uint32_t li,
                                            uint32_t lg, float (&acc)[NTT][16]) {
    using L = GLds;
    const unsigned char *arow = lds + (32 * wn + li) * PL + 16 * lg;
    // token rows tok0 + 32t + li (all with t % 16 = li % 16)
    auto brow = [&](int t) __attribute__((always_inline)) { return lds + L::B + (tok0 + 32 * t + li) * L::BP; };
    auto bslot = [&](int s) __attribute__((always_inline)) { return 16u * ((2u * s + lg) ^ (li & 15)); };
    // Token tile 0's fragments are read up front (one LDS latency, not one
    // per sub-block); tile 1's are read while tile 0's MFMA chains run, and
    // tile 0's fp32 combination runs while tile 1's chains do.
    v4i ah[8], al[8], x[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        ah[s] = as_v4i(lds4(arow + L::A0 + 32 * s));
        x[s] = as_v4i(lds4(brow(0) + bslot(s)));
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) al[s] = as_v4i(lds4(arow + L::A1 + 32 * s));
    __builtin_amdgcn_sched_barrier(0);
    // One accumulator per token tile: the hi-digit chain, then C = hi << 7
    // and the lo-digit chain on top (= 128*hi + lo exactly).
    auto chain = [&](v16i &c) __attribute__((always_inline)) {
        c = v16i{};
#pragma unroll
        for (int s = 0; s < 8; ++s) c = mfma(ah[s], x[s], c);
#pragma unroll
        for (int r = 0; r < 16; ++r) c[r] <<= 7;
#pragma unroll
        for (int s = 0; s < 8; ++s) c = mfma(al[s], x[s], c);
    };
    auto combine = [&](int t, const v16i &c) __attribute__((always_inline)) {
        const float d8 = reinterpret_cast<const float *>(lds + L::BD)[tok0 + 32 * t + li];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t rr = 32 * wn + 8 * q + 4 * lg;
            const float4 dv = *reinterpret_cast<const float4 *>(lds + L::AS + 4 * rr);
            const float dd[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * q + e;
                acc[t][r] = fmaf(d8, dd[e] * float(c[r]), acc[t][r]);
            }
        }
    };
    v16i c0;
    chain(c0);
    if constexpr (NTT == 2) {
#pragma unroll
        for (int s = 0; s < 8; ++s) x[s] = as_v4i(lds4(brow(1) + bslot(s)));
        v16i c1;
        chain(c1);
        combine(0, c0);
        combine(1, c1);
    } else {
        combine(0, c0);
    }
}

// Producer and consumer waves: 4 producer waves load superblock
// b+2 and convert b+1 into one half of a double-buffered LDS while 4 consumer
// waves run the MFMAs and the fp32 combination of superblock b from the other
// half -- the conversion's VALU work overlaps the matrix work on the same
// SIMDs, with one barrier per superblock.
// Stream-K: the (tile, superblock) units, tile-major, are split evenly over
// the workgroups (one per CU). A workgroup walks its range one tile segment
// at a time; a segment that covers a whole tile is stored to `out`, a partial
// one to the workgroup's slot in `ws` (slot 0: its first segment, 1: its
// last), and k_gemm_fixup sums the partial segments of each tile in
// workgroup order.
// Tile t -> (token tile, row block), token tiles fastest: a stream-K
// workgroup's consecutive tiles reuse one block of weight rows. (Row blocks
// fastest measured 3-13% slower.)
struct TileGeom {
    uint32_t m0, n0;
};
__device__ __forceinline__ TileGeom sk_tile(const GemmArgs &a, uint32_t t) {
    return TileGeom{(t % a.ntm) * GM, (t / a.ntm) * GN};
}

__host__ __device__ inline uint32_t sk_begin(uint32_t units, uint32_t grid, uint32_t w) {
    return uint32_t(uint64_t(units) * w / grid);
}

template <int TYPE, int CW>
__global__ __launch_bounds__(GT + 64 * CW) __attribute__((amdgpu_waves_per_eu(1 + CW / 4, 1 + CW / 4))) void k_gemm_dig(
    GemmArgs a) {
    extern __shared__ __align__(16) unsigned char lds[];
    using L = GLds;
    constexpr int NTT = 8 / CW;  // 32-token tiles per consumer wave
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool producer = wave >= CW;
    // consumer: 32-row group wn, token rows 32*NTT*wm ..
    const uint32_t wn = wave & 1, wm = (wave >> 1) & (CW / 2 - 1), tok0 = 32 * NTT * wm;
    const uint32_t li = lane & 31, lg = lane >> 5;
    const uint32_t ptid = tid - 64 * CW;  // producer thread index 0..255
    auto buf = [&](uint32_t b) __attribute__((always_inline)) { return lds + (b & 1) * L::bytes; };
    // IQ2_S codebook in LDS, past the two buffers (read by the producers' conversion)
    uint32_t *grid = reinterpret_cast<uint32_t *>(lds + 2 * L::bytes);
    if constexpr (grid_bytes(TYPE) != 0) {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(c_iq2s_grid);
        for (uint32_t i = tid; i < grid_bytes(TYPE) / 4; i += blockDim.x) grid[i] = src[i];
        __syncthreads();
    }

    const uint32_t units = a.ntiles * a.nblk;
    const uint32_t ub = sk_begin(units, gridDim.x, blockIdx.x), ue = sk_begin(units, gridDim.x, blockIdx.x + 1);
    for (uint32_t u = ub; u < ue;) {
        const uint32_t tile = u / a.nblk;
        const uint32_t b0 = u - tile * a.nblk;
        const uint32_t b1 = min(a.nblk, b0 + (ue - u));
        const bool whole = b0 == 0 && b1 == a.nblk;
        float *const part = whole ? nullptr : a.ws + (size_t(blockIdx.x) * 2 + (u == ub ? 0 : 1)) * (GM * GN);
        u += b1 - b0;
        const TileGeom tg = sk_tile(a, tile);
        const uint32_t m0 = tg.m0, n0 = tg.n0;
        // Producers step in pairs of superblocks; both sides run bend - b0 barriers.
        const uint32_t bend = b0 + ((b1 - b0 + 1) & ~1u);

        // Producer and consumer waves run separate loops with the same number
        // of barriers, so neither keeps the other's registers live.
        if (producer) {
            // Two superblocks of loads in flight per producer thread: global
            // latency under load exceeds one superblock's compute time.
            const GSrc gs = gemm_src<TYPE>(a, n0, m0, ptid);
            GPrefetch<TYPE> pa, pb;
            gemm_prefetch<TYPE>(a, gs, b0, pa);
            gemm_stage<TYPE>(pa, buf(b0), ptid, grid);
            gemm_prefetch<TYPE>(a, gs, min(b0 + 1, b1 - 1), pa);
            gemm_prefetch<TYPE>(a, gs, min(b0 + 2, b1 - 1), pb);
            __syncthreads();
            // Straight-line steps (past the end they stage into the idle buffer
            // and reload the last superblock), so the compiler's wait counts
            // stay exact.
            auto step = [&](GPrefetch<TYPE> &pf, uint32_t b) __attribute__((always_inline)) {
                gemm_stage<TYPE>(pf, buf(b + 1), ptid, grid);
                gemm_prefetch<TYPE>(a, gs, min(b + 3, b1 - 1), pf);
                __syncthreads();
            };
            for (uint32_t b = b0; b < bend; b += 2) {
                step(pa, b);
                step(pb, b + 1);
            }
            continue;
        }
        float acc[NTT][16];
#pragma unroll
        for (int t = 0; t < NTT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;
        // Consumers fill the activation planes: superblock b+1 goes into the
        // other buffer while b is multiplied (their only memory loads, so the
        // wait before each barrier waits for nothing else).
        dig_act_to_lds<TYPE, CW>(a, m0, b0, buf(b0), wave, lane);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        for (uint32_t b = b0; b < bend; ++b) {
            dig_act_to_lds<TYPE, CW>(a, m0, min(b + 1, b1 - 1), buf(b + 1), wave, lane);
            if (b < b1) dig_consume<TYPE, NTT>(buf(b), wn, tok0, li, lg, acc);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this superblock's plane is in LDS
            __syncthreads();
        }

#pragma unroll
        for (int t = 0; t < NTT; ++t) {
            const uint32_t ml = tok0 + 32 * t + li, m = m0 + ml;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t nl = 32 * wn + 8 * q + 4 * lg, n = n0 + nl;
                const float4 v = make_float4(acc[t][4 * q], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]);
                if (part != nullptr) {
                    *reinterpret_cast<float4 *>(part + ml * GN + nl) = v;  // [token][row] of the tile
                } else if (m < a.M) {
                    float *o = a.out + size_t(m) * a.N + n;
                    if (n + 3 < a.N && (a.N & 3) == 0) {
                        *reinterpret_cast<float4 *>(o) = v;
                    } else {
                        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < a.N) o[e] = vv[e];
                    }
                }
            }
        }
    }
}

// Tiles split over several stream-K workgroups: out = the partial segments
// summed in workgroup order. kFixSlices workgroups per tile (each a quarter
// of its entries), workgroup group j taking the tile that holds range
// boundary j+1, when the boundary splits it and is the first to do so.
constexpr uint32_t kFixSlices = 4;
__global__ __launch_bounds__(256) void k_gemm_fixup(GemmArgs a) {
    const uint32_t units = a.ntiles * a.nblk, G = a.skg;
    const uint32_t slice = blockIdx.x % kFixSlices;
    const uint32_t wb = blockIdx.x / kFixSlices + 1, ub = sk_begin(units, G, wb);
    const uint32_t tile = ub / a.nblk;
    if (ub % a.nblk == 0 || sk_begin(units, G, wb - 1) > tile * a.nblk) return;
    const uint32_t t0 = tile * a.nblk, t1 = t0 + a.nblk;
    // first workgroup whose range holds unit t0
    uint32_t w = uint32_t(uint64_t(t0) * G / units);
    while (w + 1 < G && sk_begin(units, G, w + 1) <= t0) ++w;
    while (w > 0 && sk_begin(units, G, w) > t0) --w;
    const TileGeom tg = sk_tile(a, tile);
    const uint32_t m0 = tg.m0, n0 = tg.n0;
    constexpr uint32_t per = GM * GN / 4 / kFixSlices;  // float4 entries per slice
    constexpr uint32_t NI = per / 256;                   // per thread
    static_assert(per % 256 == 0, "a fixup slice is a whole number of 256-thread rounds");
    float4 s[NI];
#pragma unroll
    for (uint32_t k = 0; k < NI; ++k) s[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    // The contributing workgroups in order (range boundaries computed once
    // per workgroup, not per entry); slot 1 for the one whose range starts
    // before the tile.
    uint32_t bv = sk_begin(units, G, w);
    for (uint32_t v = w; v < G && bv < t1; ++v) {
        const uint32_t bn = sk_begin(units, G, v + 1);
        if (bn > t0 && bn != bv) {
            const float *src = a.ws + (size_t(v) * 2 + (bv >= t0 ? 0u : 1u)) * (GM * GN);
#pragma unroll
            for (uint32_t k = 0; k < NI; ++k) {
                const float4 p = reinterpret_cast<const float4 *>(src)[slice * per + k * 256 + threadIdx.x];
                s[k].x += p.x;
                s[k].y += p.y;
                s[k].z += p.z;
                s[k].w += p.w;
            }
        }
        bv = bn;
    }
#pragma unroll
    for (uint32_t k = 0; k < NI; ++k) {
        const uint32_t i = slice * per + k * 256 + threadIdx.x;
        const uint32_t ml = (4 * i) / GN, nl = (4 * i) % GN;
        const uint32_t m = m0 + ml, n = n0 + nl;
        if (m >= a.M) continue;
        float *o = a.out + size_t(m) * a.N + n;
        if (n + 3 < a.N && (a.N & 3) == 0) {
            *reinterpret_cast<float4 *>(o) = s[k];
        } else {
            const float sv[4] = {s[k].x, s[k].y, s[k].z, s[k].w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n + e < a.N) o[e] = sv[e];
        }
    }
}

template <int TYPE>
hipError_t launch_gemm_t(const GemmArgs &a, dim3 grid, hipStream_t st) {
    constexpr int CW = 8;  // consumer waves (4, one per SIMD with two token blocks each, measured within 3%)
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemm_dig<TYPE, CW>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    const uint32_t lds = 2 * GLds::bytes + grid_bytes(TYPE);
    k_gemm_dig<TYPE, CW><<<grid, GT + 64 * CW, lds, st>>>(a);
    return hipGetLastError();
}

}  // namespace

// Stream-K grid: one workgroup per CU, each with at least 4 units.
uint32_t sk_grid(uint32_t M, uint32_t N, uint32_t K, int num_cu) {
    const uint32_t units = ((M + GM - 1) / GM) * ((N + GN - 1) / GN) * (K / 256);
    return std::max(1u, std::min(uint32_t(num_cu), units / 4));
}

size_t gemm_workspace_bytes(int, uint32_t M, uint32_t N, uint32_t K, int num_cu) {
    return size_t(sk_grid(M, N, K, num_cu)) * 2 * GM * GN * 4;
}

hipError_t launch_gemm(int type, const void *W, const ActView &act, float *out, uint32_t M, uint32_t N, uint32_t K,
                       int num_cu, void *workspace, hipStream_t st) {
    if (M == 0 || N == 0 || K == 0 || K % 256) return hipErrorInvalidValue;
    // IQ2_S here; the other MFMA types run k_prefill (tc_prefill.hip).
    if (type != kIQ2_S) return hipErrorInvalidValue;
    // 32-bit buffer offsets: the quantized activations (M*K bytes) and one
    // weight matrix must each stay below 4 GiB.
    if (uint64_t(M) * K >= (uint64_t(1) << 32) || uint64_t(N) * (K / 256) * unit_bytes(type) >= (uint64_t(1) << 32))
        return hipErrorInvalidValue;
    if (workspace == nullptr) return hipErrorInvalidValue;
    GemmArgs a{};
    a.W = static_cast<const uint8_t *>(W);
    a.qs = act.qs;
    a.d8 = act.d;
    a.M = M;
    a.N = N;
    a.K = K;
    a.nblk = K / 256;
    a.row_bytes = a.nblk * unit_bytes(type);
    a.ntm = (M + GM - 1) / GM;
    a.ntiles = a.ntm * ((N + GN - 1) / GN);
    const uint32_t G = sk_grid(M, N, K, num_cu);
    a.out = out;
    a.ws = static_cast<float *>(workspace);
    a.skg = G;
    const dim3 g{G, 1u, 1u};
    hipError_t e = launch_gemm_t<kIQ2_S>(a, g, st);
    if (e != hipSuccess) return e;
    // Any tile split over workgroups? (a range boundary inside a tile)
    bool split = false;
    for (uint32_t w = 1; w < G && !split; ++w) split = sk_begin(a.ntiles * a.nblk, G, w) % a.nblk != 0;
    if (!split) return hipSuccess;
    k_gemm_fixup<<<dim3{(G - 1) * kFixSlices, 1u, 1u}, 256, 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace tc
