// tc_prefill.hip -- prefill GEMM out[m][n] = W[n] . x[m] for Q4_K weights on
// the int8 matrix cores (v_mfma_i32_32x32x32_i8), each weight converted once
// per token tile of up to 256 tokens, in the registers of the lane that feeds
// it to the MFMA.
//
// Replaces the reference prefill GEMM (int8Gemm, GemmDispatch.cu:595-698 and
// its stream-K kernel GemmKernels.cuh:3707-4030) with the CPU reference's
// numerics: the activations are quantized by the bit-exact Q8_K quantizer,
// every integer dot product of a weight sub-block with an activation
// sub-block is exact, and only the per-superblock scale combination runs in
// fp32.
//
// Decomposition. A workgroup has 4 waves; wave w owns 32 weight rows
// (n0 + 32w + lane % 32) and all TT = 32 NT tokens of the tile, so no weight
// is converted twice for one tile. The activations of the tile (TT tokens x
// one 256-wide superblock: int8 values, scale and the digit sums below) are
// loaded straight into LDS, double-buffered, and read by all 4 waves as the
// MFMA A operand; the weights never pass through LDS: each lane loads the
// 80 bytes of its row and k-half it needs (header + 64 quant bytes), two
// superblocks ahead, and converts them into its B-operand registers.
//
// Q4_K (reference dequantizeQ4_KBlock, GGMLDequantize.hpp:436-477): a weight
// of sub-block s is w = d*sc_s*q - dmin*m_s with q in 0..15 and sc_s, m_s in
// 0..63. With sc_s = 8*h_s + l_s (h_s, l_s in 0..7) the products h_s*q and
// l_s*q fit int8, so the hi chain (8 MFMAs) and the lo chain (8 more, on the
// hi result shifted left by 3) give C = sum_s sc_s * (q . x)_s exactly. The
// min term sum_s m_s * S_s (S_s the sum of the 32 activations of sub-block s,
// from the quantizer as int8 digits S_s = 128*hi + lo) is one MFMA pair over 8
// k slots. Per superblock and output, in fp32: acc += d8 * (d*C - dmin*Mn).
//
// MFMA operands: lane l feeds row (l & 31) and the 16 bytes of k-group
// (l >> 5) of A and of B (any fixed pairing of k positions works, as both
// operands use it). A = activations (row = token), B = weights (column =
// weight row), so a lane's 16 results share one weight row (its scales are
// lane constants) and cover tokens 8*(r/4) + 4*(l >> 5) + (r % 4).
//
// Work split: the (tile, superblock) units, tiles ordered row block fastest,
// are divided evenly over the workgroups (stream-K); workgroup ranges are
// numbered so that the workgroups of one XCD (dispatched round robin over the
// 8 XCDs) hold one contiguous range, so they share one token tile's
// activations in their L2. A tile split over several workgroups is summed by
// k_pf_fixup in workgroup order (deterministic).
#include <type_traits>

#include "tc_kernels.hpp"

namespace tc {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));

constexpr uint32_t PW = 8;          // waves per workgroup (two per SIMD)
constexpr uint32_t PR = 32 * PW;    // weight rows per workgroup tile

template <int NT>
struct PLds {
    static constexpr uint32_t TT = 32 * NT;                 // tokens per tile
    static constexpr uint32_t QS = 0;                       // [TT][256], 16-byte chunk c of token t at slot c ^ (t & 15)
    static constexpr uint32_t DG = TT * 256;                // [TT][16] digit sums
    static constexpr uint32_t D8 = DG + TT * 16;            // [max(TT, 64)] Q8_K d
    static constexpr uint32_t W = D8 + (TT < 64 ? 64 : TT) * 4;  // [PR][144] the tile's weight blocks
    static constexpr uint32_t bytes = W + 256 * 144;        // one buffer
};

struct PfArgs {
    const uint8_t *W;
    const int8_t *qs;   // block-major [nblk][M][256]
    const float *d8;    // [nblk][M]
    const int8_t *dg;   // [nblk][M][16]
    float *out;         // [M][N]
    float *ws;          // partial tiles [G][2][TT][PR]
    uint32_t M, N, K;
    uint32_t row_bytes, nblk;
    uint32_t ntm, ntn, ntiles;  // token tiles, row blocks, tiles
    uint32_t G;                 // workgroups
#ifdef TC_PF_TRACE
    unsigned long long *trace;
#endif
};

__device__ __forceinline__ v16i mfma(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ u4 lds4(const unsigned char *p) { return *reinterpret_cast<const u4 *>(p); }
__device__ __forceinline__ v4i as_v4i(u4 v) { return __builtin_bit_cast(v4i, v); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, uint64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), short(0), int(uint32_t(bytes)), 0x00020000);
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

// Raw bytes of one superblock of this lane's weight row: the 16-byte header
// and, for k-half g, bytes 16g..16g+15 of each 32-byte quant group.
struct Q4Raw {
    u4 h, q[4];
};

// From the tile's weight blocks in LDS (row stride 144 bytes: the 16-byte
// reads of 16 consecutive rows fall on distinct banks).
__device__ __forceinline__ void q4_read(Q4Raw &r, const unsigned char *blk, uint32_t g) {
    r.h = lds4(blk);
#pragma unroll
    for (int p = 0; p < 4; ++p) r.q[p] = lds4(blk + 16 + 32 * p + 16 * g);
}

// B operands of one superblock: digit planes of sc*q per sub-block, the mins
// and the row scales.
struct Q4Frag {
    v4i bh[8], bl[8];
    v4i m;  // bytes 0-7: the 8 mins (k-half 0; zero in k-half 1)
    float d, dm;
};

__device__ __forceinline__ void q4_convert(const Q4Raw &r, uint32_t g, Q4Frag &f) {
    const u4 h = r.h;
    // 6-bit scales and mins of the 8 sub-blocks as bytes (reference
    // get_scale_min_k4, GGMLDequantize.hpp:436-447)
    const uint32_t scl = h.y & 0x3F3F3F3Fu, mnl = h.z & 0x3F3F3F3Fu;
    const uint32_t sch = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t mnh = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    const uint32_t hw[2] = {(scl >> 3) & 0x07070707u, (sch >> 3) & 0x07070707u};
    const uint32_t lw[2] = {scl & 0x07070707u, sch & 0x07070707u};
    f.d = h2f(h.x & 0xFFFFu);
    f.dm = h2f(h.x >> 16);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int s0 = 2 * p, s1 = 2 * p + 1;  // low nibbles: sub-block 2p, high: 2p+1
        const uint32_t mh0 = bcast16(hw[s0 >> 2], s0 & 3), ml0 = bcast16(lw[s0 >> 2], s0 & 3);
        const uint32_t mh1 = bcast16(hw[s1 >> 2], s1 & 3), ml1 = bcast16(lw[s1 >> 2], s1 & 3);
        const uint32_t q[4] = {r.q[p].x, r.q[p].y, r.q[p].z, r.q[p].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = (q[k] >> 4) & 0x0F0F0F0Fu;
            f.bh[s0][k] = pkmul(lo, mh0);
            f.bl[s0][k] = pkmul(lo, ml0);
            f.bh[s1][k] = pkmul(hi, mh1);
            f.bl[s1][k] = pkmul(hi, ml1);
        }
    }
    const int z = 0;
    const int a = g == 0 ? int(mnl) : z, b = g == 0 ? int(mnh) : z;
    f.m = v4i{a, b, 0, 0};
}

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

// Superblock b of token tile m0 into one LDS buffer: values (1 KB per wave
// instruction = 4 tokens, XOR-swizzled chunks), digit sums and scales. Tokens
// past M read other tokens' bytes or zeros (their outputs are never stored).
template <int NT>
__device__ __forceinline__ void act_to_lds(const PfArgs &a, uint32_t m0, uint32_t b, unsigned char *buf, uint32_t w,
                                           uint32_t lane) {
    using L = PLds<NT>;
    constexpr uint32_t TT = L::TT;
    const v4i rq = rs4(a.qs, a.M * a.K), rg = rs4(a.dg, a.M * a.nblk * 16), rd = rs4(a.d8, a.M * a.nblk * 4);
    const uint32_t base = lds_addr(buf);
    const uint32_t tb = b * a.M + m0;  // first token record of the tile in this superblock
    uint32_t ln = lane;
    asm volatile("" : "+v"(ln));  // per-call lane arithmetic (not hoisted into held registers)
    // values: instruction k (of TT/4 1-KB rows) fills tokens 4k..4k+3
    constexpr uint32_t NQ = TT / 4, NG = TT / 16, ND = (TT + 63) / 64;
#pragma unroll
    for (uint32_t i = 0; i < (NQ + PW - 1) / PW; ++i) {
        const uint32_t k = w + PW * i, t = 4 * k + ln / 16;
        if (NQ % PW == 0 || k < NQ)
            lds_load16(base + L::QS + 1024 * k, rq, (tb + t) * 256 + 16 * ((ln & 15) ^ (t & 15)));
    }
    // digit sums: 256 bytes (16 tokens) per instruction; scales: 64 tokens
#pragma unroll
    for (uint32_t i = 0; i < (NG + PW - 1) / PW; ++i) {
        const uint32_t k = w + PW * i;
        if (NG % PW == 0 || k < NG) lds_load4(base + L::DG + 256 * k, rg, (tb + 16 * k) * 16 + 4 * ln);
    }
#pragma unroll
    for (uint32_t i = 0; i < (ND + PW - 1) / PW; ++i) {
        const uint32_t k = w + PW * i;
        if (ND % PW == 0 || k < ND) lds_load4(base + L::D8 + 256 * k, rd, (tb + 64 * k + ln) * 4);
    }
}

// Superblock b of the tile's weight rows into LDS, [row][144] (9 16-byte
// chunks per row; a wave instruction covers 64 consecutive chunks, so its
// loads fall on 7-8 consecutive rows: whole cache lines). Rows past N lie
// outside the descriptor and load zeros.
template <int NT>
__device__ __forceinline__ void w_to_lds(const v4i wrs, uint32_t row_bytes,
                                         uint32_t n0, uint32_t b, unsigned char *buf, uint32_t w, uint32_t lane) {
    using L = PLds<NT>;
    constexpr uint32_t NC = PR * 9 / 64;  // wave instructions per superblock
    const uint32_t base = lds_addr(buf) + L::W;
    uint32_t ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (uint32_t i = 0; i < (NC + PW - 1) / PW; ++i) {
        const uint32_t k = w + PW * i;
        if (NC % PW == 0 || k < NC) {
            const uint32_t c = 64 * k + ln, r = c / 9, p = c - 9 * r;
            lds_load16(base + 1024 * k, wrs, (n0 + r) * row_bytes + b * 144 + 16 * p);
        }
    }
}

// One 32-token block t of the tile against this wave's converted weights.
// The hi and lo chains run interleaved as two independent accumulators (no
// MFMA waits on the previous one's result), C = 8*hi + lo after both; the
// min term's high-digit MFMA is issued first so that its shift overlaps the
// chains.
template <int NT>
__device__ __forceinline__ void q4_block(const unsigned char *buf, const Q4Frag &f, uint32_t t, uint32_t j,
                                         uint32_t g, float (&acc)[16]) {
    using L = PLds<NT>;
    const unsigned char *arow = buf + L::QS + (32 * t + j) * 256;
    const v4i dgv = as_v4i(lds4(buf + L::DG + (32 * t + j) * 16));
    // high digits in bytes 0-7 against the mins; then the low digits moved there
    v16i mn = mfma(dgv, f.m, v16i{});
    v16i ch = {}, cl = {};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const v4i af = as_v4i(lds4(arow + 16 * ((2 * s + g) ^ (j & 15))));
        ch = mfma(af, f.bh[s], ch);
        cl = mfma(af, f.bl[s], cl);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) mn[r] <<= 7;
    mn = mfma(v4i{dgv.z, dgv.w, dgv.z, dgv.w}, f.m, mn);
#pragma unroll
    for (int r = 0; r < 16; ++r) ch[r] = (ch[r] << 3) + cl[r];
    const float *d8 = reinterpret_cast<const float *>(buf + L::D8) + 32 * t + 4 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 dv = *reinterpret_cast<const float4 *>(d8 + 8 * q);
        const float dd[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 4 * q + e;
            acc[r] = fmaf(dd[e], fmaf(f.d, float(ch[r]), -f.dm * float(mn[r])), acc[r]);
        }
    }
}

__host__ __device__ inline uint32_t sk_begin(uint32_t units, uint32_t grid, uint32_t v) {
    return uint32_t(uint64_t(units) * v / grid);
}
// Range number of workgroup `bid`: the workgroups of one XCD take
// consecutive ranges (bid % 8 is the XCD under round-robin dispatch).
__device__ __forceinline__ uint32_t sk_logical(uint32_t bid, uint32_t G) {
    return (G & 7) ? bid : (bid & 7) * (G >> 3) + (bid >> 3);
}

template <int NT>
__global__ __launch_bounds__(64 * PW) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_pf_q4k(PfArgs a) {
    extern __shared__ __align__(16) unsigned char lds[];
    using L = PLds<NT>;
    constexpr uint32_t TT = L::TT;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    auto buf = [&](uint32_t b) __attribute__((always_inline)) { return lds + (b & 1) * L::bytes; };
    const v4i wrs = rs4(a.W, a.N * a.row_bytes);

    const uint32_t v = sk_logical(blockIdx.x, a.G);
#ifdef TC_PF_TRACE
    unsigned long long twait = 0, tconv = 0, tblk = 0, tgap = 0, ts3p = 0, tstore = 0, tstart = __builtin_readcyclecounter();
#endif
    const uint32_t units = a.ntiles * a.nblk;
    const uint32_t ub = sk_begin(units, a.G, v), ue = sk_begin(units, a.G, v + 1);
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
        uint32_t ln = lane;
        asm volatile("" : "+v"(ln));
        const uint32_t j = ln & 31, g = ln >> 5;
        const uint32_t tn = tile % a.ntn, tm = tile / a.ntn;
        const uint32_t n0 = tn * PR, m0 = tm * TT;

        float acc[NT][16];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;

        // Previous segment's readers of both buffers are done.
        __syncthreads();
        Q4Frag f;
        act_to_lds<NT>(a, m0, b0, buf(b0), w, lane);
        w_to_lds<NT>(wrs, a.row_bytes, n0, b0, buf(b0), w, lane);
        // Per superblock: its activations and weight blocks are waited for,
        // the next superblock's loads issued into the other LDS buffer, this
        // lane's weights converted, then the MFMAs.
        for (uint32_t b = b0; b < b1; ++b) {
#ifdef TC_PF_TRACE
            const unsigned long long ts0 = __builtin_readcyclecounter();
            if (b > b0) tgap += ts0 - ts3p;
#endif
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            __syncthreads();
#ifdef TC_PF_TRACE
            const unsigned long long ts1 = __builtin_readcyclecounter();
#endif
            act_to_lds<NT>(a, m0, min(b + 1, b1 - 1), buf(b + 1), w, lane);
            w_to_lds<NT>(wrs, a.row_bytes, n0, min(b + 1, b1 - 1), buf(b + 1), w, lane);
            {
                Q4Raw rr;
                q4_read(rr, buf(b) + L::W + (32 * w + j) * 144, g);
                q4_convert(rr, g, f);
            }
#ifdef TC_PF_TRACE
            const unsigned long long ts2 = __builtin_readcyclecounter();
#endif
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                // one token block at a time in the scheduler's window (it
                // would otherwise hoist every block's operand reads)
                __builtin_amdgcn_sched_barrier(0);
                q4_block<NT>(buf(b), f, t, j, g, acc[t]);
            }
            __builtin_amdgcn_sched_barrier(0);
#ifdef TC_PF_TRACE
            {
                const unsigned long long ts3 = __builtin_readcyclecounter();
                twait += ts1 - ts0;
                tconv += ts2 - ts1;
                tblk += ts3 - ts2;
                ts3p = ts3;
            }
#endif
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // nothing of this segment left in flight

#ifdef TC_PF_TRACE
        const unsigned long long tsst = __builtin_readcyclecounter();
#endif
        // lane: row n0 + 32w + j, tokens m0 + 32t + 8q + 4g + e
        const uint32_t nl = 32 * w + j, n = n0 + nl;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t ml = 32 * t + 8 * q + 4 * g + e, m = m0 + ml;
                    const float val = acc[t][4 * q + e];
                    if (part != nullptr)
                        part[ml * PR + nl] = val;
                    else if (m < a.M && n < a.N)
                        a.out[size_t(m) * a.N + n] = val;
                }
            }
        }
#ifdef TC_PF_TRACE
        tstore += __builtin_readcyclecounter() - tsst;
#endif
    }
#ifdef TC_PF_TRACE
    if (lane == 0) {
        unsigned long long *tr = a.trace + (size_t(blockIdx.x) * PW + w) * 8;
        tr[0] = twait; tr[1] = tconv; tr[2] = tblk; tr[3] = tgap; tr[4] = tstore;
        tr[5] = __builtin_readcyclecounter() - tstart;
    }
#endif
}

// Tiles split over several workgroups: out = the partial segments summed in
// workgroup (range) order. kFix workgroups per split tile, each a slice of
// it; group j takes the tile holding range boundary j + 1 when that boundary
// splits it and is the first to do so.
constexpr uint32_t kFix = 4;
template <int NT>
__global__ __launch_bounds__(256) void k_pf_fixup(PfArgs a) {
    constexpr uint32_t TT = PLds<NT>::TT;
    const uint32_t units = a.ntiles * a.nblk, G = a.G;
    const uint32_t slice = blockIdx.x % kFix;
    const uint32_t wb = blockIdx.x / kFix + 1, ubd = sk_begin(units, G, wb);
    const uint32_t tile = ubd / a.nblk;
    if (ubd % a.nblk == 0 || sk_begin(units, G, wb - 1) > tile * a.nblk) return;
    if (tile >= a.ntiles) return;
    const uint32_t t0 = tile * a.nblk, t1 = t0 + a.nblk;
    uint32_t v = uint32_t(uint64_t(t0) * G / units);
    while (v + 1 < G && sk_begin(units, G, v + 1) <= t0) ++v;
    while (v > 0 && sk_begin(units, G, v) > t0) --v;
    const uint32_t tn = tile % a.ntn, tm = tile / a.ntn;
    const uint32_t n0 = tn * PR, m0 = tm * TT;
    constexpr uint32_t per = TT * PR / 4 / kFix;  // float4 entries per slice
    constexpr uint32_t NI = per / 256;
    static_assert(per % 256 == 0, "a fixup slice is a whole number of 256-thread rounds");
    float4 s[NI];
#pragma unroll
    for (uint32_t k = 0; k < NI; ++k) s[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    uint32_t bv = sk_begin(units, G, v);
    for (; v < G && bv < t1; ++v) {
        const uint32_t bn = sk_begin(units, G, v + 1);
        if (bn > t0 && bn != bv) {
            const float *src = a.ws + (size_t(v) * 2 + (bv >= t0 ? 0u : 1u)) * (TT * PR);
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
        const uint32_t ml = (4 * i) / PR, nl = (4 * i) % PR;
        const uint32_t m = m0 + ml, n = n0 + nl;
        if (m >= a.M) continue;
        float *o = a.out + size_t(m) * a.N + n;
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

// Token-tile width from M (reference GemmDispatch.cu:634-643 picks its tile
// from seqLen too): the smallest of 32, 64, 128 tokens that holds M, else 256.
int pf_nt(uint32_t M) { return M <= 32 ? 1 : M <= 64 ? 2 : 4; }

struct PfGeom {
    int nt;
    uint32_t tt, ntm, ntn, ntiles, G;
};
PfGeom pf_geom(uint32_t M, uint32_t N, uint32_t K, int num_cu) {
    PfGeom g;
    g.nt = pf_nt(M);
    g.tt = 32u * g.nt;
    g.ntm = (M + g.tt - 1) / g.tt;
    g.ntn = (N + PR - 1) / PR;
    g.ntiles = g.ntm * g.ntn;
    const uint64_t units = uint64_t(g.ntiles) * (K / 256);
    // one workgroup per CU, each with at least 2 superblocks of work
    g.G = uint32_t(std::max<uint64_t>(1, std::min<uint64_t>(uint64_t(num_cu), units / 2)));
    return g;
}

template <int NT>
hipError_t pf_launch(const PfArgs &a, hipStream_t st) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_pf_q4k<NT>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    k_pf_q4k<NT><<<dim3{a.G, 1u, 1u}, 64 * PW, 2 * PLds<NT>::bytes, st>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t units = a.ntiles * a.nblk;
    bool split = false;
    for (uint32_t v = 1; v < a.G && !split; ++v) split = sk_begin(units, a.G, v) % a.nblk != 0;
    if (!split) return hipSuccess;
    k_pf_fixup<NT><<<dim3{(a.G - 1) * kFix, 1u, 1u}, 256, 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace

#ifdef TC_PF_TRACE
void *tc_pf_trace_buf = nullptr;
extern "C" void tc_pf_set_trace(void *p) { tc_pf_trace_buf = p; }
#endif
bool prefill_type(int type) { return type == kQ4_K; }

size_t prefill_workspace_bytes(int type, uint32_t M, uint32_t N, uint32_t K, int num_cu) {
    if (!prefill_type(type)) return 0;
    const PfGeom g = pf_geom(M, N, K, num_cu);
    return size_t(g.G) * 2 * g.tt * PR * 4;
}

hipError_t launch_prefill(int type, const void *W, const ActView &act, float *out, uint32_t M, uint32_t N,
                          uint32_t K, int num_cu, void *workspace, hipStream_t st) {
    if (!prefill_type(type) || M == 0 || N == 0 || K == 0 || K % 256 || workspace == nullptr || act.dg == nullptr)
        return hipErrorInvalidValue;
    if (uint64_t(M) * K >= (uint64_t(1) << 32) || uint64_t(N) * (K / 256) * unit_bytes(type) >= (uint64_t(1) << 32))
        return hipErrorInvalidValue;
    const PfGeom g = pf_geom(M, N, K, num_cu);
    PfArgs a{};
    a.W = static_cast<const uint8_t *>(W);
    a.qs = act.qs;
    a.d8 = act.d;
    a.dg = act.dg;
    a.out = out;
    a.ws = static_cast<float *>(workspace);
    a.M = M;
    a.N = N;
    a.K = K;
    a.nblk = K / 256;
    a.row_bytes = a.nblk * unit_bytes(type);
    a.ntm = g.ntm;
    a.ntn = g.ntn;
    a.ntiles = g.ntiles;
    a.G = g.G;
#ifdef TC_PF_TRACE
    a.trace = static_cast<unsigned long long *>(tc_pf_trace_buf);
#endif
    switch (g.nt) {
        case 1: return pf_launch<1>(a, st);
        case 2: return pf_launch<2>(a, st);
        default: return pf_launch<4>(a, st);
    }
}

}  // namespace tc
