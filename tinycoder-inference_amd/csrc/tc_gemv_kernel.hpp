// tc_gemv_kernel.hpp -- the decode-time quantized mat-vec kernel for gfx950
// (batch 1..8), k_gemv_t, templated on the weight type. Each weight type is
// instantiated in a translation unit of its own (tc_gemv_inst.hip, built once
// per type); the host dispatch in tc_gemv.hip picks the shape and type.
//
// One launch runs a list of jobs (matrices); each job has its own weights,
// input vector(s) and output, so q/k/v (one shared input), a gate/up pair
// (SwiGLU epilogue) or any set of independent mat-vecs go out in one launch.
// A workgroup (one per CU) owns a contiguous range of rows of one job, i.e. a
// contiguous byte range of the weight stream; its waves stream 64-unit tiles
// of raw GGUF blocks through a register ring into LDS, and every lane decodes
// one whole 256-weight unit against activation records in LDS (quantized in
// the prologue with the reference CPU rule, bit-exact).
#pragma once

#include <type_traits>

#include "tc_actquant.hpp"
#include "tc_kernels.hpp"

namespace tc {

// Cache policy of the weight stream: non-temporal (nt). Each weight byte is
// read once per launch, so its lines are marked for early eviction and the
// activations and partial sums keep their L2 and Infinity Cache residency.
// MoE expert launches keep the default policy: an expert chosen by several
// tokens is read once per (token, rank) pair, and the later reads hit the
// Infinity Cache.
constexpr int kWeightCachePolicy = 2;

namespace {
__constant__ uint32_t c_grid[256] = {
#include "iq3xxs_grid.inc"
};
__constant__ uint32_t c_grid_s[512] = {
#include "iq3s_grid.inc"
};
__constant__ uint64_t c_grid_2s[1024] = {
#include "iq2s_grid.inc"
};
__constant__ uint64_t c_grid_2xs[512] = {
#include "iq2xs_grid.inc"
};
}  // namespace

namespace gv {

constexpr int kMaxJobs = 8;

__device__ __forceinline__ uint32_t align2(uint32_t hi, uint32_t lo, uint32_t sh) {
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
}
__device__ __forceinline__ uint32_t byte_of(uint32_t w, uint32_t k) { return (w >> (8 * k)) & 0xFFu; }

// Two launch shapes (chosen per launch on the host): big streams use 512
// threads with one tile in flight per wave (the activation loads, which miss
// in L2, then see a short memory queue); small ones, and Q8_0 whose 17 KB
// wave tiles would not fit eight to a CU, use 256 threads with two.
struct CfgBig {
    static constexpr int NT = 512, DEPTH = 1;
};
struct CfgSmall {
    static constexpr int NT = 256, DEPTH = 2;
};
constexpr int kTileUnits = 64;
constexpr uint32_t XB = 304;                // LDS bytes per 256-element activation block
constexpr uint32_t XB_BS = 256, XB_D = 288;  // bsums and d offsets inside a record
// LDS bytes per 256-element activation block: the Q8_K / Q8_0 record, or the
// unquantized fp32 values for IQ2_XS (whose reference CPU path dots fp32 x),
// padded to 1072 bytes: the lanes of a wave read the records of consecutive
// blocks, and a 1024-byte stride would put them all in the same LDS banks
// (1072 = 48 mod 256, the residue of the conflict-free 304-byte record).
__host__ __device__ constexpr uint32_t xrec_bytes(int type) { return type == kIQ2_XS || type == kIQ4_NL || type == kQ5_0 ? 1072u : XB; }

// 16-byte loads per lane per tile (the last one partial for Q6_K / IQ3_XXS,
// whose 64-unit tiles are 13440 / 6272 bytes) and the LDS bytes of one tile.
__host__ __device__ constexpr int tile_dwordx4(int type) { return (unit_bytes(type) * kTileUnits + 1023) / 1024; }
__host__ __device__ constexpr int tile_slot_bytes(int type) { return tile_dwordx4(type) * 1024; }
template <class C>
__host__ __device__ constexpr int tile_depth(int type, int S) {
    // Register slots in flight per wave: fewer where the accumulators of S
    // tokens would otherwise spill at 2 waves per SIMD (a Q8_0 slot is 68
    // registers, a Q4_K slot 36).
    const int d = type == kQ4_K || type == kQ5_K ? (S <= 6 ? 2 : 1) : (S >= 4 ? 1 : 2);
    return d < C::DEPTH ? d : C::DEPTH;
}


struct TJobDev {
    const uint8_t *W, *W2;
    const float *x;
    ActView act;
    float *out, *out2;
    int32_t *dbg;
    uint32_t rows, cols, nu, out_ld;
    uint32_t rows_per_wg, wg_begin;
    int epi;
    DivMod nu_div;
    // Expert-pair mode (ids != null): the job is npairs mat-vecs, pair p using
    // expert ids[p] (matrix at W + ids[p]*wstride), input x + (p/x_div)*x_stride
    // and output out + p*out_stride; wg_per_pair workgroups each.
    const int32_t *ids;
    uint64_t wstride;
    uint32_t wg_per_pair, x_div, x_stride, out_stride, n_experts;
    // Activation tokens staged in LDS (S, or the rank-group size), and the
    // rank-group mode (rk > 0, with ids): the job's pair p is a token whose rk
    // ranks use experts ids[p*rk + k] with inputs x + p*x_stride + k*cols;
    // out = sum over k in rank order of wts[p*rk + k] * (W[e_k] x_k).
    uint32_t nx, rk;
    const float *wts;
};

struct TLaunchArgs {
    TJobDev jobs[kMaxJobs];
    uint32_t njobs;
    uint32_t off_t, off_p, off_g;  // LDS: activation records at 0, wave tiles, partials, IQ3_XXS grid
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 lds128(const unsigned char *p) { return *reinterpret_cast<const u32x4 *>(p); }

// N 16-byte registers addressed only through compile-time indices. (Native
// vectors: HIP's uint4 is a class whose copies become memcpy calls that keep
// a local array in scratch memory.)
template <int N>
struct Regs {
    u32x4 h;
    Regs<N - 1> t;
};
template <>
struct Regs<1> {
    u32x4 h;
};
template <int I, int N>
__device__ __forceinline__ u32x4 &reg(Regs<N> &r) {
    if constexpr (I == 0)
        return r.h;
    else
        return reg<I - 1, N - 1>(r.t);
}
template <int I, int N>
__device__ __forceinline__ const u32x4 &reg(const Regs<N> &r) {
    if constexpr (I == 0)
        return r.h;
    else
        return reg<I - 1, N - 1>(r.t);
}
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Raw buffer descriptor (gfx9 word 3: 32-bit raw data) over [p, p+bytes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), short(0), int(bytes), 0x00020000);
}

// (q & 0xF0F0F0F0) ^ 0x80808080: each byte = 16*high_nibble - 128 as int8.
__device__ __forceinline__ uint32_t hi_nib_s8(uint32_t q) {
    return (q & 0xF0F0F0F0u) ^ 0x80808080u;  // one v_bitop3 on gfx950
}
__device__ __forceinline__ int sdot2_ones(uint32_t pair) {
    typedef short s16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2, pair), __builtin_bit_cast(s16x2, 0x00010001u), 0, false);
}

// ---- activation prologue -------------------------------------------------------
// In two halves so that its global loads are issued ahead of the weight ring
// (vmcnt counts loads in issue order: a load issued after the weights would
// make the prologue wait for them). The loads go through a buffer descriptor
// sized to the activation, so the fixed number of preload slots costs no
// memory traffic past its end.
//
// Fused mode (x fp32): 16 lanes per 256-element block quantize with the
// reference rule (a lane owns one 16-value chunk = one bsum group); chunks
// tid + i*TNT (i < kXPre) are preloaded, any further ones are loaded after the
// weights in a loop. Pre-quantized mode: the int8 values (kXPreQ chunks of 16
// bytes per thread), the bsums or per-32 scales, and the per-block scales are
// preloaded likewise and copied into the records.
constexpr int kXPre = 3;   // fused: 64-byte x chunks per thread
constexpr int kXPreQ = 8;  // pre-quantized: 16-byte qs chunks per thread
constexpr int kXSlots = 4 * kXPre > kXPreQ + 2 ? 4 * kXPre : kXPreQ + 2;

struct XPre {
    Regs<kXSlots> r;
};

struct XRsrc {
    __amdgpu_buffer_rsrc_t a, b, c;  // fused: x; pre-quantized: qs, bsums or d32, d
};

template <int TYPE, int S>
__device__ __forceinline__ XRsrc tstage_rsrc(const TJobDev &jb) {
    const uint32_t nblk = jb.nx * (jb.cols / 256);
    XRsrc r;
    const bool fused = jb.x != nullptr;
    r.a = fused ? make_rsrc(jb.x, nblk * 1024u) : make_rsrc(jb.act.qs, nblk * 256u);
    if constexpr (TYPE == kQ8_0) {
        r.b = make_rsrc(jb.act.d, fused ? 0u : nblk * 32u);
        r.c = r.b;
    } else {
        r.b = make_rsrc(jb.act.bsums, fused ? 0u : nblk * 32u);
        r.c = make_rsrc(jb.act.d, fused ? 0u : nblk * 4u);
    }
    return r;
}

// The same kXSlots 16-byte loads in both modes (one straight-line sequence,
// so no register state merges across a branch): fused slot s holds x chunk
// tid + (s/4)*TNT, quarter s%4; pre-quantized slots 0..kXPreQ-1 hold qs chunks
// tid + s*TNT, slot kXPreQ side dwords 4tid..4tid+3, slot kXPreQ+1 block
// scales 4tid..4tid+3. Unused slots read past the descriptor (zeros, no traffic).
template <int TYPE, int S, int TNT>
__device__ __forceinline__ XPre tstage_preload(const TJobDev &jb, const XRsrc &rs) {
    XPre p;
    const uint32_t tid = threadIdx.x;
    const uint32_t wbase = __builtin_amdgcn_readfirstlane(tid & ~63u);  // first thread of this wave
    const uint32_t nblk = jb.nx * (jb.cols / 256);
    // Every load instruction costs the CU's address unit ~16 cycles whatever
    // its lanes read, so a wave issues only the slots that hold some of its
    // data (wave-uniform tests); the others stay zero.
    static_for<0, kXSlots>([&](auto sl) __attribute__((always_inline)) { reg<decltype(sl)::value>(p.r) = u32x4{0, 0, 0, 0}; });
    if (jb.x != nullptr) {
        static_for<0, kXPre>([&](auto g) __attribute__((always_inline)) {
            constexpr int G = decltype(g)::value;
            if (wbase + G * TNT < nblk * 16) {
                const uint32_t off = (tid + G * TNT) * 64u;
                static_for<0, 4>([&](auto q) __attribute__((always_inline)) {
                    reg<4 * G + decltype(q)::value>(p.r) =
                        __builtin_amdgcn_raw_buffer_load_b128(rs.a, off + 16u * decltype(q)::value, 0, 0);
                });
            }
        });
    } else {
        static_for<0, kXPreQ>([&](auto g) __attribute__((always_inline)) {
            constexpr int G = decltype(g)::value;
            if (wbase + G * TNT < nblk * 16)
                reg<G>(p.r) = __builtin_amdgcn_raw_buffer_load_b128(rs.a, (tid + G * TNT) * 16u, 0, 0);
        });
        if (4 * wbase < nblk * 8) reg<kXPreQ>(p.r) = __builtin_amdgcn_raw_buffer_load_b128(rs.b, tid * 16u, 0, 0);
        if constexpr (TYPE != kQ8_0)
            if (4 * wbase < nblk) reg<kXPreQ + 1>(p.r) = __builtin_amdgcn_raw_buffer_load_b128(rs.c, tid * 16u, 0, 0);
    }
    return p;
}

template <int TYPE>
__device__ __forceinline__ void tquant_chunk(const float (&e)[16], uint32_t g, uint32_t k, bool ok, unsigned char *xr) {
    constexpr int WIDTH = TYPE == kQ8_0 ? 2 : 16;  // lanes per activation block
    const float maxv = first_absmax<WIDTH>(e, int(16 * (k % WIDTH)));
    uint32_t w[4] = {0, 0, 0, 0};
    int bsum = 0;
    float dv = 0.0f;
    if (maxv != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, maxv);
        uint32_t qb[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) qb[i] = q8_bits(iscale, e[i]);
        uint32_t tot = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) tot += qb[i];
        bsum = int(tot - 16u * kQ8Magic);
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = q8_pack4(qb[4 * j], qb[4 * j + 1], qb[4 * j + 2], qb[4 * j + 3]);
        dv = __fdiv_rn(1.0f, iscale);
    }
    if (ok) {
        unsigned char *r = xr + size_t(g) * XB;
        *reinterpret_cast<u32x4 *>(r + 16 * k) = u32x4{w[0], w[1], w[2], w[3]};
        if constexpr (TYPE == kQ8_0) {
            if ((k & 1) == 0) reinterpret_cast<float *>(r + XB_BS)[k / 2] = dv;
        } else {
            reinterpret_cast<int16_t *>(r + XB_BS)[k] = int16_t(bsum);
            if (k == 0) *reinterpret_cast<float *>(r + XB_D) = dv;
        }
    }
}

template <int TYPE>
__device__ __forceinline__ void tquant_regs(const u32x4 &a, const u32x4 &b, const u32x4 &c, const u32x4 &d, uint32_t g,
                                            uint32_t k, bool ok, unsigned char *xr) {
// (the uint32_t copy is needed: clang's __builtin_bit_cast applied directly to
// an ext_vector element reads element 0)
#define TC_F(v) __builtin_bit_cast(float, uint32_t(v))
    const float e[16] = {TC_F(a.x), TC_F(a.y), TC_F(a.z), TC_F(a.w), TC_F(b.x), TC_F(b.y), TC_F(b.z), TC_F(b.w),
                         TC_F(c.x), TC_F(c.y), TC_F(c.z), TC_F(c.w), TC_F(d.x), TC_F(d.y), TC_F(d.z), TC_F(d.w)};
#undef TC_F
    tquant_chunk<TYPE>(e, g, k, ok, xr);
}

template <int TYPE>
__device__ __forceinline__ void tstore_side(unsigned char *xr, uint32_t i, uint32_t v) {
    // dword i of the bsums (Q8_K: 8 per block) or per-32 scales (Q8_0: 8 per block)
    reinterpret_cast<uint32_t *>(xr + size_t(i / 8) * XB + XB_BS)[i & 7] = v;
}

template <int TYPE, int S, int TNT>
__device__ __forceinline__ void tstage_finish(const TJobDev &jb, const XRsrc &rs, const XPre &p, unsigned char *xr) {
    const uint32_t tid = threadIdx.x;
    const uint32_t nblk = jb.nx * (jb.cols / 256);
    if constexpr (TYPE == kIQ2_XS || TYPE == kIQ4_NL || TYPE == kQ5_0) {
        // fp32 x as it is: 64-byte chunk c (16 floats) of block c/16 into that
        // block's record
        const uint32_t nchunk = nblk * 16;
        auto dst = [&](uint32_t c) __attribute__((always_inline)) {
            return xr + size_t(c / 16) * xrec_bytes(TYPE) + 64 * (c & 15);
        };
        static_for<0, kXPre>([&](auto i) __attribute__((always_inline)) {
            const uint32_t c = tid + i.value * TNT;
            if (c < nchunk)
                static_for<0, 4>([&](auto q) __attribute__((always_inline)) {
                    *reinterpret_cast<u32x4 *>(dst(c) + 16 * decltype(q)::value) = reg<4 * i.value + decltype(q)::value>(p.r);
                });
        });
        for (uint32_t c = tid + kXPre * TNT; c < nchunk; c += TNT)
            static_for<0, 4>([&](auto q) __attribute__((always_inline)) {
                *reinterpret_cast<u32x4 *>(dst(c) + 16 * decltype(q)::value) =
                    __builtin_amdgcn_raw_buffer_load_b128(rs.a, c * 64u + 16u * decltype(q)::value, 0, 0);
            });
        return;
    }
    if (jb.x != nullptr) {
        const uint32_t nchunk = nblk * 16;
        static_for<0, kXPre>([&](auto i) __attribute__((always_inline)) {
            if (i.value * TNT < nchunk) {
                const uint32_t c = tid + i.value * TNT;
                tquant_regs<TYPE>(reg<4 * i.value>(p.r), reg<4 * i.value + 1>(p.r), reg<4 * i.value + 2>(p.r),
                                  reg<4 * i.value + 3>(p.r), c / 16, c & 15, c < nchunk, xr);
            }
        });
        for (uint32_t c0 = kXPre * TNT; c0 < nchunk; c0 += TNT) {
            const uint32_t c = c0 + tid;
            const uint32_t off = c * 64u;
            tquant_regs<TYPE>(__builtin_amdgcn_raw_buffer_load_b128(rs.a, off, 0, 0),
                              __builtin_amdgcn_raw_buffer_load_b128(rs.a, off + 16, 0, 0),
                              __builtin_amdgcn_raw_buffer_load_b128(rs.a, off + 32, 0, 0),
                              __builtin_amdgcn_raw_buffer_load_b128(rs.a, off + 48, 0, 0), c / 16, c & 15, c < nchunk, xr);
        }
    } else {
        const uint32_t nq = nblk * 16, nside = nblk * 8;
        static_for<0, kXPreQ>([&](auto i) __attribute__((always_inline)) {
            const uint32_t c = tid + i.value * TNT;
            if (c < nq) *reinterpret_cast<u32x4 *>(xr + size_t(c / 16) * XB + 16 * (c & 15)) = reg<i.value>(p.r);
        });
        for (uint32_t c = tid + kXPreQ * TNT; c < nq; c += TNT)
            *reinterpret_cast<u32x4 *>(xr + size_t(c / 16) * XB + 16 * (c & 15)) =
                __builtin_amdgcn_raw_buffer_load_b128(rs.a, c * 16u, 0, 0);
        const u32x4 side = reg<kXPreQ>(p.r);
        const uint32_t sv[4] = {side.x, side.y, side.z, side.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * tid + i < nside) tstore_side<TYPE>(xr, 4 * tid + i, sv[i]);
        for (uint32_t c = tid + 4 * TNT; c < nside; c += TNT)
            tstore_side<TYPE>(xr, c, __builtin_amdgcn_raw_buffer_load_b32(rs.b, c * 4u, 0, 0));
        if constexpr (TYPE != kQ8_0) {
            const u32x4 dv = reg<kXPreQ + 1>(p.r);
            const uint32_t dd[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (4 * tid + i < nblk) *reinterpret_cast<uint32_t *>(xr + size_t(4 * tid + i) * XB + XB_D) = dd[i];
            for (uint32_t c = tid + 4 * TNT; c < nblk; c += TNT)
                *reinterpret_cast<uint32_t *>(xr + size_t(c) * XB + XB_D) =
                    __builtin_amdgcn_raw_buffer_load_b32(rs.c, c * 4u, 0, 0);
        }
    }
}

// ---- per-unit dot products (one lane = one 256-weight unit) -----------------------

template <int TYPE, int S>
struct TDot;

// Q4_K: the 8 sub-block integer sums are exact (reference
// SIMDMatMulVecAVX2.cpp:3690-3702); main = sum sc_i*s_i and min = sum
// m_i*(bsum pair) in int32, then d8*(d*main - dmin*min). High nibbles enter
// the dot products as 16h-128 and are corrected with 128*sum(x), which the
// bsums hold, before the exact division by 16.
template <int S>
struct TDot<kQ4_K, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               float *val, int32_t *dbg, size_t dbg_tok) {
        const u32x4 h = lds128(u);
        const uint32_t scl = h.y & 0x3F3F3F3Fu, mnl = h.z & 0x3F3F3F3Fu;
        const uint32_t sch = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t mnh = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
        const float d = h2f(h.x & 0xFFFFu), dmin = h2f(h.x >> 16);
        int mainI[S], minI[S];
#pragma unroll
        for (int s = 0; s < S; ++s) mainI[s] = minI[s] = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4 qa = lds128(u + 16 + 32 * j), qb = lds128(u + 32 + 32 * j);
            const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                lo[k] = q[k] & 0x0F0F0F0Fu;
                hi[k] = hi_nib_s8(q[k]);
            }
            const uint32_t scw = j < 2 ? scl : sch, mnw = j < 2 ? mnl : mnh;
            const int sc0 = int(byte_of(scw, (2 * j) & 3)), sc1 = int(byte_of(scw, (2 * j + 1) & 3));
            const int m0 = int(byte_of(mnw, (2 * j) & 3)), m1 = int(byte_of(mnw, (2 * j + 1) & 3));
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const unsigned char *xr = xr0 + s * xtok;
                const u32x4 x0 = lds128(xr + 64 * j), x1 = lds128(xr + 64 * j + 16);
                const u32x4 x2 = lds128(xr + 64 * j + 32), x3 = lds128(xr + 64 * j + 48);
                const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
                const uint2 bs = *reinterpret_cast<const uint2 *>(xr + XB_BS + 8 * j);
                const int bp0 = sdot2_ones(bs.x), bp1 = sdot2_ones(bs.y);
                int s0 = 0, t1 = 0;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    s0 = sdot4(int(lo[k]), int(xl[k]), s0);
                    t1 = sdot4(int(hi[k]), int(xh[k]), t1);
                }
                const int s1 = (t1 + 128 * bp1) >> 4;
                if (dbg) {
                    dbg[s * dbg_tok + 2 * j] = s0;
                    dbg[s * dbg_tok + 2 * j + 1] = s1;
                }
                mainI[s] += sc0 * s0 + sc1 * s1;
                minI[s] += m0 * bp0 + m1 * bp1;
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const float d8 = *reinterpret_cast<const float *>(xr0 + s * xtok + XB_D);
            val[s] = d8 * (d * float(mainI[s]) - dmin * float(minI[s]));
        }
    }
};

// Q5_K, one unit (176 B, 16-byte aligned) per lane: the Q4_K header and
// nibble layout (qs at 48) plus the fifth bits in qh (bit 2j+h of qh[l] for
// element l of sub-block 2j+h). The 8 sub-block sums s_g = sum q5*x are exact
// int32 (q5 in 0..31), and main = sum sc_g*s_g, min = sum m_g*(bsum pair) in
// int32, value d8*(d*main - dmin*min). The reference CPU kernel
// (SIMDMatMulVecAVX2.cpp:3842-3960) forms the same two sums per sub-block in
// fp32 (d*sc and dmin*m as float factors); the results differ by rounding
// only.
template <int S>
struct TDot<kQ5_K, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               float *val, int32_t *dbg, size_t dbg_tok) {
        const u32x4 h = lds128(u);
        const uint32_t scl = h.y & 0x3F3F3F3Fu, mnl = h.z & 0x3F3F3F3Fu;
        const uint32_t sch = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t mnh = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
        const float d = h2f(h.x & 0xFFFFu), dmin = h2f(h.x >> 16);
        const u32x4 ha = lds128(u + 16), hb = lds128(u + 32);
        const uint32_t qh[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
        int mainI[S], minI[S];
#pragma unroll
        for (int s = 0; s < S; ++s) mainI[s] = minI[s] = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4 qa = lds128(u + 48 + 32 * j), qb = lds128(u + 64 + 32 * j);
            const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                // fifth bits of sub-blocks 2j and 2j+1 (qh bits 2j, 2j+1 of each
                // byte) rotated to bit 4 of each byte (one v_alignbit each)
                const uint32_t b0 = __builtin_amdgcn_alignbit(qh[k], qh[k], (2 * j + 28) & 31) & 0x10101010u;
                const uint32_t b1 = __builtin_amdgcn_alignbit(qh[k], qh[k], (2 * j + 29) & 31) & 0x10101010u;
                lo[k] = (q[k] & 0x0F0F0F0Fu) | b0;
                hi[k] = ((q[k] >> 4) & 0x0F0F0F0Fu) | b1;
            }
            const uint32_t scw = j < 2 ? scl : sch, mnw = j < 2 ? mnl : mnh;
            const int sc0 = int(byte_of(scw, (2 * j) & 3)), sc1 = int(byte_of(scw, (2 * j + 1) & 3));
            const int m0 = int(byte_of(mnw, (2 * j) & 3)), m1 = int(byte_of(mnw, (2 * j + 1) & 3));
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const unsigned char *xr = xr0 + s * xtok;
                const u32x4 x0 = lds128(xr + 64 * j), x1 = lds128(xr + 64 * j + 16);
                const u32x4 x2 = lds128(xr + 64 * j + 32), x3 = lds128(xr + 64 * j + 48);
                const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
                const uint2 bs = *reinterpret_cast<const uint2 *>(xr + XB_BS + 8 * j);
                const int bp0 = sdot2_ones(bs.x), bp1 = sdot2_ones(bs.y);
                int s0 = 0, s1 = 0;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    s0 = sdot4(int(lo[k]), int(xl[k]), s0);
                    s1 = sdot4(int(hi[k]), int(xh[k]), s1);
                }
                if (dbg) {
                    dbg[s * dbg_tok + 2 * j] = s0;
                    dbg[s * dbg_tok + 2 * j + 1] = s1;
                }
                mainI[s] += sc0 * s0 + sc1 * s1;
                minI[s] += m0 * bp0 + m1 * bp1;
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const float d8 = *reinterpret_cast<const float *>(xr0 + s * xtok + XB_D);
            val[s] = d8 * (d * float(mainI[s]) - dmin * float(minI[s]));
        }
    }
};

// Q3_K, one unit (110 B, 2-byte aligned in LDS) per lane: w' = q + 4 (0..7)
// from 2 bits of qs (at 2j) and bit 4n+j of hmask, one dword of each per 4
// weights; isum = sum_g (sc_g - 32) * (sum_16 w'*x - 4*bsum_g) exactly (the
// reference folds the -4 through the bsums the same way,
// SIMDMatMulVecAVX2.cpp:3480-3520); value = (d*d8) * isum.
template <int S>
struct TDot<kQ3_K, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               float *val, int32_t *dbg, size_t dbg_tok) {
        const u32x4 h0 = lds128(u), h1 = lds128(u + 16);
        const uint32_t hm[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        // 12 scale bytes, then d (bytes 108-109 of the unit) in the low half of .w
        const u32x4 sv = lds128(u + 96);
        const uint32_t km1 = 0x03030303u, km2 = 0x0F0F0F0Fu, tmp = sv.z;
        const uint32_t scw[4] = {(sv.x & km2) | ((tmp & km1) << 4), (sv.y & km2) | (((tmp >> 2) & km1) << 4),
                                 ((sv.x >> 4) & km2) | (((tmp >> 4) & km1) << 4),
                                 ((sv.y >> 4) & km2) | (((tmp >> 6) & km1) << 4)};
        const float d = h2f(sv.w & 0xFFFFu);
        int tot[S];
#pragma unroll
        for (int s = 0; s < S; ++s) tot[s] = 0;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const u32x4 qa = lds128(u + 32 + 32 * n), qb = lds128(u + 48 + 32 * n);
            const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int sb = 4 * n + j;  // sub-block of 32
                uint32_t w[8];
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    w[k] = ((q[k] >> (2 * j)) & km1) | (((hm[k] >> (4 * n + j)) & 0x01010101u) << 2);
                const int sc0 = int(byte_of(scw[(2 * sb) >> 2], (2 * sb) & 3)) - 32;
                const int sc1 = int(byte_of(scw[(2 * sb + 1) >> 2], (2 * sb + 1) & 3)) - 32;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const unsigned char *xr = xr0 + s * xtok;
                    const u32x4 x0 = lds128(xr + 32 * sb), x1 = lds128(xr + 32 * sb + 16);
                    int p0 = sdot4(int(w[0]), int(x0.x), 0);
                    p0 = sdot4(int(w[1]), int(x0.y), p0);
                    p0 = sdot4(int(w[2]), int(x0.z), p0);
                    p0 = sdot4(int(w[3]), int(x0.w), p0);
                    int p1 = sdot4(int(w[4]), int(x1.x), 0);
                    p1 = sdot4(int(w[5]), int(x1.y), p1);
                    p1 = sdot4(int(w[6]), int(x1.z), p1);
                    p1 = sdot4(int(w[7]), int(x1.w), p1);
                    const uint32_t bsp = *reinterpret_cast<const uint32_t *>(xr + XB_BS + 4 * sb);
                    const int b0 = int(int16_t(bsp & 0xFFFFu)), b1 = int(int16_t(bsp >> 16));
                    tot[s] += sc0 * (p0 - 4 * b0) + sc1 * (p1 - 4 * b1);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (dbg) dbg[s * dbg_tok] = tot[s];
            const float d8 = *reinterpret_cast<const float *>(xr0 + s * xtok + XB_D);
            val[s] = (d * d8) * float(tot[s]);
        }
    }
};

// Q2_K, one unit (84 B, 4-byte aligned in LDS) per lane: 2-bit values (bits
// 2t of qs[32h + l] for sub-block 4h + t) straight into v_dot4 (0..3); per 16
// the 4-bit scale (low nibble) and min (high nibble) of scales[g]; main =
// sum sc*sum q*x and min = sum m*bsum exact in int32, value d8*(d*main -
// dmin*min) (the two sums of the compact-block kernel,
// SIMDMatMulVecAVX2.cpp:4995-5020; it rounds them per lane in fp32).
template <int S>
struct TDot<kQ2_K, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               float *val, int32_t *dbg, size_t dbg_tok) {
        const u32x4 sv = lds128(u);
        const uint32_t scb[4] = {sv.x, sv.y, sv.z, sv.w};
        const uint32_t dw = *reinterpret_cast<const uint32_t *>(u + 80);
        const float d = h2f(dw & 0xFFFFu), dmin = h2f(dw >> 16);
        int mainI[S], minI[S];
#pragma unroll
        for (int s = 0; s < S; ++s) mainI[s] = minI[s] = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const u32x4 qa = lds128(u + 16 + 32 * h), qb = lds128(u + 32 + 32 * h);
            const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int sb = 4 * h + t;
                uint32_t w[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) w[k] = (q[k] >> (2 * t)) & 0x03030303u;
                const int sc0 = int(byte_of(scb[(2 * sb) >> 2], (2 * sb) & 3) & 15u);
                const int sc1 = int(byte_of(scb[(2 * sb + 1) >> 2], (2 * sb + 1) & 3) & 15u);
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const unsigned char *xr = xr0 + s * xtok + 32 * sb;
                    const u32x4 x0 = lds128(xr), x1 = lds128(xr + 16);
                    int p0 = sdot4(int(w[0]), int(x0.x), 0);
                    p0 = sdot4(int(w[1]), int(x0.y), p0);
                    p0 = sdot4(int(w[2]), int(x0.z), p0);
                    p0 = sdot4(int(w[3]), int(x0.w), p0);
                    int p1 = sdot4(int(w[4]), int(x1.x), 0);
                    p1 = sdot4(int(w[5]), int(x1.y), p1);
                    p1 = sdot4(int(w[6]), int(x1.z), p1);
                    p1 = sdot4(int(w[7]), int(x1.w), p1);
                    mainI[s] += sc0 * p0 + sc1 * p1;
                }
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const uint32_t *bsp = reinterpret_cast<const uint32_t *>(xr0 + s * xtok + XB_BS);
            int m = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t sc2 = (scb[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;  // scale bytes 2i, 2i+1
                const uint32_t mp = ((sc2 >> 4) & 0xFu) | (((sc2 >> 12) & 0xFu) << 16);
                const uint32_t bp = bsp[i];
                m += int((mp & 0xFFFFu)) * int(int16_t(bp & 0xFFFFu)) + int(mp >> 16) * int(int16_t(bp >> 16));
            }
            minI[s] = m;
            if (dbg) {
                dbg[s * dbg_tok] = mainI[s];
                dbg[s * dbg_tok + 1] = minI[s];
            }
            const float d8 = *reinterpret_cast<const float *>(xr0 + s * xtok + XB_D);
            val[s] = d8 * (d * float(mainI[s]) - dmin * float(minI[s]));
        }
    }
};

// Q8_0, one unit (8 blocks of 34 B) per lane: value = sum_blk (d_w*d8) * isum
// (reference SIMDMatMulVecAVX2.cpp:4339-4366).
template <int S>
struct TDot<kQ8_0, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               float *val, int32_t *dbg, size_t dbg_tok) {
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0.0f;
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {  // block pairs (68 B, 4-byte aligned)
            const uint32_t *w = reinterpret_cast<const uint32_t *>(u + 68 * pr);
            uint32_t wd[17];
#pragma unroll
            for (int k = 0; k < 17; ++k) wd[k] = w[k];
            uint32_t q0[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) q0[k] = align2(wd[k + 1], wd[k], 2);
            const float dw0 = h2f(wd[0] & 0xFFFFu), dw1 = h2f(wd[8] >> 16);
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const unsigned char *xr = xr0 + s * xtok;
                const u32x4 x0 = lds128(xr + 64 * pr), x1 = lds128(xr + 64 * pr + 16);
                const u32x4 x2 = lds128(xr + 64 * pr + 32), x3 = lds128(xr + 64 * pr + 48);
                const uint32_t xa[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                const uint32_t xb[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
                int s0 = 0, s1 = 0;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    s0 = sdot4(int(q0[k]), int(xa[k]), s0);
                    s1 = sdot4(int(wd[9 + k]), int(xb[k]), s1);
                }
                if (dbg) {
                    dbg[s * dbg_tok + 2 * pr] = s0;
                    dbg[s * dbg_tok + 2 * pr + 1] = s1;
                }
                const float2 d8 = *reinterpret_cast<const float2 *>(xr + XB_BS + 8 * pr);
                acc[s] += (dw0 * d8.x) * float(s0) + (dw1 * d8.y) * float(s1);
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) val[s] = acc[s];
    }
};

// Q6_K, one unit (210 B, 2-byte aligned in LDS) per lane: 6-bit weights q
// (ql low nibbles | qh 2-bit highs), isum = sum_g sc_g * (sum_16 q*x -
// 32*bsum_g) exactly (the -32 folded through the bsums as the reference does,
// SIMDMatMulVecAVX2.cpp:4636-4667); value = (d*d8) * isum.
template <int S>
struct TDot<kQ6_K, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               float *val, int32_t *dbg, size_t dbg_tok) {
        const u32x4 scv = lds128(u + 192);
        const int8_t *sc = reinterpret_cast<const int8_t *>(u + 192);
        (void)scv;
        int tot[S];
#pragma unroll
        for (int s = 0; s < S; ++s) tot[s] = 0;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {  // 16-element halves of each 32-run
                const u32x4 la = lds128(u + 64 * n + 16 * h), lb = lds128(u + 64 * n + 32 + 16 * h);
                const u32x4 hv = lds128(u + 128 + 32 * n + 16 * h);
                const uint32_t LA[4] = {la.x, la.y, la.z, la.w}, LB[4] = {lb.x, lb.y, lb.z, lb.w};
                const uint32_t HV[4] = {hv.x, hv.y, hv.z, hv.w};
                uint32_t q[4][4];  // [k][dword]: elements 128n + 32k + 16h + 4j
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    q[0][j] = (LA[j] & 0x0F0F0F0Fu) | ((HV[j] << 4) & 0x30303030u);
                    q[1][j] = (LB[j] & 0x0F0F0F0Fu) | ((HV[j] << 2) & 0x30303030u);
                    q[2][j] = ((LA[j] >> 4) & 0x0F0F0F0Fu) | (HV[j] & 0x30303030u);
                    q[3][j] = ((LB[j] >> 4) & 0x0F0F0F0Fu) | ((HV[j] >> 2) & 0x30303030u);
                }
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const unsigned char *xr = xr0 + s * xtok;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int g = 8 * n + 2 * k + h;  // sub-block of 16
                        const u32x4 xv = lds128(xr + 128 * n + 32 * k + 16 * h);
                        int p = sdot4(int(q[k][0]), int(xv.x), 0);
                        p = sdot4(int(q[k][1]), int(xv.y), p);
                        p = sdot4(int(q[k][2]), int(xv.z), p);
                        p = sdot4(int(q[k][3]), int(xv.w), p);
                        const int bs = int(reinterpret_cast<const int16_t *>(xr + XB_BS)[g]);
                        tot[s] += int(sc[g]) * (p - 32 * bs);
                    }
                }
            }
        }
        const float d = h2f(uint32_t(u[208]) | (uint32_t(u[209]) << 8));
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (dbg) dbg[s * dbg_tok] = tot[s];
            const float d8 = *reinterpret_cast<const float *>(xr0 + s * xtok + XB_D);
            val[s] = (d * d8) * float(tot[s]);
        }
    }
};

// IQ3_XXS, one unit (98 B, 2-byte aligned in LDS) per lane: per 32-run ib,
// 8 grid indices (4 bytes of magnitudes each, codebook in LDS) and 4 7-bit
// sign indices (sign byte = idx | parity(idx) << 7) in aux = sas[ib], scale
// 2*(aux >> 28) + 1; isum = sum_ib (2ls+1) * sum_32 w*x; value = (d*d8) *
// isum, and the row is scaled by 0.25 at the end (reference
// include/GGMLDequantize.hpp:2064-2097, :2148).
template <int S>
struct TDot<kIQ3_XXS, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               const uint32_t *sgrid, float *val, int32_t *dbg, size_t dbg_tok) {
        const uint16_t *u16 = reinterpret_cast<const uint16_t *>(u);
        int tot[S];
#pragma unroll
        for (int s = 0; s < S; ++s) tot[s] = 0;
        // The codebook lookups of IB 32-runs are issued before their dot
        // products, so that several LDS round trips overlap (gate/up pair
        // 18944x3584: 20.2 -> 19.6 us with 4; 2 and 8 measured no better).
        constexpr int IB = 4;
#pragma unroll
        for (int ib0 = 0; ib0 < 8; ib0 += IB) {
            uint32_t w[IB][8];
            uint32_t auxs[IB];
#pragma unroll
            for (int i = 0; i < IB; ++i) {
                const int ib = ib0 + i;
                const uint32_t aux = uint32_t(u16[33 + 2 * ib]) | (uint32_t(u16[34 + 2 * ib]) << 16);
                const uint32_t gi0 = uint32_t(u16[1 + 4 * ib]) | (uint32_t(u16[2 + 4 * ib]) << 16);
                const uint32_t gi1 = uint32_t(u16[3 + 4 * ib]) | (uint32_t(u16[4 + 4 * ib]) << 16);
                auxs[i] = aux;
#pragma unroll
                for (int l = 0; l < 4; ++l) {
                    const uint32_t idx7 = (aux >> (7 * l)) & 127u;
                    const uint32_t s8 = idx7 | ((__builtin_popcount(idx7) & 1u) << 7);
                    const uint32_t gw = l < 2 ? gi0 : gi1;
                    // signed-grid entries (16 * index + sign nibble)
                    w[i][2 * l] = sgrid[((gw >> (16 * (l & 1))) & 0xFF) * 16 + (s8 & 15u)];
                    w[i][2 * l + 1] = sgrid[((gw >> (16 * (l & 1) + 8)) & 0xFF) * 16 + (s8 >> 4)];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < IB; ++i) {
                const int ib = ib0 + i;
                const int mult = 2 * int(auxs[i] >> 28) + 1;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const unsigned char *xr = xr0 + s * xtok + 32 * ib;
                    const u32x4 x0 = lds128(xr), x1 = lds128(xr + 16);
                    int p = sdot4(int(w[i][0]), int(x0.x), 0);
                    p = sdot4(int(w[i][1]), int(x0.y), p);
                    p = sdot4(int(w[i][2]), int(x0.z), p);
                    p = sdot4(int(w[i][3]), int(x0.w), p);
                    p = sdot4(int(w[i][4]), int(x1.x), p);
                    p = sdot4(int(w[i][5]), int(x1.y), p);
                    p = sdot4(int(w[i][6]), int(x1.z), p);
                    p = sdot4(int(w[i][7]), int(x1.w), p);
                    tot[s] += mult * p;
                }
            }
        }
        const float d = h2f(u16[0]);
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (dbg) dbg[s * dbg_tok] = tot[s];
            const float d8 = *reinterpret_cast<const float *>(xr0 + s * xtok + XB_D);
            val[s] = (d * d8) * float(tot[s]);
        }
    }
};

// IQ3_S, one unit (110 B, 2-byte aligned in LDS) per lane: per 32-run ib,
// 8 grid indices (qs bytes with bit 8 from qh[ib]; codebook of 512 words in
// LDS), 8 sign bits per 8 weights (applied bytewise as a two's-complement
// negation; magnitudes are at most 15, so no byte carries), scale 2*ls+1 from
// the nibble of scales[ib/2]; isum = sum_ib (2ls+1) * sum_32 w*x; value =
// (d*d8) * isum (include/GGMLDequantize.hpp:2102-2145).
template <int S>
struct TDot<kIQ3_S, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               const uint32_t *grid, float *val, int32_t *dbg, size_t dbg_tok) {
        const uint16_t *u16 = reinterpret_cast<const uint16_t *>(u);
        const uint32_t scw = uint32_t(u16[53]) | (uint32_t(u16[54]) << 16);
        int tot[S];
#pragma unroll
        for (int s = 0; s < S; ++s) tot[s] = 0;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            const uint32_t g0 = uint32_t(u16[1 + 4 * ib]) | (uint32_t(u16[2 + 4 * ib]) << 16);
            const uint32_t g1 = uint32_t(u16[3 + 4 * ib]) | (uint32_t(u16[4 + 4 * ib]) << 16);
            const uint32_t sw = uint32_t(u16[37 + 2 * ib]) | (uint32_t(u16[38 + 2 * ib]) << 16);
            const uint32_t qhb = (uint32_t(u16[33 + ib / 2]) >> (8 * (ib & 1))) & 0xFFu;
            uint32_t w[8];
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const uint32_t gw = l < 2 ? g0 : g1;
                const uint32_t i1 = byte_of(gw, 2 * (l & 1)) | ((qhb << (8 - 2 * l)) & 256u);
                const uint32_t i2 = byte_of(gw, 2 * (l & 1) + 1) | ((qhb << (7 - 2 * l)) & 256u);
                const uint32_t sb = byte_of(sw, l);
                const uint32_t m1 = spread_sign4(sb & 15u), m2 = spread_sign4(sb >> 4);
                w[2 * l] = (grid[i1] ^ m1) + (m1 & 0x01010101u);
                w[2 * l + 1] = (grid[i2] ^ m2) + (m2 & 0x01010101u);
            }
            const int mult = 2 * int((scw >> (4 * ib)) & 15u) + 1;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const unsigned char *xr = xr0 + s * xtok + 32 * ib;
                const u32x4 x0 = lds128(xr), x1 = lds128(xr + 16);
                int p = sdot4(int(w[0]), int(x0.x), 0);
                p = sdot4(int(w[1]), int(x0.y), p);
                p = sdot4(int(w[2]), int(x0.z), p);
                p = sdot4(int(w[3]), int(x0.w), p);
                p = sdot4(int(w[4]), int(x1.x), p);
                p = sdot4(int(w[5]), int(x1.y), p);
                p = sdot4(int(w[6]), int(x1.z), p);
                p = sdot4(int(w[7]), int(x1.w), p);
                tot[s] += mult * p;
            }
        }
        const float d = h2f(u16[0]);
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (dbg) dbg[s * dbg_tok] = tot[s];
            const float d8 = *reinterpret_cast<const float *>(xr0 + s * xtok + XB_D);
            val[s] = (d * d8) * float(tot[s]);
        }
    }
};

// IQ2_S, one unit (82 B, 2-byte aligned in LDS) per lane: per 8 weights one
// codebook entry of 8 magnitudes (index qs byte | 2 bits of qh[ib], codebook
// of 1024 x 8 bytes in LDS), 8 sign bits applied bytewise as a two's-
// complement negation (magnitudes 8..43, no carries), scale 1+2*ls per 16
// from the nibbles of scales[ib]; isum = sum_ib ls1*sum_16 + ls2*sum_16;
// value = (d*d8) * isum, and the row is scaled by 0.125 at the end
// (include/GGMLDequantize.hpp:2028-2057, :2148-2159).
template <int S>
struct TDot<kIQ2_S, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               const uint32_t *grid, float *val, int32_t *dbg, size_t dbg_tok) {
        const uint16_t *u16 = reinterpret_cast<const uint16_t *>(u);
        int tot[S];
#pragma unroll
        for (int s = 0; s < S; ++s) tot[s] = 0;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            const uint32_t gw = uint32_t(u16[1 + 2 * ib]) | (uint32_t(u16[2 + 2 * ib]) << 16);
            const uint32_t sw = uint32_t(u16[17 + 2 * ib]) | (uint32_t(u16[18 + 2 * ib]) << 16);
            const uint32_t qhb = (uint32_t(u16[33 + ib / 2]) >> (8 * (ib & 1))) & 0xFFu;
            const uint32_t scb = (uint32_t(u16[37 + ib / 2]) >> (8 * (ib & 1))) & 0xFFu;
            uint32_t w[8];
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const uint32_t idx = byte_of(gw, l) | ((qhb << (8 - 2 * l)) & 0x300u);
                const uint32_t sb = byte_of(sw, l);
                const uint32_t m1 = spread_sign4(sb & 15u), m2 = spread_sign4(sb >> 4);
                w[2 * l] = (grid[2 * idx] ^ m1) + (m1 & 0x01010101u);
                w[2 * l + 1] = (grid[2 * idx + 1] ^ m2) + (m2 & 0x01010101u);
            }
            const int ls1 = 1 + 2 * int(scb & 15u), ls2 = 1 + 2 * int(scb >> 4);
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const unsigned char *xr = xr0 + s * xtok + 32 * ib;
                const u32x4 x0 = lds128(xr), x1 = lds128(xr + 16);
                int p1 = sdot4(int(w[0]), int(x0.x), 0);
                p1 = sdot4(int(w[1]), int(x0.y), p1);
                p1 = sdot4(int(w[2]), int(x0.z), p1);
                p1 = sdot4(int(w[3]), int(x0.w), p1);
                int p2 = sdot4(int(w[4]), int(x1.x), 0);
                p2 = sdot4(int(w[5]), int(x1.y), p2);
                p2 = sdot4(int(w[6]), int(x1.z), p2);
                p2 = sdot4(int(w[7]), int(x1.w), p2);
                tot[s] += ls1 * p1 + ls2 * p2;
            }
        }
        const float d = h2f(u16[0]);
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (dbg) dbg[s * dbg_tok] = tot[s];
            const float d8 = *reinterpret_cast<const float *>(xr0 + s * xtok + XB_D);
            val[s] = (d * d8) * float(tot[s]);
        }
    }
};

// IQ4_XS, one unit (136 B, 8-byte aligned in LDS) per lane: d at 0, 16 bits
// of scale high parts at 2, scale low nibbles at 4, 128 nibble bytes at 8.
// Sub-block ib (32 weights): ls = low nibble ib | high bits 2ib << 4, scale
// ls - 32; weight j < 16 is kvalues[low nibble of byte 16ib + j], j >= 16
// kvalues[high nibble of byte 16ib + j - 16] (include/GGMLDequantize.hpp:
// 1044-1080). Four nibbles become four table bytes with three v_perm_b32:
// the entries 0-7 and 8-15 by the nibble's low 3 bits, then a per-byte pick
// by bit 3. value = d*d8*sum_ib (ls-32)*sum_32 w*q8, exact in int32 (the
// reference kernel, SIMDMatMulVecAVX2.cpp:3988-4119, rounds per 32 in fp32).
__device__ __forceinline__ uint32_t iq4nl_lut(uint32_t n) {
    // kvalues_iq4nl (include/GGMLDequantize.hpp:55-57) as four words of bytes
    constexpr uint32_t T0 = 0xBFAD9881u, T1 = 0xF6EADDCFu, T2 = 0x26190D01u, T3 = 0x71594535u;
    const uint32_t lo3 = n & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(T1, T0, lo3), b = __builtin_amdgcn_perm(T3, T2, lo3);
    return __builtin_amdgcn_perm(b, a, ((n >> 1) & 0x04040404u) | 0x03020100u);
}

template <int S>
struct TDot<kIQ4_XS, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               float *val, int32_t *dbg, size_t dbg_tok) {
        const uint32_t *u32 = reinterpret_cast<const uint32_t *>(u);
        const uint32_t h0 = u32[0], sl = u32[1];
        int tot[S];
#pragma unroll
        for (int s = 0; s < S; ++s) tot[s] = 0;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            uint32_t w[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t q = u32[2 + 4 * ib + k];
                w[k] = iq4nl_lut(q & 0x0F0F0F0Fu);
                w[4 + k] = iq4nl_lut((q >> 4) & 0x0F0F0F0Fu);
            }
            const int ls = int(((sl >> (4 * ib)) & 15u) | (((h0 >> (16 + 2 * ib)) & 3u) << 4)) - 32;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const unsigned char *xr = xr0 + s * xtok + 32 * ib;
                const u32x4 x0 = lds128(xr), x1 = lds128(xr + 16);
                int p = sdot4(int(w[0]), int(x0.x), 0);
                p = sdot4(int(w[1]), int(x0.y), p);
                p = sdot4(int(w[2]), int(x0.z), p);
                p = sdot4(int(w[3]), int(x0.w), p);
                p = sdot4(int(w[4]), int(x1.x), p);
                p = sdot4(int(w[5]), int(x1.y), p);
                p = sdot4(int(w[6]), int(x1.z), p);
                p = sdot4(int(w[7]), int(x1.w), p);
                tot[s] += ls * p;
            }
        }
        const float d = h2f(h0 & 0xFFFFu);
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (dbg) dbg[s * dbg_tok] = tot[s];
            const float d8 = *reinterpret_cast<const float *>(xr0 + s * xtok + XB_D);
            val[s] = (d * d8) * float(tot[s]);
        }
    }
};

// IQ4_NL, one unit (8 blocks of 18 B: d, then 16 nibble bytes; 144 B, so
// 16-byte aligned in LDS) per lane, on fp32 x (the reference's CPU kernel for
// this type, matMulVecBatchIQ4NL_Q8K_AVX2, SIMDMatMulVecAVX2.cpp:4126-4200,
// dots unquantized x). Table bytes as in IQ4_XS; per block the reference's
// order: 8 lanes of a 4-deep fma chain over elements l, 8+l, 16+l, 24+l,
// reduced ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)), then fma(d, sum, acc). The
// unit's value chains its 8 blocks from 0, so a row differs from the
// reference's one chain over all blocks by fp32 summation order only.
template <int S>
struct TDot<kIQ4_NL, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               float *val, int32_t *dbg, size_t dbg_tok) {
        (void)dbg;
        (void)dbg_tok;
        const uint32_t *u32 = reinterpret_cast<const uint32_t *>(u);
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0.0f;
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {  // block pairs: 36 B = 9 dwords
            uint32_t wd[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) wd[k] = u32[9 * pr + k];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int blk = 2 * pr + h;
                uint32_t q[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) q[k] = h == 0 ? align2(wd[k + 1], wd[k], 2) : wd[5 + k];
                const float d = h2f(h == 0 ? (wd[0] & 0xFFFFu) : (wd[4] >> 16));
                uint32_t wt[8];  // table bytes of elements 4k.. (k < 4: low nibbles) and 16 + 4(k-4).. (high)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    wt[k] = iq4nl_lut(q[k] & 0x0F0F0F0Fu);
                    wt[4 + k] = iq4nl_lut((q[k] >> 4) & 0x0F0F0F0Fu);
                }
                float w[32];
#pragma unroll
                for (int e = 0; e < 32; ++e) w[e] = float(int8_t(uint8_t(wt[e >> 2] >> (8 * (e & 3)))));
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const float4 *xp = reinterpret_cast<const float4 *>(xr0 + s * xtok) + 8 * blk;
                    float x[32];
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const float4 v = xp[c];
                        x[4 * c] = v.x;
                        x[4 * c + 1] = v.y;
                        x[4 * c + 2] = v.z;
                        x[4 * c + 3] = v.w;
                    }
                    float v[8];
#pragma unroll
                    for (int l = 0; l < 8; ++l) {
                        float t = w[l] * x[l];
                        t = fmaf(w[8 + l], x[8 + l], t);
                        t = fmaf(w[16 + l], x[16 + l], t);
                        v[l] = fmaf(w[24 + l], x[24 + l], t);
                    }
                    const float sum = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
                    acc[s] = fmaf(d, sum, acc[s]);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) val[s] = acc[s];
    }
};

// Q5_0, one unit (8 blocks of 22 B: d, 32 high bits, 16 nibble bytes; 176 B,
// so 16-byte aligned in LDS) per lane, on fp32 x (the reference's CPU path
// for this type, dotProductQ5_0, include/GGMLDequantize.hpp:1820-1836, dots
// unquantized x). Weight j < 16 is the low nibble of byte j with bit j of the
// high bits as bit 4, weight 16 + j the high nibble with bit 16 + j; value
// q - 16. Per block d * sum(x * (q - 16)) in fp32 (the reference sums in
// double), the unit's 8 blocks added in order.
template <int S>
struct TDot<kQ5_0, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               float *val, int32_t *dbg, size_t dbg_tok) {
        (void)dbg;
        (void)dbg_tok;
        const uint32_t *u32 = reinterpret_cast<const uint32_t *>(u);
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0.0f;
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {  // block pairs: 44 B = 11 dwords
            uint32_t wd[11];
#pragma unroll
            for (int k = 0; k < 11; ++k) wd[k] = u32[11 * pr + k];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int blk = 2 * pr + h;
                uint32_t q[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) q[k] = h == 0 ? align2(wd[k + 2], wd[k + 1], 2) : wd[7 + k];
                const uint32_t qh = h == 0 ? align2(wd[1], wd[0], 2) : wd[6];
                const float d = h2f(h == 0 ? (wd[0] & 0xFFFFu) : (wd[5] >> 16));
                // bytes 0..31 of the block's weights: w[k] elements 4k.., w[4+k] 16+4k..
                uint32_t wb[8];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t lo = (qh >> (4 * k)) & 15u, hi = (qh >> (16 + 4 * k)) & 15u;
                    wb[k] = (q[k] & 0x0F0F0F0Fu) | (((lo * 0x00204081u) & 0x01010101u) << 4);
                    wb[4 + k] = ((q[k] >> 4) & 0x0F0F0F0Fu) | (((hi * 0x00204081u) & 0x01010101u) << 4);
                }
                float w[32];
#pragma unroll
                for (int e = 0; e < 32; ++e) w[e] = float(int((wb[e >> 2] >> (8 * (e & 3))) & 0xFFu) - 16);
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const float4 *xp = reinterpret_cast<const float4 *>(xr0 + s * xtok) + 8 * blk;
                    float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const float4 a = xp[c], b = xp[4 + c];
                        p0 = fmaf(a.x, w[4 * c], p0);
                        p0 = fmaf(a.y, w[4 * c + 1], p0);
                        p0 = fmaf(a.z, w[4 * c + 2], p0);
                        p0 = fmaf(a.w, w[4 * c + 3], p0);
                        p1 = fmaf(b.x, w[16 + 4 * c], p1);
                        p1 = fmaf(b.y, w[16 + 4 * c + 1], p1);
                        p1 = fmaf(b.z, w[16 + 4 * c + 2], p1);
                        p1 = fmaf(b.w, w[16 + 4 * c + 3], p1);
                    }
                    acc[s] = fmaf(d, p0 + p1, acc[s]);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) val[s] = acc[s];
    }
};

// IQ2_XS, one unit (74 B, 2-byte aligned in LDS) per lane, on fp32 x (the
// reference's CPU path for this type, dotProductIQ2_XS, dots unquantized x;
// include/GGMLDequantize.hpp:1901-1927): per 8 weights one 16-bit entry --
// codebook index (bits 0-8, 512 x 8 bytes in LDS) and a 7-bit sign index whose
// 8th sign is its parity --, weight = ((d*(0.5+ls))*0.25) * magnitude with the
// sign applied to the float's sign bit; the scale is applied once per 8
// weights (value = sum of dl * sum_8 x * signed magnitude), which rounds
// differently from the reference's per-weight products only in fp32 order.
template <int S>
struct TDot<kIQ2_XS, S> {
    __device__ __forceinline__ static void run(const unsigned char *u, const unsigned char *xr0, size_t xtok,
                                               const uint32_t *grid, float *val, int32_t *dbg, size_t dbg_tok) {
        (void)dbg;
        (void)dbg_tok;
        const uint16_t *u16 = reinterpret_cast<const uint16_t *>(u);
        const float d = h2f(u16[0]);
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0.0f;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            const uint32_t scb = (uint32_t(u16[33 + ib / 2]) >> (8 * (ib & 1))) & 0xFFu;
            const float dl0 = d * (0.5f + float(scb & 15u)) * 0.25f;
            const float dl1 = d * (0.5f + float(scb >> 4)) * 0.25f;
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const uint32_t q = u16[1 + 4 * ib + l];
                const uint32_t si = q >> 9;
                const uint32_t sg = si | ((__builtin_popcount(si) & 1u) << 7);
                const uint32_t g0 = grid[2 * (q & 511u)], g1 = grid[2 * (q & 511u) + 1];
                const float dl = l < 2 ? dl0 : dl1;
                // signed magnitudes (the scale dl is applied once per 8 weights)
                float w[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t gb = ((j < 4 ? g0 : g1) >> (8 * (j & 3))) & 0xFFu;
                    w[j] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, float(gb)) ^ (((sg >> j) & 1u) << 31));
                }
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const float *xp = reinterpret_cast<const float *>(xr0 + s * xtok) + 32 * ib + 8 * l;
                    const float4 xa = *reinterpret_cast<const float4 *>(xp);
                    const float4 xb = *reinterpret_cast<const float4 *>(xp + 4);
                    float p = xa.x * w[0];
                    p = fmaf(xa.y, w[1], p);
                    p = fmaf(xa.z, w[2], p);
                    p = fmaf(xa.w, w[3], p);
                    p = fmaf(xb.x, w[4], p);
                    p = fmaf(xb.y, w[5], p);
                    p = fmaf(xb.z, w[6], p);
                    p = fmaf(xb.w, w[7], p);
                    acc[s] = fmaf(dl, p, acc[s]);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) val[s] = acc[s];
    }
};

// ONE: a single-job launch (on fp32 x, without expert ids in the plain
// form), whose first-needed descriptor fields arrive as preloaded arguments.
template <int TYPE, int S, bool DBG, class C, bool RG = false, bool KEEP = false, bool ONE = false>
__global__ __launch_bounds__(C::NT) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_gemv_t(
    // Leading scalar arguments, built with kernarg preloading so that they
    // arrive in SGPRs at wave start. One-job launches (ONE): job 0's
    // first-needed fields (x, W, W2 as bits, cols, tokens, rows, rows per
    // workgroup, units per row), so the activation and weight loads issue
    // without waiting for a kernel-argument fetch. Other launches: the first
    // workgroup of jobs 1..5 in p_a..p_e and of jobs 6, 7 in the two halves of
    // p_w2 (~0u past the last job), so a workgroup finds its job without a
    // fetch and loads only that job's descriptor.
    const float *p_x, const uint8_t *p_W, uint64_t p_w2, uint32_t p_a, uint32_t p_b, uint32_t p_c, uint32_t p_d,
    uint32_t p_e, TLaunchArgs L) {
    constexpr int TNT = C::NT, TNW = TNT / 64;
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char *xr = smem;
    constexpr uint32_t UB = unit_bytes(TYPE);
    constexpr uint32_t TILE_BYTES = kTileUnits * UB;
    constexpr int NX = tile_dwordx4(TYPE);  // 16-byte loads per lane per tile
    constexpr int D = tile_depth<C>(TYPE, S);
    // The wave index is read as a scalar so that the tile schedule, the
    // descriptor choice and the buffer offsets stay in SGPRs.
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    unsigned char *tile = smem + L.off_t + wave * tile_slot_bytes(TYPE);
    float *spart = reinterpret_cast<float *>(smem + L.off_p);

    uint32_t j = 0;
    if constexpr (!ONE) {
        static_assert(kMaxJobs == 8, "job starts in the leading arguments");
        const uint32_t wgb[7] = {p_a, p_b, p_c, p_d, p_e, uint32_t(p_w2), uint32_t(p_w2 >> 32)};
#pragma unroll
        for (int k = 1; k < kMaxJobs; ++k)
            if (blockIdx.x >= wgb[k - 1]) j = k;
    }
    TJobDev jb = L.jobs[j];
    if constexpr (ONE && !KEEP && !RG) {
        jb.x = p_x;
        jb.W = p_W;
        jb.W2 = reinterpret_cast<const uint8_t *>(p_w2);
        jb.cols = p_a;
        jb.nx = p_b;
        jb.rows = p_c;
        jb.rows_per_wg = p_d;
        jb.nu = p_e;
        jb.wg_begin = 0;
        jb.act = ActView{};  // fp32 x: no pre-quantized activations (the host picks this variant only then)
    }
    uint32_t lw = blockIdx.x - jb.wg_begin;
    bool no_expert = false;
    // Expert ids are loaded here and first used after the activation loads
    // are issued, so their latency overlaps the activations'.
    int32_t eid = 0;                // expert-pair mode: this pair's expert
    typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
    i32x8 reid = {-1, -1, -1, -1, -1, -1, -1, -1};  // rank-group mode: this token's experts (-1 past rk)
    const float *rwts = nullptr;
    // (the plain one-job launches have no expert ids)
    if (!(ONE && !KEEP && !RG) && jb.ids != nullptr) {
        const uint32_t p = lw / jb.wg_per_pair;
        lw -= p * jb.wg_per_pair;
        if constexpr (!RG) {
            eid = jb.ids[p];
            jb.x += size_t(p / jb.x_div) * jb.x_stride;
        } else {
            const int32_t *rids = jb.ids + size_t(p) * jb.rk;
            static_for<0, 8>([&](auto k) __attribute__((always_inline)) {
                constexpr uint32_t K = decltype(k)::value;
                const int32_t v = rids[K < jb.rk ? K : 0];  // always in bounds
                reid[K] = K < jb.rk ? v : -1;
            });
            rwts = jb.wts + size_t(p) * jb.rk;
            jb.x += size_t(p) * jb.x_stride;
        }
        jb.out += size_t(p) * jb.out_stride;
        if (jb.out2 != nullptr) jb.out2 += size_t(p) * jb.out_stride;
    }
    const uint32_t nu = jb.nu;
    // matrices per workgroup: 2 for a gate/up pair, rk in rank-group mode
    const uint32_t pairs = RG ? jb.rk : jb.W2 != nullptr ? 2 : 1;
    const uint32_t r0 = lw * jb.rows_per_wg;
    const uint32_t nr = min(jb.rows_per_wg, jb.rows - r0);
    const uint32_t per_mat = nr * nu;
    const uint32_t ntiles_mat = (per_mat + kTileUnits - 1) / kTileUnits;
    const uint32_t ntiles = ntiles_mat * pairs;
    const size_t nbr = TYPE == kQ8_0 ? jb.cols / 32 : jb.cols / 256;
    const size_t per = TYPE == kQ4_K || TYPE == kQ5_K ? 8 : TYPE == kQ2_K ? 2 : 1;
    const size_t dbg_tok = size_t(jb.rows) * nbr * per;
    const size_t xtok = size_t(nu) * xrec_bytes(TYPE);
    // Expert of rank m (rank-group mode; m is wave-uniform).
    auto rank_expert = [&](uint32_t m) __attribute__((always_inline)) {
        int32_t e = reid[0];
        static_for<1, 8>([&](auto k) __attribute__((always_inline)) {
            e = m == uint32_t(decltype(k)::value) ? reid[decltype(k)::value] : e;
        });
        return e;
    };
    // Matrix of tile t (0 or 1 for a pair, the rank in rank-group mode).
    auto mat_of = [&](uint32_t t) __attribute__((always_inline)) {
        uint32_t m = 0;
#pragma unroll
        for (int k = 1; k < 8; ++k) m += t >= uint32_t(k) * ntiles_mat ? 1u : 0u;
        return m;
    };


    // Register ring: the wave's tiles are t = wave, wave+TNW, ...; slot i holds
    // tile k (k mod D == i) from its load until it is copied to the wave's LDS
    // buffer, after which the slot refills with tile k+D. D-1 tiles stay in
    // flight while one is decoded. Copies and refills are unconditional so
    // every path issues the same loads and the in-order vmcnt bookkeeping never
    // drains at a control-flow join. (A dynamic schedule -- waves taking tiles
    // from an LDS counter -- measured no faster: a workgroup finishes when its
    // last bytes arrive, whichever wave decodes them.)
    const uint32_t nmine = wave < ntiles ? (ntiles - wave + TNW - 1) / TNW : 0;
    // IQ3_XXS grid words, requested ahead of everything else
    uint32_t gword = 0;
    if constexpr (TYPE == kIQ3_XXS) gword = c_grid[tid & 255];
    const XRsrc xrs = tstage_rsrc<TYPE, S>(jb);
    const XPre xp = tstage_preload<TYPE, S, TNT>(jb, xrs);
    // Every wave's activation loads enter the CU's memory queue before any
    // wave's weight loads (a barrier without a memory fence: it does not wait
    // for the loads).
    __builtin_amdgcn_s_barrier();
    if constexpr (!RG) {
        if (!(ONE && !KEEP && !RG) && jb.ids != nullptr) {
            no_expert = eid < 0 || uint32_t(eid) >= jb.n_experts;
            const uint64_t off = no_expert ? 0 : uint64_t(eid) * jb.wstride;
            jb.W += off;
            if (jb.W2 != nullptr) jb.W2 += off;
        }
    }
    // Descriptors over exactly this workgroup's rows of each matrix.
    const uint8_t *const wbase1 = jb.W + size_t(r0) * nu * UB;
    const uint8_t *const wbase2 = (jb.W2 != nullptr ? jb.W2 : jb.W) + size_t(r0) * nu * UB;
    Regs<D * NX> buf;
    // Loads past the workgroup's tiles (the ring's last refills) go through a
    // descriptor of size 0, and lanes past a partial tile's end carry a
    // per-lane offset beyond the range: both return zeros and touch no memory.
    // (The range check covers the per-lane offset, not the scalar one, so the
    // scalar offset never carries an out-of-range marker.)
    auto ld = [&](auto i, uint32_t t) __attribute__((always_inline)) {
        bool live = t < ntiles;
        const uint8_t *base;
        uint32_t tt;
        if constexpr (!RG) {
            const bool second = t >= ntiles_mat;
            tt = second ? t - ntiles_mat : t;
            base = second ? wbase2 : wbase1;
        } else {
            const uint32_t m = live ? mat_of(t) : 0u;
            tt = t - m * ntiles_mat;
            const int32_t e = rank_expert(m);
            live = live && e >= 0 && uint32_t(e) < jb.n_experts;
            base = wbase1 + (live ? uint64_t(e) * jb.wstride : 0);
        }
        const uint32_t soff = live ? tt * TILE_BYTES : 0u;
        // whole dwords: the range check zeroes a dword only partly in range,
        // and 2-byte-aligned units end 2 bytes into one when a workgroup's
        // unit count is odd (the matrix's last dword stays in its last page)
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, live ? (per_mat * UB + 3u) & ~3u : 0u);
        static_for<0, NX>([&](auto c) __attribute__((always_inline)) {
            uint32_t voff = lane * 16 + c.value * 1024;
            if constexpr (c.value == NX - 1 && TILE_BYTES % 1024 != 0) voff = voff < TILE_BYTES ? voff : 0x80000000u;
            reg<decltype(i)::value * NX + c.value>(buf) = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, KEEP ? 0 : kWeightCachePolicy);
        });
    };
    // Staged ring: D0 slots are requested before the activations are
    // quantized, the rest after. A short memory queue at kernel start lets
    // the activation loads (which miss in L2: every launch streams the
    // weights through it) return in about one unloaded latency; the full
    // depth then keeps HBM busy for the rest of the stream.
    constexpr int D0 = 1;
    static_for<0, D0>([&](auto i) __attribute__((always_inline)) { ld(i, wave + i.value * TNW); });
    if constexpr (TYPE == kIQ3_XXS) {
        // Signed grid: entry 16*i + n is grid[i] with the signs of the 4-bit
        // pattern n applied bytewise (n's bit k negates byte k).
        if (tid < 256) {
            u32x4 *sg = reinterpret_cast<u32x4 *>(smem + L.off_g + tid * 64);
            static_for<0, 4>([&](auto q) __attribute__((always_inline)) {
                uint32_t e[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t m = spread_sign4(4u * decltype(q)::value + j);
                    e[j] = (gword ^ m) + (m & 0x01010101u);  // grid bytes are nonzero: no carries
                }
                sg[decltype(q)::value] = u32x4{e[0], e[1], e[2], e[3]};
            });
        }
    }
    if constexpr (TYPE == kIQ3_S) {
        uint32_t *sg = reinterpret_cast<uint32_t *>(smem + L.off_g);
        for (uint32_t i = tid; i < 512; i += TNT) sg[i] = c_grid_s[i];
    }
    if constexpr (TYPE == kIQ2_S) {
        uint64_t *sg = reinterpret_cast<uint64_t *>(smem + L.off_g);
        for (uint32_t i = tid; i < 1024; i += TNT) sg[i] = c_grid_2s[i];
    }
    if constexpr (TYPE == kIQ2_XS) {
        uint64_t *sg = reinterpret_cast<uint64_t *>(smem + L.off_g);
        for (uint32_t i = tid; i < 512; i += TNT) sg[i] = c_grid_2xs[i];
    }
    tstage_finish<TYPE, S, TNT>(jb, xrs, xp, xr);
    static_for<D0, D>([&](auto i) __attribute__((always_inline)) { ld(i, wave + i.value * TNW); });
    __syncthreads();

    for (uint32_t k0 = 0; k0 < nmine; k0 += D) {
        static_for<0, D>([&](auto i) __attribute__((always_inline)) {
            const uint32_t kk = k0 + i.value;
            const uint32_t t = wave + kk * TNW;
            static_for<0, NX>([&](auto c) __attribute__((always_inline)) {
                *reinterpret_cast<u32x4 *>(tile + (c.value * 64 + lane) * 16) = reg<i.value * NX + c.value>(buf);
            });
            ld(i, t + D * TNW);
            if (kk < nmine) {
                const uint32_t m = RG ? mat_of(t) : t >= ntiles_mat ? 1u : 0u;
                const uint32_t um = (t - m * ntiles_mat) * kTileUnits + lane;
                if (um < per_mat) {
                    const uint32_t rl = div_fast(um, jb.nu_div);
                    const uint32_t b = um - rl * nu;
                    int32_t *dbg = nullptr;
                    if constexpr (DBG)
                        dbg = jb.dbg + (size_t(r0 + rl) * nbr + (TYPE == kQ8_0 ? size_t(b) * 8 : b)) * per;
                    float val[S];
                    // rank-group mode: tile of rank m against that rank's activations (S == 1)
                    const unsigned char *xb = xr + (RG ? size_t(m) * xtok : 0) + size_t(b) * xrec_bytes(TYPE);
                    if constexpr (TYPE == kIQ3_XXS || TYPE == kIQ3_S || TYPE == kIQ2_S || TYPE == kIQ2_XS)
                        TDot<TYPE, S>::run(tile + lane * UB, xb, xtok,
                                           reinterpret_cast<const uint32_t *>(smem + L.off_g), val, dbg, dbg_tok);
                    else
                        TDot<TYPE, S>::run(tile + lane * UB, xb, xtok, val, dbg, dbg_tok);
#pragma unroll
                    for (int s = 0; s < S; ++s) spart[((size_t(m) * S + s) * nr + rl) * nu + b] = val[s];
                }
            }
        });
    }
    __syncthreads();
    // Row sums: 4 lanes per (token, row), each summing a strided quarter of
    // the row's units, combined with DPP quad sums (fixed order).
    const uint32_t nout = S * nr;
    if constexpr (RG) {
        // rank-group mode: out = sum_k w_k * rowsum_k in rank order (as the
        // separate reference reduction, ModelMoE.cpp:990-1002)
        for (uint32_t o0 = 0; o0 < nr; o0 += TNT / 4) {
            const uint32_t o = o0 + tid / 4, q = tid & 3;
            const uint32_t rl = o < nr ? o : nr - 1;
            float acc = 0.0f;
            for (uint32_t k = 0; k < pairs; ++k) {
                const float *pg = spart + (size_t(k) * nr + rl) * nu;
                float g = 0.0f;
                for (uint32_t bb = q; bb < nu; bb += 4) g += pg[bb];
                g = quad_sum(g);
                if constexpr (TYPE == kIQ3_XXS) g = 0.25f * g;
                if constexpr (TYPE == kIQ2_S) g = 0.125f * g;
                const int32_t e = rank_expert(k);
                if (e < 0 || uint32_t(e) >= jb.n_experts) g = 0.0f;
                acc = fmaf(rwts[k], g, acc);
            }
            if (o < nr && q == 0) jb.out[r0 + rl] = acc;
        }
        return;
    }
    // A row's sum is a fixed tree that depends only on the row's unit count,
    // never on the launch shape, so every launch of a matrix gives the same
    // bits. Up to 16 units: 4 strided partials (units q, q+4, ... in order)
    // and their quad sum, 4 lanes per row. More: 16 strided partials, then
    // quads, then pairs of quads, on 16 lanes per row when the workgroup has
    // few rows (the down projection's 74 units per row then take 5 adds per
    // lane instead of 19), else on 4 lanes with 4 partials each.
    const bool p16 = nu > 16;
    const bool wide = p16 && nout * 16 <= uint32_t(TNT);
    const uint32_t lpr = wide ? 16u : 4u;
    for (uint32_t o0 = 0; o0 < nout; o0 += TNT / lpr) {
        const uint32_t o = o0 + tid / lpr, q = tid & (lpr - 1);
        const uint32_t oc = o < nout ? o : nout - 1;
        const uint32_t s = oc / nr, rl = oc - s * nr;
        auto row_sum = [&](const float *pr) __attribute__((always_inline)) {
            if (!p16) {
                float v = 0.0f;
                for (uint32_t bb = q; bb < nu; bb += 4) v += pr[bb];
                return quad_sum(v);
            }
            if (wide) {
                float v = 0.0f;
                for (uint32_t bb = q; bb < nu; bb += 16) v += pr[bb];
                v = quad_sum(v);
                v += __shfl_xor(v, 4);
                return v + __shfl_xor(v, 8);
            }
            float pj[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                float v = 0.0f;
                for (uint32_t bb = q + 4 * j; bb < nu; bb += 16) v += pr[bb];
                pj[j] = quad_sum(v);
            }
            return (pj[0] + pj[1]) + (pj[2] + pj[3]);
        };
        float g = row_sum(spart + (size_t(s) * nr + rl) * nu);
        float u = 0.0f;
        if (pairs == 2) u = row_sum(spart + ((size_t(S) + s) * nr + rl) * nu);
        if constexpr (TYPE == kIQ3_XXS) {
            g = 0.25f * g;
            u = 0.25f * u;
        }
        if constexpr (TYPE == kIQ2_S) {  // the row scale of the IQ2_S fused path (GGMLDequantize.hpp:2148-2159)
            g = 0.125f * g;
            u = 0.125f * u;
        }
        if (o < nout && q == 0) {
            if (pairs == 2) {
                if (no_expert) u = 0.0f;
                jb.out2[size_t(s) * jb.out_ld + r0 + rl] = u;
                if (jb.epi == 1) g = g / (1.0f + expf(-g)) * u;
            }
            // An out-of-range expert id contributes nothing (the reference skips it).
            jb.out[size_t(s) * jb.out_ld + r0 + rl] = no_expert ? 0.0f : g;
        }
    }
}

template <int TYPE, int S, bool DBG, class C, bool RG = false, bool KEEP = false, bool ONE = false>
hipError_t launch_tiled_sd(const TLaunchArgs &a, dim3 g, uint32_t lds, hipStream_t st) {
    // Dynamic LDS above 64 KB needs the per-kernel opt-in, once per process.
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_t<TYPE, S, DBG, C, RG, KEEP, ONE>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    const TJobDev &j0 = a.jobs[0];
    if constexpr (ONE) {
        k_gemv_t<TYPE, S, DBG, C, RG, KEEP, ONE><<<g, C::NT, lds, st>>>(
            j0.x, j0.W, uint64_t(reinterpret_cast<uintptr_t>(j0.W2)), j0.cols, j0.nx, j0.rows, j0.rows_per_wg, j0.nu, a);
    } else {
        uint32_t w[7];
        for (uint32_t k = 1; k < uint32_t(kMaxJobs); ++k) w[k - 1] = k < a.njobs ? a.jobs[k].wg_begin : ~0u;
        k_gemv_t<TYPE, S, DBG, C, RG, KEEP, ONE><<<g, C::NT, lds, st>>>(
            nullptr, nullptr, uint64_t(w[5]) | (uint64_t(w[6]) << 32), w[0], w[1], w[2], w[3], w[4], a);
    }
    return hipSuccess;
}

template <int TYPE, int S, class C>
hipError_t launch_tiled_s(const TLaunchArgs &a, dim3 g, uint32_t lds, hipStream_t st) {
    // The per-block integer-sum test hook is its own instantiation: its
    // global stores would otherwise sit in the production loop. So is the
    // MoE rank-group mode (Q4_K experts, one token per launch), and the
    // Q4_K one-token expert-pair launches (default cache policy).
    bool dbg = false, rg = false, experts = false;
    for (uint32_t j = 0; j < a.njobs; ++j) {
        dbg = dbg || a.jobs[j].dbg != nullptr;
        rg = rg || a.jobs[j].rk != 0;
        experts = experts || a.jobs[j].ids != nullptr;
    }
    if (rg) {
        if constexpr (TYPE == kQ4_K && S == 1) {
            if (dbg || a.njobs != 1) return hipErrorInvalidValue;
            return launch_tiled_sd<TYPE, S, false, C, true, true, true>(a, g, lds, st);
        }
        return hipErrorInvalidValue;
    }
    if constexpr (TYPE == kQ4_K && S == 1)
        if (experts && !dbg) {
            if (a.njobs != 1) return hipErrorInvalidValue;
            return launch_tiled_sd<TYPE, S, false, C, false, true, true>(a, g, lds, st);
        }
    if (dbg) return launch_tiled_sd<TYPE, S, true, C>(a, g, lds, st);
    // one-token single-job launches on fp32 x (most decode launches): the
    // descriptor without the job-table lookup, its first fields preloaded
    if constexpr (S == 1)
        if (a.njobs == 1 && a.jobs[0].x != nullptr && a.jobs[0].ids == nullptr)
            return launch_tiled_sd<TYPE, S, false, C, false, false, true>(a, g, lds, st);
    return launch_tiled_sd<TYPE, S, false, C>(a, g, lds, st);
}

template <int TYPE, class C>
hipError_t launch_tiled(uint32_t S, const TLaunchArgs &a, uint32_t grid, uint32_t lds, hipStream_t st) {
    const dim3 g{grid, 1u, 1u};
    hipError_t e = hipSuccess;
    switch (S) {
#define TC_CASE(n) \
    case n: e = launch_tiled_s<TYPE, n, C>(a, g, lds, st); break;
        TC_CASE(1) TC_CASE(2) TC_CASE(3) TC_CASE(4) TC_CASE(5) TC_CASE(6) TC_CASE(7) TC_CASE(8)
#undef TC_CASE
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

// One workgroup per CU: its LDS holds the activation records, the wave
// tiles and the partial sums.
constexpr uint32_t kTLdsBudget = 152 * 1024;

template <class C>
uint32_t tlds_layout(int type, uint32_t S, uint32_t cols, TLaunchArgs *a) {
    uint32_t o = S * (cols / 256) * xrec_bytes(type);
    a->off_g = o;
    if (type == kIQ3_XXS) o += 16384;  // signed grid, 256 x 16 words
    if (type == kIQ3_S) o += 2048;     // IQ3_S codebook, 512 words
    if (type == kIQ2_S) o += 8192;     // IQ2_S codebook, 1024 x 8 bytes
    if (type == kIQ2_XS) o += 4096;    // IQ2_XS codebook, 512 x 8 bytes
    a->off_t = o;
    o += (C::NT / 64) * tile_slot_bytes(type);
    a->off_p = o;
    return o;
}

// Launch of the kernel for one weight type (defined per type in
// tc_gemv_inst.hip): the 512-thread shape when big, else the 256-thread one.
template <int TYPE>
hipError_t launch_type(bool big, uint32_t S, const TLaunchArgs &a, uint32_t grid, uint32_t lds, hipStream_t st);
// The explicit specializations, one per type the Makefile builds
// (GEMV_TYPES): declared here, so that every caller sees them before use.
#define TC_GV_DECLARE(T) \
    template <>          \
    hipError_t launch_type<T>(bool big, uint32_t S, const TLaunchArgs &a, uint32_t grid, uint32_t lds, hipStream_t st);
TC_GV_DECLARE(kQ5_0)
TC_GV_DECLARE(kQ8_0)
TC_GV_DECLARE(kQ2_K)
TC_GV_DECLARE(kQ3_K)
TC_GV_DECLARE(kQ4_K)
TC_GV_DECLARE(kQ5_K)
TC_GV_DECLARE(kQ6_K)
TC_GV_DECLARE(kIQ2_XS)
TC_GV_DECLARE(kIQ3_XXS)
TC_GV_DECLARE(kIQ4_NL)
TC_GV_DECLARE(kIQ3_S)
TC_GV_DECLARE(kIQ2_S)
TC_GV_DECLARE(kIQ4_XS)
#undef TC_GV_DECLARE

}  // namespace gv
}  // namespace tc
