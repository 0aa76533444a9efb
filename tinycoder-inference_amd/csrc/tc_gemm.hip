// tc_gemm.hip -- prefill GEMM: out[m][n] = W[n] . x[m] for M tokens against raw
// GGUF Q4_K / Q8_0 weight rows, on the int8 matrix cores (v_mfma_i32_32x32x32_i8).
//
// Replaces the reference prefill GEMM (int8Gemm, GemmDispatch.cu:595-698) with
// the CPU reference's numerics: the activations are quantized by the same
// bit-exact quantizers as the mat-vec path (Q8_K for Q4_K weights, 32-wide
// Q8_0-style for Q8_0 weights), every integer dot product of a weight block
// with an activation block is exact, and only the final per-block scale
// combination runs in fp32.
//
// Decomposition. One workgroup (8 waves) owns a tile of 128 weight rows x 128
// tokens and walks K one 256-element superblock at a time (optionally a
// K-slice of them, for split-K). Per superblock the raw weight rows, the
// quantized activations and their scales are staged through LDS:
//
//  * Q4_K: a weight of sub-block s is w = d*sc_s*q - dmin*m_s (q in 0..15,
//    sc_s, m_s in 0..63). The product sc_s*q (<= 945) is written to two int8
//    planes, hi = (sc_s*q) >> 7 and lo = (sc_s*q) & 127, so that one chain of
//    MFMAs over the 8 sub-blocks gives main = sum_s sc_s * (q . x)_s exactly as
//    128*acc(hi) + acc(lo). The min term sum_s m_s * (x-sum of sub-block s) is
//    one more pair of MFMAs over 8 useful k-slots, with the activation pair
//    sums split into int8 digits the same way. Per superblock and output:
//    acc += d8 * (d*main - dmin*min).
//  * Q8_0: the int8 weights are the A operand directly; each 32-block gives
//    one MFMA and acc += (dw*d8) * isum.
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

constexpr int GT = 512;       // threads per workgroup (8 waves)
constexpr int GN = 128;       // weight rows per workgroup tile
constexpr int GM = 128;       // tokens per workgroup tile
constexpr int PL = 272;       // LDS plane row stride (256 + 16: conflict-free b128 reads)

// LDS layout (bytes), shared by both weight types where the field exists.
struct GLds {
    static constexpr uint32_t A0 = 0;                      // Q4_K hi plane / Q8_0 weights [GN][PL]
    static constexpr uint32_t A1 = A0 + GN * PL;           // Q4_K lo plane [GN][PL]
    static constexpr uint32_t AM = A1 + GN * PL;           // Q4_K mins, 8 bytes + 8 zero [GN][16]
    static constexpr uint32_t AS = AM + GN * 16;           // Q4_K d [GN] | Q8_0 dw [GN][8]
    static constexpr uint32_t AD = AS + GN * 32;           // Q4_K dmin [GN]
    static constexpr uint32_t B = AD + GN * 4;             // activation int8 [GM][PL]
    static constexpr uint32_t BL = B + GM * PL;            // Q4_K pair-sum low digits [GM][16]
    static constexpr uint32_t BH = BL + GM * 16;           // Q4_K pair-sum high digits [GM][16]
    static constexpr uint32_t BD = BH + GM * 16;           // Q8_K d [GM] | Q8_0 d [GM][8]
    static constexpr uint32_t RAW = BD + GM * 32;          // raw weight tile [GN][unit bytes]
    static constexpr uint32_t bytes(int type) { return RAW + GN * unit_bytes(type); }
};

struct GemmArgs {
    const uint8_t *W;
    const int8_t *qs;       // activations [M][K]
    const float *d8;        // [M][K/256] (Q8_K) or [M][K/32] (Q8_0)
    const int16_t *bsums;   // [M][K/16] (Q8_K)
    float *out;             // [M][N] when nsplit == 1, else partials [nsplit][M][N]
    uint32_t M, N, K;
    uint32_t row_bytes;     // bytes per weight row
    uint32_t ntm;           // token tiles
    uint32_t nblk;          // superblocks per row
    uint32_t split_blk;     // superblocks per K-slice
};

__device__ __forceinline__ u4 lds4(const unsigned char *p) { return *reinterpret_cast<const u4 *>(p); }
__device__ __forceinline__ v4i as_v4i(u4 v) { return __builtin_bit_cast(v4i, v); }

// Q4_K 6-bit scale/min of sub-block j (reference get_scale_min_k4,
// GGMLDequantize.hpp:436-447), from the 12 scale bytes.
__device__ __forceinline__ void q4k_scale_min(const uint8_t *q, int j, uint32_t &sc, uint32_t &mn) {
    if (j < 4) {
        sc = q[j] & 63;
        mn = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// sc * (4 nibbles packed one per byte) -> (hi, lo) digit bytes: byte b of the
// result pair holds (sc*q_b) >> 7 and (sc*q_b) & 127.
__device__ __forceinline__ void digits4(uint32_t q, uint32_t sc, uint32_t &hi, uint32_t &lo) {
    const uint32_t e = (q & 0x000F000Fu) * sc;          // bytes 0, 2 as 16-bit lanes
    const uint32_t o = ((q >> 8) & 0x000F000Fu) * sc;   // bytes 1, 3
    lo = (e & 0x007F007Fu) | ((o & 0x007F007Fu) << 8);
    hi = ((e >> 7) & 0x00070007u) | (((o >> 7) & 0x00070007u) << 8);
}

template <int TYPE>
struct GPrefetch {
    static constexpr int RAWC = (GN * unit_bytes(TYPE) / 16 + GT - 1) / GT;  // raw weight chunks / thread
    u4 raw[RAWC];
    u4 act[4];   // 2048 chunks of 16 activation bytes
    u4 side;     // Q8_K bsums (256 chunks) or Q8_0 d (256 chunks)
    float d8;    // Q8_K d (128 tokens)
};

template <int TYPE>
__device__ __forceinline__ void gemm_prefetch(const GemmArgs &a, uint32_t n0, uint32_t m0, uint32_t b,
                                              GPrefetch<TYPE> &p) {
    constexpr uint32_t UB = unit_bytes(TYPE);
    constexpr uint32_t CPR = UB / 16;  // raw chunks per row
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < GPrefetch<TYPE>::RAWC; ++i) {
        const uint32_t c = min(tid + i * GT, GN * CPR - 1);
        const uint32_t r = c / CPR, w = c - r * CPR;
        const uint32_t n = min(n0 + r, a.N - 1);
        p.raw[i] = *reinterpret_cast<const u4 *>(a.W + size_t(n) * a.row_bytes + size_t(b) * UB + 16 * w);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t c = tid + i * GT;
        const uint32_t m = min(m0 + c / 16, a.M - 1);
        p.act[i] = *reinterpret_cast<const u4 *>(a.qs + size_t(m) * a.K + size_t(b) * 256 + 16 * (c & 15));
    }
    {
        const uint32_t c = tid & 255;
        const uint32_t m = min(m0 + c / 2, a.M - 1);
        if constexpr (TYPE == kQ8_0)
            p.side = *reinterpret_cast<const u4 *>(a.d8 + size_t(m) * (a.K / 32) + size_t(b) * 8 + 4 * (c & 1));
        else
            p.side = *reinterpret_cast<const u4 *>(a.bsums + size_t(m) * (a.K / 16) + size_t(b) * 16 + 8 * (c & 1));
    }
    if constexpr (TYPE == kQ4_K) {
        const uint32_t m = min(m0 + (tid & 127), a.M - 1);
        p.d8 = a.d8[size_t(m) * (a.K / 256) + b];
    }
}

// Staged data -> LDS (raw weights, activation plane, activation side data).
template <int TYPE>
__device__ __forceinline__ void gemm_stage(const GPrefetch<TYPE> &p, unsigned char *lds) {
    constexpr uint32_t UB = unit_bytes(TYPE);
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < GPrefetch<TYPE>::RAWC; ++i) {
        const uint32_t c = tid + i * GT;
        if (c < GN * UB / 16) *reinterpret_cast<u4 *>(lds + GLds::RAW + 16 * c) = p.raw[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t c = tid + i * GT;
        *reinterpret_cast<u4 *>(lds + GLds::B + (c / 16) * PL + 16 * (c & 15)) = p.act[i];
    }
    if (tid < 256) {
        const uint32_t m = tid / 2, h = tid & 1;
        if constexpr (TYPE == kQ8_0) {
            *reinterpret_cast<u4 *>(lds + GLds::BD + m * 32 + 16 * h) = p.side;
        } else {
            // bsums (16 int16) -> 8 pair sums; this thread has pairs 4h..4h+3
            uint32_t lo = 0, hi = 0;
            const uint32_t w[4] = {p.side.x, p.side.y, p.side.z, p.side.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ps = int(int16_t(w[i] & 0xFFFF)) + int(int16_t(w[i] >> 16));
                lo |= uint32_t(ps & 127) << (8 * i);
                hi |= uint32_t(uint8_t(int8_t(ps >> 7))) << (8 * i);
            }
            reinterpret_cast<uint32_t *>(lds + GLds::BL + m * 16)[h] = lo;
            reinterpret_cast<uint32_t *>(lds + GLds::BH + m * 16)[h] = hi;
            if (h == 0) {
                reinterpret_cast<uint32_t *>(lds + GLds::BL + m * 16)[2] = 0;
                reinterpret_cast<uint32_t *>(lds + GLds::BL + m * 16)[3] = 0;
                reinterpret_cast<uint32_t *>(lds + GLds::BH + m * 16)[2] = 0;
                reinterpret_cast<uint32_t *>(lds + GLds::BH + m * 16)[3] = 0;
            }
        }
    }
    if constexpr (TYPE == kQ4_K) {
        if (tid < GM) reinterpret_cast<float *>(lds + GLds::BD)[tid] = p.d8;
    }
}

// Raw weight tile in LDS -> MFMA operand planes and per-row scales.
template <int TYPE>
__device__ __forceinline__ void gemm_convert(unsigned char *lds) {
    const uint32_t tid = threadIdx.x;
    const uint32_t r = tid / 4, qq = tid & 3;
    if constexpr (TYPE == kQ4_K) {
        // 4 threads per row; thread qq converts sub-blocks 2qq (low nibbles)
        // and 2qq+1 (high nibbles) of qs[32qq .. 32qq+31].
        const unsigned char *raw = lds + GLds::RAW + r * 144;
        const uint32_t dh = *reinterpret_cast<const uint32_t *>(raw);
        const uint8_t *sc12 = raw + 4;
        uint32_t sc0, mn0, sc1, mn1;
        q4k_scale_min(sc12, 2 * qq, sc0, mn0);
        q4k_scale_min(sc12, 2 * qq + 1, sc1, mn1);
        const u4 qa = lds4(raw + 16 + 32 * qq), qb = lds4(raw + 32 + 32 * qq);
        const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        uint32_t hl[8], ll[8], hh[8], lh[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            digits4(q[k] & 0x0F0F0F0Fu, sc0, hl[k], ll[k]);
            digits4((q[k] >> 4) & 0x0F0F0F0Fu, sc1, hh[k], lh[k]);
        }
        unsigned char *a0 = lds + GLds::A0 + r * PL, *a1 = lds + GLds::A1 + r * PL;
        const uint32_t s0 = 64 * qq, s1 = 64 * qq + 32;  // k offsets of sub-blocks 2qq, 2qq+1
        *reinterpret_cast<u4 *>(a0 + s0) = u4{hl[0], hl[1], hl[2], hl[3]};
        *reinterpret_cast<u4 *>(a0 + s0 + 16) = u4{hl[4], hl[5], hl[6], hl[7]};
        *reinterpret_cast<u4 *>(a1 + s0) = u4{ll[0], ll[1], ll[2], ll[3]};
        *reinterpret_cast<u4 *>(a1 + s0 + 16) = u4{ll[4], ll[5], ll[6], ll[7]};
        *reinterpret_cast<u4 *>(a0 + s1) = u4{hh[0], hh[1], hh[2], hh[3]};
        *reinterpret_cast<u4 *>(a0 + s1 + 16) = u4{hh[4], hh[5], hh[6], hh[7]};
        *reinterpret_cast<u4 *>(a1 + s1) = u4{lh[0], lh[1], lh[2], lh[3]};
        *reinterpret_cast<u4 *>(a1 + s1 + 16) = u4{lh[4], lh[5], lh[6], lh[7]};
        reinterpret_cast<uint16_t *>(lds + GLds::AM + r * 16)[qq] = uint16_t(mn0 | (mn1 << 8));
        reinterpret_cast<uint16_t *>(lds + GLds::AM + r * 16)[4 + qq] = 0;
        if (qq == 0) {
            reinterpret_cast<float *>(lds + GLds::AS)[r] = h2f(dh & 0xFFFF);
            reinterpret_cast<float *>(lds + GLds::AD)[r] = h2f(dh >> 16);
        }
    } else {
        // Q8_0: 8 blocks of 34 bytes per row (2-byte aligned); thread qq
        // handles blocks 2qq, 2qq+1.
        const unsigned char *raw = lds + GLds::RAW + r * 272;
        unsigned char *a0 = lds + GLds::A0 + r * PL;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t blk = 2 * qq + j;
            const uint16_t *src = reinterpret_cast<const uint16_t *>(raw + 34 * blk);
            uint32_t w[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) w[k] = uint32_t(src[1 + 2 * k]) | (uint32_t(src[2 + 2 * k]) << 16);
            *reinterpret_cast<u4 *>(a0 + 32 * blk) = u4{w[0], w[1], w[2], w[3]};
            *reinterpret_cast<u4 *>(a0 + 32 * blk + 16) = u4{w[4], w[5], w[6], w[7]};
            reinterpret_cast<float *>(lds + GLds::AS + r * 32)[blk] = h2f(src[0]);
        }
    }
}

__device__ __forceinline__ v16i mfma(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

template <int TYPE>
__global__ __launch_bounds__(GT) void k_gemm(GemmArgs a) {
    extern __shared__ __align__(16) unsigned char lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wn = wave & 3, wm = wave >> 2;  // 32-row group, 64-token group
    const uint32_t li = lane & 31, lg = lane >> 5;

    const uint32_t tile = blockIdx.x;
    const uint32_t split = blockIdx.y;
    const uint32_t tm = tile % a.ntm, tn = tile / a.ntm;
    const uint32_t n0 = tn * GN, m0 = tm * GM;
    const uint32_t b0 = split * a.split_blk;
    const uint32_t b1 = min(b0 + a.split_blk, a.nblk);

    float acc[2][16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;

    GPrefetch<TYPE> pf;
    if (b0 < b1) gemm_prefetch<TYPE>(a, n0, m0, b0, pf);
    for (uint32_t b = b0; b < b1; ++b) {
        gemm_stage<TYPE>(pf, lds);
        if (b + 1 < b1) gemm_prefetch<TYPE>(a, n0, m0, b + 1, pf);
        __syncthreads();
        gemm_convert<TYPE>(lds);
        __syncthreads();

        const unsigned char *arow = lds + (32 * wn + li) * PL + 16 * lg;
        const unsigned char *brow0 = lds + GLds::B + (64 * wm + li) * PL + 16 * lg;
        const unsigned char *brow1 = brow0 + 32 * PL;
        if constexpr (TYPE == kQ4_K) {
            v16i hi0 = {}, lo0 = {}, hi1 = {}, lo1 = {};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const v4i ah = as_v4i(lds4(arow + GLds::A0 + 32 * s));
                const v4i al = as_v4i(lds4(arow + GLds::A1 + 32 * s));
                const v4i x0 = as_v4i(lds4(brow0 + 32 * s));
                const v4i x1 = as_v4i(lds4(brow1 + 32 * s));
                hi0 = mfma(ah, x0, hi0);
                lo0 = mfma(al, x0, lo0);
                hi1 = mfma(ah, x1, hi1);
                lo1 = mfma(al, x1, lo1);
            }
            // min term over 8 useful k slots (k-group 0, bytes 0..7)
            const v4i zero = {0, 0, 0, 0};
            const v4i am = lg == 0 ? as_v4i(lds4(lds + GLds::AM + (32 * wn + li) * 16)) : zero;
            const uint32_t tb0 = 64 * wm + li, tb1 = tb0 + 32;
            const v4i bl0 = lg == 0 ? as_v4i(lds4(lds + GLds::BL + tb0 * 16)) : zero;
            const v4i bh0 = lg == 0 ? as_v4i(lds4(lds + GLds::BH + tb0 * 16)) : zero;
            const v4i bl1 = lg == 0 ? as_v4i(lds4(lds + GLds::BL + tb1 * 16)) : zero;
            const v4i bh1 = lg == 0 ? as_v4i(lds4(lds + GLds::BH + tb1 * 16)) : zero;
            const v16i z16 = {};
            const v16i ml0 = mfma(am, bl0, z16), mh0 = mfma(am, bh0, z16);
            const v16i ml1 = mfma(am, bl1, z16), mh1 = mfma(am, bh1, z16);
            const float d80 = reinterpret_cast<const float *>(lds + GLds::BD)[tb0];
            const float d81 = reinterpret_cast<const float *>(lds + GLds::BD)[tb1];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t rr = 32 * wn + 8 * q + 4 * lg;
                const float4 dv = *reinterpret_cast<const float4 *>(lds + GLds::AS + 4 * rr);
                const float4 mv = *reinterpret_cast<const float4 *>(lds + GLds::AD + 4 * rr);
                const float dd[4] = {dv.x, dv.y, dv.z, dv.w}, dm[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * q + e;
                    const int main0 = (hi0[r] << 7) + lo0[r], min0 = (mh0[r] << 7) + ml0[r];
                    const int main1 = (hi1[r] << 7) + lo1[r], min1 = (mh1[r] << 7) + ml1[r];
                    acc[0][r] = fmaf(d80, dd[e] * float(main0) - dm[e] * float(min0), acc[0][r]);
                    acc[1][r] = fmaf(d81, dd[e] * float(main1) - dm[e] * float(min1), acc[1][r]);
                }
            }
        } else {
            const uint32_t tb0 = 64 * wm + li, tb1 = tb0 + 32;
#pragma unroll 2
            for (int s = 0; s < 8; ++s) {
                const v4i aw = as_v4i(lds4(arow + GLds::A0 + 32 * s));
                const v4i x0 = as_v4i(lds4(brow0 + 32 * s));
                const v4i x1 = as_v4i(lds4(brow1 + 32 * s));
                const v16i z16 = {};
                const v16i c0 = mfma(aw, x0, z16), c1 = mfma(aw, x1, z16);
                const float d80 = reinterpret_cast<const float *>(lds + GLds::BD + tb0 * 32)[s];
                const float d81 = reinterpret_cast<const float *>(lds + GLds::BD + tb1 * 32)[s];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 4 * q + e;
                        const float dw = reinterpret_cast<const float *>(
                            lds + GLds::AS + (32 * wn + 8 * q + 4 * lg + e) * 32)[s];
                        acc[0][r] = fmaf(dw * d80, float(c0[r]), acc[0][r]);
                        acc[1][r] = fmaf(dw * d81, float(c1[r]), acc[1][r]);
                    }
                }
            }
        }
        __syncthreads();
    }

    // Store: this lane holds tokens m0 + 64wm + 32t + li, rows n0 + 32wn +
    // 8q + 4lg + e. Rows of a register quad are consecutive.
    float *out = a.out + size_t(split) * a.M * a.N;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t m = m0 + 64 * wm + 32 * t + li;
        if (m >= a.M) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t n = n0 + 32 * wn + 8 * q + 4 * lg;
            float *o = out + size_t(m) * a.N + n;
            if (n + 3 < a.N && (a.N & 3) == 0) {
                *reinterpret_cast<float4 *>(o) = make_float4(acc[t][4 * q], acc[t][4 * q + 1], acc[t][4 * q + 2],
                                                             acc[t][4 * q + 3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n + e < a.N) o[e] = acc[t][4 * q + e];
            }
        }
    }
}

// Split-K partials [nsplit][M][N] -> out[M][N], summed in slice order.
__global__ __launch_bounds__(256) void k_gemm_reduce(const float *__restrict__ part, float *__restrict__ out,
                                                     size_t mn, uint32_t nsplit) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= mn) return;
    float s = part[i];
    for (uint32_t k = 1; k < nsplit; ++k) s += part[k * mn + i];
    out[i] = s;
}

template <int TYPE>
hipError_t launch_gemm_t(const GemmArgs &a, dim3 grid, hipStream_t st) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemm<TYPE>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    k_gemm<TYPE><<<grid, GT, GLds::bytes(TYPE), st>>>(a);
    return hipGetLastError();
}

}  // namespace

uint32_t gemm_splits(int type, uint32_t M, uint32_t N, uint32_t K, int num_cu) {
    (void)type;
    const uint32_t tiles = ((M + GM - 1) / GM) * ((N + GN - 1) / GN);
    const uint32_t nblk = K / 256;
    uint32_t s = 1;
    // Fill the chip: split K while there are fewer tiles than CUs and each
    // slice keeps at least 4 superblocks.
    while (tiles * s * 2 <= uint32_t(num_cu) * 2 && nblk / (s * 2) >= 4 && tiles * s < uint32_t(num_cu)) s *= 2;
    return s;
}

size_t gemm_workspace_bytes(int type, uint32_t M, uint32_t N, uint32_t K, int num_cu) {
    const uint32_t s = gemm_splits(type, M, N, K, num_cu);
    return s > 1 ? size_t(s) * M * N * 4 : 0;
}

hipError_t launch_gemm(int type, const void *W, const ActView &act, float *out, uint32_t M, uint32_t N, uint32_t K,
                       int num_cu, void *workspace, hipStream_t st) {
    if (M == 0 || N == 0 || K == 0 || K % 256) return hipErrorInvalidValue;
    if (type != kQ4_K && type != kQ8_0) return hipErrorInvalidValue;
    const uint32_t nsplit = gemm_splits(type, M, N, K, num_cu);
    if (nsplit > 1 && workspace == nullptr) return hipErrorInvalidValue;
    GemmArgs a{};
    a.W = static_cast<const uint8_t *>(W);
    a.qs = act.qs;
    a.d8 = act.d;
    a.bsums = act.bsums;
    a.M = M;
    a.N = N;
    a.K = K;
    a.nblk = K / 256;
    a.row_bytes = a.nblk * unit_bytes(type);
    a.ntm = (M + GM - 1) / GM;
    a.split_blk = (a.nblk + nsplit - 1) / nsplit;
    a.out = nsplit > 1 ? static_cast<float *>(workspace) : out;
    const dim3 grid{a.ntm * ((N + GN - 1) / GN), nsplit, 1u};
    hipError_t e = type == kQ4_K ? launch_gemm_t<kQ4_K>(a, grid, st) : launch_gemm_t<kQ8_0>(a, grid, st);
    if (e != hipSuccess || nsplit == 1) return e;
    const size_t mn = size_t(M) * N;
    k_gemm_reduce<<<dim3{uint32_t((mn + 255) / 256), 1u, 1u}, 256, 0, st>>>(static_cast<const float *>(workspace),
                                                                           out, mn, nsplit);
    return hipGetLastError();
}

}  // namespace tc
