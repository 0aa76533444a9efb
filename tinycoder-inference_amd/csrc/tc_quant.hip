// tc_quant.hip -- activation quantizers and weight encoders for gfx950.
//
// This translation unit is compiled with -ffp-contract=off: every multiply and
// add below is one IEEE rounding, and division goes through __fdiv_rn, so the
// results are bit-identical to the reference CPU code they follow.
#include "tc_common.hpp"
#include "tc_actquant.hpp"
#include "tc_kernels.hpp"

namespace tc {

__constant__ uint32_t c_iq3xxs_grid[256] = {
#include "iq3xxs_grid.inc"
};
__constant__ uint32_t c_iq3s_grid[512] = {
#include "iq3s_grid.inc"
};
__constant__ uint64_t c_iq2s_grid[1024] = {
#include "iq2s_grid.inc"
};
__constant__ uint64_t c_iq2xs_grid[512] = {
#include "iq2xs_grid.inc"
};

// ---- activation quantizers ---------------------------------------------------

// Destination block of source block g (token g / nbk, block g % nbk): the
// same index (token-major), or block-major (all tokens of 256-column block j
// together, j * S + token) when S != 0.
__device__ __forceinline__ uint32_t act_dst_block(uint32_t g, uint32_t nbk, uint32_t S) {
    if (S == 0) return g;
    const uint32_t t = g / nbk;
    return (g - t * nbk) * S + t;
}

// Q8_K (reference include/GGMLDequantize.hpp:2769-2807): one wave per BPW
// consecutive 256-element blocks, all of their loads issued before the first
// block is quantized (large batches: a wave per block would keep too few bytes
// in flight). nblk_total = S * cols / 256 (token rows are contiguous, so block
// g covers x[256g, 256g+256)).
template <int BPW>
__global__ __launch_bounds__(256) void k_quant_q8k(const float *__restrict__ x, int8_t *__restrict__ qs,
                                                   float *__restrict__ d, int16_t *__restrict__ bsums,
                                                   uint16_t *__restrict__ dg, uint32_t nblk_total, uint32_t nbk,
                                                   uint32_t bm_S, uint32_t *zero, uint32_t nzero) {
    if (blockIdx.x == 0)
        for (uint32_t i = threadIdx.x; i < nzero; i += 256)
            __hip_atomic_store(zero + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const uint32_t g0 = (blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * BPW;
    if (g0 >= nblk_total) return;
    const uint32_t lane = threadIdx.x & 63;
    float4 v[BPW];
#pragma unroll
    for (int i = 0; i < BPW; ++i)
        v[i] = g0 + i < nblk_total ? reinterpret_cast<const float4 *>(x + size_t(g0 + i) * 256)[lane]
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const uint32_t g = g0 + i;
        if (g >= nblk_total) break;  // wave-uniform
        const uint32_t o = act_dst_block(g, nbk, bm_S);
        quant_q8k_block_wave_v(v[i], qs + size_t(o) * 256, d + o, bsums + size_t(o) * 16, dg + size_t(o) * 16);
    }
}

// The same with a row gather: output row s quantizes x row rows[s] (MoE
// activations in expert-sorted order).
__global__ __launch_bounds__(256) void k_quant_q8k_rows(const float *__restrict__ x, const uint32_t *__restrict__ rows,
                                                        int8_t *__restrict__ qs, float *__restrict__ d,
                                                        int16_t *__restrict__ bsums, uint16_t *__restrict__ dg,
                                                        uint32_t nblk_total, uint32_t nbk, uint32_t bm_S,
                                                        uint32_t *zero, uint32_t nzero) {
    if (blockIdx.x == 0)
        for (uint32_t i = threadIdx.x; i < nzero; i += 256)
            __hip_atomic_store(zero + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const uint32_t g = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (g >= nblk_total) return;
    const uint32_t s = g / nbk, j = g - s * nbk;
    const uint32_t o = act_dst_block(g, nbk, bm_S);
    const uint32_t r = rows[s] == ~0u ? 0u : rows[s];  // unrouted rows: any valid row (never stored)
    quant_q8k_block_wave(x + (size_t(r) * nbk + j) * 256, qs + size_t(o) * 256, d + o, bsums + size_t(o) * 16,
                         dg + size_t(o) * 16);
}

// 32-wide rule used for Q8_0 weights (reference
// src/cpp/core/SIMDMatMulVecAVX2.cpp:4296-4326): one wave per BPW groups of 8
// blocks, loads first as in k_quant_q8k.
template <int BPW>
__global__ __launch_bounds__(256) void k_quant_q8_0(const float *__restrict__ x, int8_t *__restrict__ qs,
                                                    float *__restrict__ d, uint16_t *__restrict__ dp,
                                                    uint32_t ngroups, uint32_t nbk, uint32_t bm_S, uint32_t *zero,
                                                    uint32_t nzero) {
    if (blockIdx.x == 0)
        for (uint32_t i = threadIdx.x; i < nzero; i += 256)
            __hip_atomic_store(zero + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const uint32_t g0 = (blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * BPW;
    if (g0 >= ngroups) return;
    const uint32_t lane = threadIdx.x & 63;
    float4 v[BPW];
#pragma unroll
    for (int i = 0; i < BPW; ++i)
        v[i] = g0 + i < ngroups ? reinterpret_cast<const float4 *>(x + size_t(g0 + i) * 256)[lane]
                                : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const uint32_t g = g0 + i;
        if (g >= ngroups) break;  // wave-uniform
        const uint32_t o = act_dst_block(g, nbk, bm_S);
        quant_q8_0_blocks_wave_v(v[i], qs + size_t(o) * 256, d + size_t(o) * 8, dp + size_t(o) * 32);
    }
}

// Row copy into a wider, zero-padded row: dst[r][i] = src[r][i] for i < sbytes,
// 0 for sbytes <= i < dbytes. One thread per destination dword (dbytes is a
// multiple of 4; the source rows may sit at any byte offset).
__global__ __launch_bounds__(256) void k_pad_rows(const uint8_t *__restrict__ src, uint32_t sbytes,
                                                  uint32_t *__restrict__ dst, uint32_t dwords, uint32_t rows) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= size_t(rows) * dwords) return;
    const size_t r = i / dwords;
    const uint32_t c = uint32_t(i - r * dwords) * 4;
    const uint8_t *s = src + r * sbytes;
    uint32_t v = 0;
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k)
        if (c + k < sbytes) v |= uint32_t(s[c + k]) << (8 * k);
    dst[i] = v;
}

// ---- fp16 encodings ----------------------------------------------------------

// The reference's fp32 -> fp16 (include/GGMLDequantize.hpp:61-87): mantissa
// truncation; its subnormal branch also takes exponent -14, so values below
// 2^-13 become signed zero. Reproduced as-is for the Q4_K encoder.
__device__ uint16_t f2h_trunc_ref(float f) {
    const uint32_t b = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (b >> 31) & 1u;
    const int exp = int((b >> 23) & 0xFFu) - 127;
    uint32_t mant = b & 0x7FFFFFu;
    uint32_t h;
    if (exp > 15) {
        h = (sign << 15) | (0x1Fu << 10) | (mant != 0 ? 0x200u : 0u);
    } else if (exp > -14) {
        h = (sign << 15) | (uint32_t(exp + 15) << 10) | (mant >> 13);
    } else if (exp > -24) {
        mant = (mant | 0x800000u) >> (14 - exp);
        h = (sign << 15) | (mant >> 13);
    } else {
        h = sign << 15;
    }
    return uint16_t(h);
}

// IEEE fp32 -> fp16, round to nearest even (this build's own encoders).
__device__ uint16_t f2h_rne(float f) {
    const uint32_t x = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return uint16_t(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return uint16_t(sign | 0x7C00u);
    if (ax < 0x38800000u) {
        const float a = __builtin_bit_cast(float, ax);
        return uint16_t(sign | uint32_t(rintf(a * 16777216.0f)));
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return uint16_t(sign | h);
}

__device__ __forceinline__ float first_abs_max(const float *x, int n, float *amax_out) {
    float amax = 0.0f, maxv = 0.0f;
    for (int j = 0; j < n; ++j) {
        const float a = fabsf(x[j]);
        if (a > amax) {
            amax = a;
            maxv = x[j];
        }
    }
    *amax_out = amax;
    return maxv;
}

// ---- weight encoders (one thread per 256-weight unit) ------------------------

// Q4_K: the reference's quantizeQ4KBlock (src/cpp/core/GGMLQuantize.cpp:47-95).
__device__ void enc_q4k(const float *x, uint8_t *out) {
    float scale[8], minv[8];
    uint8_t q[256];
    float maxScale = 0.0f, maxMin = 0.0f;
    for (int g = 0; g < 8; ++g) {
        const float *xp = x + 32 * g;
        float mn = 0.0f, mx = 0.0f;
        for (int i = 0; i < 32; ++i) {
            mn = xp[i] < mn ? xp[i] : mn;
            mx = mx < xp[i] ? xp[i] : mx;
        }
        const float sc = __fdiv_rn(mx - mn, 15.0f);
        scale[g] = sc;
        minv[g] = -mn;
        maxScale = maxScale < sc ? sc : maxScale;
        maxMin = maxMin < minv[g] ? minv[g] : maxMin;
        for (int i = 0; i < 32; ++i) {
            int v = sc > 1e-30f ? int(rintf(__fdiv_rn(xp[i] - mn, sc))) : 0;
            v = v < 0 ? 0 : (v > 15 ? 15 : v);
            q[32 * g + i] = uint8_t(v);
        }
    }
    const uint16_t hd = maxScale > 0.0f ? f2h_trunc_ref(__fdiv_rn(maxScale, 63.0f)) : 0;
    const uint16_t hdm = maxMin > 0.0f ? f2h_trunc_ref(__fdiv_rn(maxMin, 63.0f)) : 0;
    const float d = h2f(hd), dm = h2f(hdm);
    uint8_t sc6[8], m6[8];
    for (int g = 0; g < 8; ++g) {
        const int s = d > 1e-30f ? int(rintf(__fdiv_rn(scale[g], d))) : 0;
        const int m = dm > 1e-30f ? int(rintf(__fdiv_rn(minv[g], dm))) : 0;
        sc6[g] = uint8_t(s < 0 ? 0 : (s > 63 ? 63 : s));
        m6[g] = uint8_t(m < 0 ? 0 : (m > 63 ? 63 : m));
    }
    out[0] = uint8_t(hd);
    out[1] = uint8_t(hd >> 8);
    out[2] = uint8_t(hdm);
    out[3] = uint8_t(hdm >> 8);
    for (int j = 0; j < 4; ++j) {
        out[4 + j] = uint8_t(sc6[j] | ((sc6[j + 4] >> 4) << 6));
        out[8 + j] = uint8_t(m6[j] | ((m6[j + 4] >> 4) << 6));
        out[12 + j] = uint8_t((sc6[j + 4] & 0x0F) | ((m6[j + 4] & 0x0F) << 4));
    }
    for (int i = 0; i < 128; ++i) {
        const int g0 = 2 * (i >> 5), l = i & 31;
        out[16 + i] = uint8_t(q[32 * g0 + l] | (q[32 * (g0 + 1) + l] << 4));
    }
}

// Q5_K (this build's encoder; the reference ships none): per-32 affine scale
// (max-min)/31 and min -min, fp16 (RNE) super-scales max/63, 6-bit sub-scales
// and mins packed like Q4_K's, q = clamp(rne((x + dmin*m)/(d*sc)), 0, 31) with
// the low nibbles in qs and the fifth bits in qh, as the reference decoder
// reads them (include/GGMLDequantize.hpp:346-380).
__device__ void enc_q5k(const float *x, uint8_t *out) {
    float scale[8], minv[8];
    float maxScale = 0.0f, maxMin = 0.0f;
    for (int g = 0; g < 8; ++g) {
        const float *xp = x + 32 * g;
        float mn = 0.0f, mx = 0.0f;
        for (int i = 0; i < 32; ++i) {
            mn = xp[i] < mn ? xp[i] : mn;
            mx = mx < xp[i] ? xp[i] : mx;
        }
        scale[g] = __fdiv_rn(mx - mn, 31.0f);
        minv[g] = -mn;
        maxScale = maxScale < scale[g] ? scale[g] : maxScale;
        maxMin = maxMin < minv[g] ? minv[g] : maxMin;
    }
    const uint16_t hd = maxScale > 0.0f ? f2h_rne(__fdiv_rn(maxScale, 63.0f)) : 0;
    const uint16_t hdm = maxMin > 0.0f ? f2h_rne(__fdiv_rn(maxMin, 63.0f)) : 0;
    const float d = h2f(hd), dm = h2f(hdm);
    uint8_t sc6[8], m6[8];
    for (int g = 0; g < 8; ++g) {
        const int s = d > 0.0f ? int(rintf(__fdiv_rn(scale[g], d))) : 0;
        const int m = dm > 0.0f ? int(rintf(__fdiv_rn(minv[g], dm))) : 0;
        sc6[g] = uint8_t(s < 0 ? 0 : (s > 63 ? 63 : s));
        m6[g] = uint8_t(m < 0 ? 0 : (m > 63 ? 63 : m));
    }
    out[0] = uint8_t(hd);
    out[1] = uint8_t(hd >> 8);
    out[2] = uint8_t(hdm);
    out[3] = uint8_t(hdm >> 8);
    for (int j = 0; j < 4; ++j) {
        out[4 + j] = uint8_t(sc6[j] | ((sc6[j + 4] >> 4) << 6));
        out[8 + j] = uint8_t(m6[j] | ((m6[j + 4] >> 4) << 6));
        out[12 + j] = uint8_t((sc6[j + 4] & 0x0F) | ((m6[j + 4] & 0x0F) << 4));
    }
    uint8_t *qh = out + 16, *qs = out + 48;
    for (int i = 0; i < 160; ++i) out[16 + i] = 0;
    for (int g = 0; g < 8; ++g) {
        const float es = d * float(sc6[g]), em = dm * float(m6[g]);
        const int c = g >> 1, h = g & 1;
        for (int l = 0; l < 32; ++l) {
            int v = es > 0.0f ? int(rintf(__fdiv_rn(x[32 * g + l] + em, es))) : 0;
            v = v < 0 ? 0 : (v > 31 ? 31 : v);
            qs[32 * c + l] |= uint8_t((v & 15) << (4 * h));
            qh[l] |= uint8_t((v >> 4) << (2 * c + h));
        }
    }
}

// Q8_0 (8 blocks of 32): d = max|w|/127 as fp16 (RNE), q = rne(w/d), +-127.
__device__ void enc_q8_0(const float *x, uint8_t *out) {
    for (int b = 0; b < 8; ++b) {
        const float *xb = x + 32 * b;
        uint8_t *o = out + 34 * b;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fabsf(xb[i]) > amax ? fabsf(xb[i]) : amax;
        const uint16_t hd = f2h_rne(__fdiv_rn(amax, 127.0f));
        const float d = h2f(hd);
        o[0] = uint8_t(hd);
        o[1] = uint8_t(hd >> 8);
        for (int i = 0; i < 32; ++i) {
            int q = d > 0.0f ? int(rintf(__fdiv_rn(xb[i], d))) : 0;
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            o[2 + i] = uint8_t(int8_t(q));
        }
    }
}

// Q2_K (this build's encoder; the reference ships none): per-16 affine
// scale (max-min)/3 and min -min (0 included in the range), fp16 (RNE)
// super-scales max/15, 4-bit scales and mins (low / high nibble of
// scales[g]), q = clamp(rne((x + dmin*m)/(d*sc)), 0, 3), packed as the
// reference decoder reads them (include/GGMLDequantize.hpp:550-590).
__device__ void enc_q2k(const float *x, uint8_t *out) {
    float scale[16], minv[16], maxScale = 0.0f, maxMin = 0.0f;
    for (int g = 0; g < 16; ++g) {
        float mn = 0.0f, mx = 0.0f;
        for (int i = 0; i < 16; ++i) {
            mn = x[16 * g + i] < mn ? x[16 * g + i] : mn;
            mx = mx < x[16 * g + i] ? x[16 * g + i] : mx;
        }
        scale[g] = __fdiv_rn(mx - mn, 3.0f);
        minv[g] = -mn;
        maxScale = maxScale < scale[g] ? scale[g] : maxScale;
        maxMin = maxMin < minv[g] ? minv[g] : maxMin;
    }
    for (int i = 0; i < 84; ++i) out[i] = 0;
    const uint16_t hd = maxScale > 0.0f ? f2h_rne(__fdiv_rn(maxScale, 15.0f)) : 0;
    const uint16_t hm = maxMin > 0.0f ? f2h_rne(__fdiv_rn(maxMin, 15.0f)) : 0;
    out[80] = uint8_t(hd);
    out[81] = uint8_t(hd >> 8);
    out[82] = uint8_t(hm);
    out[83] = uint8_t(hm >> 8);
    const float d = h2f(hd), dm = h2f(hm);
    for (int g = 0; g < 16; ++g) {
        int sv = d > 0.0f ? int(rintf(__fdiv_rn(scale[g], d))) : 0;
        int mv = dm > 0.0f ? int(rintf(__fdiv_rn(minv[g], dm))) : 0;
        sv = sv < 0 ? 0 : (sv > 15 ? 15 : sv);
        mv = mv < 0 ? 0 : (mv > 15 ? 15 : mv);
        out[g] = uint8_t(sv | (mv << 4));
        const float es = d * float(sv), em = dm * float(mv);
        for (int i = 0; i < 16; ++i) {
            const int e = 16 * g + i;
            int q = es > 0.0f ? int(rintf(__fdiv_rn(x[e] + em, es))) : 0;
            q = q < 0 ? 0 : (q > 3 ? 3 : q);
            const int h = e >> 7, t = (e >> 5) & 3, l = e & 31;
            out[16 + 32 * h + l] |= uint8_t(q << (2 * t));
        }
    }
}

// Q3_K (this build's encoder; the reference ships none): per-16 group scale
// m/-4 from the signed first-abs-max, block iscale = -32/M over the group
// scales, 6-bit signed scales (stored +32), fp16 (RNE) d = 1/iscale, q =
// clamp(rne(x/(d*s)), -4, 3) stored as q+4 (2 bits in qs, the third in
// hmask), packed as the reference decoder reads them
// (include/GGMLDequantize.hpp:612-648).
__device__ void enc_q3k(const float *x, uint8_t *out) {
    float gs[16];
    for (int g = 0; g < 16; ++g) {
        float amax;
        const float m = first_abs_max(x + 16 * g, 16, &amax);
        gs[g] = amax == 0.0f ? 0.0f : __fdiv_rn(m, -4.0f);
    }
    float amaxs;
    const float M = first_abs_max(gs, 16, &amaxs);
    for (int i = 0; i < 110; ++i) out[i] = 0;
    int s6[16];
    uint8_t L[256];
    if (amaxs == 0.0f) {
        for (int g = 0; g < 16; ++g) s6[g] = 32;
        for (int e = 0; e < 256; ++e) L[e] = 4;
    } else {
        const float iscale = __fdiv_rn(-32.0f, M);
        for (int g = 0; g < 16; ++g) {
            int v = int(rintf(iscale * gs[g]));
            v = v < -32 ? -32 : (v > 31 ? 31 : v);
            s6[g] = v + 32;
        }
        const uint16_t hd = f2h_rne(__fdiv_rn(1.0f, iscale));
        out[108] = uint8_t(hd);
        out[109] = uint8_t(hd >> 8);
        const float dh = h2f(hd);
        for (int e = 0; e < 256; ++e) {
            const float dg = dh * float(s6[e >> 4] - 32);
            int q = dg != 0.0f ? int(rintf(__fdiv_rn(x[e], dg))) : 0;
            q = q < -4 ? -4 : (q > 3 ? 3 : q);
            L[e] = uint8_t(q + 4);
        }
    }
    for (int i = 0; i < 4; ++i) {
        out[96 + i] = uint8_t((s6[i] & 15) | ((s6[8 + i] & 15) << 4));
        out[100 + i] = uint8_t((s6[4 + i] & 15) | ((s6[12 + i] & 15) << 4));
        out[104 + i] =
            uint8_t((s6[i] >> 4) | ((s6[4 + i] >> 4) << 2) | ((s6[8 + i] >> 4) << 4) | ((s6[12 + i] >> 4) << 6));
    }
    for (int e = 0; e < 256; ++e) {
        const int n = e >> 7, j = (e >> 5) & 3, l = e & 31;
        out[32 + 32 * n + l] |= uint8_t((L[e] & 3) << (2 * j));
        out[l] |= uint8_t((L[e] >> 2) << (4 * n + j));
    }
}

// Q6_K (this build's encoder; the reference ships none): per-16 group scale
// m/-32 from the signed first-abs-max, block iscale = -128/M over the group
// scales, int8 sub-scales, fp16 (RNE) d = 1/iscale, q = clamp(rne(x/(d*sc)),
// -32, 31) + 32, packed as the reference decoder reads
// (include/GGMLDequantize.hpp:503-527).
__device__ void enc_q6k(const float *x, uint8_t *out) {
    float gs[16];
    for (int g = 0; g < 16; ++g) {
        float amax;
        const float m = first_abs_max(x + 16 * g, 16, &amax);
        gs[g] = amax == 0.0f ? 0.0f : __fdiv_rn(m, -32.0f);
    }
    float amaxs;
    const float M = first_abs_max(gs, 16, &amaxs);
    for (int i = 0; i < 210; ++i) out[i] = 0;
    uint8_t L[256];
    if (amaxs == 0.0f) {
        for (int e = 0; e < 256; ++e) L[e] = 32;
    } else {
        const float iscale = __fdiv_rn(-128.0f, M);
        int8_t sc[16];
        for (int g = 0; g < 16; ++g) {
            const int v = int(rintf(iscale * gs[g]));
            sc[g] = int8_t(v > 127 ? 127 : v);
            out[192 + g] = uint8_t(sc[g]);
        }
        const uint16_t hd = f2h_rne(__fdiv_rn(1.0f, iscale));
        out[208] = uint8_t(hd);
        out[209] = uint8_t(hd >> 8);
        const float dh = h2f(hd);
        for (int e = 0; e < 256; ++e) {
            const float dg = dh * float(sc[e >> 4]);
            int q = dg != 0.0f ? int(rintf(__fdiv_rn(x[e], dg))) : 0;
            q = q < -32 ? -32 : (q > 31 ? 31 : q);
            L[e] = uint8_t(q + 32);
        }
    }
    for (int half = 0; half < 2; ++half) {
        uint8_t *ql = out + 64 * half;
        uint8_t *qh = out + 128 + 32 * half;
        const uint8_t *Lh = L + 128 * half;
        for (int l = 0; l < 32; ++l) {
            const int q1 = Lh[l], q2 = Lh[l + 32], q3 = Lh[l + 64], q4 = Lh[l + 96];
            ql[l] = uint8_t((q1 & 0xF) | ((q3 & 0xF) << 4));
            ql[l + 32] = uint8_t((q2 & 0xF) | ((q4 & 0xF) << 4));
            qh[l] = uint8_t((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    }
}

// IQ3_XXS (this build's encoder; the reference ships none): per-32 scale
// s = max|x|/62, block d = max s / 7.75 (fp16 RNE), ls = clamp(rne(s/(0.5d) -
// 0.5), 0, 15), db = d*(0.5+ls)*0.5; per 8 the negative signs with the
// smallest-|x| one flipped on odd count (even parity is implied by the
// format); per 4 the grid entry nearest |x|/db in squared error (first wins).
__device__ void enc_iq3xxs(const float *x, uint8_t *out) {
    float sc[8], smax = 0.0f;
    for (int c = 0; c < 8; ++c) {
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fabsf(x[32 * c + i]) > amax ? fabsf(x[32 * c + i]) : amax;
        sc[c] = __fdiv_rn(amax, 62.0f);
        smax = sc[c] > smax ? sc[c] : smax;
    }
    for (int i = 0; i < 98; ++i) out[i] = 0;
    const uint16_t hd = f2h_rne(__fdiv_rn(smax, 7.75f));
    const float d = h2f(hd);
    if (d == 0.0f) return;
    out[0] = uint8_t(hd);
    out[1] = uint8_t(hd >> 8);
    uint8_t *qs = out + 2;
    uint8_t *sas = out + 66;
    for (int c = 0; c < 8; ++c) {
        const int lsl = int(rintf(__fdiv_rn(sc[c], 0.5f * d) - 0.5f));
        const int ls = lsl < 0 ? 0 : (lsl > 15 ? 15 : lsl);
        const float db = d * (0.5f + float(ls)) * 0.5f;
        uint32_t aux = uint32_t(ls) << 28;
        for (int l = 0; l < 4; ++l) {
            const float *xv = x + 32 * c + 8 * l;
            uint32_t neg = 0;
            int minj = 0;
            for (int j = 0; j < 8; ++j) {
                if (xv[j] < 0.0f) neg |= 1u << j;
                if (fabsf(xv[j]) < fabsf(xv[minj])) minj = j;
            }
            if (__builtin_popcount(neg) & 1) neg ^= 1u << minj;
            aux |= (neg & 127u) << (7 * l);
            for (int h = 0; h < 2; ++h) {
                float t[4];
                for (int j = 0; j < 4; ++j) t[j] = __fdiv_rn(fabsf(xv[4 * h + j]), db);
                int best = 0;
                float berr = 0.0f;
                for (int gi = 0; gi < 256; ++gi) {
                    const uint32_t gv = c_iq3xxs_grid[gi];
                    float err = 0.0f;
                    for (int j = 0; j < 4; ++j) {
                        const float diff = float((gv >> (8 * j)) & 0xFFu) - t[j];
                        err = err + diff * diff;
                    }
                    if (gi == 0 || err < berr) {
                        berr = err;
                        best = gi;
                    }
                }
                qs[8 * c + 2 * l + h] = uint8_t(best);
            }
        }
        for (int k = 0; k < 4; ++k) sas[4 * c + k] = uint8_t(aux >> (8 * k));
    }
}

// IQ3_S (this build's encoder; the reference ships none): per-32 s =
// max|x|/15, d = max s / 31 (fp16 RNE), ls = clamp(rne((s/d - 1)/2), 0, 15),
// db = d*(1+2ls); a sign bit per weight; per 4 the codebook entry (of 512)
// nearest |x|/db in squared error (first wins), its bit 8 in qh, as the
// reference decoder reads them (include/GGMLDequantize.hpp:1164-1212).
__device__ void enc_iq3s(const float *x, uint8_t *out) {
    float sc[8], smax = 0.0f;
    for (int c = 0; c < 8; ++c) {
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fabsf(x[32 * c + i]) > amax ? fabsf(x[32 * c + i]) : amax;
        sc[c] = __fdiv_rn(amax, 15.0f);
        smax = sc[c] > smax ? sc[c] : smax;
    }
    for (int i = 0; i < 110; ++i) out[i] = 0;
    const uint16_t hd = f2h_rne(__fdiv_rn(smax, 31.0f));
    const float d = h2f(hd);
    if (d == 0.0f) return;
    out[0] = uint8_t(hd);
    out[1] = uint8_t(hd >> 8);
    uint8_t *qs = out + 2, *qh = out + 66, *signs = out + 74, *scales = out + 106;
    for (int c = 0; c < 8; ++c) {
        int ls = int(rintf(__fdiv_rn(__fdiv_rn(sc[c], d) - 1.0f, 2.0f)));
        ls = ls < 0 ? 0 : (ls > 15 ? 15 : ls);
        scales[c >> 1] |= uint8_t(ls << (4 * (c & 1)));
        const float db = d * (1.0f + 2.0f * float(ls));
        for (int l = 0; l < 4; ++l) {
            const float *xv = x + 32 * c + 8 * l;
            for (int j = 0; j < 8; ++j)
                if (xv[j] < 0.0f) signs[4 * c + l] |= uint8_t(1u << j);
            for (int h = 0; h < 2; ++h) {
                float t[4];
                for (int j = 0; j < 4; ++j) t[j] = __fdiv_rn(fabsf(xv[4 * h + j]), db);
                int best = 0;
                float berr = 0.0f;
                for (int gi = 0; gi < 512; ++gi) {
                    const uint32_t gv = c_iq3s_grid[gi];
                    float err = 0.0f;
                    for (int j = 0; j < 4; ++j) {
                        const float diff = float((gv >> (8 * j)) & 0xFFu) - t[j];
                        err = err + diff * diff;
                    }
                    if (gi == 0 || err < berr) {
                        berr = err;
                        best = gi;
                    }
                }
                qs[8 * c + 2 * l + h] = uint8_t(best & 255);
                qh[c] |= uint8_t((best >> 8) << (2 * l + h));
            }
        }
    }
}

// IQ2_S (this build's encoder; the reference ships none): per-16 s =
// max|x|/43, d = 8 * max s / 31 (fp16 RNE), ls = clamp(rne((8s/d - 1)/2), 0,
// 15), db = (d*(0.5+ls))*0.25; a sign bit per weight; per 8 the codebook
// entry (of 1024) nearest |x|/db in squared error (first wins), index bits
// 8-9 in qh, as the reference decoder reads them
// (include/GGMLDequantize.hpp:1215-1242).
__device__ void enc_iq2s(const float *x, uint8_t *out) {
    float sc[16], smax = 0.0f;
    for (int c = 0; c < 16; ++c) {
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i) amax = fabsf(x[16 * c + i]) > amax ? fabsf(x[16 * c + i]) : amax;
        sc[c] = __fdiv_rn(amax, 43.0f);
        smax = sc[c] > smax ? sc[c] : smax;
    }
    for (int i = 0; i < 82; ++i) out[i] = 0;
    const uint16_t hd = f2h_rne(__fdiv_rn(8.0f * smax, 31.0f));
    const float d = h2f(hd);
    if (d == 0.0f) return;
    out[0] = uint8_t(hd);
    out[1] = uint8_t(hd >> 8);
    uint8_t *qs = out + 2, *signs = out + 34, *qh = out + 66, *scales = out + 74;
    for (int c = 0; c < 16; ++c) {
        const int ib = c >> 1, h = c & 1;
        int ls = int(rintf(__fdiv_rn(__fdiv_rn(8.0f * sc[c], d) - 1.0f, 2.0f)));
        ls = ls < 0 ? 0 : (ls > 15 ? 15 : ls);
        scales[ib] |= uint8_t(ls << (4 * h));
        const float db = d * (0.5f + float(ls)) * 0.25f;
        for (int q = 0; q < 2; ++q) {
            const int l = 2 * h + q;
            const float *xv = x + 32 * ib + 8 * l;
            float t[8];
            for (int j = 0; j < 8; ++j) {
                if (xv[j] < 0.0f) signs[4 * ib + l] |= uint8_t(1u << j);
                t[j] = __fdiv_rn(fabsf(xv[j]), db);
            }
            int best = 0;
            float berr = 0.0f;
            for (int gi = 0; gi < 1024; ++gi) {
                const uint64_t gv = c_iq2s_grid[gi];
                float err = 0.0f;
                for (int j = 0; j < 8; ++j) {
                    const float diff = float(uint32_t(gv >> (8 * j)) & 0xFFu) - t[j];
                    err = err + diff * diff;
                }
                if (gi == 0 || err < berr) {
                    berr = err;
                    best = gi;
                }
            }
            qs[4 * ib + l] = uint8_t(best & 255);
            qh[ib] |= uint8_t((best >> 8) << (2 * l));
        }
    }
}

// IQ4_XS (this build's encoder; the reference ships none): per 32, s = m /
// -127 with m the first element of largest |x|; d = M / -32 (fp16 RNE) with M
// the first s of largest |s|; ls - 32 = clamp(rne(s / d), -32, 31); per
// weight the table entry nearest x / (d * (ls - 32)) in squared error (first
// wins), packed as the reference decoder reads it
// (include/GGMLDequantize.hpp:1044-1080).
__constant__ int8_t c_kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

// IQ4_NL (this build's encoder; the reference ships none): per 32-block d =
// m / -127 (fp16 RNE) with m the first element of largest |x|; per weight the
// table entry nearest x in squared error of d * kvalue (first wins), packed as
// the reference decoder reads it (include/GGMLDequantize.hpp:1304-1312). One
// unit is 8 consecutive blocks (144 bytes).
__device__ void enc_iq4nl(const float *x, uint8_t *out) {
    for (int b = 0; b < 8; ++b) {
        const float *xb = x + 32 * b;
        uint8_t *o = out + 18 * b;
        float m = 0.0f;
        for (int i = 0; i < 32; ++i) m = fabsf(xb[i]) > fabsf(m) ? xb[i] : m;
        for (int i = 0; i < 18; ++i) o[i] = 0;
        const uint16_t hd = f2h_rne(__fdiv_rn(m, -127.0f));
        const float d = h2f(hd);
        if (d == 0.0f || d != d) continue;
        o[0] = uint8_t(hd);
        o[1] = uint8_t(hd >> 8);
        for (int j = 0; j < 32; ++j) {
            int best = 0;
            float berr = 0.0f;
            for (int n = 0; n < 16; ++n) {
                const float diff = d * float(c_kvalues_iq4nl[n]) - xb[j];
                const float err = diff * diff;
                if (n == 0 || err < berr) {
                    berr = err;
                    best = n;
                }
            }
            o[2 + (j & 15)] |= uint8_t(j < 16 ? best : best << 4);
        }
    }
}

// Q5_0 (this build's encoder; the reference ships none): per 32-block d =
// m / -16 (fp16 RNE) with m the first element of largest |x|; q =
// clamp(rne(x / d) + 16, 0, 31), packed as the reference decoder reads it
// (include/GGMLDequantize.hpp:163-185). One unit is 8 blocks (176 bytes).
__device__ void enc_q50(const float *x, uint8_t *out) {
    for (int b = 0; b < 8; ++b) {
        const float *xb = x + 32 * b;
        uint8_t *o = out + 22 * b;
        float m = 0.0f;
        for (int i = 0; i < 32; ++i) m = fabsf(xb[i]) > fabsf(m) ? xb[i] : m;
        for (int i = 0; i < 22; ++i) o[i] = 0;
        const uint16_t hd = f2h_rne(__fdiv_rn(m, -16.0f));
        const float d = h2f(hd);
        if (d == 0.0f || d != d) continue;
        o[0] = uint8_t(hd);
        o[1] = uint8_t(hd >> 8);
        uint32_t qh = 0;
        for (int j = 0; j < 32; ++j) {
            int q = int(rintf(__fdiv_rn(xb[j], d))) + 16;
            q = q < 0 ? 0 : (q > 31 ? 31 : q);
            o[6 + (j & 15)] |= uint8_t(j < 16 ? (q & 15) : (q & 15) << 4);
            qh |= uint32_t(q >> 4) << j;
        }
        for (int i = 0; i < 4; ++i) o[2 + i] = uint8_t(qh >> (8 * i));
    }
}

// Index of the table entry whose multiple of dl is nearest to xv (first on ties).
__device__ int iq4_nearest(float dl, float xv) {
    int best = 0;
    float berr = 0.0f;
    for (int n = 0; n < 16; ++n) {
        const float diff = dl * float(c_kvalues_iq4nl[n]) - xv;
        const float err = diff * diff;
        if (n == 0 || err < berr) {
            berr = err;
            best = n;
        }
    }
    return best;
}

// Out of line: inlined into its kernel this encoder takes the compiler minutes.
__device__ __attribute__((noinline)) void enc_iq4xs(const float *x, uint8_t *out) {
    float sc[8], smax = 0.0f;
    for (int c = 0; c < 8; ++c) {
        float m = 0.0f;
        for (int i = 0; i < 32; ++i) m = fabsf(x[32 * c + i]) > fabsf(m) ? x[32 * c + i] : m;
        sc[c] = __fdiv_rn(m, -127.0f);
        smax = fabsf(sc[c]) > fabsf(smax) ? sc[c] : smax;
    }
    for (int i = 0; i < 136; ++i) out[i] = 0;
    const uint16_t hd = f2h_rne(__fdiv_rn(smax, -32.0f));
    const float d = h2f(hd);
    if (d == 0.0f || d != d) return;
    out[0] = uint8_t(hd);
    out[1] = uint8_t(hd >> 8);
    uint32_t sh = 0;
    for (int c = 0; c < 8; ++c) {
        int l = int(rintf(__fdiv_rn(sc[c], d)));
        l = l < -32 ? -32 : (l > 31 ? 31 : l);
        const int ls = l + 32;
        out[4 + c / 2] |= uint8_t((ls & 15) << (4 * (c % 2)));
        sh |= uint32_t(ls >> 4) << (2 * c);
        const float dl = d * float(l);
        for (int j = 0; j < 32; ++j) {
            const int best = iq4_nearest(dl, x[32 * c + j]);
            out[8 + 16 * c + (j & 15)] |= uint8_t(j < 16 ? best : best << 4);
        }
    }
    out[2] = uint8_t(sh);
    out[3] = uint8_t(sh >> 8);
}

// IQ2_XS (this build's encoder; the reference ships none): scales as IQ2_S;
// per 8 the negative signs with the smallest-|x| one flipped on odd count (the
// format implies even parity) and the codebook entry (of 512) nearest |x|/db
// (first wins); entry = index | (signs & 127) << 9, as the reference decoder
// reads it (include/GGMLDequantize.hpp:1245-1271).
__device__ void enc_iq2xs(const float *x, uint8_t *out) {
    float sc[16], smax = 0.0f;
    for (int c = 0; c < 16; ++c) {
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i) amax = fabsf(x[16 * c + i]) > amax ? fabsf(x[16 * c + i]) : amax;
        sc[c] = __fdiv_rn(amax, 43.0f);
        smax = sc[c] > smax ? sc[c] : smax;
    }
    for (int i = 0; i < 74; ++i) out[i] = 0;
    const uint16_t hd = f2h_rne(__fdiv_rn(8.0f * smax, 31.0f));
    const float d = h2f(hd);
    if (d == 0.0f) return;
    out[0] = uint8_t(hd);
    out[1] = uint8_t(hd >> 8);
    for (int c = 0; c < 16; ++c) {
        const int ib = c >> 1, h = c & 1;
        int ls = int(rintf(__fdiv_rn(__fdiv_rn(8.0f * sc[c], d) - 1.0f, 2.0f)));
        ls = ls < 0 ? 0 : (ls > 15 ? 15 : ls);
        out[66 + ib] |= uint8_t(ls << (4 * h));
        const float db = d * (0.5f + float(ls)) * 0.25f;
        for (int q = 0; q < 2; ++q) {
            const int l = 2 * h + q;
            const float *xv = x + 32 * ib + 8 * l;
            uint32_t neg = 0;
            int minj = 0;
            float t[8];
            for (int j = 0; j < 8; ++j) {
                if (xv[j] < 0.0f) neg |= 1u << j;
                if (fabsf(xv[j]) < fabsf(xv[minj])) minj = j;
                t[j] = __fdiv_rn(fabsf(xv[j]), db);
            }
            if (__builtin_popcount(neg) & 1) neg ^= 1u << minj;
            int best = 0;
            float berr = 0.0f;
            for (int gi = 0; gi < 512; ++gi) {
                const uint64_t gv = c_iq2xs_grid[gi];
                float err = 0.0f;
                for (int j = 0; j < 8; ++j) {
                    const float diff = float(uint32_t(gv >> (8 * j)) & 0xFFu) - t[j];
                    err = err + diff * diff;
                }
                if (gi == 0 || err < berr) {
                    berr = err;
                    best = gi;
                }
            }
            const uint32_t qv = uint32_t(best) | ((neg & 127u) << 9);
            out[2 + 2 * (4 * ib + l)] = uint8_t(qv);
            out[3 + 2 * (4 * ib + l)] = uint8_t(qv >> 8);
        }
    }
}

// One kernel per weight type (one thread per 256-weight unit): kept apart so
// that no kernel inlines every encoder.
template <int TYPE>
__global__ __launch_bounds__(64) void k_encode(const float *__restrict__ x, uint8_t *__restrict__ out,
                                               uint32_t nunits) {
    const uint32_t u = blockIdx.x * 64 + threadIdx.x;
    if (u >= nunits) return;
    const float *xu = x + size_t(u) * 256;
    uint8_t *o = out + size_t(u) * unit_bytes(TYPE);
    if constexpr (TYPE == kQ4_K) enc_q4k(xu, o);
    else if constexpr (TYPE == kQ8_0) enc_q8_0(xu, o);
    else if constexpr (TYPE == kQ2_K) enc_q2k(xu, o);
    else if constexpr (TYPE == kQ3_K) enc_q3k(xu, o);
    else if constexpr (TYPE == kQ5_K) enc_q5k(xu, o);
    else if constexpr (TYPE == kQ6_K) enc_q6k(xu, o);
    else if constexpr (TYPE == kIQ3_S) enc_iq3s(xu, o);
    else if constexpr (TYPE == kIQ2_S) enc_iq2s(xu, o);
    else if constexpr (TYPE == kIQ2_XS) enc_iq2xs(xu, o);
    else if constexpr (TYPE == kIQ4_XS) enc_iq4xs(xu, o);
    else if constexpr (TYPE == kIQ4_NL) enc_iq4nl(xu, o);
    else if constexpr (TYPE == kQ5_0) enc_q50(xu, o);
    else enc_iq3xxs(xu, o);
}

// ---- launchers -----------------------------------------------------------------

hipError_t launch_quant_act(int wtype, const float *x, uint32_t S, uint32_t cols, const ActLayout &L,
                            void *buf, hipStream_t st, bool block_major, uint32_t *zero, uint32_t nzero) {
    const uint32_t nbk = cols / 256, bm_S = block_major ? S : 0;
    int8_t *qs = reinterpret_cast<int8_t *>(static_cast<char *>(buf) + L.qs_off);
    float *d = reinterpret_cast<float *>(static_cast<char *>(buf) + L.d_off);
    if (wtype == kQ8_0) {
        uint16_t *dp = reinterpret_cast<uint16_t *>(static_cast<char *>(buf) + L.dg_off);
        const uint32_t ng = S * (cols / 256);
        if (ng >= 131072) k_quant_q8_0<4><<<(ng + 15) / 16, 256, 0, st>>>(x, qs, d, dp, ng, nbk, bm_S, zero, nzero);
        else k_quant_q8_0<1><<<(ng + 3) / 4, 256, 0, st>>>(x, qs, d, dp, ng, nbk, bm_S, zero, nzero);
    } else {
        int16_t *bs = reinterpret_cast<int16_t *>(static_cast<char *>(buf) + L.bs_off);
        uint16_t *dg = reinterpret_cast<uint16_t *>(static_cast<char *>(buf) + L.dg_off);
        const uint32_t nb = S * (cols / 256);
        // 4 blocks per wave from 131072 blocks on (measured: slower than a
        // wave per block at 29k-41k blocks, faster at 139k and more)
        if (nb >= 131072) k_quant_q8k<4><<<(nb + 15) / 16, 256, 0, st>>>(x, qs, d, bs, dg, nb, nbk, bm_S, zero, nzero);
        else k_quant_q8k<1><<<(nb + 3) / 4, 256, 0, st>>>(x, qs, d, bs, dg, nb, nbk, bm_S, zero, nzero);
    }
    return hipGetLastError();
}

hipError_t launch_quant_act_rows(const float *x, const uint32_t *rows, uint32_t S, uint32_t cols, const ActLayout &L,
                                 void *buf, hipStream_t st, uint32_t *zero, uint32_t nzero) {
    const uint32_t nbk = cols / 256, nb = S * nbk;
    char *b = static_cast<char *>(buf);
    k_quant_q8k_rows<<<(nb + 3) / 4, 256, 0, st>>>(x, rows, reinterpret_cast<int8_t *>(b + L.qs_off),
                                                   reinterpret_cast<float *>(b + L.d_off),
                                                   reinterpret_cast<int16_t *>(b + L.bs_off),
                                                   reinterpret_cast<uint16_t *>(b + L.dg_off), nb, nbk, S, zero, nzero);
    return hipGetLastError();
}

hipError_t launch_pad_rows(const void *src, uint32_t src_row_bytes, void *dst, uint32_t dst_row_bytes, uint32_t rows,
                           hipStream_t st) {
    if (dst_row_bytes % 4 || dst_row_bytes < src_row_bytes) return hipErrorInvalidValue;
    const size_t n = size_t(rows) * (dst_row_bytes / 4);
    if (n == 0) return hipSuccess;
    k_pad_rows<<<uint32_t((n + 255) / 256), 256, 0, st>>>(static_cast<const uint8_t *>(src), src_row_bytes,
                                                           static_cast<uint32_t *>(dst), dst_row_bytes / 4, rows);
    return hipGetLastError();
}

hipError_t launch_encode(int type, const float *x, void *out, uint32_t nunits, hipStream_t st) {
    const uint32_t g = (nunits + 63) / 64;
    uint8_t *o = static_cast<uint8_t *>(out);
    switch (type) {
#define TC_CASE(t) \
    case t: k_encode<t><<<g, 64, 0, st>>>(x, o, nunits); break;
        TC_CASE(kQ4_K) TC_CASE(kQ8_0) TC_CASE(kQ2_K) TC_CASE(kQ3_K) TC_CASE(kQ5_K) TC_CASE(kQ6_K) TC_CASE(kIQ3_S)
        TC_CASE(kIQ2_S) TC_CASE(kIQ2_XS) TC_CASE(kIQ4_XS) TC_CASE(kIQ4_NL) TC_CASE(kQ5_0) TC_CASE(kIQ3_XXS)
#undef TC_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace tc
