// tc_actquant.hpp -- device code of the activation quantizers, shared by the
// standalone quantizer kernels and the mat-vec kernels that quantize their
// input in the workgroup prologue.
//
// Both rules are bit-identical to the reference CPU: the first element with
// the largest |x| (lowest index on ties) gives max, iscale = -127/max (IEEE
// division), q = min(127, rne(iscale*x)), d = 1/iscale (IEEE). The one sum
// (the rounding trick in q8_bits) is kept apart from its product.
#pragma once

#include "tc_common.hpp"

namespace tc {

// Lane-group reductions with DPP lane moves (no LDS crossbar): xor 1 and
// xor 2 inside quads, then the mirror of each 8- and 16-lane row segment.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_move(uint32_t x) {
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(x), CTRL, 0xF, 0xF, false));
}
template <int WIDTH, typename Op>
__device__ __forceinline__ uint32_t group_reduce(uint32_t x, Op op) {
    static_assert(WIDTH == 2 || WIDTH == 4 || WIDTH == 8 || WIDTH == 16, "groups of 2 to 16 lanes");
    x = op(x, dpp_move<0xB1>(x));                          // quad_perm [1,0,3,2]
    if constexpr (WIDTH >= 4) x = op(x, dpp_move<0x4E>(x));   // quad_perm [2,3,0,1]
    if constexpr (WIDTH >= 8) x = op(x, dpp_move<0x141>(x));  // row_half_mirror
    if constexpr (WIDTH >= 16) x = op(x, dpp_move<0x140>(x)); // row_mirror
    return x;
}

// The block's signed max (its first element of largest |x|) when the block
// is spread over WIDTH lanes, lane values e[0..N) at block indices base ..
// base+N-1: the lane's largest |x| and the key 2i + sign of its first element
// reaching it; across the lanes the largest |x|, then the smallest key among
// the lanes holding it (lowest index). +-0 for an all-zero block.
template <int WIDTH, int N>
__device__ __forceinline__ float first_absmax(const float (&e)[N], int base) {
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < N; ++i) am = fmaxf(am, fabsf(e[i]));
    uint32_t key = 0xFFFFFFFFu;
#pragma unroll
    for (int i = N - 1; i >= 0; --i)
        if (fabsf(e[i]) == am) key = uint32_t(2 * (base + i)) | (__builtin_bit_cast(uint32_t, e[i]) >> 31);
    // the |x| are non-negative floats (never NaN: fmaxf drops NaN), whose
    // bits order as unsigned integers
    auto umax = [](uint32_t p, uint32_t q) { return p > q ? p : q; };
    auto umin = [](uint32_t p, uint32_t q) { return p < q ? p : q; };
    const uint32_t ab = __builtin_bit_cast(uint32_t, am);
    if constexpr (WIDTH == 64) {
        // the whole wave is one block: the 16-lane rows' maxima, then the
        // lowest lane holding the max (lanes hold increasing indices, so it
        // holds the smallest key)
        const uint32_t r = group_reduce<16>(ab, umax);
        const uint32_t gb = umax(umax(__builtin_amdgcn_readlane(r, 0), __builtin_amdgcn_readlane(r, 16)),
                                 umax(__builtin_amdgcn_readlane(r, 32), __builtin_amdgcn_readlane(r, 48)));
        const float gm = __builtin_bit_cast(float, gb);
        const uint64_t hit = __ballot(ab == gb);
        const uint32_t k0 = __builtin_amdgcn_readlane(key, __builtin_ctzll(hit));
        return (k0 & 1u) ? -gm : gm;
    } else {
        const uint32_t gb = group_reduce<WIDTH>(ab, umax);
        const uint32_t kk = group_reduce<WIDTH>(ab == gb ? key : 0xFFFFFFFFu, umin);
        const float gm = __builtin_bit_cast(float, gb);
        return (kk & 1u) ? -gm : gm;
    }
}

// rne(iscale * x) (the product rounded once, then to the nearest integer,
// ties to even) as the low byte of the float bits of the product + 1.5*2^23:
// |product| <= 127.00002, so the sum lies in [2^23, 2^24), where the float
// spacing is 1, and its bits are 0x4B400000 + rne(product). No clamp is
// needed: |iscale| <= 127/|max| (1 + 2^-24), so the product never rounds
// above 127 (the reference's min(127, .) never applies).
constexpr uint32_t kQ8Magic = 0x4B400000u;
__device__ __forceinline__ uint32_t q8_bits(float iscale, float x) {
#pragma clang fp contract(off)
    const float p = iscale * x;
    return __builtin_bit_cast(uint32_t, p + 12582912.0f);
}

// Low bytes of four q8_bits values packed in order.
__device__ __forceinline__ uint32_t q8_pack4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_amdgcn_perm(b, a, 0x0c0c0400u) | __builtin_amdgcn_perm(d, c, 0x04000c0cu);
}

// Four values of one block quantized with iscale: the packed bytes, and
// their sum in *sum.
__device__ __forceinline__ uint32_t quant4_sum(float4 v, float iscale, int *sum) {
    const uint32_t a = q8_bits(iscale, v.x), b = q8_bits(iscale, v.y), c = q8_bits(iscale, v.z), d = q8_bits(iscale, v.w);
    *sum = int(a + b + c + d - 4u * kQ8Magic);
    return q8_pack4(a, b, c, d);
}

// One 256-element Q8_K block by one full wave, lane values already loaded
// (lane l holds elements 4l..4l+3). Writes qs[0..255], *d and bsums[0..15],
// and with dg the 32-wide sums s_p = bsums[2p] + bsums[2p + 1] as two exact
// bf16 pieces: dg[p] = 128 * (s_p >> 7), dg[8 + p] = s_p & 127.
__device__ __forceinline__ void quant_q8k_block_wave_v(float4 v, int8_t *qs, float *d, int16_t *bsums,
                                                       uint16_t *dg = nullptr) {
    const uint32_t lane = threadIdx.x & 63;
    const float e[4] = {v.x, v.y, v.z, v.w};
    const float maxv = first_absmax<64>(e, 4 * int(lane));
    uint32_t packed = 0;
    int sum = 0;
    float dv = 0.0f;
    if (maxv != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, maxv);
        packed = quant4_sum(v, iscale, &sum);
        dv = __fdiv_rn(1.0f, iscale);
    }
    reinterpret_cast<uint32_t *>(qs)[lane] = packed;
    const int s16 = quad_sum(sum);
    if ((lane & 3) == 0) bsums[lane >> 2] = int16_t(s16);
    if (lane == 0) *d = dv;
    if (dg != nullptr) {
        const int s32 = s16 + __shfl_xor(s16, 4);  // lanes 8p: bsums 2p and 2p+1
        if ((lane & 7) == 0) {
            // |s| <= 4064: 128 * (s >> 7) has at most 6 significant bits and
            // s & 127 at most 7, so both are exact in bf16
            dg[lane >> 3] = uint16_t(__builtin_bit_cast(uint32_t, float((s32 >> 7) * 128)) >> 16);
            dg[8 + (lane >> 3)] = uint16_t(__builtin_bit_cast(uint32_t, float(s32 & 127)) >> 16);
        }
    }
}

__device__ __forceinline__ void quant_q8k_block_wave(const float *x, int8_t *qs, float *d, int16_t *bsums,
                                                     uint16_t *dg = nullptr) {
    quant_q8k_block_wave_v(reinterpret_cast<const float4 *>(x)[threadIdx.x & 63], qs, d, bsums, dg);
}

// Eight 32-element blocks by one full wave (8 lanes per block), lane values
// already loaded. With dp, also each block's d as three bf16 pieces that sum
// to it exactly (top 8 significant bits, the next 8, the rest), plus a zero:
// dp[4b .. 4b+3] (the prefill GEMM forms dw*d from them on the matrix cores).
__device__ __forceinline__ void quant_q8_0_blocks_wave_v(float4 v, int8_t *qs, float *d, uint16_t *dp = nullptr) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t sub = lane & 7;
    const float e[4] = {v.x, v.y, v.z, v.w};
    const float maxv = first_absmax<8>(e, 4 * int(sub));
    uint32_t packed = 0;
    float dv = 0.0f;
    if (maxv != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, maxv);
        int sum;
        packed = quant4_sum(v, iscale, &sum);
        dv = __fdiv_rn(1.0f, iscale);
    }
    reinterpret_cast<uint32_t *>(qs)[lane] = packed;
    if (sub == 0) d[lane >> 3] = dv;
    if (dp != nullptr && sub == 0) {
#pragma clang fp contract(off)
        const uint32_t hb = __builtin_bit_cast(uint32_t, dv) & 0xFFFF0000u;
        const float r = dv - __builtin_bit_cast(float, hb);
        const uint32_t mb = __builtin_bit_cast(uint32_t, r) & 0xFFFF0000u;
        const float l = r - __builtin_bit_cast(float, mb);
        const uint32_t lb = __builtin_bit_cast(uint32_t, l);
        uint2 pk;
        pk.x = (hb >> 16) | mb;
        pk.y = lb >> 16;
        reinterpret_cast<uint2 *>(dp)[lane >> 3] = pk;
    }
}

__device__ __forceinline__ void quant_q8_0_blocks_wave(const float *x, int8_t *qs, float *d) {
    quant_q8_0_blocks_wave_v(reinterpret_cast<const float4 *>(x)[threadIdx.x & 63], qs, d);
}

}  // namespace tc
