// tc_actquant.hpp -- device code of the activation quantizers, shared by the
// standalone quantizer kernels and the mat-vec kernels that quantize their
// input in the workgroup prologue.
//
// Both rules are bit-identical to the reference CPU: the first element with
// the largest |x| (lowest index on ties) gives max, iscale = -127/max (IEEE
// division), q = min(127, rne(iscale*x)), d = 1/iscale (IEEE). Only products
// feed the rounding, so FP contraction cannot change any result.
#pragma once

#include "tc_common.hpp"

namespace tc {

struct AbsMax {
    float amax, maxv;
    int idx;
};

__device__ __forceinline__ AbsMax absmax_combine(AbsMax a, AbsMax b) {
    const bool take = (b.amax > a.amax) || (b.amax == a.amax && b.idx < a.idx);
    return take ? b : a;
}

template <int WIDTH>
__device__ __forceinline__ AbsMax absmax_reduce(AbsMax v) {
#pragma unroll
    for (int m = 1; m < WIDTH; m <<= 1) {
        AbsMax o;
        o.amax = __shfl_xor(v.amax, m);
        o.maxv = __shfl_xor(v.maxv, m);
        o.idx = __shfl_xor(v.idx, m);
        v = absmax_combine(v, o);
    }
    return v;
}

__device__ __forceinline__ AbsMax absmax4(float4 v, int base) {
    AbsMax r{0.0f, 0.0f, 1 << 20};
    const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float a = fabsf(e[k]);
        if (a > r.amax) {
            r.amax = a;
            r.maxv = e[k];
            r.idx = base + k;
        }
    }
    return r;
}

__device__ __forceinline__ uint32_t quant4(float4 v, float iscale) {
    const float e[4] = {v.x, v.y, v.z, v.w};
    uint32_t packed = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        int q = int(rintf(iscale * e[k]));
        q = q < 127 ? q : 127;
        packed |= uint32_t(uint8_t(int8_t(q))) << (8 * k);
    }
    return packed;
}

__device__ __forceinline__ int bytesum4(uint32_t p) {
    return int(int8_t(p)) + int(int8_t(p >> 8)) + int(int8_t(p >> 16)) + int(int8_t(p >> 24));
}

// One 256-element Q8_K block by one full wave, lane values already loaded
// (lane l holds elements 4l..4l+3). Writes qs[0..255], *d and bsums[0..15].
__device__ __forceinline__ void quant_q8k_block_wave_v(float4 v, int8_t *qs, float *d, int16_t *bsums) {
    const uint32_t lane = threadIdx.x & 63;
    const AbsMax m = absmax_reduce<64>(absmax4(v, 4 * lane));
    uint32_t packed = 0;
    float dv = 0.0f;
    if (m.amax != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, m.maxv);
        packed = quant4(v, iscale);
        dv = __fdiv_rn(1.0f, iscale);
    }
    reinterpret_cast<uint32_t *>(qs)[lane] = packed;
    const int s16 = quad_sum(bytesum4(packed));
    if ((lane & 3) == 0) bsums[lane >> 2] = int16_t(s16);
    if (lane == 0) *d = dv;
}

__device__ __forceinline__ void quant_q8k_block_wave(const float *x, int8_t *qs, float *d, int16_t *bsums) {
    quant_q8k_block_wave_v(reinterpret_cast<const float4 *>(x)[threadIdx.x & 63], qs, d, bsums);
}

// Eight 32-element blocks by one full wave (8 lanes per block), lane values
// already loaded.
__device__ __forceinline__ void quant_q8_0_blocks_wave_v(float4 v, int8_t *qs, float *d) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t sub = lane & 7;
    const AbsMax m = absmax_reduce<8>(absmax4(v, 4 * sub));
    uint32_t packed = 0;
    float dv = 0.0f;
    if (m.amax != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, m.maxv);
        packed = quant4(v, iscale);
        dv = __fdiv_rn(1.0f, iscale);
    }
    reinterpret_cast<uint32_t *>(qs)[lane] = packed;
    if (sub == 0) d[lane >> 3] = dv;
}

__device__ __forceinline__ void quant_q8_0_blocks_wave(const float *x, int8_t *qs, float *d) {
    quant_q8_0_blocks_wave_v(reinterpret_cast<const float4 *>(x)[threadIdx.x & 63], qs, d);
}

}  // namespace tc
