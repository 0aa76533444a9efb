// tc_common.hpp -- shared device definitions for the gfx950 quantized mat-vec
// and GEMM kernels: GGUF block geometry, the activation layout in HBM, wave-64
// reductions and small bit utilities.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tc {

// GGML type ids (reference include/IModelLoader.hpp:51-62).
enum : int { kQ5_0 = 6, kQ8_0 = 8, kQ2_K = 10, kQ3_K = 11, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kIQ2_XS = 17, kIQ3_XXS = 18, kIQ3_S = 21, kIQ4_NL = 20, kIQ2_S = 22, kIQ4_XS = 23 };

// Every format is handled in "units" of 256 weights. For the K-quants and
// IQ3_XXS a unit is one GGUF block; for Q8_0 it is 8 consecutive 34-byte
// blocks (272 bytes, which keeps every unit 16-byte aligned).
__host__ __device__ constexpr int unit_bytes(int type) {
    return type == kQ2_K ? 84 : type == kQ3_K ? 110 : type == kQ4_K ? 144 : type == kQ5_K ? 176 : type == kQ6_K ? 210 : type == kIQ3_XXS ? 98 : type == kIQ3_S ? 110 : type == kIQ2_S ? 82 : type == kIQ2_XS ? 74 : type == kIQ4_XS ? 136 : type == kIQ4_NL ? 144 : type == kQ5_0 ? 176 : type == kQ8_0 ? 272 : 0;
}
__host__ __device__ constexpr int block_bytes(int type) {
    return type == kQ8_0 ? 34 : type == kIQ4_NL ? 18 : type == kQ5_0 ? 22 : unit_bytes(type);
}
__host__ __device__ constexpr int block_elems(int type) { return type == kQ8_0 || type == kIQ4_NL || type == kQ5_0 ? 32 : 256; }

// Activations quantized for one call live in one device buffer, per token s:
//   qs    int8  [S][cols]            (the quantized values)
//   d     fp32  [S][cols / blk]      (blk = 256 for Q8_K, 32 for Q8_0-style)
//   bsums int16 [S][cols / 16]       (Q8_K only: sums of 16 consecutive qs)
//   dg    bf16  [S][cols / 256][16]  (Q8_K: the 8 sums s of 32 consecutive qs
//                                     as two exact bf16 pieces, 0-7 the high
//                                     128 * (s >> 7), 8-15 the low s & 127)
//         bf16  [S][cols / 32][4]    (Q8_0: each block's d as 3 bf16 pieces
//                                     summing to it exactly, and a zero)
// Bytes of dg per token and 256 columns.
__host__ __device__ constexpr uint32_t dg_bytes(int wtype) { return wtype == kQ8_0 ? 64u : 32u; }

struct ActView {
    const int8_t *qs;
    const float *d;
    const int16_t *bsums;
    const int8_t *dg = nullptr;
};

struct ActLayout {
    size_t qs_off, d_off, bs_off, dg_off, bytes;
};

__host__ inline ActLayout act_layout(int wtype, uint32_t S, uint32_t cols) {
    ActLayout L;
    const uint32_t blk = wtype == kQ8_0 ? 32u : 256u;
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    L.qs_off = 0;
    L.d_off = up(size_t(S) * cols);
    L.bs_off = L.d_off + up(size_t(S) * (cols / blk) * 4);
    L.dg_off = L.bs_off + up(size_t(S) * (cols / 16) * 2);
    L.bytes = L.dg_off + up(size_t(S) * (cols / 256) * dg_bytes(wtype));
    return L;
}

// Fast unsigned division by a runtime constant (Granlund-Montgomery): q = n/d
// for n < 2^31, using a 32x32->64 multiply-high.
struct DivMod {
    uint32_t d, mul, shift;
};

__host__ inline DivMod make_divmod(uint32_t d) {
    DivMod r{d, 0, 0};
    uint32_t s = 0;
    while ((1u << s) < d) ++s;
    r.shift = s;
    // mul = ceil(2^(32+s) / d) - 2^32
    const uint64_t one = 1;
    r.mul = uint32_t(((one << 32) * ((one << s) - d)) / d + 1);
    return r;
}

__device__ __forceinline__ uint32_t div_fast(uint32_t n, const DivMod &m) {
    if (m.d == 1) return n;
    const uint32_t t = __umulhi(n, m.mul);
    return (t + ((n - t) >> 1)) >> (m.shift - 1);
}

// fp16 bits -> fp32 (exact, including subnormals).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return float(__builtin_bit_cast(_Float16, uint16_t(bits16)));
}

// ---- wave-64 reductions through DPP / permutes --------------------------------

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}

// Sum over aligned groups of 4 lanes (quad_perm [1,0,3,2] then [2,3,0,1]):
// every lane of the quad receives the quad total.
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    return v;
}
__device__ __forceinline__ int quad_sum(int v) {
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    return v;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Byte-wise spread of 4 sign bits (bit j -> byte j set to 0xFF).
__device__ __forceinline__ uint32_t spread_sign4(uint32_t s4) {
    return ((s4 * 0x00204081u) & 0x01010101u) * 0xFFu;
}

}  // namespace tc
