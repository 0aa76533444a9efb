// tc_simd_matmul.hpp -- the reference's CPU mat-vec entry points
// (namespace tinycoder, include/SIMDMatMulVec.hpp:426-606 of the reference)
// with the same names, arguments and bool result, backed by the gfx950
// kernels of libtc_hip.so through tc_host_matmul (include/tc_qmatmul.h).
//
// All pointers are host pointers, as in the reference. Each call copies X to
// the device, runs the decode mat-vec (seqLen <= 8) or the prefill GEMM, and
// copies out back before it returns. W is read from a device copy when it lies
// inside a range registered with tc_host_weights_register (do that once per
// weight matrix); otherwise it is copied on every call. `false` means no
// gfx950 device, an unsupported shape, or a failed copy or launch: the caller
// takes its own fallback, as it does when the reference returns false for a
// host without AVX2. The numerics are the GPU path's: activations quantized
// with the reference rule (bit-exact), per-block integer sums exact, fp32
// outputs within 1e-3 relative / 1e-4 absolute of the reference CPU kernels.
#pragma once

#include <cstdint>

#include "tc_qmatmul.h"

namespace tinycoder {

/// fp32 weights, the router's F32 matrix (reference SIMDMatMulVec.hpp:426):
/// the outputs carry the reference AVX2 kernel's bits (same FMA order).
inline bool matMulVecBatchF32_SIMD(const float *W_f32, const float *X, uint32_t seqLen, uint32_t rows,
                                   uint32_t cols, float *out) {
    return tc_host_matmul_f32(W_f32, X, seqLen, rows, cols, out) == TC_OK;
}

/// Q4_K (reference SIMDMatMulVec.hpp:448).
inline bool matMulVecBatchQ4K_SIMD(const uint8_t *W_q4k, const float *X, uint32_t seqLen, uint32_t rows,
                                   uint32_t cols, float *out) {
    return tc_host_matmul(TC_Q4_K, W_q4k, X, seqLen, rows, cols, out, nullptr) == TC_OK;
}

/// Q3_K with the optional residual-fused store out = W.x + residual
/// (reference SIMDMatMulVec.hpp:479).
inline bool matMulVecBatchQ3K_SIMD(const uint8_t *W_q3k, const float *X, uint32_t seqLen, uint32_t rows,
                                   uint32_t cols, float *out, const float *residual = nullptr) {
    return tc_host_matmul(TC_Q3_K, W_q3k, X, seqLen, rows, cols, out, residual) == TC_OK;
}

/// Q6_K (reference SIMDMatMulVec.hpp:504).
inline bool matMulVecBatchQ6K_SIMD(const uint8_t *W_q6k, const float *X, uint32_t seqLen, uint32_t rows,
                                   uint32_t cols, float *out) {
    return tc_host_matmul(TC_Q6_K, W_q6k, X, seqLen, rows, cols, out, nullptr) == TC_OK;
}

/// Q5_K (reference SIMDMatMulVec.hpp:527).
inline bool matMulVecBatchQ5K_SIMD(const uint8_t *W_q5k, const float *X, uint32_t seqLen, uint32_t rows,
                                   uint32_t cols, float *out) {
    return tc_host_matmul(TC_Q5_K, W_q5k, X, seqLen, rows, cols, out, nullptr) == TC_OK;
}

/// IQ4_XS (reference SIMDMatMulVec.hpp:547).
inline bool matMulVecBatchIQ4XS_SIMD(const uint8_t *W_iq4xs, const float *X, uint32_t seqLen, uint32_t rows,
                                     uint32_t cols, float *out) {
    return tc_host_matmul(TC_IQ4_XS, W_iq4xs, X, seqLen, rows, cols, out, nullptr) == TC_OK;
}

/// IQ4_NL (reference SIMDMatMulVec.hpp:566).
inline bool matMulVecBatchIQ4NL_SIMD(const uint8_t *W_iq4nl, const float *X, uint32_t seqLen, uint32_t rows,
                                     uint32_t cols, float *out) {
    return tc_host_matmul(TC_IQ4_NL, W_iq4nl, X, seqLen, rows, cols, out, nullptr) == TC_OK;
}

/// Q8_0, cols % 32 == 0 (reference SIMDMatMulVec.hpp:580).
inline bool matMulVecBatchQ8_0_SIMD(const uint8_t *W_q8_0, const float *X, uint32_t seqLen, uint32_t rows,
                                    uint32_t cols, float *out) {
    return tc_host_matmul(TC_Q8_0, W_q8_0, X, seqLen, rows, cols, out, nullptr) == TC_OK;
}

/// Compact Q2_K, i.e. raw 84-byte GGUF Q2_K blocks (reference
/// SIMDMatMulVec.hpp:606, the re-quantized LM head).
inline bool matMulVecBatchQ2K_Compact_SIMD(const uint8_t *W_q2k, const float *X, uint32_t seqLen, uint32_t rows,
                                           uint32_t cols, float *out) {
    return tc_host_matmul(TC_Q2_K, W_q2k, X, seqLen, rows, cols, out, nullptr) == TC_OK;
}

}  // namespace tinycoder
