// tc_int8gemm.hpp -- the reference's GPU quantized-matmul interface
// (namespace tinycoder::gpu, include/Int8Gemm.hpp:42-107 of the reference)
// with the same names, argument meaning and return convention, implemented as
// inline wrappers over this library's C ABI (tc_qmatmul.h). A reference build
// that includes this header instead of its own Int8Gemm.hpp and links
// libtc_hip.so runs the gfx950 kernels behind every call site
// (GpuGemvIQInt8.hpp:771-962, MoeBatch.cu:146-168, GPUComputeForward.cu).
//
// Return convention (as in the reference): false means "unsupported type or
// shape, or a launch failure"; the caller then takes its fallback. A message
// is written to stderr only for launch failures (GemmDispatch.cu:691); the
// reason for any false is also available from tc_last_error().
#pragma once

#include <cstdint>
#include <cstdio>

#include "tc_qmatmul.h"

namespace tinycoder::gpu {

namespace detail {
inline bool ok(int rc) {
    if (rc == TC_E_LAUNCH) std::fprintf(stderr, "tinycoder::gpu: %s\n", tc_last_error());
    return rc == TC_OK;
}
}  // namespace detail

/// True when a gfx950 device is present (reference int8GemmAvailable,
/// Int8Gemm.hpp:45).
inline bool int8GemmAvailable() { return tc_available() != 0; }

/// out[seqLen][rows] = x[seqLen][cols] @ W[rows][cols]^T on the int8 matrix
/// cores (Q4_K, Q5_K, Q6_K, Q8_0, IQ3_XXS, IQ3_S, IQ2_S) or the exact batched
/// mat-vec (Q2_K, Q3_K, IQ2_XS, IQ4_XS, IQ4_NL, Q5_0)
/// (reference int8Gemm, Int8Gemm.hpp:57-59).
inline bool int8Gemm(int type, const void *w, const float *x, float *out, uint32_t seqLen, uint32_t rows,
                     uint32_t cols, uint32_t blocksPerRow, void *stream) {
    return detail::ok(tc_gemm(type, w, x, out, seqLen, rows, cols, blocksPerRow, stream));
}

/// Int8 path preferred over an fp16 twin for this shape (reference
/// int8GemmPreferred, Int8Gemm.hpp:73). No fp16 twin exists here: true for
/// every supported type.
inline bool int8GemmPreferred(uint32_t type, uint32_t rows, uint32_t cols) {
    return tc_gemm_preferred(type, rows, cols) != 0;
}

/// Decode mat-vec for 1..8 tokens (reference int8Gemv, Int8Gemm.hpp:78-79).
inline bool int8Gemv(int type, const void *w, const float *x, float *out, uint32_t seqLen, uint32_t rows,
                     uint32_t cols, void *stream) {
    return detail::ok(tc_gemv(type, w, x, out, seqLen, rows, cols, stream));
}

/// Pre-size the activation scratch (reference int8GemvReserve, Int8Gemm.hpp:82).
inline void int8GemvReserve(uint32_t cols, uint32_t seqLen) { (void)tc_gemv_reserve(cols, seqLen); }

/// Enable/disable the Q8_0 GEMM path (reference int8GemmSetQ8Enabled,
/// Int8Gemm.hpp:88).
inline void int8GemmSetQ8Enabled(bool enabled) { tc_gemm_set_q8_enabled(enabled ? 1 : 0); }

/// Fused gate+up mat-vecs with SwiGLU: gout = silu(Wg x) * (Wu x), uout = Wu x
/// (reference int8GemvDualIQ3 / int8GemvDualQ4K, Int8Gemm.hpp:93-107).
inline bool int8GemvDualIQ3(const void *wg, const void *wu, const float *x, float *gout, float *uout,
                            uint32_t rows, uint32_t cols, void *stream) {
    return detail::ok(tc_gemv_dual(TC_IQ3_XXS, wg, wu, x, gout, uout, rows, cols, stream));
}

inline bool int8GemvDualQ4K(const void *wg, const void *wu, const float *x, float *gout, float *uout,
                            uint32_t rows, uint32_t cols, void *stream) {
    return detail::ok(tc_gemv_dual(TC_Q4_K, wg, wu, x, gout, uout, rows, cols, stream));
}

/// IQ2_XS gate/up pair (reference int8GemvDualIQ2XS, Int8Gemm.hpp:99), on
/// fp32 activations as the reference CPU path for IQ2_XS computes it.
inline bool int8GemvDualIQ2XS(const void *wg, const void *wu, const float *x, float *gout, float *uout,
                              uint32_t rows, uint32_t cols, void *stream) {
    return detail::ok(tc_gemv_dual(TC_IQ2_XS, wg, wu, x, gout, uout, rows, cols, stream));
}

}  // namespace tinycoder::gpu
