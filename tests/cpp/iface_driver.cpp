// iface_driver.cpp -- test driver: the reference-named C++ interfaces of this
// library (include/tc_int8gemm.hpp: tinycoder::gpu, device pointers;
// include/tc_simd_matmul.hpp: tinycoder::matMulVecBatch*_SIMD, host
// pointers) called exactly as a reference call site calls them, exported
// under plain C names so that the parity tests can pass buffers in from
// Python. Each function returns the interface's bool as 0/1.
#include "tc_int8gemm.hpp"
#include "tc_simd_matmul.hpp"

namespace g = tinycoder::gpu;

extern "C" {

int drv_int8GemmAvailable() { return g::int8GemmAvailable(); }
int drv_int8GemmPreferred(uint32_t type, uint32_t rows, uint32_t cols) { return g::int8GemmPreferred(type, rows, cols); }
void drv_int8GemvReserve(uint32_t cols, uint32_t seqLen) { g::int8GemvReserve(cols, seqLen); }
void drv_int8GemmSetQ8Enabled(int on) { g::int8GemmSetQ8Enabled(on != 0); }

int drv_int8Gemv(int type, const void *w, const float *x, float *out, uint32_t seqLen, uint32_t rows, uint32_t cols,
                 void *stream) {
    return g::int8Gemv(type, w, x, out, seqLen, rows, cols, stream);
}

int drv_int8Gemm(int type, const void *w, const float *x, float *out, uint32_t seqLen, uint32_t rows, uint32_t cols,
                 uint32_t blocksPerRow, void *stream) {
    return g::int8Gemm(type, w, x, out, seqLen, rows, cols, blocksPerRow, stream);
}

int drv_int8GemvDual(int which, const void *wg, const void *wu, const float *x, float *gout, float *uout,
                     uint32_t rows, uint32_t cols, void *stream) {
    switch (which) {
        case 0: return g::int8GemvDualQ4K(wg, wu, x, gout, uout, rows, cols, stream);
        case 1: return g::int8GemvDualIQ3(wg, wu, x, gout, uout, rows, cols, stream);
        default: return g::int8GemvDualIQ2XS(wg, wu, x, gout, uout, rows, cols, stream);
    }
}

int drv_matMulVecBatch_SIMD(int type, const uint8_t *W, const float *X, uint32_t seqLen, uint32_t rows, uint32_t cols,
                            float *out, const float *residual) {
    switch (type) {
        case TC_Q4_K: return tinycoder::matMulVecBatchQ4K_SIMD(W, X, seqLen, rows, cols, out);
        case TC_Q3_K: return tinycoder::matMulVecBatchQ3K_SIMD(W, X, seqLen, rows, cols, out, residual);
        case TC_Q6_K: return tinycoder::matMulVecBatchQ6K_SIMD(W, X, seqLen, rows, cols, out);
        case TC_Q5_K: return tinycoder::matMulVecBatchQ5K_SIMD(W, X, seqLen, rows, cols, out);
        case TC_IQ4_XS: return tinycoder::matMulVecBatchIQ4XS_SIMD(W, X, seqLen, rows, cols, out);
        case TC_IQ4_NL: return tinycoder::matMulVecBatchIQ4NL_SIMD(W, X, seqLen, rows, cols, out);
        case TC_Q8_0: return tinycoder::matMulVecBatchQ8_0_SIMD(W, X, seqLen, rows, cols, out);
        case TC_Q2_K: return tinycoder::matMulVecBatchQ2K_Compact_SIMD(W, X, seqLen, rows, cols, out);
        default: return 0;
    }
}

int drv_matMulVecBatchF32_SIMD(const float *W, const float *X, uint32_t seqLen, uint32_t rows, uint32_t cols,
                               float *out) {
    return tinycoder::matMulVecBatchF32_SIMD(W, X, seqLen, rows, cols, out);
}

}  // extern "C"
