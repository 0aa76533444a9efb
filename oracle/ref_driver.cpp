// ref_driver.cpp -- C-ABI wrappers over the reference's OWN CPU functions,
// linked against the reference translation units compiled in place from the
// reference tree (see oracle/Makefile). TEST INFRASTRUCTURE ONLY: used to write
// the golden vectors under tests/golden and as the "reference" CPU baseline in
// bench.py; never linked into the product.
//
// Nothing here restates arithmetic: each wrapper forwards to the reference
// function named in its comment (paths relative to the reference root).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <utility>
#include <vector>

#include "GGMLDequantize.hpp"
#include "GGMLQuantize.hpp"
#include "GGUFLoader.hpp"
#include "SIMDMatMulVecInternal.hpp"
#include "ThreadPool.hpp"

using namespace tinycoder;

extern "C" {

// src/cpp/core/ThreadPool.cpp:236 (initialize) with
// ThreadPool::recommendedThreadCount() (:68) when n == 0. Returns the count.
int ref_init_threads(int n) {
    size_t t = n > 0 ? static_cast<size_t>(n) : ThreadPool::recommendedThreadCount();
    ThreadPool::instance().initialize(t);
    return static_cast<int>(ThreadPool::instance().numThreads());
}

// include/GGMLDequantize.hpp:89
float ref_half_to_float(uint16_t h) { return GGMLDequantize::halfToFloat(h); }
// include/GGMLDequantize.hpp:61
uint16_t ref_float_to_half(float f) { return GGMLDequantize::floatToHalf(f); }

// include/GGMLDequantize.hpp:2769 -> unpacked qs[n], d[n/256], bsums[n/16].
void ref_quantize_q8k(const float *x, uint32_t n, int8_t *qs, float *d, int16_t *bsums) {
    std::vector<Q8KBlock> b(n / 256);
    GGMLDequantize::quantizeQ8K(x, n, b.data());
    for (uint32_t i = 0; i < n / 256; ++i) {
        std::memcpy(qs + 256 * i, b[i].qs, 256);
        d[i] = b[i].d;
        std::memcpy(bsums + 16 * i, b[i].bsums, 32);
    }
}

// include/GGMLDequantize.hpp:243 / :436 / :503 / :1135 (one block each).
void ref_dequant_block(int type, const uint8_t *blk, float *out) {
    switch (type) {
        case 8: GGMLDequantize::dequantizeQ8_0Block(blk, out); break;
        case 10: GGMLDequantize::dequantizeQ2_KBlock(blk, out); break;  // include/GGMLDequantize.hpp:550
        case 11: GGMLDequantize::dequantizeQ3_KBlock(blk, out); break;  // include/GGMLDequantize.hpp:612
        case 12: GGMLDequantize::dequantizeQ4_KBlock(blk, out); break;
        case 13: GGMLDequantize::dequantizeQ5_KBlock(blk, out); break;  // include/GGMLDequantize.hpp:346
        case 14: GGMLDequantize::dequantizeQ6_KBlock(blk, out); break;
        case 18: GGMLDequantize::dequantizeIQ3_XXSBlock(blk, out); break;
        case 21: GGMLDequantize::dequantizeIQ3_SBlock(blk, out); break;  // include/GGMLDequantize.hpp:1164
        case 22: GGMLDequantize::dequantizeIQ2_SBlock(blk, out); break;  // include/GGMLDequantize.hpp:1215
        case 17: GGMLDequantize::dequantizeIQ2_XSBlock(blk, out); break;  // include/GGMLDequantize.hpp:1245
        case 23: GGMLDequantize::dequantizeIQ4_XSBlock(blk, out); break;  // include/GGMLDequantize.hpp:1319
        case 20: GGMLDequantize::dequantizeIQ4_NLBlock(blk, out); break;  // include/GGMLDequantize.hpp:1304
        case 6: GGMLDequantize::dequantizeQ5_0Block(blk, out); break;  // include/GGMLDequantize.hpp:163
        default: break;
    }
}

// src/cpp/core/GGMLQuantize.cpp:47
void ref_quantize_q4k_block(const float *x, uint8_t *out) {
    GGMLQuantize::quantizeQ4KBlock(x, out);
}

// include/GGMLDequantize.hpp:2064 (per-block d*bsum, unscaled).
float ref_dot_iq3xxs_q8k(const uint8_t *blk, const float *x256) {
    Q8KBlock q;
    GGMLDequantize::quantizeQ8K(x256, 256, &q);
    return GGMLDequantize::dotProductIQ3_XXS_Q8K(blk, &q);
}

// The CPU kernels the reference dispatches to for each type:
//   Q4_K  src/cpp/core/SIMDMatMulVecAVX2.cpp:3614
//   Q8_0  src/cpp/core/SIMDMatMulVecAVX2.cpp:4239
//   Q6_K  src/cpp/core/SIMDMatMulVecAVX2.cpp:4410
//   IQ3_XXS include/GGMLDequantize.hpp:2231 (scalar matMulVecBatchQ8K; the
//         type has no SIMD kernel, src/cpp/core/ModelInternal.cpp:499)
// out[seqLen][rows]. Returns 0 on success.
// src/cpp/core/SIMDMatMulVecAVX2.cpp:2982 (matMulVecBatchF32_AVX2: the
// qwen35moe router logits, ModelMoE.cpp:372-386).
void ref_matmul_f32(const float *W, const float *X, uint32_t seqLen, uint32_t rows, uint32_t cols, float *out) {
    simd::matMulVecBatchF32_AVX2(W, X, seqLen, rows, cols, out);
}

// The router's selection, src/cpp/core/ModelMoE.cpp:387-424, on given logits.
// Those lines are the body of Model::computeQwen35MoERouterOnly, a member of
// Model whose config (expert counts) only a loaded model sets, so the member
// itself cannot be called here; the lines are repeated verbatim in effect on
// the same types (float probabilities, std::pair<float, uint32_t> entries)
// and the same std::partial_sort call of this toolchain's C++ library, whose
// tie order the GPU router and the C oracle must match.
void ref_moe_select(const float *logits, uint32_t seqLen, uint32_t expertCount, uint32_t eu, int32_t *expertIdxOut,
                    float *expertWgtOut) {
    std::vector<float> probs(expertCount);
    std::vector<std::pair<float, uint32_t>> scored(expertCount);
    for (uint32_t s = 0; s < seqLen; ++s) {
        const float *routerLogitsS = logits + static_cast<size_t>(s) * expertCount;
        float maxL = -std::numeric_limits<float>::infinity();
        for (uint32_t e = 0; e < expertCount; ++e) maxL = std::max(maxL, routerLogitsS[e]);
        double sumExp = 0.0;
        for (uint32_t e = 0; e < expertCount; ++e) {
            probs[e] = std::exp(static_cast<double>(routerLogitsS[e]) - maxL);
            sumExp += probs[e];
        }
        const float invSum = static_cast<float>(1.0 / sumExp);
        for (uint32_t e = 0; e < expertCount; ++e) probs[e] *= invSum;
        for (uint32_t e = 0; e < expertCount; ++e) scored[e] = {probs[e], e};
        std::partial_sort(scored.begin(), scored.begin() + eu, scored.end(),
                          [](const auto &a, const auto &b) { return a.first > b.first; });
        double wsum = 0.0;
        for (uint32_t r = 0; r < eu; ++r) wsum += scored[r].first;
        const float wsumClamped = static_cast<float>(std::max(wsum, 6.103515625e-5));
        for (uint32_t r = 0; r < eu; ++r) {
            expertIdxOut[static_cast<size_t>(s) * eu + r] = static_cast<int32_t>(scored[r].second);
            expertWgtOut[static_cast<size_t>(s) * eu + r] = scored[r].first / wsumClamped;
        }
    }
}

int ref_matmul(int type, const uint8_t *W, const float *X, uint32_t seqLen, uint32_t rows,
               uint32_t cols, float *out) {
    switch (type) {
        case 12: simd::matMulVecBatchQ4K_Q8K_AVX2(W, X, seqLen, rows, cols, out); return 0;
        // src/cpp/core/SIMDMatMulVecAVX2.cpp:3988 (the IQ4_XS Q8_K kernel)
        case 23: simd::matMulVecBatchIQ4XS_Q8K_AVX2(W, X, seqLen, rows, cols, out); return 0;
        // src/cpp/core/SIMDMatMulVecAVX2.cpp:4126 (IQ4_NL: fp32 x despite the name)
        case 20: simd::matMulVecBatchIQ4NL_Q8K_AVX2(W, X, seqLen, rows, cols, out); return 0;
        // src/cpp/core/SIMDMatMulVecAVX2.cpp:4757 (the compact-block Q2_K kernel)
        case 10: simd::matMulVecBatchQ2K_Compact_Q8K_AVX2(W, X, seqLen, rows, cols, out); return 0;
        // src/cpp/core/SIMDMatMulVecAVX2.cpp:3220 (no residual)
        case 11: simd::matMulVecBatchQ3K_Q8K_AVX2(W, X, seqLen, rows, cols, out, nullptr); return 0;
        // src/cpp/core/SIMDMatMulVecAVX2.cpp:3842
        case 13: simd::matMulVecBatchQ5K_Q8K_AVX2(W, X, seqLen, rows, cols, out); return 0;
        case 8: simd::matMulVecBatchQ8_0_Q8K_AVX2(W, X, seqLen, rows, cols, out); return 0;
        case 14: simd::matMulVecBatchQ6K_Q8K_AVX2(W, X, seqLen, rows, cols, out); return 0;
        case 18:
            GGMLDequantize::matMulVecBatchQ8K(GGML_TYPE_IQ3_XXS, W, X, seqLen, rows, cols, out);
            return 0;
        // IQ3_S: the same scalar fused Q8_K path (include/GGMLDequantize.hpp:2102 block dot)
        case 21:
            GGMLDequantize::matMulVecBatchQ8K(GGML_TYPE_IQ3_S, W, X, seqLen, rows, cols, out);
            return 0;
        // IQ2_S: the same path (block dot include/GGMLDequantize.hpp:2028, row scale 0.125)
        case 22:
            GGMLDequantize::matMulVecBatchQ8K(GGML_TYPE_IQ2_S, W, X, seqLen, rows, cols, out);
            return 0;
        // IQ2_XS has no Q8_K dot: the float fused path, whose row loop
        // (include/GGMLDequantize.hpp:2449-2461: double sum of the per-block
        // float dots, one float conversion per row) is composed here around
        // the reference's own block dot dotProductIQ2_XS (:1901-1927).
        // (matMulVecFused itself links a helper of SIMDMatMulVec.cpp, which
        // does not build here; that helper serves partial blocks only.)
        case 17:
            for (uint32_t s = 0; s < seqLen; ++s)
                for (uint32_t j = 0; j < rows; ++j) {
                    double dot = 0.0;
                    for (uint32_t b = 0; b < cols / 256; ++b)
                        dot += static_cast<double>(GGMLDequantize::dotProductIQ2_XS(
                            W + (size_t(j) * (cols / 256) + b) * 74, X + size_t(s) * cols + size_t(b) * 256));
                    out[size_t(s) * rows + j] = static_cast<float>(dot);
                }
            return 0;
        // Q5_0: the same float fused row loop around the reference's own block
        // dot dotProductQ5_0 (include/GGMLDequantize.hpp:1820), 32-wide blocks.
        case 6:
            for (uint32_t s = 0; s < seqLen; ++s)
                for (uint32_t j = 0; j < rows; ++j) {
                    double dot = 0.0;
                    for (uint32_t b = 0; b < cols / 32; ++b)
                        dot += static_cast<double>(GGMLDequantize::dotProductQ5_0(
                            W + (size_t(j) * (cols / 32) + b) * 22, X + size_t(s) * cols + size_t(b) * 32));
                    out[size_t(s) * rows + j] = static_cast<float>(dot);
                }
            return 0;
        default: return -1;
    }
}

// The IQ3_S codebook (include/GGMLDequantize.hpp:815, 512 words): format
// data, exported to write this build's table file.
void ref_iq3s_grid(uint32_t *out) { std::memcpy(out, GGMLDequantize::IQ3S_GRID, 512 * sizeof(uint32_t)); }
// The IQ2_S codebook (include/GGMLDequantize.hpp:807, 1024 x 8 bytes), likewise.
void ref_iq2s_grid(uint64_t *out) { std::memcpy(out, GGMLDequantize::IQ2S_GRID, 1024 * sizeof(uint64_t)); }
// The IQ2_XS codebook (include/GGMLDequantize.hpp:821, 512 x 8 bytes), likewise.
void ref_iq2xs_grid(uint64_t *out) { std::memcpy(out, GGMLDequantize::iq2xs_grid, 512 * sizeof(uint64_t)); }

// ---- GGUF reader (include/GGUFLoader.hpp:48) ---------------------------------
// A loader handle; load() or loadMetadata() per `metadata_only`. NULL on failure.
void *ref_gguf_open(const char *path, int metadata_only) {
    auto *g = new GGUFLoader();
    const bool ok = metadata_only ? g->loadMetadata(path) : g->load(path);
    if (!ok) {
        delete g;
        return nullptr;
    }
    return g;
}
void ref_gguf_close(void *h) { delete static_cast<GGUFLoader *>(h); }
// tensorRecords() (GGUFLoader.cpp:1020): count, then record i.
uint64_t ref_gguf_count(void *h) { return static_cast<GGUFLoader *>(h)->tensorRecords().size(); }
int ref_gguf_record(void *h, uint64_t i, char *name, uint64_t cap, uint32_t *type, uint32_t *n_dims,
                    uint32_t *dims, uint64_t *offset) {
    const auto &recs = static_cast<GGUFLoader *>(h)->tensorRecords();
    if (i >= recs.size()) return -1;
    const TensorInfo &r = recs[i];
    std::snprintf(name, cap, "%s", r.name.c_str());
    *type = r.type;
    *n_dims = static_cast<uint32_t>(r.shape.size());
    for (size_t d = 0; d < r.shape.size() && d < 4; ++d) dims[d] = r.shape[d];
    *offset = r.offset;
    return 0;
}
// getTensor (GGUFLoader.cpp:987).
const uint8_t *ref_gguf_tensor(void *h, const char *name) { return static_cast<GGUFLoader *>(h)->getTensor(name); }
// config() fields parsed from the metadata (GGUFLoader.cpp:595-690):
// u[0..15] = numLayers, maxSeqLen, hiddenSize, intermediateSize,
// numAttentionHeads, numKVHeads, vocabSize, expertCount, expertUsedCount,
// expertFeedForwardLength, ropeDimensionCount, ropeDimensionSections[0..3],
// headDim; f[0..1] = ropeTheta, finalLogitSoftcapping; arch / name strings.
void ref_gguf_config(void *h, uint32_t *u, float *f, char *arch, char *name, uint64_t cap) {
    const ModelConfig &c = static_cast<GGUFLoader *>(h)->config();
    const uint32_t v[16] = {c.numLayers, c.maxSeqLen, c.hiddenSize, c.intermediateSize, c.numAttentionHeads,
                            c.numKVHeads, c.vocabSize, c.expertCount, c.expertUsedCount, c.expertFeedForwardLength,
                            c.ropeDimensionCount, c.ropeDimensionSections[0], c.ropeDimensionSections[1],
                            c.ropeDimensionSections[2], c.ropeDimensionSections[3], c.headDim};
    std::memcpy(u, v, sizeof v);
    f[0] = c.ropeTheta;
    f[1] = c.finalLogitSoftcapping;
    std::snprintf(arch, cap, "%s", c.architecture.c_str());
    std::snprintf(name, cap, "%s", c.modelName.c_str());
}
// ggmlTypeSize / ggmlBlockSize (GGUFLoader.cpp:64, :130).
uint32_t ref_ggml_type_size(uint32_t t) { return ggmlTypeSize(t); }
uint32_t ref_ggml_block_size(uint32_t t) { return ggmlBlockSize(t); }

}  // extern "C"
