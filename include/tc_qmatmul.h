/*
 * tc_qmatmul.h -- C-ABI of the MI355X (gfx950) quantized mat-vec / GEMM
 * library (libtc_hip.so). Plain pointers and sizes only.
 *
 * Conventions shared by every entry point:
 *   - Device pointers: weights `w` are raw row-major GGUF blocks
 *     (row bytes = cols / block_elems * block_bytes), activations `x` are fp32
 *     [seq_len][cols], outputs are fp32 [seq_len][rows] (token-major), exactly
 *     the layouts of the reference's int8Gemm/int8Gemv (include/Int8Gemm.hpp:42-107).
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - Weight type ids are GGML's: TC_Q8_0 = 8, TC_Q2_K = 10, TC_Q3_K = 11, TC_Q4_K = 12, TC_Q5_K = 13,
 *     TC_Q6_K = 14, TC_IQ2_XS = 17, TC_IQ3_XXS = 18, TC_IQ4_NL = 20, TC_IQ3_S = 21, TC_IQ2_S = 22, TC_IQ4_XS = 23, TC_Q5_0 = 6 (reference include/IModelLoader.hpp:51-62).
 *   - Return value: TC_OK (0) on success, a negative TC_E_* code otherwise;
 *     nothing is written to outputs when a shape or type is refused.
 *     tc_last_error() gives a message for the calling thread's last failure.
 *   - Numerics: activations are quantized with the reference CPU rule for the
 *     weight type (Q8_K, 256-wide, for Q2_K / Q3_K / Q4_K / Q5_K / Q6_K / IQ3_XXS / IQ3_S / IQ2_S / IQ4_XS;
 *     IQ2_XS, IQ4_NL and Q5_0 take fp32 activations unquantized, as their
 *     reference CPU paths (dotProductIQ2_XS, matMulVecBatchIQ4NL_Q8K_AVX2,
 *     dotProductQ5_0) do, so the quantized-activation entry points
 *     (tc_act_quantize, tc_gemv_q8, tc_quantize_act, tc_block_isums,
 *     tc_debug_q8k_blocks) refuse them; 32-wide with an
 *     fp32 scale for Q8_0), bit-identical to the CPU; per-block integer sums are
 *     exact; fp32 outputs agree with the CPU reference within 1e-3 relative /
 *     1e-4 absolute.
 *   - Not thread-safe per device: calls share the library's grow-only scratch
 *     and must be serialized (as the reference's, GemmDispatch.cu:236-252).
 */
#ifndef TC_QMATMUL_H
#define TC_QMATMUL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TC_Q5_0 = 6, TC_Q8_0 = 8, TC_Q2_K = 10, TC_Q3_K = 11, TC_Q4_K = 12, TC_Q5_K = 13, TC_Q6_K = 14, TC_IQ2_XS = 17, TC_IQ3_XXS = 18, TC_IQ4_NL = 20, TC_IQ3_S = 21, TC_IQ2_S = 22, TC_IQ4_XS = 23 };

enum {
    TC_OK = 0,
    TC_E_UNSUPPORTED = -1, /* type or shape not handled: caller falls back */
    TC_E_LAUNCH = -2,      /* a HIP launch or allocation failed */
    TC_E_ARG = -3,         /* null pointer or inconsistent argument */
};

/* Device query (once per process, like GemmDispatch.cu:208-234 ctx()).
 * Replaces tinycoder::gpu::int8GemmAvailable (include/Int8Gemm.hpp:45):
 * 1 when a gfx950 device is present and TINYCODER_INT8_GEMM is not "0". */
int tc_available(void);

/* Decode mat-vec, seq_len 1..8: out[s][r] = x[s] . W[r].
 * Replaces tinycoder::gpu::int8Gemv (include/Int8Gemm.hpp:77-78,
 * src/cpp/core/cuda/gemm/GemmDispatch.cu:788). cols % 256 == 0. */
int tc_gemv(int type, const void *w, const float *x, float *out, uint32_t seq_len, uint32_t rows,
            uint32_t cols, void *stream);

/* Several decode mat-vecs of one weight type in ONE launch, each with its own
 * input: out[i][s][r] = x[i][s] . W[i][r] for i < n (n <= 8). Host arrays of
 * device pointers / sizes. The reference's fused Q+K+V decode kernel
 * (TINYCODER_FUSE_QKV, ENVIRONMENT.md:29; include/gpu/GpuGemvIQ.hpp:806) is
 * the case n = 3 with x[0] = x[1] = x[2]. seq_len 1..8. */
int tc_gemv_multi(int type, uint32_t n, const void *const *w, const float *const *x, float *const *out,
                  const uint32_t *rows, const uint32_t *cols, uint32_t seq_len, void *stream);

/* Two-phase decode: quantize once, reuse for every matrix that reads the same
 * activation (q/k/v, gate/up). `act` is a caller-owned device buffer of
 * tc_act_bytes(type, seq_len, cols) bytes (256-byte aligned). Activations
 * quantized for Q4_K, Q6_K and IQ3_XXS are interchangeable (Q8_K); Q8_0 needs
 * its own (32-wide). */
size_t tc_act_bytes(int type, uint32_t seq_len, uint32_t cols);
int tc_act_quantize(int type, const float *x, uint32_t seq_len, uint32_t cols, void *act, void *stream);

/* Decode mat-vec on pre-quantized activations (filled by tc_act_quantize for
 * the same seq_len and cols). Replaces launchQGemvQ81
 * (include/gpu/GpuGemvIQInt8.hpp:891), which takes a pre-quantized
 * activation buffer. seq_len 1..8. */
int tc_gemv_q8(int type, const void *w, const void *act, float *out, uint32_t seq_len, uint32_t rows,
               uint32_t cols, void *stream);

/* Pre-size the activation scratch so that later tc_gemv / tc_gemm calls of
 * at most this size allocate nothing (e.g. before a hipGraph capture).
 * Replaces tinycoder::gpu::int8GemvReserve (include/Int8Gemm.hpp:82). */
int tc_gemv_reserve(uint32_t cols, uint32_t seq_len);

/* Fused gate/up decode mat-vec (seq_len 1): uout = Wu x, gout = silu(Wg x) * uout.
 * Replaces int8GemvDualQ4K / int8GemvDualIQ3 (include/Int8Gemm.hpp:90-107). */
int tc_gemv_dual(int type, const void *wg, const void *wu, const float *x, float *gout, float *uout,
                 uint32_t rows, uint32_t cols, void *stream);

/* Prefill GEMM, seq_len >= 1: out[seq_len][rows] = x[seq_len][cols] @ W^T.
 * Replaces tinycoder::gpu::int8Gemm (include/Int8Gemm.hpp:57-59,
 * GemmDispatch.cu:595). Int8 MFMA for the types the reference's GEMM takes
 * (Q4_K, Q5_K, Q6_K, Q8_0, IQ3_XXS, IQ3_S, IQ2_S; GemmDispatch.cu:600-602);
 * the other types run the decode kernel over groups of 8 tokens.
 * blocks_per_row must equal cols / block_elems. */
int tc_gemm(int type, const void *w, const float *x, float *out, uint32_t seq_len, uint32_t rows,
            uint32_t cols, uint32_t blocks_per_row, void *stream);

/* Prefill GEMM that allocates nothing: the same kernels and results as
 * tc_gemm for its MFMA types (cols % 256 == 0), with its scratch (quantized
 * activations, split / stream-K partials) in a fixed per-device array of
 * tc_gemm_noalloc_scratch_bytes() (128 MiB) instead of the library's buffers.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Shapes whose scratch exceeds the array are refused
 * (TC_E_UNSUPPORTED, nothing written). Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU race; calls ordered on a stream
 * do not. */
int tc_gemm_noalloc(int type, const void *w, const float *x, float *out, uint32_t seq_len, uint32_t rows,
                    uint32_t cols, uint32_t blocks_per_row, void *stream);
size_t tc_gemm_noalloc_scratch_bytes(void);

/* Shape-based preference of the int8 path over an fp16 twin. The fp16-twin
 * path does not exist in this build, so it answers 1 for every supported type.
 * Replaces tinycoder::gpu::int8GemmPreferred (include/Int8Gemm.hpp:73). */
int tc_gemm_preferred(uint32_t type, uint32_t rows, uint32_t cols);

/* Enable / disable the Q8_0 GEMM path at run time.
 * Replaces tinycoder::gpu::int8GemmSetQ8Enabled (include/Int8Gemm.hpp:88). */
void tc_gemm_set_q8_enabled(int enabled);

/* Activation quantizer for weight type `type`, into caller buffers:
 * qs int8 [seq_len][cols], d fp32 [seq_len][cols/256] (Q8_K) or [cols/32]
 * (Q8_0 weights), bsums int16 [seq_len][cols/16] (Q8_K only; may be NULL for
 * Q8_0). Test/parity hook equal to the CPU's quantizeQ8K
 * (include/GGMLDequantize.hpp:2769) / the Q8_0 kernel's quantizer
 * (SIMDMatMulVecAVX2.cpp:4296). */
int tc_quantize_act(int type, const float *x, uint32_t seq_len, uint32_t cols, int8_t *qs, float *d,
                    int16_t *bsums, void *stream);

/* Per-block integer sums of the decode kernel (the GPU side of the
 * reference's parity hooks GPUModel::debugQ8KBlocks / debugQ8_0Blocks,
 * include/GPUCompute.hpp:399-460, as a free function over a whole matrix):
 * isums[seq_len][rows][nblk][k], k = 8 sub-block sums for Q4_K, else 1
 * (nblk = cols/32 for Q8_0). The same kernel as tc_gemv computes them. */
int tc_block_isums(int type, const void *w, const float *x, int32_t *isums, uint32_t seq_len,
                   uint32_t rows, uint32_t cols, void *stream);

/* Weight encoder: fp32 [rows][cols] -> raw GGUF blocks of `type`. Q4_K is the
 * reference's own quantizer (src/cpp/core/GGMLQuantize.cpp:47, bit-exact);
 * Q8_0 / Q6_K / IQ3_XXS are this library's encoders (the reference has none).
 * Replaces GGMLQuantize::quantizeQ4KBlock (include/GGMLQuantize.hpp:56). */
int tc_encode(int type, const float *x, void *out, uint32_t rows, uint32_t cols, void *stream);

/* Bytes of one row of `type` with `cols` weights (0 when unsupported). */
size_t tc_row_bytes(int type, uint32_t cols);

/* MoE expert FFN over Q4_K experts (qwen35moe routed experts, reference
 * src/cpp/core/ModelMoE.cpp:660-672 and :990-1002): for every token s and
 * rank r < top_k, e = ids[s][r]: h = silu(Wg[e] x_s) * (Wu[e] x_s),
 * out[s] += wts[s][r] * (Wd[e] h), summed over r in rank order.
 * wg, wu: [n_experts][ff][hidden]; wd: [n_experts][hidden][ff] (Q4_K blocks).
 * ids int32 [seq_len][top_k], wts fp32 [seq_len][top_k], x [seq_len][hidden],
 * out [seq_len][hidden]; all device pointers.
 * From tc_moe_set_gemm_min_tokens tokens on (default 160; the prefill case
 * of the reference's moeBatchExperts, MoeBatch.cu:37-197) the pairs are
 * sorted by expert on the device and each matrix runs as ONE grouped int8
 * MFMA GEMM over all experts; below it, one mat-vec per (token, rank) pair. */
int tc_moe_ffn(const float *x, const int32_t *ids, const float *wts, uint32_t seq_len, uint32_t top_k,
               const void *wg, const void *wu, const void *wd, uint32_t n_experts, uint32_t hidden,
               uint32_t ff, float *out, void *stream);

/* MoE router of qwen35moe: logits[s][e] = x[s] . w_router[e] over the fp32
 * router matrix w_router [n_experts][hidden], then per token the softmax over
 * all experts, the top_k experts by probability and their renormalised
 * weights into ids[s][r], wts[s][r] (rank order; the ids/wts inputs of
 * tc_moe_ffn). Replaces Model::computeQwen35MoERouterOnly
 * (src/cpp/core/ModelMoE.cpp:341-425) and the reference's GPU router
 * kQ35MoeRouter (include/gpu/GpuQwen35Kernels.hpp:931). Bit-identical to the
 * CPU router: the logits in its AVX2 FMA order (SIMDMatMulVecAVX2.cpp:2982),
 * exp and the softmax sum in double, std::partial_sort's order of equal
 * probabilities, the 6.103515625e-5 clamp. logits is a caller buffer of
 * [seq_len][n_experts] fp32 (written). n_experts <= 4096, top_k <= n_experts. */
int tc_moe_router(const float *w_router, const float *x, uint32_t seq_len, uint32_t n_experts, uint32_t hidden,
                  uint32_t top_k, float *logits, int32_t *ids, float *wts, void *stream);

/* The selection step of tc_moe_router alone, on given logits
 * [seq_len][n_experts] (ModelMoE.cpp:387-424). */
int tc_moe_select(const float *logits, uint32_t seq_len, uint32_t n_experts, uint32_t top_k, int32_t *ids, float *wts,
                  void *stream);

/* Token count from which tc_moe_ffn takes the grouped-GEMM path (no
 * reference counterpart: a tuning knob like int8GemmSetQ8Enabled; 0 = always,
 * UINT32_MAX = never). Process-wide. */
void tc_moe_set_gemm_min_tokens(uint32_t n);

/* Parity hooks over host data (the reference's GPUModel::debugQ8KRow,
 * debugQ8_0Row, debugQ8KBlocks and debugQ8_0Blocks, include/GPUCompute.hpp:
 * 399-460, as free functions; GPUModel itself is outside this library).
 * w_row: one host row of raw blocks; x: host fp32 [cols]; cols % 256 == 0.
 * *_row: *result = the decode kernel's output for that row.
 * *_blocks: out_quant = the GPU-quantized activation blocks, block_q8_K
 * {float d; int8 qs[256]; int16 bsums[16]} (292 B) or {float d; int8 qs[32]}
 * (36 B) for Q8_0; out_blk[b] = block b's float contribution as the decode
 * kernel forms it (the kernel run on the row with every other block's scale
 * zeroed, so those blocks add exactly 0). q8k: Q4_K, Q6_K, IQ3_XXS. */
int tc_debug_q8k_row(int type, const uint8_t *w_row, uint32_t blocks_per_row, const float *x, uint32_t cols,
                     float *result);
int tc_debug_q8_0_row(const uint8_t *w_row, uint32_t blocks_per_row, const float *x, uint32_t cols,
                      float *result);
int tc_debug_q8k_blocks(int type, const uint8_t *w_row, uint32_t blocks_per_row, const float *x, uint32_t cols,
                        float *out_blk, uint8_t *out_quant);
int tc_debug_q8_0_blocks(const uint8_t *w_row, uint32_t blocks_per_row, const float *x, uint32_t cols,
                         float *out_blk, uint8_t *out_quant);

/* Host-pointer products: the boundary of the reference's CPU entry points
 * matMulVecBatch{Q4K,Q3K,Q6K,Q5K,IQ4XS,IQ4NL,Q8_0}_SIMD
 * (include/SIMDMatMulVec.hpp:448-584; include/tc_simd_matmul.hpp restates
 * them over this call). W (raw GGUF rows), X [seq_len][cols], out
 * [seq_len][rows] and residual (optional, [seq_len][rows]: out = W.x +
 * residual, the Q3_K entry point's residual-fused store) are HOST pointers.
 * The call copies X to the device, runs tc_gemv (seq_len <= 8) or tc_gemm,
 * and copies out back; it returns when out is written. W is read from a
 * registered device copy when it lies inside a range given to
 * tc_host_weights_register, else it is copied to the device on every call.
 * Calls are serialized by the library. */
int tc_host_matmul(int type, const uint8_t *W, const float *X, uint32_t seq_len, uint32_t rows, uint32_t cols,
                   float *out, const float *residual);
/* fp32 weights: out[s][j] = W[j] . X[s] over host pointers (W [rows][cols],
 * X [seq_len][cols], out [seq_len][rows]), the boundary of the reference's
 * matMulVecBatchF32_SIMD (include/SIMDMatMulVec.hpp:426; its one caller is
 * the qwen35moe router). Each output is formed in the reference AVX2
 * kernel's FMA order (SIMDMatMulVecAVX2.cpp:2982), so the results are its
 * bits, as tc_moe_router's logits. W is read from a registered device copy
 * as for tc_host_matmul. seq_len <= 65535. */
int tc_host_matmul_f32(const float *W, const float *X, uint32_t seq_len, uint32_t rows, uint32_t cols, float *out);
/* Keep a device copy of the host range [host, host + bytes) (weights that
 * later tc_host_matmul calls read); the copy is taken now, so later writes to
 * the host range are not seen until it is registered again. A copy belongs
 * to the device current at registration and serves calls made on that
 * device. No counterpart in the reference (its CPU kernels read host memory
 * in place). */
int tc_host_weights_register(const void *host, size_t bytes);
int tc_host_weights_unregister(const void *host);

/* Message for the calling thread's last failed call ("" if none). */
const char *tc_last_error(void);

/* Roof probes (no counterpart in the reference: measurement aids for reading
 * the kernels' rates). `sink` is device scratch of tc_probe_sink_bytes().
 * tc_probe_mfma_i8: workgroups x 256 threads, each wave issuing 4*iters
 * v_mfma_i32_32x32x32_i8 (65536 int8 ops each) from registers.
 * tc_probe_read: reads `bytes` of `buf` once with 16-byte non-temporal loads,
 * one contiguous chunk per workgroup of 512 threads. Time them with events. */
size_t tc_probe_sink_bytes(void);
int tc_probe_mfma_i8(uint32_t workgroups, uint32_t iters, void *sink, void *stream);
int tc_probe_read(const void *buf, size_t bytes, uint32_t workgroups, void *sink, void *stream);

#ifdef __cplusplus
}
#endif
#endif
