/*
 * oracle.h -- CPU restatement of the reference's quantized mat-vec path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library, its C-ABI
 * or its host mirror) may include, link or call this. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as
 * the checker or the timed CPU baseline.
 *
 * Every function restates one piece of the reference CPU path; the citation on
 * each names the reference file:line it follows (paths relative to the
 * reference repository root).
 *
 * Parity status per function (how it is pinned):
 *   oc_half_to_float / oc_float_to_half  pinned: exhaustive 65536-pattern check
 *       against the compiled reference (tests/golden) + IEEE closed forms.
 *   oc_quantize_q8k / oc_quantize_q8_0_act  pinned: golden vectors from the
 *       compiled reference + invariants (|q|<=127, bsums, q(max)=-127).
 *   oc_dequant_row  pinned: golden vectors + closed forms on hand-built blocks.
 *   oc_block_isums  pinned: brute-force integer dot of dequantized integer
 *       weights x quantized activations (order-free integer identity).
 *   oc_matmul (Q8_0/Q2_K/Q3_K/Q4_K/Q5_K/Q6_K/IQ3_XXS/IQ3_S/IQ2_S/IQ2_XS/IQ4_XS/IQ4_NL/Q5_0)  pinned: bit-exact against
 *       golden outputs of the compiled reference AVX2 / scalar kernels.
 *   oc_encode_q4k_block  pinned: bit-exact against the compiled reference
 *       quantizeQ4KBlock (golden) + the reference's own round-trip test.
 *   oc_encode_q8_0_block / oc_encode_q2k_block / oc_encode_q3k_block / oc_encode_q5k_block / oc_encode_q6k_block /
 *   oc_encode_iq3xxs_block / oc_encode_iq3s_block / oc_encode_iq2s_block /
 *   oc_encode_iq2xs_block / oc_encode_iq4xs_block / oc_encode_iq4nl_block /
 *   oc_encode_q50_block:
 *       the reference has no encoder for these formats (this build defines
 *       them); pinned by decode round-trip error bounds only.
 *   oc_moe_ffn  pinned: composed of the pinned pieces; golden vectors from the
 *       compiled reference kernels composed the same way (rank-order sum).
 */
#ifndef TC_ORACLE_H
#define TC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    OC_TYPE_Q5_0 = 6,
    OC_TYPE_Q8_0 = 8,
    OC_TYPE_Q2_K = 10,
    OC_TYPE_Q3_K = 11,
    OC_TYPE_Q4_K = 12,
    OC_TYPE_Q5_K = 13,
    OC_TYPE_Q6_K = 14,
    OC_TYPE_IQ2_XS = 17,
    OC_TYPE_IQ3_XXS = 18,
    OC_TYPE_IQ4_NL = 20,
    OC_TYPE_IQ3_S = 21,
    OC_TYPE_IQ2_S = 22,
    OC_TYPE_IQ4_XS = 23,
};

uint32_t oc_type_size(int type);   /* bytes per block */
uint32_t oc_block_size(int type);  /* weights per block */

float oc_half_to_float(uint16_t h);
uint16_t oc_float_to_half(float f);

/* Q8_K activation quantizer (256-wide). n % 256 == 0.
 * qs[n], d[n/256], bsums[n/16]. */
void oc_quantize_q8k(const float *x, uint32_t n, int8_t *qs, float *d, int16_t *bsums);
/* Q8_0-style 32-wide activation quantizer used by the Q8_0 kernel.
 * n % 32 == 0. qs[n], d[n/32]. */
void oc_quantize_q8_0_act(const float *x, uint32_t n, int8_t *qs, float *d);

/* Dequantize n weights (n multiple of the block size) of one row. */
int oc_dequant_row(int type, const uint8_t *w, uint32_t n, float *out);

/* Per-block integer dot sums of W[rows][cols] against the quantized activations
 * of X[S][cols]. Output layout [S][rows][nblk][k]: k = 8 sub-block sums for
 * Q4_K and Q5_K, k = 2 (main, min) for Q2_K, k = 1 otherwise (Q8_0 blocks
 * are the 32-wide ones; IQ2_XS, whose CPU path does not quantize x, has none:
 * -1). */
int oc_block_isums(int type, const uint8_t *W, const float *X, uint32_t S,
                   uint32_t rows, uint32_t cols, int32_t *isums);

/* out[S][rows] = X[S][cols] @ W^T, same float evaluation order as the
 * reference CPU kernel for the type. Returns 0 on success. */
int oc_matmul(int type, const uint8_t *W, const float *X, uint32_t S,
              uint32_t rows, uint32_t cols, float *out);

/* Weight encoders. */
void oc_encode_q4k_block(const float *x, uint8_t *out);
void oc_encode_q8_0_block(const float *x, uint8_t *out);
void oc_encode_q2k_block(const float *x, uint8_t *out);
void oc_encode_q3k_block(const float *x, uint8_t *out);
void oc_encode_q5k_block(const float *x, uint8_t *out);
void oc_encode_q6k_block(const float *x, uint8_t *out);
void oc_encode_iq3xxs_block(const float *x, uint8_t *out);
void oc_encode_iq3s_block(const float *x, uint8_t *out);
void oc_encode_iq2s_block(const float *x, uint8_t *out);
void oc_encode_iq2xs_block(const float *x, uint8_t *out);
void oc_encode_iq4xs_block(const float *x, uint8_t *out);
void oc_encode_iq4nl_block(const float *x, uint8_t *out);
void oc_encode_q50_block(const float *x, uint8_t *out);
int oc_encode_rows(int type, const float *x, uint32_t rows, uint32_t cols, uint8_t *out);

/* MoE expert FFN (Q4_K experts), rank-order reduction.
 * x[S][H]; ids[S][K] expert ids; wts[S][K] routing weights;
 * wg/wu: [E][FF rows][H cols] Q4_K; wd: [E][H rows][FF cols] Q4_K; out[S][H]. */
int oc_moe_ffn(const float *x, const int32_t *ids, const float *wts, uint32_t S,
               uint32_t K, const uint8_t *wg, const uint8_t *wu, const uint8_t *wd,
               uint32_t E, uint32_t H, uint32_t FF, float *out);

/* MoE router. oc_matmul_f32: out[S][rows] = X[S][cols] @ W^T for an fp32
 * matrix, in the reference AVX2 kernel's evaluation order (the router
 * logits). oc_moe_route: softmax, top-K and renormalisation of logits[S][E]
 * into ids[S][K] and wts[S][K]; returns 0 on success. */
void oc_matmul_f32(const float *W, const float *X, uint32_t S, uint32_t rows, uint32_t cols, float *out);
int oc_moe_route(const float *logits, uint32_t S, uint32_t E, uint32_t K, int32_t *ids, float *wts);

#ifdef __cplusplus
}
#endif
#endif
