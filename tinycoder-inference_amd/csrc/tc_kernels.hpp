// tc_kernels.hpp -- launchers shared between the kernel translation units and
// the host dispatch (tc_api.cpp).
#pragma once

#include "tc_common.hpp"

namespace tc {

// Activation quantizer for weight type `wtype` (Q8_K for the K-quants and
// IQ3_XXS, 32-wide Q8_0-style for Q8_0) of x[S][cols] into `buf` laid out by
// act_layout(wtype, S, cols).
// With block_major the blocks are stored block-major (block j of token t at
// j * S + t), the layout launch_prefill reads.
// The launch also zeroes zero[0 .. nzero) (the prefill GEMM's arrival
// counters, which must be zero when the GEMM that follows starts).
hipError_t launch_quant_act(int wtype, const float *x, uint32_t S, uint32_t cols, const ActLayout &L,
                            void *buf, hipStream_t st, bool block_major = false, uint32_t *zero = nullptr,
                            uint32_t nzero = 0);

// Weight encoder: x[nunits][256] fp32 -> nunits units of `type`.
// Q8_K block-major quantization of the gathered rows x[rows[s]], s < S.
hipError_t launch_quant_act_rows(const float *x, const uint32_t *rows, uint32_t S, uint32_t cols, const ActLayout &L,
                                 void *buf, hipStream_t st, uint32_t *zero = nullptr, uint32_t nzero = 0);

hipError_t launch_encode(int type, const float *x, void *out, uint32_t nunits, hipStream_t st);

// rows x src_row_bytes -> rows x dst_row_bytes (a multiple of 4), each row
// copied and zero-filled past src_row_bytes.
hipError_t launch_pad_rows(const void *src, uint32_t src_row_bytes, void *dst, uint32_t dst_row_bytes, uint32_t rows,
                           hipStream_t st);

// One mat-vec job: out[s][r] (row stride out_ld per token) = W[r] . x[s].
// With W2 set the job is a pair over the same rows (gate/up): out2 = W2 x and,
// for epi == 1, out = silu(W x) * out2. Activations come from `x` (fp32,
// quantized in the kernel prologue) or, when x is null, from `act`
// (quantized by launch_quant_act).
struct GemvJob {
    const uint8_t *W = nullptr, *W2 = nullptr;
    const float *x = nullptr;
    ActView act{};
    float *out = nullptr, *out2 = nullptr;
    int32_t *dbg = nullptr;  // optional per-block integer sums (test hook)
    uint32_t rows = 0, cols = 0, out_ld = 0;
    int epi = 0;
    // Expert-pair mode (tiled types, fused x only): npairs mat-vecs, pair p
    // using the matrix at W (and W2) + ids[p]*wstride, input x +
    // (p/x_div)*x_stride, outputs out (and out2) + p*out_stride. An id outside
    // [0, n_experts) gives zero outputs.
    const int32_t *ids = nullptr;
    uint64_t wstride = 0;
    uint32_t npairs = 1, x_div = 1, x_stride = 0, out_stride = 0, n_experts = 0;
    // Rank-group mode (rk > 0, with ids, single-token launch): pair p is a
    // token with rk ranks; rank k uses the matrix at W + ids[p*rk+k]*wstride
    // and input x + p*x_stride + k*cols, and out + p*out_stride receives
    // sum over k in rank order of wts[p*rk+k] * (that product).
    uint32_t rk = 0;
    const float *wts = nullptr;
};

// out[t][i] = sum over r < top_k, in rank order, of wts[t][r] * y[t*top_k + r][i].
hipError_t launch_moe_combine(const float *y, const float *wts, float *out, uint32_t T, uint32_t top_k, uint32_t H,
                              hipStream_t st);

// Up to 8 jobs of one weight type and token count in one launch. Returns
// hipErrorInvalidValue when a shape does not fit the kernel.
hipError_t launch_gemv_jobs(int type, uint32_t S, const GemvJob *jobs, uint32_t njobs, int num_cu,
                            hipStream_t st);

// Largest token count per mat-vec launch for this width (LDS budget).
// Weight bytes one mat-vec launch streams over the jobs (both matrices of a pair).
uint64_t jobs_weight_bytes(int type, const GemvJob *jobs, uint32_t njobs);
// Largest S*cols a mat-vec launch over `weight_bytes` quantizes in-kernel
// without loading x after the weights; wider inputs are quantized by a
// separate launch first.
uint32_t gemv_fused_quant_limit(int type, uint64_t weight_bytes);
uint32_t gemv_max_tokens(int type, uint32_t cols);

// Prefill GEMM (int8 MFMA): out[M][N] = W x^T with the activations already
// quantized (launch_quant_act over M tokens, block-major) and the weights
// converted in the MFMA lanes' registers, once per token tile of up to 128
// tokens (tc_prefill.hip; Q4_K, Q5_K, Q6_K, Q8_0, IQ3_XXS, IQ3_S, IQ2_S).
// Stream-K over one workgroup per CU. Q4_K, Q5_K and Q8_0 need the
// activations' scale data (act.dg); every type prefill_workspace_bytes() of scratch
// whose first prefill_counter_words() 32-bit words are zero when the launch
// starts (every launch leaves them zero again).
bool prefill_type(int type);
uint32_t prefill_counter_words(int type, uint32_t M, uint32_t N, uint32_t K, int num_cu);
size_t prefill_workspace_bytes(int type, uint32_t M, uint32_t N, uint32_t K, int num_cu);
hipError_t launch_prefill(int type, const void *W, const ActView &act, float *out, uint32_t M, uint32_t N,
                          uint32_t K, int num_cu, void *workspace, hipStream_t st);

// Grouped (MoE) form over expert-sorted rows: out[i][n] = act row i . W[e(i)]
// row n for the token tiles of mt (count *ntm, at most ntm_max; tiles of at
// most `tile` rows, tile from prefill_grouped_tile). ctr: the arrival
// counters, prefill_grouped_counter_words() of them, zero when the launch
// starts (every launch leaves them zero again); workspace:
// prefill_grouped_workspace_bytes() for the partial tiles. With W2 and
// out2 (mats = 2) a second matrix of the same shape and expert stride (MoE
// gate and up) goes in the same launch: out2 = act . W2.
uint32_t prefill_grouped_tile(uint32_t rows_total, uint32_t n_experts);
uint32_t prefill_grouped_counter_words(uint32_t ntm_max, uint32_t N, uint32_t mats = 1);
size_t prefill_grouped_workspace_bytes(uint32_t tile, uint32_t ntm_max, uint32_t N, uint32_t K, int num_cu,
                                       uint32_t mats = 1);
hipError_t launch_prefill_grouped(const void *W, uint64_t wstride, const ActView &act, float *out,
                                  uint32_t rows_total, uint32_t N, uint32_t K, const uint32_t *mt, const uint32_t *ntm,
                                  uint32_t ntm_max, uint32_t tile, int num_cu, uint32_t *ctr, void *workspace,
                                  hipStream_t st, const void *W2 = nullptr, float *out2 = nullptr);

// ---- MoE prefill over expert-sorted rows ----
// Device-side router: pairs p = t*top_k + r (ids[p] in [0, E), others
// skipped) sorted by expert; each expert's segment starts at a multiple of
// `pad` rows and is cut into tiles of at most `tile` rows. pos[p] = the
// pair's row (-1 for a skipped pair), row_tok[i] = the token of row i (~0 for
// rows no pair lands on), mt = (row begin, row end, expert) per tile, *ntm =
// the tile count. Sizes: moe_max_rows rows and moe_max_tiles tiles.
uint32_t moe_max_tiles(uint32_t npairs, uint32_t n_experts, uint32_t tile);
uint32_t moe_max_rows(uint32_t npairs, uint32_t n_experts, uint32_t pad);
hipError_t launch_moe_route(const int32_t *ids, uint32_t npairs, uint32_t top_k, uint32_t n_experts, uint32_t pad,
                            uint32_t tile, int32_t *pos, uint32_t *row_tok, uint32_t *mt, uint32_t *ntm,
                            hipStream_t st);
// h = silu(g) * u elementwise over nrows_max rows of ff values, written over g
// (rows past the routed ones hold values nothing reads).
// MoE: h = silu(g) * u over g, u [S][cols] quantized to Q8_K block-major
// into buf (layout L, as launch_quant_act with block_major); h itself is not
// stored.
hipError_t launch_swiglu_quant_q8k(const float *g, const float *u, uint32_t S, uint32_t cols, const ActLayout &L,
                                   void *buf, hipStream_t st);
// out[t] = sum over r in rank order of wts[t*top_k+r] * y[pos[t*top_k+r]]
// (pairs with pos < 0 skipped), from 0.
hipError_t launch_moe_combine_rows(const float *y, const int32_t *pos, const float *wts, float *out, uint32_t T,
                                   uint32_t top_k, uint32_t H, hipStream_t st);
// ---- MoE router (F32 router matrix; the CPU router's exact evaluation) ----
// logits out[S][rows] = X[S][cols] . W[rows][cols] in the reference AVX2
// kernel's FMA order.
hipError_t launch_router_logits(const float *W, const float *X, uint32_t S, uint32_t rows, uint32_t cols, float *out,
                                hipStream_t st);
// Softmax, top-K (std::partial_sort's order) and renormalised weights of
// logits[S][E] into ids[S][K], wts[S][K].
hipError_t launch_router_select(const float *logits, uint32_t S, uint32_t E, uint32_t K, int32_t *ids, float *wts,
                                hipStream_t st);



// ---- host-side helpers shared by the entry-point files (tc_api.cpp) ----
int device_cu_count();
int gemm_mfma_check(int type, uint32_t S, uint32_t rows, uint32_t cols);
size_t gemm_mfma_scratch(int type, uint32_t S, uint32_t rows, uint32_t cols, int num_cu, size_t *act_bytes);
int gemm_mfma_into(int type, const void *w, const float *x, float *out, uint32_t S, uint32_t rows, uint32_t cols,
                   int num_cu, void *act, void *ws, hipStream_t st);
int gemm_entry_check(int type, const void *w, const float *x, const float *out, uint32_t S, uint32_t rows,
                     uint32_t cols, uint32_t blocks_per_row);
int fail_code(int code, const char *msg);

}  // namespace tc
