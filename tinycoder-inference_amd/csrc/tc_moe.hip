// tc_moe.hip -- MoE prefill over expert-sorted rows: the device-side router,
// the SwiGLU between the grouped gate/up and down GEMMs, and the rank-order
// combination of the down outputs.
//
// The reference's batched MoE (src/cpp/core/cuda/forward/MoeBatch.cu:37-197)
// gathers each expert's tokens on the host and runs one int8Gemm per expert
// and matrix; its device-resident variant keeps expert-sorted token lists
// (moePreStart_/moePreTok_, include/GPUCompute.hpp:730-738). Here the sort is
// done on the device from the router's ids, and ONE grouped GEMM launch per
// matrix covers every expert (tiles never straddle two experts), so no host
// round trip or per-expert launch sits between the router and the experts.
#include "tc_kernels.hpp"

namespace tc {
namespace {

constexpr uint32_t kRouteThreads = 1024;
constexpr uint32_t kRouteMaxExperts = 4096;

// One workgroup: per-expert counts (LDS atomics), their prefix sums, the tile
// table, then each pair's row (an LDS cursor per expert). An expert's segment
// starts at a multiple of `pad` rows and is cut into tiles of `tile` rows.
// Rows of one expert come in no fixed order, which changes nothing: every row
// is computed alone and the combination reads rows by pair.
__global__ __launch_bounds__(kRouteThreads) void k_moe_route(const int32_t *__restrict__ ids, uint32_t npairs,
                                                             uint32_t top_k, uint32_t E, uint32_t pad, uint32_t tile,
                                                             uint32_t rows_max,
                                                             int32_t *__restrict__ pos, uint32_t *__restrict__ row_tok,
                                                             uint32_t *__restrict__ mt, uint32_t *__restrict__ ntm) {
    __shared__ uint32_t cnt[kRouteMaxExperts], start[kRouteMaxExperts];
    __shared__ uint32_t wsum[kRouteThreads / 64], wtile[kRouteThreads / 64];
    const uint32_t tid = threadIdx.x;
    for (uint32_t e = tid; e < E; e += kRouteThreads) cnt[e] = 0;
    // rows that no pair lands on (padding, skipped pairs) are marked ~0
    for (uint32_t i = tid; i < rows_max; i += kRouteThreads) row_tok[i] = ~0u;
    __syncthreads();
    for (uint32_t p = tid; p < npairs; p += kRouteThreads) {
        const int32_t e = ids[p];
        if (e >= 0 && uint32_t(e) < E) atomicAdd(&cnt[e], 1u);
    }
    __syncthreads();
    // Exclusive prefix sums of rows and of tiles over the experts: each thread
    // owns a contiguous range of experts, then the per-thread totals are
    // scanned across the workgroup.
    const uint32_t per = (E + kRouteThreads - 1) / kRouteThreads;
    const uint32_t e0 = min(E, tid * per), e1 = min(E, e0 + per);
    uint32_t rows = 0, tiles = 0;
    for (uint32_t e = e0; e < e1; ++e) {
        rows += (cnt[e] + pad - 1) / pad * pad;
        tiles += (cnt[e] + tile - 1) / tile;
    }
    const uint32_t lane = tid & 63, wave = tid >> 6;
    uint32_t ir = rows, it = tiles;  // inclusive scans within the wave
    for (uint32_t o = 1; o < 64; o <<= 1) {
        const uint32_t vr = __shfl_up(ir, o), vt = __shfl_up(it, o);
        if (lane >= o) {
            ir += vr;
            it += vt;
        }
    }
    if (lane == 63) {
        wsum[wave] = ir;
        wtile[wave] = it;
    }
    __syncthreads();
    uint32_t br = 0, bt = 0;
    for (uint32_t w = 0; w < wave; ++w) {
        br += wsum[w];
        bt += wtile[w];
    }
    uint32_t r0 = br + ir - rows, t0 = bt + it - tiles;
    for (uint32_t e = e0; e < e1; ++e) {
        start[e] = r0;
        const uint32_t c = cnt[e];
        for (uint32_t j = 0; j * tile < c; ++j) {
            uint32_t *m = mt + 3 * size_t(t0 + j);
            m[0] = r0 + j * tile;
            m[1] = r0 + min(c, (j + 1) * tile);
            m[2] = e;
        }
        r0 += (c + pad - 1) / pad * pad;
        t0 += (c + tile - 1) / tile;
    }
    if (tid == kRouteThreads - 1) *ntm = t0;  // the last thread's end is the total
    // (the row_tok marks above are ordered before the stores below by this barrier)
    __syncthreads();
    for (uint32_t p = tid; p < npairs; p += kRouteThreads) {
        const int32_t e = ids[p];
        int32_t q = -1;
        if (e >= 0 && uint32_t(e) < E) {
            q = int32_t(atomicAdd(&start[e], 1u));
            row_tok[q] = p / top_k;
        }
        pos[p] = q;
    }
}

__global__ __launch_bounds__(256) void k_moe_swiglu(float *__restrict__ g, const float *__restrict__ u, size_t n) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    g[i] = gv / (1.0f + expf(-gv)) * u[i];
}

// Rank-order weighted sum (ModelMoE.cpp:990-1002): from 0, fma per rank.
__global__ __launch_bounds__(256) void k_moe_combine_rows(const float *__restrict__ y, const int32_t *__restrict__ pos,
                                                          const float *__restrict__ wts, float *__restrict__ out,
                                                          uint32_t top_k, uint32_t H, uint32_t nchunk) {
    const uint32_t t = blockIdx.x / nchunk;
    const uint32_t i = (blockIdx.x - t * nchunk) * 256 + threadIdx.x;
    if (i >= H) return;
    float acc = 0.0f;
    for (uint32_t r = 0; r < top_k; ++r) {
        const int32_t q = pos[size_t(t) * top_k + r];
        if (q >= 0) acc = fmaf(wts[size_t(t) * top_k + r], y[size_t(q) * H + i], acc);
    }
    out[size_t(t) * H + i] = acc;
}

}  // namespace

uint32_t moe_max_tiles(uint32_t npairs, uint32_t n_experts, uint32_t tile) {
    // every expert's last tile may be partial
    return (npairs + tile - 1) / tile + std::min(npairs, n_experts);
}

uint32_t moe_max_rows(uint32_t npairs, uint32_t n_experts, uint32_t pad) {
    return npairs + (pad - 1) * std::min(npairs, n_experts);
}

hipError_t launch_moe_route(const int32_t *ids, uint32_t npairs, uint32_t top_k, uint32_t n_experts, uint32_t pad,
                            uint32_t tile, int32_t *pos, uint32_t *row_tok, uint32_t *mt, uint32_t *ntm,
                            hipStream_t st) {
    if (npairs == 0 || top_k == 0 || n_experts == 0 || n_experts > kRouteMaxExperts || pad == 0 || tile == 0)
        return hipErrorInvalidValue;
    k_moe_route<<<1, kRouteThreads, 0, st>>>(ids, npairs, top_k, n_experts, pad, tile,
                                             moe_max_rows(npairs, n_experts, pad), pos, row_tok, mt, ntm);
    return hipGetLastError();
}

hipError_t launch_moe_swiglu(float *g, const float *u, uint32_t nrows_max, uint32_t ff, hipStream_t st) {
    const size_t n = size_t(nrows_max) * ff;
    if (n == 0) return hipErrorInvalidValue;
    k_moe_swiglu<<<uint32_t((n + 255) / 256), 256, 0, st>>>(g, u, n);
    return hipGetLastError();
}

hipError_t launch_moe_combine_rows(const float *y, const int32_t *pos, const float *wts, float *out, uint32_t T,
                                   uint32_t top_k, uint32_t H, hipStream_t st) {
    const uint32_t nchunk = (H + 255) / 256;
    if (T == 0 || H == 0 || uint64_t(T) * nchunk >= (uint64_t(1) << 31)) return hipErrorInvalidValue;
    k_moe_combine_rows<<<T * nchunk, 256, 0, st>>>(y, pos, wts, out, top_k, H, nchunk);
    return hipGetLastError();
}

}  // namespace tc
