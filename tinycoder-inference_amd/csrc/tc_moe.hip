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
#include "tc_actquant.hpp"
#include "tc_kernels.hpp"

namespace tc {
namespace {

constexpr uint32_t kRouteThreads = 1024;
constexpr uint32_t kRouteMaxExperts = 4096;
constexpr uint32_t kRouteMapWords = 8192;  // per-expert token bitmaps kept in LDS up to E * ceil(T / 32) words
constexpr uint32_t kRouteLdsIds = 8192;    // ids read once into LDS up to this many pairs

// One workgroup: per-expert counts (LDS atomics), their prefix sums, the tile
// table, then each pair's row. An expert's segment starts at a multiple of
// `pad` rows and is cut into tiles of `tile` rows. Within its segment an
// expert's pairs take rows in pair order (token order): a row's place in the
// tiles decides how the GEMM splits its K range, and so the rounding of its
// sum, so the order is fixed rather than left to the atomics. A pair's row is
// its segment start plus the number of earlier tokens routed to its expert:
// from a bitmap per expert over the tokens and its per-word prefix counts in
// LDS. (Calls whose bitmaps exceed LDS, or whose ids repeat an expert within
// a token, count the earlier pairs of the segment instead.)
__global__ __launch_bounds__(kRouteThreads) void k_moe_route(const int32_t *__restrict__ ids, uint32_t npairs,
                                                             uint32_t top_k, uint32_t E, uint32_t pad, uint32_t tile,
                                                             uint32_t rows_max,
                                                             int32_t *__restrict__ pos, uint32_t *__restrict__ row_tok,
                                                             uint32_t *__restrict__ mt, uint32_t *__restrict__ ntm) {
    __shared__ uint32_t cnt[kRouteMaxExperts], start[kRouteMaxExperts];
    __shared__ uint32_t bmap[kRouteMapWords], bpre[kRouteMapWords];
    __shared__ uint32_t wsum[kRouteThreads / 64], wtile[kRouteThreads / 64];
    __shared__ uint32_t dup;
    __shared__ int32_t sids[kRouteLdsIds];
    const uint32_t tid = threadIdx.x;
    // the pairs' experts, read once (every loop below walks them; from
    // global memory each iteration waited a full round trip)
    const bool ids_lds = npairs <= kRouteLdsIds;
    if (ids_lds) {
        constexpr uint32_t NI = kRouteLdsIds / kRouteThreads;
        int32_t v[NI];  // all loads in flight before the first store
#pragma unroll
        for (uint32_t k = 0; k < NI; ++k) {
            const uint32_t p = tid + k * kRouteThreads;
            v[k] = p < npairs ? ids[p] : 0;
        }
#pragma unroll
        for (uint32_t k = 0; k < NI; ++k) {
            const uint32_t p = tid + k * kRouteThreads;
            if (p < npairs) sids[p] = v[k];
        }
    }
    const int32_t *const eid = ids_lds ? sids : ids;
    // bitmap words per expert, padded to an odd count: a wave's lanes reading
    // one word index of different experts then fall on different banks
    const uint32_t ntok = npairs / top_k, W = ((ntok + 31) / 32) | 1u;  // npairs = tokens x top_k
    // token of pair p: p / top_k as a multiply-high by ceil(2^32 / top_k)
    // (exact for p < 2^32 / top_k: the error term p * (m*top_k - 2^32) / 2^32
    // stays below the gap to the next multiple)
    const uint32_t tdiv = 0xFFFFFFFFu / top_k + 1u;
    auto tok_of = [&](uint32_t p) __attribute__((always_inline)) {
        return top_k == 1 ? p : __umulhi(p, tdiv);
    };
    const bool use_map = uint64_t(E) * W <= kRouteMapWords;
    for (uint32_t e = tid; e < E; e += kRouteThreads) cnt[e] = 0;
    if (use_map)
        for (uint32_t i = tid; i < E * W; i += kRouteThreads) bmap[i] = 0;
    if (tid == 0) dup = 0;
    // rows that no pair lands on (padding, skipped pairs) are marked ~0
    for (uint32_t i = tid; i < rows_max; i += kRouteThreads) row_tok[i] = ~0u;
    __syncthreads();
    for (uint32_t p = tid; p < npairs; p += kRouteThreads) {
        const int32_t e = eid[p];
        if (e >= 0 && uint32_t(e) < E) {
            atomicAdd(&cnt[e], 1u);
            if (use_map) {
                const uint32_t t = tok_of(p), bit = 1u << (t & 31);
                if (atomicOr(&bmap[uint32_t(e) * W + t / 32], bit) & bit) dup = 1;  // the expert twice in a token
            }
        }
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
    if (use_map && dup == 0) {
        // per expert, the earlier tokens' count at each bitmap word
        for (uint32_t e = tid; e < E; e += kRouteThreads) {
            uint32_t run = 0;
            for (uint32_t w = 0; w < W; ++w) {
                bpre[e * W + w] = run;
                run += __builtin_popcount(bmap[e * W + w]);
            }
        }
        __syncthreads();
        for (uint32_t p = tid; p < npairs; p += kRouteThreads) {
            const int32_t e = eid[p];
            int32_t q = -1;
            if (e >= 0 && uint32_t(e) < E) {
                const uint32_t t = tok_of(p), i = uint32_t(e) * W + t / 32;
                q = int32_t(start[e] + bpre[i] + __builtin_popcount(bmap[i] & ((1u << (t & 31)) - 1u)));
                row_tok[q] = t;
            }
            pos[p] = q;
        }
    } else {
        // the pair index at some row of its expert's segment (row_tok as
        // scratch), then each pair's rank among the segment's pairs
        for (uint32_t p = tid; p < npairs; p += kRouteThreads) {
            const int32_t e = eid[p];
            if (e >= 0 && uint32_t(e) < E) row_tok[atomicAdd(&start[e], 1u)] = p;
        }
        __syncthreads();
        for (uint32_t p = tid; p < npairs; p += kRouteThreads) {
            const int32_t e = eid[p];
            int32_t q = -1;
            if (e >= 0 && uint32_t(e) < E) {
                const uint32_t s1 = start[e], s0 = s1 - cnt[e];  // start[e] is now the segment's end
                uint32_t rank = 0;
                for (uint32_t r = s0; r < s1; ++r) rank += row_tok[r] < p ? 1u : 0u;
                q = int32_t(s0 + rank);
            }
            pos[p] = q;
        }
        __syncthreads();  // every scratch record read before row_tok is written
        for (uint32_t p = tid; p < npairs; p += kRouteThreads) {
            const int32_t q = pos[p];
            if (q >= 0) row_tok[q] = p / top_k;
        }
    }
}

// MoE: h = silu(g) * u elementwise (the FFN's SwiGLU, as the decode kernels'
// epilogue forms it) quantized to Q8_K straight from registers, one wave per
// 256-element block of h, block-major: h never goes to memory. (Compiled with
// the mat-vec kernels' flags, so that h is bit for bit the decode SwiGLU
// epilogue's; the quantizer keeps its one sum apart from its product itself.)
__global__ __launch_bounds__(256) void k_swiglu_quant_q8k(const float *__restrict__ g, const float *__restrict__ u,
                                                          int8_t *__restrict__ qs, float *__restrict__ d,
                                                          int16_t *__restrict__ bsums, uint16_t *__restrict__ dg,
                                                          uint32_t nblk_total, uint32_t nbk, uint32_t bm_S) {
    const uint32_t gb = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (gb >= nblk_total) return;
    const uint32_t lane = threadIdx.x & 63;
    const float4 gv = reinterpret_cast<const float4 *>(g + size_t(gb) * 256)[lane];
    const float4 uv = reinterpret_cast<const float4 *>(u + size_t(gb) * 256)[lane];
    float4 h;
    h.x = gv.x / (1.0f + expf(-gv.x)) * uv.x;
    h.y = gv.y / (1.0f + expf(-gv.y)) * uv.y;
    h.z = gv.z / (1.0f + expf(-gv.z)) * uv.z;
    h.w = gv.w / (1.0f + expf(-gv.w)) * uv.w;
    const uint32_t o = (gb % nbk) * bm_S + gb / nbk;  // block-major
    quant_q8k_block_wave_v(h, qs + size_t(o) * 256, d + o, bsums + size_t(o) * 16, dg + size_t(o) * 16);
}

// Rank-order weighted sum (ModelMoE.cpp:990-1002): from 0, fma per rank.
// A thread sums 4 consecutive outputs (16-byte loads); with top_k <= 8 the
// loads of every rank are issued before the first fma (the same fma order).
template <bool VEC>
__global__ __launch_bounds__(256) void k_moe_combine_rows(const float *__restrict__ y, const int32_t *__restrict__ pos,
                                                          const float *__restrict__ wts, float *__restrict__ out,
                                                          uint32_t top_k, uint32_t H, uint32_t nchunk) {
    const uint32_t t = blockIdx.x / nchunk;
    const uint32_t i = ((blockIdx.x - t * nchunk) * 256 + threadIdx.x) * 4;
    if (i >= H) return;
    const int32_t *pt = pos + size_t(t) * top_k;
    const float *wt = wts + size_t(t) * top_k;
    if constexpr (VEC) {
        // H % 4 == 0 and top_k <= 8
        float4 v[8];
        float w[8];
#pragma unroll
        for (uint32_t r = 0; r < 8; ++r) {
            const int32_t q = r < top_k ? pt[r] : -1;
            w[r] = q >= 0 ? wt[r] : 0.0f;
            v[r] = q >= 0 ? *reinterpret_cast<const float4 *>(y + size_t(q) * H + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (uint32_t r = 0; r < 8; ++r) {
            if (r < top_k && pt[r] >= 0) {
                acc.x = fmaf(w[r], v[r].x, acc.x);
                acc.y = fmaf(w[r], v[r].y, acc.y);
                acc.z = fmaf(w[r], v[r].z, acc.z);
                acc.w = fmaf(w[r], v[r].w, acc.w);
            }
        }
        *reinterpret_cast<float4 *>(out + size_t(t) * H + i) = acc;
    } else {
        for (uint32_t e = 0; e < 4 && i + e < H; ++e) {
            float acc = 0.0f;
            for (uint32_t r = 0; r < top_k; ++r) {
                const int32_t q = pt[r];
                if (q >= 0) acc = fmaf(wt[r], y[size_t(q) * H + i + e], acc);
            }
            out[size_t(t) * H + i + e] = acc;
        }
    }
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
    if (npairs == 0 || top_k == 0 || n_experts == 0 || n_experts > kRouteMaxExperts || pad == 0 || tile == 0 ||
        uint64_t(npairs) * top_k >= (uint64_t(1) << 32))  // (the kernel's token-of-pair division)
        return hipErrorInvalidValue;
    k_moe_route<<<1, kRouteThreads, 0, st>>>(ids, npairs, top_k, n_experts, pad, tile,
                                             moe_max_rows(npairs, n_experts, pad), pos, row_tok, mt, ntm);
    return hipGetLastError();
}

hipError_t launch_swiglu_quant_q8k(const float *g, const float *u, uint32_t S, uint32_t cols, const ActLayout &L,
                                   void *buf, hipStream_t st) {
    if (S == 0 || cols == 0 || cols % 256) return hipErrorInvalidValue;
    const uint32_t nbk = cols / 256, nb = S * nbk;
    char *b = static_cast<char *>(buf);
    k_swiglu_quant_q8k<<<(nb + 3) / 4, 256, 0, st>>>(g, u, reinterpret_cast<int8_t *>(b + L.qs_off),
                                                     reinterpret_cast<float *>(b + L.d_off),
                                                     reinterpret_cast<int16_t *>(b + L.bs_off),
                                                     reinterpret_cast<uint16_t *>(b + L.dg_off), nb, nbk, S);
    return hipGetLastError();
}

hipError_t launch_moe_combine_rows(const float *y, const int32_t *pos, const float *wts, float *out, uint32_t T,
                                   uint32_t top_k, uint32_t H, hipStream_t st) {
    const uint32_t nchunk = (H + 1023) / 1024;  // 4 outputs per thread
    if (T == 0 || H == 0 || uint64_t(T) * nchunk >= (uint64_t(1) << 31)) return hipErrorInvalidValue;
    // (y is the library's own buffer: 16-byte aligned; out is the caller's)
    if (H % 4 == 0 && top_k <= 8 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0)
        k_moe_combine_rows<true><<<T * nchunk, 256, 0, st>>>(y, pos, wts, out, top_k, H, nchunk);
    else
        k_moe_combine_rows<false><<<T * nchunk, 256, 0, st>>>(y, pos, wts, out, top_k, H, nchunk);
    return hipGetLastError();
}

}  // namespace tc
