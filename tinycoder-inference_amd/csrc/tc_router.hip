// tc_router.hip -- the qwen35moe MoE router on the device: the F32 router
// mat-vec (logits), the softmax over all experts, the top-k selection and the
// clamped renormalisation, bit-identical to the reference CPU router
// (src/cpp/core/ModelMoE.cpp:341-425, computeQwen35MoERouterOnly).
//
// The CPU router is the reference's exact path; its GPU kernel
// (include/gpu/GpuQwen35Kernels.hpp:931, kQ35MoeRouter) uses float exp and
// an insertion top-k and so differs from it on close and tied
// probabilities. Here every step follows the CPU's evaluation:
//  * logits: the AVX2 F32 kernel's order (SIMDMatMulVecAVX2.cpp:2982-3090):
//    32 FMA lanes (four 8-wide chains) over the 32-column steps, the leftover
//    8-column groups into chain 0, its fixed horizontal tree, then the
//    cols % 8 tail as serial FMAs;
//  * probabilities: float(exp(double(l) - maxL)), summed in double in expert
//    order, scaled by float(1 / sum) in float;
//  * selection: std::partial_sort's order, ties included (a k-entry binary
//    heap whose top is the smallest probability, replaced by each later entry
//    with a strictly larger one, then heap-sorted; the sift moves of the GNU
//    C++ library, whose tie order the result depends on);
//  * weights: p / float(max(double sum of the k, 6.103515625e-5)).
#include "tc_kernels.hpp"

namespace tc {
namespace {

constexpr uint32_t kRowsPerBlock = 8;  // router rows per 256-thread workgroup (32 lanes each)
constexpr uint32_t kSelectMaxExperts = 4096;

// out[s][r] = x[s] . W[r] for 8 rows per workgroup, token blockIdx.y.
__global__ __launch_bounds__(256) void k_router_logits(const float *__restrict__ W, const float *__restrict__ X,
                                                       uint32_t rows, uint32_t cols, float *__restrict__ out) {
    __shared__ float acc[kRowsPerBlock][33];
    const uint32_t lane = threadIdx.x & 31, rl = threadIdx.x >> 5;
    const uint32_t r = blockIdx.x * kRowsPerBlock + rl, s = blockIdx.y;
    const float *x = X + size_t(s) * cols;
    const float *w = W + size_t(r < rows ? r : 0) * cols;
    const uint32_t vec = cols / 8 * 8;
    float a = 0.0f;
    uint32_t i = 0;
    for (; i + 31 < vec; i += 32) a = fmaf(x[i + lane], w[i + lane], a);
    for (; i + 7 < vec; i += 8)  // whole 8-column groups left: chain 0 only
        if (lane < 8) a = fmaf(x[i + lane], w[i + lane], a);
    acc[rl][lane] = a;
    __syncthreads();
    if (lane == 0 && r < rows) {
        const float *c = acc[rl];  // chain k lane j at c[8k + j]
        float sv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) sv[j] = (c[j] + c[8 + j]) + (c[16 + j] + c[24 + j]);
        float t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = sv[j] + sv[j + 4];
        float v = (t[0] + t[1]) + (t[2] + t[3]);
        for (uint32_t k = vec; k < cols; ++k) v = fmaf(x[k], w[k], v);
        out[size_t(s) * rows + r] = v;
    }
}

struct Scored {
    float p;
    uint32_t e;
};

__device__ __forceinline__ bool before(const Scored &a, const Scored &b) { return a.p > b.p; }

__device__ void heap_push_up(Scored *h, uint32_t hole, uint32_t top, Scored v) {
    uint32_t parent = (hole - 1) / 2;
    while (hole > top && before(h[parent], v)) {
        h[hole] = h[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    h[hole] = v;
}

// Sift-down of the hole to a leaf along the child not before its sibling,
// then sift-up of v.
__device__ void heap_adjust(Scored *h, uint32_t hole, uint32_t len, Scored v) {
    const uint32_t top = hole;
    uint32_t child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (before(h[child], h[child - 1])) child--;
        h[hole] = h[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        h[hole] = h[child - 1];
        hole = child - 1;
    }
    heap_push_up(h, hole, top, v);
}

// One wave per token: softmax, selection and weights.
__global__ __launch_bounds__(64) void k_router_select(const float *__restrict__ logits, uint32_t E, uint32_t K,
                                                      int32_t *__restrict__ ids, float *__restrict__ wts) {
    extern __shared__ __align__(16) unsigned char smem[];
    float *prob = reinterpret_cast<float *>(smem);               // [E]
    Scored *heap = reinterpret_cast<Scored *>(smem + 4 * E);     // [K]
    const uint32_t s = blockIdx.x, lane = threadIdx.x;
    const float *l = logits + size_t(s) * E;
    float m = -__builtin_inff();
    for (uint32_t e = lane; e < E; e += 64) m = fmaxf(m, l[e]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const double maxL = double(m);
    for (uint32_t e = lane; e < E; e += 64) prob[e] = float(exp(double(l[e]) - maxL));
    __syncthreads();
    if (lane != 0) return;
    double sum = 0.0;
    for (uint32_t e = 0; e < E; ++e) sum += double(prob[e]);
    const float inv = float(1.0 / sum);
    // std::partial_sort over entries (prob[e] * inv, e): the heap of the first K,
    // each later strictly larger entry replacing the top, then the heap sort.
    for (uint32_t e = 0; e < K; ++e) heap[e] = Scored{prob[e] * inv, e};
    if (K > 1)
        for (uint32_t parent = (K - 2) / 2;; --parent) {
            heap_adjust(heap, parent, K, heap[parent]);
            if (parent == 0) break;
        }
    for (uint32_t e = K; e < E; ++e) {
        const Scored v{prob[e] * inv, e};
        if (before(v, heap[0])) heap_adjust(heap, 0, K, v);
    }
    for (uint32_t last = K; last > 1;) {
        --last;
        const Scored v = heap[last];
        heap[last] = heap[0];
        heap_adjust(heap, 0, last, v);
    }
    double wsum = 0.0;
    for (uint32_t r = 0; r < K; ++r) wsum += double(heap[r].p);
    const float wc = float(wsum > 6.103515625e-5 ? wsum : 6.103515625e-5);
    for (uint32_t r = 0; r < K; ++r) {
        ids[size_t(s) * K + r] = int32_t(heap[r].e);
        wts[size_t(s) * K + r] = __fdiv_rn(heap[r].p, wc);
    }
}

}  // namespace

hipError_t launch_router_logits(const float *W, const float *X, uint32_t S, uint32_t rows, uint32_t cols, float *out,
                                hipStream_t st) {
    if (S == 0 || rows == 0 || cols == 0 || S > 65535) return hipErrorInvalidValue;
    k_router_logits<<<dim3{(rows + kRowsPerBlock - 1) / kRowsPerBlock, S, 1u}, 256, 0, st>>>(W, X, rows, cols, out);
    return hipGetLastError();
}

hipError_t launch_router_select(const float *logits, uint32_t S, uint32_t E, uint32_t K, int32_t *ids, float *wts,
                                hipStream_t st) {
    if (S == 0 || E == 0 || K == 0 || K > E || E > kSelectMaxExperts) return hipErrorInvalidValue;
    const uint32_t lds = 4 * E + 8 * K;
    k_router_select<<<S, 64, lds, st>>>(logits, E, K, ids, wts);
    return hipGetLastError();
}

}  // namespace tc
