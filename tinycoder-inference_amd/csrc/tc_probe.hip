// tc_probe.hip -- roof probes of this part, for reading the kernels' measured
// rates against what the hardware sustains (not on any compute path).
//
//  * int8 MFMA: v_mfma_i32_32x32x32_i8 back to back, four independent
//    accumulator chains per wave, two waves per SIMD, register operands only.
//  * HBM read: every byte of a buffer read once with 16-byte non-temporal
//    buffer loads, one contiguous chunk per workgroup (the decode kernels'
//    access pattern without any decode work).
#include "tc_common.hpp"

#include "tc_qmatmul.h"

namespace tc {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_probe_mfma(int *sink, uint32_t iters) {
    const v4i a = {int(threadIdx.x), 1, 2, 3}, b = {3, int(threadIdx.x), 1, 2};
    v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (uint32_t i = 0; i < iters; ++i) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c3, 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
    sink[blockIdx.x * 256 + threadIdx.x] = s;
}

__global__ __launch_bounds__(512) void k_probe_read(const uint8_t *buf, uint64_t chunk, uint64_t bytes,
                                                    uint32_t *sink) {
    const uint64_t begin = uint64_t(blockIdx.x) * chunk;
    const uint64_t n = begin < bytes ? (bytes - begin < chunk ? bytes - begin : chunk) : 0;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(buf + begin), short(0), int(uint32_t(n)), 0x00020000);
    u32x4 acc = {0, 0, 0, 0};
    // 8 loads of 16 B per lane in flight per round: 64 KB per workgroup round
    for (uint32_t off = threadIdx.x * 16u; off < n; off += 8u * 512u * 16u) {
        u32x4 v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + k * 512u * 16u, 0, 2);
#pragma unroll
        for (int k = 0; k < 8; ++k) acc ^= v[k];
    }
    sink[blockIdx.x * 512 + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

}  // namespace
}  // namespace tc

extern "C" {

size_t tc_probe_sink_bytes(void) { return size_t(8192) * 512 * 4; }

int tc_probe_mfma_i8(uint32_t workgroups, uint32_t iters, void *sink, void *stream) {
    if (sink == nullptr || workgroups == 0 || workgroups > 8192) return TC_E_ARG;
    tc::k_probe_mfma<<<workgroups, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<int *>(sink), iters);
    return hipGetLastError() == hipSuccess ? TC_OK : TC_E_LAUNCH;
}

int tc_probe_read(const void *buf, size_t bytes, uint32_t workgroups, void *sink, void *stream) {
    if (buf == nullptr || sink == nullptr || workgroups == 0 || workgroups > 8192) return TC_E_ARG;
    const uint64_t chunk = ((uint64_t(bytes) + workgroups - 1) / workgroups + 16383) & ~uint64_t(16383);
    if (chunk >= (uint64_t(1) << 31)) return TC_E_ARG;
    tc::k_probe_read<<<workgroups, 512, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const uint8_t *>(buf),
                                                                              chunk, bytes, static_cast<uint32_t *>(sink));
    return hipGetLastError() == hipSuccess ? TC_OK : TC_E_LAUNCH;
}

}  // extern "C"
