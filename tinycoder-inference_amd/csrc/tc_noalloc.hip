// tc_noalloc.hip -- the prefill GEMM for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc): tc_gemm_noalloc runs the same kernels as tc_gemm with its
// scratch (the quantized activations and the split / stream-K partials) in a
// fixed file-scope device array instead of the library's grow-only buffers.
//
// The array lives once per GPU for the life of the process. Host code never
// uses its name as a device address: its address on each device is read once,
// with that device current, through hipGetSymbolAddress, and kept per device.
// Every call on a GPU shares that GPU's array, so calls that overlap on one GPU
// (different streams, no ordering between them) race; calls on one stream, or
// otherwise ordered, do not. Nothing in the array needs to start at zero: each
// call writes every byte it later reads.
#include <hip/hip_runtime.h>

#include <mutex>

#include "tc_kernels.hpp"
#include "tc_qmatmul.h"

namespace {

constexpr size_t kScratchBytes = size_t(128) << 20;  // TC_GEMM_NOALLOC_SCRATCH_BYTES

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch` (looked up once per device).
int scratch_on_device(void **ptr) {
    int id = 0;
    if (hipGetDevice(&id) != hipSuccess || id < 0 || id >= kMaxDevices)
        return tc::fail_code(TC_E_UNSUPPORTED, "no usable device");
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_scratch_ptr[id] == nullptr) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return tc::fail_code(TC_E_LAUNCH, "hipGetSymbolAddress(scratch) failed");
        g_scratch_ptr[id] = p;
    }
    *ptr = g_scratch_ptr[id];
    return TC_OK;
}

}  // namespace

extern "C" {

size_t tc_gemm_noalloc_scratch_bytes(void) { return kScratchBytes; }

int tc_gemm_noalloc(int type, const void *w, const float *x, float *out, uint32_t seq_len, uint32_t rows,
                    uint32_t cols, uint32_t blocks_per_row, void *stream) {
    const int num_cu = tc::device_cu_count();
    if (num_cu == 0) return tc::fail_code(TC_E_UNSUPPORTED, "no gfx950 device");
    int rc = tc::gemm_entry_check(type, w, x, out, seq_len, rows, cols, blocks_per_row);
    if (rc) return rc;
    if ((rc = tc::gemm_mfma_check(type, seq_len, rows, cols))) return rc;
    size_t act_bytes = 0;
    const size_t ws_bytes = tc::gemm_mfma_scratch(type, seq_len, rows, cols, num_cu, &act_bytes);
    const size_t act_room = (act_bytes + 255) & ~size_t(255);
    if (act_room + ws_bytes > kScratchBytes)
        return tc::fail_code(TC_E_UNSUPPORTED, "shape needs more than the 128 MiB no-alloc scratch (use tc_gemm)");
    void *base = nullptr;
    if ((rc = scratch_on_device(&base))) return rc;
    unsigned char *b = static_cast<unsigned char *>(base);
    return tc::gemm_mfma_into(type, w, x, out, seq_len, rows, cols, num_cu, b, ws_bytes ? b + act_room : nullptr,
                              static_cast<hipStream_t>(stream));
}

}  // extern "C"
