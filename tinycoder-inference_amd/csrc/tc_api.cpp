// tc_api.cpp -- host side of libtc_hip.so: device query, grow-only scratch,
// argument checks and the extern "C" entry points declared in
// include/tc_qmatmul.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "tc_kernels.hpp"
#include "tc_qmatmul.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(e == hipErrorInvalidValue ? TC_E_UNSUPPORTED : TC_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

struct Device {
    bool ok = false;
    int id = 0, num_cu = 0;
    void *act = nullptr;  // quantized activations
    size_t act_bytes = 0;
    void *aux = nullptr;  // kernel intermediates (MoE hidden, GEMM partials)
    size_t aux_bytes = 0;
    void *pad = nullptr;  // zero-padded copies of Q8_0 rows of a width not a multiple of 256
    size_t pad_bytes = 0;
};

std::mutex g_mu;
std::vector<Device> g_dev;

// Device attributes are read once per device (the reference's ctx(),
// GemmDispatch.cu:208-234).
Device *device() {
    int id = 0;
    if (hipGetDevice(&id) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_dev.size() <= size_t(id)) g_dev.resize(id + 1);
    Device &d = g_dev[id];
    if (!d.ok) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, id) != hipSuccess) return nullptr;
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return nullptr;
        d.id = id;
        d.num_cu = prop.multiProcessorCount;
        d.ok = true;
    }
    return &d;
}

bool ensure(void *&p, size_t &cap, size_t need) {
    if (cap >= need) return true;
    if (p != nullptr) {
        // The buffer may still be read by work queued earlier on any stream.
        (void)hipDeviceSynchronize();
        (void)hipFree(p);
    }
    p = nullptr;
    cap = 0;
    if (hipMalloc(&p, need) != hipSuccess) {
        p = nullptr;
        return false;
    }
    cap = need;
    return true;
}

// Bytes past a GEMM activation buffer that the MFMA kernel's tail loads may
// touch: one 128-token tile of 256-byte rows.
constexpr size_t kGemmActSlack = 128 * 256;

// IQ2_XS, IQ4_NL and Q5_0 take fp32 activations (their reference CPU paths do not quantize x):
// the entry points that hand over quantized activations refuse it.
bool int8_act_type(int t) { return t != TC_IQ2_XS && t != TC_IQ4_NL && t != TC_Q5_0; }

bool type_ok(int t) { return t == TC_Q8_0 || t == TC_Q5_0 || t == TC_IQ4_NL || t == TC_IQ4_XS || t == TC_IQ2_XS || t == TC_Q2_K || t == TC_IQ2_S || t == TC_IQ3_S || t == TC_Q3_K || t == TC_Q4_K || t == TC_Q5_K || t == TC_Q6_K || t == TC_IQ3_XXS; }

bool g_q8_gemm_enabled = true;

// Weight types of the int8 MFMA prefill GEMM (the others run the decode
// kernel over groups of 8 tokens).
bool mfma_gemm_type(int t) {
    return t == TC_Q4_K || t == TC_Q5_K || t == TC_Q6_K || t == TC_IQ3_XXS || t == TC_IQ3_S || t == TC_IQ2_S || t == TC_Q8_0;
}

tc::ActView act_view(void *buf, const tc::ActLayout &L, size_t tok, int type, uint32_t cols) {
    const uint32_t blk = type == TC_Q8_0 ? 32u : 256u;
    char *b = static_cast<char *>(buf);
    tc::ActView v;
    v.qs = reinterpret_cast<const int8_t *>(b + L.qs_off) + tok * cols;
    v.d = reinterpret_cast<const float *>(b + L.d_off) + tok * (cols / blk);
    v.bsums = reinterpret_cast<const int16_t *>(b + L.bs_off) + tok * (cols / 16);
    v.dg = reinterpret_cast<const int8_t *>(b + L.dg_off) + tok * (cols / 256) * tc::dg_bytes(type);
    return v;
}

// Activations wider than the mat-vec prologue preloads (S*cols beyond 3
// 16-value chunks per thread: 24576 values for the 512-thread shape, 12288
// for the 256-thread one) are quantized once by a small kernel into the
// device scratch instead of in every workgroup of the mat-vec (whose
// prologue would repeat the work hundreds of times). The fp32-activation
// types (IQ2_XS, IQ4_NL, Q5_0) always stage x in-kernel.
bool prequantize_wide(int type, uint32_t S, uint32_t cols, uint64_t weight_bytes) {
    return size_t(S) * cols > tc::gemv_fused_quant_limit(type, weight_bytes);
}

int launch_jobs(Device *dev, int type, uint32_t S, tc::GemvJob *jobs, uint32_t n, hipStream_t st) {
    const uint64_t wbytes = tc::jobs_weight_bytes(type, jobs, n);
    size_t need = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (jobs[i].x && prequantize_wide(type, S, jobs[i].cols, wbytes)) need += tc::act_layout(type, S, jobs[i].cols).bytes;
    if (need) {
        if (!ensure(dev->act, dev->act_bytes, need)) return fail(TC_E_LAUNCH, "hipMalloc(%zu) failed", need);
        size_t off = 0;
        for (uint32_t i = 0; i < n; ++i) {
            if (!(jobs[i].x && prequantize_wide(type, S, jobs[i].cols, wbytes))) continue;
            const tc::ActLayout L = tc::act_layout(type, S, jobs[i].cols);
            void *buf = static_cast<char *>(dev->act) + off;
            hipError_t e = tc::launch_quant_act(type, jobs[i].x, S, jobs[i].cols, L, buf, st);
            if (e != hipSuccess) return hip_fail(e, "activation quantizer");
            jobs[i].act = act_view(buf, L, 0, type, jobs[i].cols);
            jobs[i].x = nullptr;
            off += L.bytes;
        }
    }
    const hipError_t e = tc::launch_gemv_jobs(type, S, jobs, n, dev->num_cu, st);
    if (e != hipSuccess) return hip_fail(e, "decode mat-vec");
    return TC_OK;
}

// Run one decode job over token chunks that fit the kernel's LDS budget.
// `x` (fp32) is quantized inside the kernel; with x == null the activations
// come from the pre-quantized buffer `act`.
int run_gemv(Device *dev, int type, const void *w, const void *w2, const float *x, const void *act, float *out,
             float *out2, int epi, int32_t *dbg, uint32_t S, uint32_t rows, uint32_t cols, hipStream_t st) {
    const uint32_t smax = tc::gemv_max_tokens(type, cols);
    if (smax == 0) return fail(TC_E_UNSUPPORTED, "cols=%u too wide for the decode kernel", cols);
    const tc::ActLayout L = tc::act_layout(type, S, cols);
    const uint32_t nbr = type == TC_Q8_0 ? cols / 32 : cols / 256;
    const size_t per = type == TC_Q4_K || type == TC_Q5_K ? 8 : type == TC_Q2_K ? 2 : 1;
    for (uint32_t s0 = 0; s0 < S; s0 += smax) {
        const uint32_t n = std::min(smax, S - s0);
        tc::GemvJob job;
        job.W = static_cast<const uint8_t *>(w);
        job.W2 = static_cast<const uint8_t *>(w2);
        if (x)
            job.x = x + size_t(s0) * cols;
        else
            job.act = act_view(const_cast<void *>(act), L, s0, type, cols);
        job.out = out + size_t(s0) * rows;
        job.out2 = out2 ? out2 + size_t(s0) * rows : nullptr;
        job.epi = epi;
        job.rows = rows;
        job.cols = cols;
        job.out_ld = rows;
        job.dbg = dbg ? dbg + size_t(s0) * rows * nbr * per : nullptr;
        const int rc = launch_jobs(dev, type, n, &job, 1, st);
        if (rc) return rc;
    }
    return TC_OK;
}

// Q8_0 rows of a width that is a multiple of 32 but not of 256: the
// reference's Q8_0 dispatch takes any cols % 32 == 0
// (QuantizedMatrix.cpp:96-103), the kernels work on 256-column units.
bool ragged_q80(int type, uint32_t cols) { return type == TC_Q8_0 && cols % 256 != 0 && cols % 32 == 0; }

int check_common(int type, const void *w, const void *x, const void *out, uint32_t S, uint32_t rows,
                 uint32_t cols, bool ragged_ok = false) {
    if (!type_ok(type)) return fail(TC_E_UNSUPPORTED, "unsupported type %d", type);
    if (!w || !x || !out) return fail(TC_E_ARG, "null pointer");
    if (S == 0 || rows == 0 || cols == 0) return fail(TC_E_UNSUPPORTED, "empty shape");
    if (cols % 256 != 0 && !(ragged_ok && ragged_q80(type, cols)))
        return fail(TC_E_UNSUPPORTED, "cols=%u is not a multiple of %u", cols, type == TC_Q8_0 ? 32u : 256u);
    if ((reinterpret_cast<uintptr_t>(w) & 15) || (reinterpret_cast<uintptr_t>(x) & 15))
        return fail(TC_E_UNSUPPORTED, "weights and activations must be 16-byte aligned");
    return TC_OK;
}

// The ragged Q8_0 case runs on zero-padded copies: each weight row and each
// activation row is copied into a row of the next multiple of 256 columns
// (one small copy kernel per operand, into the device's pad scratch). A
// padded weight block has d = 0 and a padded activation block is all zero,
// so it adds exactly 0 to every output; the real blocks are quantized and
// multiplied as they would be in place.
struct Padded {
    const void *w[2] = {nullptr, nullptr};
    const float *x = nullptr;
    uint32_t cols = 0;
};

int pad_q80(Device *dev, const void *w0, const void *w1, uint32_t rows, const float *x, uint32_t S, uint32_t cols,
            Padded *p, hipStream_t st) {
    const uint32_t cp = (cols + 255) / 256 * 256;
    const uint32_t rb = cols / 32 * 34, rbp = cp / 32 * 34;
    const size_t wbytes = (size_t(rows) * rbp + 255) & ~size_t(255);
    const size_t need = wbytes * (w1 ? 2 : 1) + size_t(S) * cp * 4;
    if (!ensure(dev->pad, dev->pad_bytes, need)) return fail(TC_E_LAUNCH, "hipMalloc(%zu) failed", need);
    char *b = static_cast<char *>(dev->pad);
    hipError_t e = tc::launch_pad_rows(w0, rb, b, rbp, rows, st);
    if (e == hipSuccess && w1) e = tc::launch_pad_rows(w1, rb, b + wbytes, rbp, rows, st);
    if (e == hipSuccess && x) e = tc::launch_pad_rows(x, cols * 4, b + wbytes * (w1 ? 2 : 1), cp * 4, S, st);
    if (e != hipSuccess) return hip_fail(e, "Q8_0 row padding");
    p->w[0] = b;
    p->w[1] = w1 ? b + wbytes : nullptr;
    p->x = reinterpret_cast<const float *>(b + wbytes * (w1 ? 2 : 1));
    p->cols = cp;
    return TC_OK;
}

}  // namespace

namespace tc {
// Error text for the calling thread's tc_last_error() (used by tc_gguf.cpp).
void set_error(const std::string &msg) { g_err = msg; }

// Compute units of the current device, 0 when it is not a gfx950.
int device_cu_count() {
    Device *d = device();
    return d ? d->num_cu : 0;
}

// Shape limits of the MFMA prefill GEMM (the int8-activation K-quant and IQ
// types and Q8_0; cols % 256 == 0).
int gemm_mfma_check(int type, uint32_t S, uint32_t rows, uint32_t cols) {
    if (!mfma_gemm_type(type)) return fail(TC_E_UNSUPPORTED, "type %d has no MFMA GEMM", type);
    if (cols % 256) return fail(TC_E_UNSUPPORTED, "cols=%u is not a multiple of 256", cols);
    // 32-bit buffer offsets in the MFMA kernels
    if (uint64_t(S) * cols >= (uint64_t(1) << 32) || uint64_t(rows) * tc_row_bytes(type, cols) >= (uint64_t(1) << 32))
        return fail(TC_E_UNSUPPORTED, "activations or weights of 4 GiB or more");
    return TC_OK;
}

// Device scratch of one MFMA GEMM call: *act_bytes for the block-major
// quantized activations, the return value for the split / stream-K partials.
size_t gemm_mfma_scratch(int type, uint32_t S, uint32_t rows, uint32_t cols, int num_cu, size_t *act_bytes) {
    // + kGemmActSlack: the MFMA kernel's loads for token rows past M in the
    // last superblock run up to one token tile past the buffer (values never
    // stored; the buffer range check covers only the per-lane offset).
    *act_bytes = tc::act_layout(type, S, cols).bytes + kGemmActSlack;
    return tc::prefill_workspace_bytes(type, S, rows, cols, num_cu);
}

// Quantize all tokens once (block-major, into act), then the MFMA kernel
// (partials in ws when the split needs them). No allocation.
int gemm_mfma_into(int type, const void *w, const float *x, float *out, uint32_t S, uint32_t rows, uint32_t cols,
                   int num_cu, void *act, void *ws, hipStream_t st) {
    const tc::ActLayout L = tc::act_layout(type, S, cols);
    // the quantizer also zeroes the prefill GEMM's arrival counters (the
    // head of ws)
    const uint32_t nctr = ws ? tc::prefill_counter_words(type, S, rows, cols, num_cu) : 0;
    hipError_t e = tc::launch_quant_act(type, x, S, cols, L, act, st, true, static_cast<uint32_t *>(ws), nctr);
    if (e != hipSuccess) return hip_fail(e, "activation quantizer");
    e = tc::launch_prefill(type, w, act_view(act, L, 0, type, cols), out, S, rows, cols, num_cu, ws, st);
    if (e != hipSuccess) return hip_fail(e, "int8 MFMA GEMM");
    return TC_OK;
}

int gemm_entry_check(int type, const void *w, const float *x, const float *out, uint32_t S, uint32_t rows,
                     uint32_t cols, uint32_t blocks_per_row) {
    int rc = check_common(type, w, x, out, S, rows, cols);
    if (rc) return rc;
    if (blocks_per_row != cols / uint32_t(tc::block_elems(type)))
        return fail(TC_E_ARG, "blocks_per_row=%u does not match cols=%u", blocks_per_row, cols);
    if (type == TC_Q8_0 && !g_q8_gemm_enabled) return fail(TC_E_UNSUPPORTED, "Q8_0 GEMM disabled");
    return TC_OK;
}

int fail_code(int code, const char *msg) { return fail(code, "%s", msg); }
}  // namespace tc

extern "C" {

int tc_available(void) {
    static const int avail = [] {
        const char *e = std::getenv("TINYCODER_INT8_GEMM");
        if (e != nullptr && e[0] == '0') return 0;
        return device() != nullptr ? 1 : 0;
    }();
    return avail;
}

size_t tc_row_bytes(int type, uint32_t cols) {
    if (!type_ok(type)) return 0;
    const uint32_t be = tc::block_elems(type);
    if (cols % be) return 0;
    return size_t(cols / be) * tc::block_bytes(type);
}

int tc_gemv(int type, const void *w, const float *x, float *out, uint32_t seq_len, uint32_t rows, uint32_t cols,
            void *stream) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    int rc = check_common(type, w, x, out, seq_len, rows, cols, true);
    if (rc) return rc;
    if (seq_len > 8) return fail(TC_E_UNSUPPORTED, "seq_len=%u > 8 (use tc_gemm)", seq_len);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (ragged_q80(type, cols)) {
        Padded p;
        if ((rc = pad_q80(dev, w, nullptr, rows, x, seq_len, cols, &p, st))) return rc;
        return run_gemv(dev, type, p.w[0], nullptr, p.x, nullptr, out, nullptr, 0, nullptr, seq_len, rows, p.cols, st);
    }
    return run_gemv(dev, type, w, nullptr, x, nullptr, out, nullptr, 0, nullptr, seq_len, rows, cols, st);
}

int tc_gemv_multi(int type, uint32_t n, const void *const *w, const float *const *x, float *const *out,
                  const uint32_t *rows, const uint32_t *cols, uint32_t seq_len, void *stream) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    if (!w || !x || !out || !rows || !cols) return fail(TC_E_ARG, "null pointer");
    if (n == 0 || n > 8) return fail(TC_E_UNSUPPORTED, "n=%u matrices (1..8)", n);
    if (seq_len > 8) return fail(TC_E_UNSUPPORTED, "seq_len=%u > 8", seq_len);
    tc::GemvJob jobs[8];
    for (uint32_t i = 0; i < n; ++i) {
        int rc = check_common(type, w[i], x[i], out[i], seq_len, rows[i], cols[i]);
        if (rc) return rc;
        if (seq_len > tc::gemv_max_tokens(type, cols[i]))
            return fail(TC_E_UNSUPPORTED, "seq_len=%u too large for cols=%u in one launch", seq_len, cols[i]);
        jobs[i].W = static_cast<const uint8_t *>(w[i]);
        jobs[i].x = x[i];
        jobs[i].out = out[i];
        jobs[i].rows = rows[i];
        jobs[i].cols = cols[i];
        jobs[i].out_ld = rows[i];
    }
    return launch_jobs(dev, type, seq_len, jobs, n, static_cast<hipStream_t>(stream));
}

size_t tc_act_bytes(int type, uint32_t seq_len, uint32_t cols) {
    if (!type_ok(type) || !int8_act_type(type) || cols % 256) return 0;
    return tc::act_layout(type, seq_len, cols).bytes;
}

int tc_act_quantize(int type, const float *x, uint32_t seq_len, uint32_t cols, void *act, void *stream) {
    if (!device()) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    int rc = check_common(type, act, x, act, seq_len, 1, cols);
    if (rc) return rc;
    if (!int8_act_type(type)) return fail(TC_E_UNSUPPORTED, "type %d takes fp32 activations", type);
    if (reinterpret_cast<uintptr_t>(act) & 255) return fail(TC_E_ARG, "act must be 256-byte aligned");
    const tc::ActLayout L = tc::act_layout(type, seq_len, cols);
    hipError_t e = tc::launch_quant_act(type, x, seq_len, cols, L, act, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "activation quantizer");
    return TC_OK;
}

int tc_gemv_q8(int type, const void *w, const void *act, float *out, uint32_t seq_len, uint32_t rows, uint32_t cols,
               void *stream) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    int rc = check_common(type, w, act, out, seq_len, rows, cols);
    if (rc) return rc;
    if (seq_len > 8) return fail(TC_E_UNSUPPORTED, "seq_len=%u > 8 (use tc_gemm)", seq_len);
    if (!int8_act_type(type)) return fail(TC_E_UNSUPPORTED, "type %d takes fp32 activations", type);
    if (reinterpret_cast<uintptr_t>(act) & 255) return fail(TC_E_ARG, "act must be 256-byte aligned");
    return run_gemv(dev, type, w, nullptr, nullptr, act, out, nullptr, 0, nullptr, seq_len, rows, cols,
                    static_cast<hipStream_t>(stream));
}

int tc_gemv_reserve(uint32_t cols, uint32_t seq_len) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    size_t need = 0;
    for (int t : {TC_Q8_0, TC_Q4_K}) need = std::max(need, tc::act_layout(t, seq_len, cols).bytes);
    if (!ensure(dev->act, dev->act_bytes, need)) return fail(TC_E_LAUNCH, "hipMalloc(%zu) failed", need);
    return TC_OK;
}

int tc_gemv_dual(int type, const void *wg, const void *wu, const float *x, float *gout, float *uout, uint32_t rows,
                 uint32_t cols, void *stream) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    int rc = check_common(type, wg, x, gout, 1, rows, cols, true);
    if (rc) return rc;
    if (!wu || !uout) return fail(TC_E_ARG, "null pointer");
    if ((reinterpret_cast<uintptr_t>(wu) & 15)) return fail(TC_E_UNSUPPORTED, "weights must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (ragged_q80(type, cols)) {
        Padded p;
        if ((rc = pad_q80(dev, wg, wu, rows, x, 1, cols, &p, st))) return rc;
        return run_gemv(dev, type, p.w[0], p.w[1], p.x, nullptr, gout, uout, 1, nullptr, 1, rows, p.cols, st);
    }
    return run_gemv(dev, type, wg, wu, x, nullptr, gout, uout, 1, nullptr, 1, rows, cols, st);
}

int tc_gemm(int type, const void *w, const float *x, float *out, uint32_t seq_len, uint32_t rows, uint32_t cols,
            uint32_t blocks_per_row, void *stream) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    int rc = check_common(type, w, x, out, seq_len, rows, cols, true);
    if (rc) return rc;
    if (blocks_per_row != cols / uint32_t(tc::block_elems(type)))
        return fail(TC_E_ARG, "blocks_per_row=%u does not match cols=%u", blocks_per_row, cols);
    if (type == TC_Q8_0 && !g_q8_gemm_enabled) return fail(TC_E_UNSUPPORTED, "Q8_0 GEMM disabled");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (ragged_q80(type, cols)) {
        if (uint64_t(seq_len) * cols >= (uint64_t(1) << 30))
            return fail(TC_E_UNSUPPORTED, "activations of 4 GiB or more");
        Padded p;
        if ((rc = pad_q80(dev, w, nullptr, rows, x, seq_len, cols, &p, st))) return rc;
        w = p.w[0];
        x = p.x;
        cols = p.cols;
    }
    if (!mfma_gemm_type(type)) {
        // Q2_K / Q3_K / IQ4_XS and the fp32-activation IQ2_XS / IQ4_NL / Q5_0:
        // the exact batched path (the reference's launchQGemm,
        // GpuGemvIQInt8.hpp:771-847) -- the decode kernel over token groups.
        for (uint32_t s0 = 0; s0 < seq_len; s0 += 8) {
            const uint32_t S = std::min(8u, seq_len - s0);
            rc = run_gemv(dev, type, w, nullptr, x + size_t(s0) * cols, nullptr, out + size_t(s0) * rows, nullptr, 0,
                          nullptr, S, rows, cols, st);
            if (rc) return rc;
        }
        return TC_OK;
    }
    if ((rc = tc::gemm_mfma_check(type, seq_len, rows, cols))) return rc;
    size_t act_bytes = 0;
    const size_t ws = tc::gemm_mfma_scratch(type, seq_len, rows, cols, dev->num_cu, &act_bytes);
    if (!ensure(dev->act, dev->act_bytes, act_bytes)) return fail(TC_E_LAUNCH, "hipMalloc(%zu) failed", act_bytes);
    if (ws && !ensure(dev->aux, dev->aux_bytes, ws)) return fail(TC_E_LAUNCH, "hipMalloc(%zu) failed", ws);
    return tc::gemm_mfma_into(type, w, x, out, seq_len, rows, cols, dev->num_cu, dev->act, ws ? dev->aux : nullptr, st);
}

int tc_gemm_preferred(uint32_t type, uint32_t, uint32_t) { return type_ok(int(type)) ? 1 : 0; }

void tc_gemm_set_q8_enabled(int enabled) { g_q8_gemm_enabled = enabled != 0; }

int tc_quantize_act(int type, const float *x, uint32_t seq_len, uint32_t cols, int8_t *qs, float *d, int16_t *bsums,
                    void *stream) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    if (!type_ok(type)) return fail(TC_E_UNSUPPORTED, "unsupported type %d", type);
    if (!int8_act_type(type)) return fail(TC_E_UNSUPPORTED, "type %d takes fp32 activations", type);
    if (!x || !qs || !d || (type != TC_Q8_0 && !bsums)) return fail(TC_E_ARG, "null pointer");
    const uint32_t blk = type == TC_Q8_0 ? 32 : 256;
    if (seq_len == 0 || cols == 0 || cols % blk) return fail(TC_E_UNSUPPORTED, "cols=%u", cols);
    hipStream_t st = static_cast<hipStream_t>(stream);
    // Q8_0 at a width that is not a multiple of 256: quantize zero-padded
    // rows (each 32-block is quantized on its own, so the real blocks come
    // out as they would in place), then copy out the real columns.
    uint32_t cq = cols;
    if (ragged_q80(type, cols)) {
        Padded p;
        int rc = pad_q80(dev, nullptr, nullptr, 0, x, seq_len, cols, &p, st);
        if (rc) return rc;
        x = p.x;
        cq = p.cols;
    }
    const tc::ActLayout L = tc::act_layout(type, seq_len, cq);
    if (!ensure(dev->act, dev->act_bytes, L.bytes)) return fail(TC_E_LAUNCH, "hipMalloc failed");
    hipError_t e = tc::launch_quant_act(type, x, seq_len, cq, L, dev->act, st);
    if (e != hipSuccess) return hip_fail(e, "activation quantizer");
    const char *b = static_cast<const char *>(dev->act);
    e = hipMemcpy2DAsync(qs, cols, b + L.qs_off, cq, cols, seq_len, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(d, size_t(cols / blk) * 4, b + L.d_off, size_t(cq / blk) * 4, size_t(cols / blk) * 4,
                             seq_len, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess && type != TC_Q8_0)
        e = hipMemcpyAsync(bsums, b + L.bs_off, size_t(seq_len) * (cols / 16) * 2, hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return hip_fail(e, "copy");
    return TC_OK;
}

int tc_block_isums(int type, const void *w, const float *x, int32_t *isums, uint32_t seq_len, uint32_t rows,
                   uint32_t cols, void *stream) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    int rc = check_common(type, w, x, isums, seq_len, rows, cols);
    if (rc) return rc;
    if (!int8_act_type(type)) return fail(TC_E_UNSUPPORTED, "type %d has no integer block sums (fp32 path)", type);
    hipStream_t st = static_cast<hipStream_t>(stream);
    // The decode kernel writes the integer sums as a side output; its fp32
    // results land in a scratch row buffer.
    const size_t need = size_t(seq_len) * rows * 4;
    if (!ensure(dev->aux, dev->aux_bytes, need)) return fail(TC_E_LAUNCH, "hipMalloc failed");
    return run_gemv(dev, type, w, nullptr, x, nullptr, static_cast<float *>(dev->aux), nullptr, 0, isums, seq_len,
                    rows, cols, st);
}

int tc_encode(int type, const float *x, void *out, uint32_t rows, uint32_t cols, void *stream) {
    if (!device()) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    if (!type_ok(type)) return fail(TC_E_UNSUPPORTED, "unsupported type %d", type);
    if (!x || !out) return fail(TC_E_ARG, "null pointer");
    if (cols % 256) return fail(TC_E_UNSUPPORTED, "cols=%u is not a multiple of 256", cols);
    const uint64_t units = uint64_t(rows) * (cols / 256);
    if (units >= (1ull << 32)) return fail(TC_E_UNSUPPORTED, "too many blocks");
    hipError_t e = tc::launch_encode(type, x, out, uint32_t(units), static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "encoder");
    return TC_OK;
}

}  // extern "C"

namespace {

// Token count from which tc_moe_ffn runs the grouped GEMM. Below it the
// per-pair mat-vecs win: the GEMM path's eight launches cost more than the
// mat-vecs' work at a few (token, rank) pairs per expert. Measured for 128
// experts x top-8 (2048 x 768 experts): 16 tokens 106 us grouped vs 49 us
// pairs, 64 tokens 151 vs 187 us.
uint32_t g_moe_gemm_min_tokens = 40;

// MoE prefill over expert-sorted rows: device-side routing, the grouped Q4_K
// MFMA GEMM for gate and up (one launch each over all experts), SwiGLU, the
// grouped down GEMM, and the rank-order combination.
int moe_grouped(Device *dev, const float *x, const int32_t *ids, const float *wts, uint32_t T, uint32_t top_k,
                const void *wg, const void *wu, const void *wd, uint32_t E, uint32_t H, uint32_t FF, float *out,
                hipStream_t st) {
    const uint32_t P = T * top_k;
    const uint32_t tile = tc::prefill_grouped_tile(P, E);
    const uint32_t ntm_max = tc::moe_max_tiles(P, E, tile);
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    const tc::ActLayout LX = tc::act_layout(TC_Q4_K, P, H), LH = tc::act_layout(TC_Q4_K, P, FF);
    const size_t ws = std::max(tc::prefill_grouped_workspace_bytes(tile, ntm_max, FF, H, dev->num_cu, 2),
                               tc::prefill_grouped_workspace_bytes(tile, ntm_max, H, FF, dev->num_cu));
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += up(bytes);
        return o;
    };
    const size_t o_pos = take(size_t(P) * 4), o_tok = take(size_t(P) * 4), o_mt = take(size_t(ntm_max) * 12),
                 o_ntm = take(4), o_g = take(size_t(P) * FF * 4), o_u = take(size_t(P) * FF * 4),
                 o_y = take(size_t(P) * H * 4), o_ax = take(LX.bytes + kGemmActSlack),
                 o_ah = take(LH.bytes + kGemmActSlack), o_ws = take(ws);
    // the GEMMs' arrival counters (zeroed by the gather below; each GEMM
    // launch leaves them zero for the next)
    const uint32_t nctr =
        std::max(tc::prefill_grouped_counter_words(ntm_max, FF, 2), tc::prefill_grouped_counter_words(ntm_max, H));
    const size_t o_ctr = take(size_t(nctr) * 4);
    if (!ensure(dev->aux, dev->aux_bytes, off)) return fail(TC_E_LAUNCH, "hipMalloc(%zu) failed", off);
    char *b = static_cast<char *>(dev->aux);
    int32_t *pos = reinterpret_cast<int32_t *>(b + o_pos);
    uint32_t *tok = reinterpret_cast<uint32_t *>(b + o_tok), *mt = reinterpret_cast<uint32_t *>(b + o_mt);
    uint32_t *ntm = reinterpret_cast<uint32_t *>(b + o_ntm);
    float *g = reinterpret_cast<float *>(b + o_g), *u = reinterpret_cast<float *>(b + o_u);
    float *y = reinterpret_cast<float *>(b + o_y);
    const uint64_t gstride = uint64_t(FF) * (H / 256) * 144, dstride = uint64_t(H) * (FF / 256) * 144;

    hipError_t e = tc::launch_moe_route(ids, P, top_k, E, 1, tile, pos, tok, mt, ntm, st);
    if (e != hipSuccess) return hip_fail(e, "MoE router");
    uint32_t *ctr = reinterpret_cast<uint32_t *>(b + o_ctr);
    e = tc::launch_quant_act_rows(x, tok, P, H, LX, b + o_ax, st, ctr, nctr);
    if (e != hipSuccess) return hip_fail(e, "MoE activation gather");
    const tc::ActView ax = act_view(b + o_ax, LX, 0, TC_Q4_K, H);
    // gate and up in one launch (their tiles share the activations)
    e = tc::launch_prefill_grouped(wg, gstride, ax, g, P, FF, H, mt, ntm, ntm_max, tile, dev->num_cu, ctr, b + o_ws,
                                   st, wu, u);
    if (e != hipSuccess) return hip_fail(e, "MoE gate/up GEMM");
    e = tc::launch_swiglu_quant_q8k(g, u, P, FF, LH, b + o_ah, st);
    if (e != hipSuccess) return hip_fail(e, "MoE SwiGLU");
    const tc::ActView ah = act_view(b + o_ah, LH, 0, TC_Q4_K, FF);
    e = tc::launch_prefill_grouped(wd, dstride, ah, y, P, H, FF, mt, ntm, ntm_max, tile, dev->num_cu, ctr, b + o_ws,
                                   st);
    if (e != hipSuccess) return hip_fail(e, "MoE down GEMM");
    e = tc::launch_moe_combine_rows(y, pos, wts, out, T, top_k, H, st);
    if (e != hipSuccess) return hip_fail(e, "MoE combine");
    return TC_OK;
}

}  // namespace

extern "C" {

void tc_moe_set_gemm_min_tokens(uint32_t n) { g_moe_gemm_min_tokens = n; }

int tc_moe_ffn(const float *x, const int32_t *ids, const float *wts, uint32_t seq_len, uint32_t top_k,
               const void *wg, const void *wu, const void *wd, uint32_t n_experts, uint32_t hidden, uint32_t ff,
               float *out, void *stream) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    if (!x || !ids || !wts || !wg || !wu || !wd || !out) return fail(TC_E_ARG, "null pointer");
    if (seq_len == 0 || top_k == 0 || n_experts == 0) return fail(TC_E_ARG, "empty MoE call");
    if (hidden % 256 || ff % 256) return fail(TC_E_UNSUPPORTED, "hidden=%u / ff=%u not multiples of 256", hidden, ff);
    for (const void *p : {wg, wu, wd})
        if (reinterpret_cast<uintptr_t>(p) & 15) return fail(TC_E_UNSUPPORTED, "weights must be 16-byte aligned");
    const uint64_t npairs = uint64_t(seq_len) * top_k;
    if (npairs > (1u << 20)) return fail(TC_E_UNSUPPORTED, "too many (token, rank) pairs");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (seq_len >= g_moe_gemm_min_tokens && n_experts <= 4096 &&
        uint64_t(npairs) * std::max(hidden, ff) < (uint64_t(1) << 32))
        return moe_grouped(dev, x, ids, wts, seq_len, top_k, wg, wu, wd, n_experts, hidden, ff, out, st);
    // Scratch: h and u [pairs][ff], per-pair down outputs [pairs][hidden].
    const size_t hb = (npairs * ff * 4 + 255) & ~size_t(255);
    const size_t need = 2 * hb + npairs * hidden * 4;
    if (!ensure(dev->aux, dev->aux_bytes, need)) return fail(TC_E_LAUNCH, "hipMalloc(%zu) failed", need);
    float *h = static_cast<float *>(dev->aux);
    float *u = reinterpret_cast<float *>(static_cast<char *>(dev->aux) + hb);
    float *y = reinterpret_cast<float *>(static_cast<char *>(dev->aux) + 2 * hb);
    const uint64_t gstride = uint64_t(ff) * (hidden / 256) * 144;
    const uint64_t dstride = uint64_t(hidden) * (ff / 256) * 144;

    tc::GemvJob up{};
    up.W = static_cast<const uint8_t *>(wg);
    up.W2 = static_cast<const uint8_t *>(wu);
    up.x = x;
    up.out = h;
    up.out2 = u;
    up.rows = ff;
    up.cols = hidden;
    up.out_ld = ff;
    up.epi = 1;
    up.ids = ids;
    up.wstride = gstride;
    up.npairs = uint32_t(npairs);
    up.x_div = top_k;
    up.x_stride = hidden;
    up.out_stride = ff;
    up.n_experts = n_experts;
    hipError_t e = tc::launch_gemv_jobs(TC_Q4_K, 1, &up, 1, dev->num_cu, st);
    if (e != hipSuccess) return hip_fail(e, "MoE gate/up");

    tc::GemvJob dn{};
    dn.W = static_cast<const uint8_t *>(wd);
    dn.x = h;
    dn.rows = hidden;
    dn.cols = ff;
    dn.out_ld = hidden;
    dn.ids = ids;
    dn.wstride = dstride;
    dn.n_experts = n_experts;
    if (top_k <= 8) {
        // down projections of a token's ranks and their rank-order weighted
        // sum in one launch (rank-group mode)
        dn.out = out;
        dn.npairs = seq_len;
        dn.x_stride = top_k * ff;
        dn.out_stride = hidden;
        dn.rk = top_k;
        dn.wts = wts;
        e = tc::launch_gemv_jobs(TC_Q4_K, 1, &dn, 1, dev->num_cu, st);
        if (e != hipSuccess) return hip_fail(e, "MoE down");
        return TC_OK;
    }
    dn.out = y;
    dn.npairs = uint32_t(npairs);
    dn.x_div = 1;
    dn.x_stride = ff;
    dn.out_stride = hidden;
    e = tc::launch_gemv_jobs(TC_Q4_K, 1, &dn, 1, dev->num_cu, st);
    if (e != hipSuccess) return hip_fail(e, "MoE down");

    e = tc::launch_moe_combine(y, wts, out, seq_len, top_k, hidden, st);
    if (e != hipSuccess) return hip_fail(e, "MoE combine");
    return TC_OK;
}

int tc_moe_select(const float *logits, uint32_t seq_len, uint32_t n_experts, uint32_t top_k, int32_t *ids, float *wts,
                  void *stream) {
    if (!device()) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    if (!logits || !ids || !wts) return fail(TC_E_ARG, "null pointer");
    if (seq_len == 0 || n_experts == 0 || top_k == 0 || top_k > n_experts)
        return fail(TC_E_ARG, "seq_len=%u n_experts=%u top_k=%u", seq_len, n_experts, top_k);
    if (n_experts > 4096) return fail(TC_E_UNSUPPORTED, "n_experts=%u > 4096", n_experts);
    hipError_t e = tc::launch_router_select(logits, seq_len, n_experts, top_k, ids, wts, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "MoE router selection");
    return TC_OK;
}

int tc_moe_router(const float *w_router, const float *x, uint32_t seq_len, uint32_t n_experts, uint32_t hidden,
                  uint32_t top_k, float *logits, int32_t *ids, float *wts, void *stream) {
    if (!device()) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    if (!w_router || !x || !logits || !ids || !wts) return fail(TC_E_ARG, "null pointer");
    if (seq_len == 0 || n_experts == 0 || hidden == 0 || top_k == 0 || top_k > n_experts)
        return fail(TC_E_ARG, "seq_len=%u n_experts=%u hidden=%u top_k=%u", seq_len, n_experts, hidden, top_k);
    if (n_experts > 4096 || seq_len > 65535) return fail(TC_E_UNSUPPORTED, "n_experts > 4096 or seq_len > 65535");
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = tc::launch_router_logits(w_router, x, seq_len, n_experts, hidden, logits, st);
    if (e != hipSuccess) return hip_fail(e, "MoE router logits");
    e = tc::launch_router_select(logits, seq_len, n_experts, top_k, ids, wts, st);
    if (e != hipSuccess) return hip_fail(e, "MoE router selection");
    return TC_OK;
}

// ---- parity hooks (reference GPUModel::debugQ8KRow / debugQ8_0Row /
// debugQ8KBlocks / debugQ8_0Blocks, include/GPUCompute.hpp:399-460, as free
// functions over host data) --------------------------------------------------

namespace {

struct DevBuf {
    void *p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

// Scale fields of one block zeroed: the block then contributes exactly 0 in
// every kernel (Q2_K d and dmin, Q3_K d, Q4_K / Q5_K d and dmin, IQ3_S / IQ2_S / IQ4_XS d, Q6_K d, IQ3_XXS d, Q8_0 d).
void zero_block_scales(int type, uint8_t *blk) {
    switch (type) {
        case TC_Q4_K:
        case TC_Q5_K: std::memset(blk, 0, 4); break;
        case TC_Q2_K: std::memset(blk + 80, 0, 4); break;
        case TC_Q3_K: std::memset(blk + 108, 0, 2); break;
        case TC_Q6_K: std::memset(blk + 208, 0, 2); break;
        default: std::memset(blk, 0, 2); break;
    }
}

// Row results of `nrows` host rows against one host activation vector.
int debug_rows(int type, const uint8_t *w_host, uint32_t nrows, const float *x_host, uint32_t cols, float *res) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    const size_t rb = tc_row_bytes(type, cols);
    DevBuf w, x, o;
    if (hipMalloc(&w.p, rb * nrows) != hipSuccess || hipMalloc(&x.p, cols * 4) != hipSuccess ||
        hipMalloc(&o.p, nrows * 4) != hipSuccess)
        return fail(TC_E_LAUNCH, "hipMalloc failed");
    if (hipMemcpy(w.p, w_host, rb * nrows, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(x.p, x_host, cols * 4, hipMemcpyHostToDevice) != hipSuccess)
        return fail(TC_E_LAUNCH, "copy to device failed");
    int rc = run_gemv(dev, type, w.p, nullptr, static_cast<const float *>(x.p), nullptr, static_cast<float *>(o.p),
                      nullptr, 0, nullptr, 1, nrows, cols, nullptr);
    if (rc) return rc;
    if (hipMemcpy(res, o.p, nrows * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(TC_E_LAUNCH, "copy to host failed");
    return TC_OK;
}

// Per-block contributions: row b of a scratch matrix is the input row with
// every block but b zeroed (unit u = 8 Q8_0 blocks is split the same way).
int debug_blocks(int type, const uint8_t *w_row, uint32_t nblk, const float *x_host, uint32_t cols, float *out_blk) {
    const size_t rb = tc_row_bytes(type, cols), bb = tc::block_bytes(type);
    std::vector<uint8_t> m(rb * nblk);
    for (uint32_t b = 0; b < nblk; ++b) {
        uint8_t *row = m.data() + rb * b;
        std::memcpy(row, w_row, rb);
        for (uint32_t k = 0; k < nblk; ++k)
            if (k != b) zero_block_scales(type, row + bb * k);
    }
    return debug_rows(type, m.data(), nblk, x_host, cols, out_blk);
}

int debug_quant(int type, const float *x_host, uint32_t cols, uint8_t *out_quant) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    const tc::ActLayout L = tc::act_layout(type, 1, cols);
    DevBuf x, a;
    if (hipMalloc(&x.p, cols * 4) != hipSuccess || hipMalloc(&a.p, L.bytes) != hipSuccess)
        return fail(TC_E_LAUNCH, "hipMalloc failed");
    if (hipMemcpy(x.p, x_host, cols * 4, hipMemcpyHostToDevice) != hipSuccess)
        return fail(TC_E_LAUNCH, "copy to device failed");
    hipError_t e = tc::launch_quant_act(type, static_cast<const float *>(x.p), 1, cols, L, a.p, nullptr);
    if (e != hipSuccess) return hip_fail(e, "activation quantizer");
    std::vector<uint8_t> h(L.bytes);
    if (hipMemcpy(h.data(), a.p, L.bytes, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(TC_E_LAUNCH, "copy to host failed");
    const int8_t *qs = reinterpret_cast<const int8_t *>(h.data() + L.qs_off);
    const float *d = reinterpret_cast<const float *>(h.data() + L.d_off);
    const int16_t *bs = reinterpret_cast<const int16_t *>(h.data() + L.bs_off);
    if (type == TC_Q8_0) {
        for (uint32_t b = 0; b < cols / 32; ++b) {  // {float d; int8 qs[32]}
            std::memcpy(out_quant + 36 * b, d + b, 4);
            std::memcpy(out_quant + 36 * b + 4, qs + 32 * b, 32);
        }
    } else {
        for (uint32_t b = 0; b < cols / 256; ++b) {  // block_q8_K {float d; int8 qs[256]; int16 bsums[16]}
            std::memcpy(out_quant + 292 * b, d + b, 4);
            std::memcpy(out_quant + 292 * b + 4, qs + 256 * b, 256);
            std::memcpy(out_quant + 292 * b + 260, bs + 16 * b, 32);
        }
    }
    return TC_OK;
}

}  // namespace

int tc_debug_q8k_row(int type, const uint8_t *w_row, uint32_t blocks_per_row, const float *x, uint32_t cols,
                     float *result) {
    if (type == TC_Q8_0 || !type_ok(type) || !int8_act_type(type))
        return fail(TC_E_UNSUPPORTED, "type %d is not a Q8_K-activation type", type);
    if (!w_row || !x || !result) return fail(TC_E_ARG, "null pointer");
    if (cols % 256 || blocks_per_row != cols / 256) return fail(TC_E_ARG, "blocks_per_row/cols mismatch");
    return debug_rows(type, w_row, 1, x, cols, result);
}

int tc_debug_q8_0_row(const uint8_t *w_row, uint32_t blocks_per_row, const float *x, uint32_t cols, float *result) {
    if (!w_row || !x || !result) return fail(TC_E_ARG, "null pointer");
    if (cols % 256 || blocks_per_row != cols / 32) return fail(TC_E_ARG, "blocks_per_row/cols mismatch");
    return debug_rows(TC_Q8_0, w_row, 1, x, cols, result);
}

int tc_debug_q8k_blocks(int type, const uint8_t *w_row, uint32_t blocks_per_row, const float *x, uint32_t cols,
                        float *out_blk, uint8_t *out_quant) {
    if (type == TC_Q8_0 || !type_ok(type) || !int8_act_type(type))
        return fail(TC_E_UNSUPPORTED, "type %d is not a Q8_K-activation type", type);
    if (!w_row || !x || !out_blk || !out_quant) return fail(TC_E_ARG, "null pointer");
    if (cols % 256 || blocks_per_row != cols / 256) return fail(TC_E_ARG, "blocks_per_row/cols mismatch");
    int rc = debug_quant(type, x, cols, out_quant);
    return rc ? rc : debug_blocks(type, w_row, blocks_per_row, x, cols, out_blk);
}

int tc_debug_q8_0_blocks(const uint8_t *w_row, uint32_t blocks_per_row, const float *x, uint32_t cols,
                         float *out_blk, uint8_t *out_quant) {
    if (!w_row || !x || !out_blk || !out_quant) return fail(TC_E_ARG, "null pointer");
    if (cols % 256 || blocks_per_row != cols / 32) return fail(TC_E_ARG, "blocks_per_row/cols mismatch");
    int rc = debug_quant(TC_Q8_0, x, cols, out_quant);
    return rc ? rc : debug_blocks(TC_Q8_0, w_row, blocks_per_row, x, cols, out_blk);
}

// ---- host-pointer products (the reference CPU entry points' boundary,
// include/SIMDMatMulVec.hpp:448-584) ------------------------------------------

namespace {

struct HostRange {
    const uint8_t *host;
    size_t bytes;
    void *dev;
    int device;  // the HIP device holding the copy
};

std::mutex g_host_mu;
std::vector<HostRange> g_host_ranges;  // registered host weight ranges and their device copies

int current_device() {
    int id = -1;
    return hipGetDevice(&id) == hipSuccess ? id : -1;
}

// Device address of [p, p + bytes) when it lies inside a range registered on
// the current device.
const void *registered_copy(const void *p, size_t bytes) {
    const uint8_t *q = static_cast<const uint8_t *>(p);
    const int id = current_device();
    for (const HostRange &r : g_host_ranges)
        if (r.device == id && q >= r.host && q + bytes <= r.host + r.bytes) {
            const uint8_t *d = static_cast<const uint8_t *>(r.dev) + (q - r.host);
            // The kernels take 16-byte-aligned weights; a sub-range starting
            // elsewhere (e.g. row 1 of 1540-byte Q3_K rows) is staged instead.
            return (reinterpret_cast<uintptr_t>(d) & 15) == 0 ? d : nullptr;
        }
    return nullptr;
}

struct HostScratch {
    void *p = nullptr;
    size_t cap = 0;
};
HostScratch g_hw, g_hx, g_ho;  // weights / activations / outputs staged for host-pointer calls

}  // namespace

int tc_host_weights_register(const void *host, size_t bytes) {
    if (!device()) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    if (!host || bytes == 0) return fail(TC_E_ARG, "null or empty range");
    std::lock_guard<std::mutex> lk(g_host_mu);
    const int id = current_device();
    for (const HostRange &r : g_host_ranges)
        if (r.host == host && r.device == id) return fail(TC_E_ARG, "range already registered");
    void *d = nullptr;
    if (hipMalloc(&d, bytes) != hipSuccess) return fail(TC_E_LAUNCH, "hipMalloc(%zu) failed", bytes);
    if (hipMemcpy(d, host, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        return fail(TC_E_LAUNCH, "copy to device failed");
    }
    g_host_ranges.push_back({static_cast<const uint8_t *>(host), bytes, d, id});
    return TC_OK;
}

int tc_host_weights_unregister(const void *host) {
    std::lock_guard<std::mutex> lk(g_host_mu);
    const int id = current_device();
    for (size_t i = 0; i < g_host_ranges.size(); ++i)
        if (g_host_ranges[i].host == host && g_host_ranges[i].device == id) {
            (void)hipDeviceSynchronize();
            (void)hipFree(g_host_ranges[i].dev);
            g_host_ranges.erase(g_host_ranges.begin() + long(i));
            return TC_OK;
        }
    return fail(TC_E_ARG, "range not registered");
}

int tc_host_matmul(int type, const uint8_t *W, const float *X, uint32_t seq_len, uint32_t rows, uint32_t cols,
                   float *out, const float *residual) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    if (!type_ok(type)) return fail(TC_E_UNSUPPORTED, "unsupported type %d", type);
    if (!W || !X || !out) return fail(TC_E_ARG, "null pointer");
    if (seq_len == 0 || rows == 0 || cols == 0) return fail(TC_E_UNSUPPORTED, "empty shape");
    const size_t rb = tc_row_bytes(type, cols);
    if (rb == 0) return fail(TC_E_UNSUPPORTED, "cols=%u", cols);
    const size_t wbytes = rb * rows, xbytes = size_t(seq_len) * cols * 4, obytes = size_t(seq_len) * rows * 4;
    std::lock_guard<std::mutex> lk(g_host_mu);
    const void *wd = registered_copy(W, wbytes);
    if (!wd) {
        if (!ensure(g_hw.p, g_hw.cap, wbytes)) return fail(TC_E_LAUNCH, "hipMalloc(%zu) failed", wbytes);
        if (hipMemcpy(g_hw.p, W, wbytes, hipMemcpyHostToDevice) != hipSuccess)
            return fail(TC_E_LAUNCH, "weight copy to device failed");
        wd = g_hw.p;
    }
    if (!ensure(g_hx.p, g_hx.cap, xbytes) || !ensure(g_ho.p, g_ho.cap, obytes))
        return fail(TC_E_LAUNCH, "hipMalloc failed");
    if (hipMemcpy(g_hx.p, X, xbytes, hipMemcpyHostToDevice) != hipSuccess)
        return fail(TC_E_LAUNCH, "activation copy to device failed");
    float *od = static_cast<float *>(g_ho.p);
    const float *xd = static_cast<const float *>(g_hx.p);
    const int rc = seq_len <= 8 ? tc_gemv(type, wd, xd, od, seq_len, rows, cols, nullptr)
                                : tc_gemm(type, wd, xd, od, seq_len, rows, cols, cols / uint32_t(tc::block_elems(type)),
                                          nullptr);
    if (rc) return rc;
    if (!residual) {
        if (hipMemcpy(out, od, obytes, hipMemcpyDeviceToHost) != hipSuccess)
            return fail(TC_E_LAUNCH, "output copy to host failed");
        return TC_OK;
    }
    // out = dot + residual, as the reference's residual-fused store; out may
    // be the residual buffer itself (the attnO in-place residual,
    // SIMDMatMulVec.hpp:472-476), so the products land in a host buffer first
    // and every residual value is read before its output is written.
    std::vector<float> dot(size_t(seq_len) * rows);
    if (hipMemcpy(dot.data(), od, obytes, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(TC_E_LAUNCH, "output copy to host failed");
    for (size_t i = 0; i < dot.size(); ++i) out[i] = dot[i] + residual[i];
    return TC_OK;
}

int tc_host_matmul_f32(const float *W, const float *X, uint32_t seq_len, uint32_t rows, uint32_t cols, float *out) {
    Device *dev = device();
    if (!dev) return fail(TC_E_UNSUPPORTED, "no gfx950 device");
    if (!W || !X || !out) return fail(TC_E_ARG, "null pointer");
    if (seq_len == 0 || rows == 0 || cols == 0) return fail(TC_E_UNSUPPORTED, "empty shape");
    if (seq_len > 65535) return fail(TC_E_UNSUPPORTED, "seq_len=%u > 65535", seq_len);
    const size_t wbytes = size_t(rows) * cols * 4, xbytes = size_t(seq_len) * cols * 4,
                 obytes = size_t(seq_len) * rows * 4;
    std::lock_guard<std::mutex> lk(g_host_mu);
    const void *wd = registered_copy(W, wbytes);
    if (!wd) {
        if (!ensure(g_hw.p, g_hw.cap, wbytes)) return fail(TC_E_LAUNCH, "hipMalloc(%zu) failed", wbytes);
        if (hipMemcpy(g_hw.p, W, wbytes, hipMemcpyHostToDevice) != hipSuccess)
            return fail(TC_E_LAUNCH, "weight copy to device failed");
        wd = g_hw.p;
    }
    if (!ensure(g_hx.p, g_hx.cap, xbytes) || !ensure(g_ho.p, g_ho.cap, obytes))
        return fail(TC_E_LAUNCH, "hipMalloc failed");
    if (hipMemcpy(g_hx.p, X, xbytes, hipMemcpyHostToDevice) != hipSuccess)
        return fail(TC_E_LAUNCH, "activation copy to device failed");
    hipError_t e = tc::launch_router_logits(static_cast<const float *>(wd), static_cast<const float *>(g_hx.p), seq_len,
                                            rows, cols, static_cast<float *>(g_ho.p), nullptr);
    if (e != hipSuccess) return hip_fail(e, "fp32 mat-vec");
    if (hipMemcpy(out, g_ho.p, obytes, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(TC_E_LAUNCH, "output copy to host failed");
    return TC_OK;
}

const char *tc_last_error(void) { return g_err.c_str(); }

}  // extern "C"
