// tc_gemv.hip -- host dispatch of the decode-time quantized mat-vec
// (k_gemv_t in tc_gemv_kernel.hpp): job layout, row split over the CUs,
// launch-shape choice and the per-type launch.
#include <algorithm>
#include <cmath>

#include "tc_gemv_kernel.hpp"

namespace tc {

namespace {
using namespace gv;
// Streams of at least this many weight bytes use the 512-thread shape.
constexpr uint64_t kBigBytes = 24ull << 20;
// MoE expert launches (expert ids on the device) from 4 MB: their weight
// loads wait for the ids, and more waves per CU hide that (batch 1: 14.4
// against 15.1 us; plain 7 MB launches were slower on the 512-thread shape).
constexpr uint64_t kBigBytesExperts = 4ull << 20;

bool tiled_type(int type) { return type == kQ5_0 || type == kIQ4_NL || type == kIQ4_XS || type == kIQ2_XS || type == kQ2_K || type == kIQ2_S || type == kIQ3_S || type == kQ3_K || type == kQ4_K || type == kQ5_K || type == kQ8_0 || type == kQ6_K || type == kIQ3_XXS; }

// Matrices one workgroup streams per row range: 2 for a gate/up pair, rk in
// rank-group mode, else 1.
uint32_t job_mats(const GemvJob &g) { return g.rk ? g.rk : g.W2 ? 2 : 1; }

bool use_big(int type, uint64_t weight_bytes) { return type != kQ8_0 && weight_bytes >= kBigBytes; }

template <class C>
hipError_t launch_gemv_tiled_c(int type, uint32_t S, const GemvJob *jobs, uint32_t njobs, int num_cu,
                               hipStream_t st) {
    TLaunchArgs a{};
    a.njobs = njobs;
    uint32_t maxcols = 0, maxnx = S;
    uint64_t total_units = 0;
    for (uint32_t j = 0; j < njobs; ++j) {
        maxcols = std::max(maxcols, jobs[j].cols);
        if (jobs[j].rk) maxnx = std::max(maxnx, jobs[j].rk);
        total_units += uint64_t(jobs[j].rows) * (jobs[j].cols / 256) * job_mats(jobs[j]) * jobs[j].npairs;
    }
    const uint32_t fixed = tlds_layout<C>(type, maxnx, maxcols, &a);
    if (fixed >= kTLdsBudget) return hipErrorInvalidValue;
    const uint32_t part_avail = kTLdsBudget - fixed;
    // One workgroup per CU, each with at least 2 tiles of work.
    const uint64_t want = std::max<uint64_t>(
        1, std::min<uint64_t>(uint64_t(num_cu), (total_units + 2 * kTileUnits - 1) / (2 * kTileUnits)));
    // Workgroups per job. A workgroup first stages its job's activations
    // (nu records per token; wide inputs cost several times more than narrow
    // ones) and then streams its units, so in a launch of plain jobs with
    // different widths the shares are chosen so that every workgroup's
    // staging + units come out equal: g_j = units_j / (T - stage_j), with the
    // smallest T for which the counts fit on the chip.
    uint64_t gplan[kMaxJobs] = {};
    bool plan = njobs > 1;
    for (uint32_t j = 0; j < njobs; ++j) plan = plan && jobs[j].npairs == 1 && jobs[j].ids == nullptr;
    if (plan) {
        // staging one activation record costs about as much time as
        // streaming 10 weight units (measured on the 7-matrix Q4_K layer)
        constexpr double kStage = 10.0;
        double st[kMaxJobs], smax = 0.0;
        for (uint32_t j = 0; j < njobs; ++j) {
            st[j] = kStage * (jobs[j].cols / 256) * S;
            smax = std::max(smax, st[j]);
        }
        auto count = [&](double T, uint64_t *g) {
            uint64_t tot = 0;
            for (uint32_t j = 0; j < njobs; ++j) {
                const double u = double(jobs[j].rows) * (jobs[j].cols / 256) * job_mats(jobs[j]);
                g[j] = std::min<uint64_t>(jobs[j].rows, std::max<uint64_t>(1, uint64_t(std::ceil(u / (T - st[j])))));
                tot += g[j];
            }
            return tot;
        };
        double lo = smax, hi = smax + double(total_units) + 1.0;  // count(hi) == njobs
        for (int it = 0; it < 60; ++it) {
            const double mid = 0.5 * (lo + hi);
            uint64_t g[kMaxJobs];
            if (count(mid, g) > want) lo = mid;
            else hi = mid;
        }
        count(hi, gplan);
    }
    uint32_t wg = 0, max_part = 0;
    for (uint32_t j = 0; j < njobs; ++j) {
        const GemvJob &g = jobs[j];
        TJobDev &d = a.jobs[j];
        const uint32_t pairs = job_mats(g);
        d.W = g.W;
        d.W2 = g.W2;
        d.x = g.x;
        d.act = g.act;
        d.out = g.out;
        d.out2 = g.out2;
        d.dbg = g.dbg;
        d.rows = g.rows;
        d.cols = g.cols;
        d.nu = g.cols / 256;
        d.out_ld = g.out_ld;
        d.epi = g.epi;
        d.nu_div = make_divmod(d.nu);
        d.ids = g.ids;
        d.wstride = g.wstride;
        d.x_div = g.x_div;
        d.x_stride = g.x_stride;
        d.out_stride = g.out_stride;
        d.n_experts = g.n_experts;
        d.rk = g.rk;
        d.wts = g.wts;
        d.nx = g.rk ? g.rk : S;
        const uint64_t units = uint64_t(g.rows) * d.nu * pairs * g.npairs;
        // workgroups per mat-vec (per expert pair in expert-pair mode)
        // (rounded down: one workgroup more than the CUs would run as a
        // second round)
        uint64_t gj = plan ? gplan[j] : std::max<uint64_t>(1, want * units / total_units / g.npairs);
        gj = std::min<uint64_t>(gj, g.rows);
        uint32_t rpw = uint32_t((g.rows + gj - 1) / gj);
        const uint32_t fit = part_avail / (pairs * S * d.nu * 4);
        if (fit == 0) return hipErrorInvalidValue;
        rpw = std::min(rpw, fit);
        // Rows of Q2_K / Q3_K / Q6_K / IQ3_XXS / IQ3_S / IQ2_S / IQ2_XS /
        // IQ4_XS are not always 16-byte multiples: every workgroup's first row
        // stays 16-byte aligned with row groups of the fewest rows whose bytes
        // are a multiple of 16 (at most 8: 8*84, 8*110, 8*210, 8*98, 8*82,
        // 8*74 and 8*136 bytes per 256 columns are).
        if (rpw < g.rows) {
            const uint64_t row_bytes = uint64_t(d.nu) * unit_bytes(type);
            uint32_t grp = 1;
            while (grp < 8 && (grp * row_bytes) % 16 != 0) grp *= 2;
            rpw = (rpw + grp - 1) / grp * grp;
            if (rpw > fit) rpw = fit / grp * grp;
            if (rpw == 0) return hipErrorInvalidValue;
        }
        d.rows_per_wg = rpw;
        gj = (g.rows + rpw - 1) / rpw;
        d.wg_per_pair = uint32_t(gj);
        d.wg_begin = wg;
        wg += uint32_t(gj) * g.npairs;
        max_part = std::max(max_part, pairs * S * rpw * d.nu * 4);
    }
    const uint32_t lds = fixed + max_part;
    constexpr bool big = C::NT == CfgBig::NT;
    switch (type) {
#define TC_CASE(t) \
    case t: return launch_type<t>(big, S, a, wg, lds, st);
        TC_CASE(kQ4_K) TC_CASE(kQ5_K) TC_CASE(kQ3_K) TC_CASE(kIQ3_S) TC_CASE(kIQ2_S) TC_CASE(kQ2_K)
        TC_CASE(kIQ2_XS) TC_CASE(kIQ4_XS) TC_CASE(kIQ4_NL) TC_CASE(kQ5_0) TC_CASE(kQ6_K) TC_CASE(kIQ3_XXS)
        TC_CASE(kQ8_0)
#undef TC_CASE
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

uint64_t jobs_weight_bytes(int type, const GemvJob *jobs, uint32_t njobs) {
    uint64_t b = 0;
    for (uint32_t j = 0; j < njobs; ++j)
        b += uint64_t(jobs[j].rows) * (jobs[j].cols / 256) * unit_bytes(type) * job_mats(jobs[j]) * jobs[j].npairs;
    return b;
}

namespace {

// Types whose activations are staged as fp32 (1072 bytes per 256): at wide
// inputs (the 18944-column down projection) only the 256-thread shape, with
// half the wave tile slots, fits its records in LDS.
bool fp32_act_type(int type) { return type == kIQ2_XS || type == kIQ4_NL || type == kQ5_0; }

template <class C>
bool tiled_fits(int type, uint32_t S, uint32_t cols) {
    TLaunchArgs a;
    return tlds_layout<C>(type, S, cols, &a) + 2 * 8 * S * (cols / 256) * 4 <= kTLdsBudget;
}

hipError_t launch_gemv_tiled(int type, uint32_t S, const GemvJob *jobs, uint32_t njobs, int num_cu,
                             hipStream_t st) {
    bool big_fits = true;
    if (fp32_act_type(type))
        for (uint32_t i = 0; i < njobs; ++i) big_fits = big_fits && tiled_fits<CfgBig>(type, S, jobs[i].cols);
    bool experts = false;
    for (uint32_t i = 0; i < njobs; ++i) experts = experts || jobs[i].ids != nullptr;
    const uint64_t wb = jobs_weight_bytes(type, jobs, njobs);
    return big_fits && (use_big(type, wb) || (experts && type != kQ8_0 && wb >= kBigBytesExperts))
               ? launch_gemv_tiled_c<CfgBig>(type, S, jobs, njobs, num_cu, st)
               : launch_gemv_tiled_c<CfgSmall>(type, S, jobs, njobs, num_cu, st);
}

}  // namespace

uint32_t gemv_fused_quant_limit(int type, uint64_t weight_bytes) {
    // S*cols up to which the tiled kernels preload all of x ahead of the weights
    if (!tiled_type(type) || type == kIQ2_XS || type == kIQ4_NL || type == kQ5_0) return 0xFFFFFFFFu;  // fp32 x, never pre-quantized
    return uint32_t(kXPre) * (use_big(type, weight_bytes) ? CfgBig::NT : CfgSmall::NT) * 16u;
}

uint32_t gemv_max_tokens(int type, uint32_t cols) {
    uint32_t best = 0;
    if (tiled_type(type)) {
        for (uint32_t S = 1; S <= 8; ++S) {
            TLaunchArgs a;
            const uint32_t f = std::max(tlds_layout<CfgBig>(type, S, cols, &a), tlds_layout<CfgSmall>(type, S, cols, &a));
            // Q8_0 and (when the 512-thread shape does not fit) the fp32
            // activation types launch the 256-thread shape only
            const bool small_only = type == kQ8_0 || fp32_act_type(type);
            if ((small_only ? tlds_layout<CfgSmall>(type, S, cols, &a) : f) + 2 * 8 * S * (cols / 256) * 4 <=
                kTLdsBudget)
                best = S;
        }
    }
    return best;
}

hipError_t launch_gemv_jobs(int type, uint32_t S, const GemvJob *jobs, uint32_t njobs, int num_cu,
                            hipStream_t st) {
    if (S == 0 || S > 8 || njobs == 0 || njobs > uint32_t(kMaxJobs)) return hipErrorInvalidValue;
    for (uint32_t j = 0; j < njobs; ++j) {
        const GemvJob &g = jobs[j];
        if (g.rows == 0 || g.cols == 0 || g.cols % 256 != 0) return hipErrorInvalidValue;
        if ((reinterpret_cast<uintptr_t>(g.W) & 15) || (g.W2 && (reinterpret_cast<uintptr_t>(g.W2) & 15)))
            return hipErrorInvalidValue;
    }
    if (!tiled_type(type)) return hipErrorInvalidValue;
    return launch_gemv_tiled(type, S, jobs, njobs, num_cu, st);
}

namespace {

// Rank-order weighted sum of the per-(token, rank) expert outputs
// (reference ModelMoE.cpp:990-1002: the output starts at 0 and adds
// w_r * down_r for r = 0..top_k-1 in order).
__global__ __launch_bounds__(256) void k_moe_combine(const float *__restrict__ y, const float *__restrict__ wts,
                                                     float *__restrict__ out, uint32_t top_k, uint32_t H) {
    const uint32_t t = blockIdx.y;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= H) return;
    float acc = 0.0f;
    for (uint32_t r = 0; r < top_k; ++r)
        acc = fmaf(wts[size_t(t) * top_k + r], y[(size_t(t) * top_k + r) * H + i], acc);
    out[size_t(t) * H + i] = acc;
}

}  // namespace

hipError_t launch_moe_combine(const float *y, const float *wts, float *out, uint32_t T, uint32_t top_k, uint32_t H,
                              hipStream_t st) {
    if (T == 0 || H == 0) return hipErrorInvalidValue;
    k_moe_combine<<<dim3{(H + 255) / 256, T, 1u}, 256, 0, st>>>(y, wts, out, top_k, H);
    return hipGetLastError();
}

}  // namespace tc
