// tc_gemv_inst.hip -- the decode kernel instantiated for ONE weight type,
// TC_GEMV_TYPE (a GGML type id), given on the compiler command line. The
// Makefile builds this file once per type, so the types compile in parallel.
#include "tc_gemv_kernel.hpp"

#ifndef TC_GEMV_TYPE
#error "TC_GEMV_TYPE (GGML type id) must be defined"
#endif

namespace tc::gv {

template <>
hipError_t launch_type<TC_GEMV_TYPE>(bool big, uint32_t S, const TLaunchArgs &a, uint32_t grid, uint32_t lds,
                                     hipStream_t st) {
    // Q8_0's 17 KB wave tiles fit only the 256-thread shape.
    if constexpr (TC_GEMV_TYPE == kQ8_0) {
        if (big) return hipErrorInvalidValue;
        return launch_tiled<kQ8_0, CfgSmall>(S, a, grid, lds, st);
    } else {
        return big ? launch_tiled<TC_GEMV_TYPE, CfgBig>(S, a, grid, lds, st)
                   : launch_tiled<TC_GEMV_TYPE, CfgSmall>(S, a, grid, lds, st);
    }
}

}  // namespace tc::gv
