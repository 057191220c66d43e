// sq8_wdirect_inst.hip — instantiates the weight-direct kernels for one weight type (SQ8_WT),
// compiled once per type so the two sets build in parallel.
#include "sq8_wdirect_kernel.h"

#if !defined(SQ8_WT)
#error "compile with -DSQ8_WT=<0 int8 | 1 fp8>"
#endif

#define SQ8_CAT2(a, b) a##b
#define SQ8_CAT(a, b) SQ8_CAT2(a, b)

namespace sq8 {

hipError_t SQ8_CAT(launch_wdirect_, SQ8_WT)(const GemmArgs &p, int tile, int wl, int epi, int out,
                                            hipStream_t stream) {
    if (tile == WD_256 && wl == W_NK) return wd::dispatch_wd<256, 4, SQ8_WT, W_NK>(p, epi, out, stream);
    if (tile == WD_256 && wl == W_PACKED) return wd::dispatch_wd<256, 4, SQ8_WT, W_PACKED>(p, epi, out, stream);
    if (tile == WD_128 && wl == W_NK) return wd::dispatch_wd<128, 4, SQ8_WT, W_NK>(p, epi, out, stream);
    if (tile == WD_128 && wl == W_PACKED) return wd::dispatch_wd<128, 4, SQ8_WT, W_PACKED>(p, epi, out, stream);
    return hipErrorInvalidValue;
}

}  // namespace sq8
