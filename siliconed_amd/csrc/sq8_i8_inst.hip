// sq8_i8_inst.hip — instantiations of the W8A8 product kernel (sq8_i8_kernel.h): 128 × 256 tiles,
// two workgroups per CU, three activation stages, packed or [N, K] int8 weights, every epilogue and
// output type.
#include "sq8_gemm.h"
#include "sq8_i8_kernel.h"

namespace sq8 {

hipError_t launch_i8gemm(const GemmArgs &p, int wl, int epi, int out, hipStream_t stream) {
    // Three activation stages: C1 on the W8A8 route 2012 → 2025 TOP/s (three interleaved pairs).
    if (wl == W_PACKED) return wd::dispatch_i8<128, 4, W_PACKED, 3>(p, epi, out, stream);
    if (wl == W_NK) return wd::dispatch_i8<128, 4, W_NK, 3>(p, epi, out, stream);
    return hipErrorInvalidValue;
}

}  // namespace sq8
