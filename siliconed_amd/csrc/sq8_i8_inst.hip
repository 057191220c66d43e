// sq8_i8_inst.hip — instantiations of the W8A8 product kernel (sq8_i8_kernel.h): 128 × 256 tiles,
// two workgroups per CU, packed or [N, K] int8 weights, every epilogue and output type.
#include "sq8_gemm.h"
#include "sq8_i8_kernel.h"

namespace sq8 {

hipError_t launch_i8gemm(const GemmArgs &p, int wl, int epi, int out, hipStream_t stream) {
    if (wl == W_PACKED) return wd::dispatch_i8<128, 4, W_PACKED>(p, epi, out, stream);
    if (wl == W_NK) return wd::dispatch_i8<128, 4, W_NK>(p, epi, out, stream);
    return hipErrorInvalidValue;
}

}  // namespace sq8
