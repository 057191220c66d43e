// sq8_gemm_general.hip — the guarded GEMM kernels (every element checked, zeros past the edges)
// for ragged or unaligned operands: 128 × 128 tiles, every weight type, layout and epilogue.
#include "sq8_gemm_kernel.h"

namespace sq8 {

hipError_t launch_general(const GemmArgs &p, int wt, int wl, int epi, int out, hipStream_t stream) {
    if (wt == W_INT8 && wl == W_KN) return kern::dispatch_epi_out<128, 128, W_INT8, W_KN, false>(p, epi, out, stream);
    if (wt == W_INT8 && wl == W_NK) return kern::dispatch_epi_out<128, 128, W_INT8, W_NK, false>(p, epi, out, stream);
    if (wt == W_FP8 && wl == W_KN) return kern::dispatch_epi_out<128, 128, W_FP8, W_KN, false>(p, epi, out, stream);
    if (wt == W_FP8 && wl == W_NK) return kern::dispatch_epi_out<128, 128, W_FP8, W_NK, false>(p, epi, out, stream);
    return hipErrorInvalidValue;
}

}  // namespace sq8
