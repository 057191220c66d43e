// sq8_gemm_inst.hip — instantiates the branch-free (FAST) GEMM kernels for one weight type and
// layout, chosen at compile time: the build compiles this file once per (SQ8_WT, SQ8_WL) so the
// four sets compile in parallel.
#include "sq8_gemm_kernel.h"

#if !defined(SQ8_WT) || !defined(SQ8_WL)
#error "compile with -DSQ8_WT=<0 int8 | 1 fp8> -DSQ8_WL=<0 KN | 1 NK>"
#endif

#define SQ8_CAT2(a, b) a##b
#define SQ8_CAT(a, b) SQ8_CAT2(a, b)
#define SQ8_NAME SQ8_CAT(launch_fast_, SQ8_CAT(SQ8_WT, SQ8_CAT(_, SQ8_WL)))

namespace sq8 {

hipError_t SQ8_NAME(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream) {
    switch (tile) {
    case TILE_256x256: return kern::dispatch_epi_out<256, 256, SQ8_WT, SQ8_WL, true>(p, epi, out, stream);
    case TILE_128x128: return kern::dispatch_epi_out<128, 128, SQ8_WT, SQ8_WL, true>(p, epi, out, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace sq8
