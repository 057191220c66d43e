// sq8_gemm.hip — picks the GEMM kernel for a product: the branch-free kernels when the operands
// allow them (sq8_gemm_inst.hip), the guarded ones otherwise (sq8_gemm_general.hip).
#include "sq8_gemm.h"

namespace sq8 {

hipError_t launch_fast_0_0(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream);
hipError_t launch_fast_0_1(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream);
hipError_t launch_fast_1_0(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream);
hipError_t launch_fast_1_1(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream);
hipError_t launch_general(const GemmArgs &p, int wt, int wl, int epi, int out, hipStream_t stream);
hipError_t launch_wdirect_0_1(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream);
hipError_t launch_wdirect_0_2(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream);
hipError_t launch_wdirect_1_1(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream);
hipError_t launch_wdirect_1_2(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream);

hipError_t launch_wdirect(const GemmArgs &p, int tile, int wt, int wl, int epi, int out, hipStream_t stream) {
    if (wt == W_INT8) return wl == W_NK ? launch_wdirect_0_1(p, tile, epi, out, stream) : launch_wdirect_0_2(p, tile, epi, out, stream);
    return wl == W_NK ? launch_wdirect_1_1(p, tile, epi, out, stream) : launch_wdirect_1_2(p, tile, epi, out, stream);
}

int choose_wd_tile(int M, int N, bool glu) {
    // 128 × 256 tiles of 64-column slabs (GLU: 32 output columns a slab). Below 96 of them (M = 1024
    // at N = 3072, where the two kernels tie on MI355X) the skinny kernel's 32-row tiles with K split
    // over four waves are faster: 5× at M = 1, 1.7× at M = 512.
    const long slabs = glu ? (N / 2 + 31) / 32 : (N + 63) / 64;
    const long tiles = (long)((M + 127) / 128) * ((slabs + 3) / 4);
    return tiles >= 96 ? WD_128 : WD_SKINNY32;
}

int choose_tile(int M, int N_out, bool glu) {
    // Tiles of 256 × 256 while they fill the 256 CUs at least 3/4 of the way; 128 × 128 below.
    const int n_virtual = glu ? 2 * N_out : N_out;
    const long big = (long)((M + 255) / 256) * ((n_virtual + 255) / 256);
    return big >= 192 ? TILE_256x256 : TILE_128x128;
}

hipError_t launch_gemm(const GemmArgs &p, bool fast, int tile, int wt, int wl, int epi, int out, hipStream_t stream) {
    if (!fast) return launch_general(p, wt, wl, epi, out, stream);
    if (wt == W_INT8 && wl == W_KN) return launch_fast_0_0(p, tile, epi, out, stream);
    if (wt == W_INT8 && wl == W_NK) return launch_fast_0_1(p, tile, epi, out, stream);
    if (wt == W_FP8 && wl == W_KN) return launch_fast_1_0(p, tile, epi, out, stream);
    if (wt == W_FP8 && wl == W_NK) return launch_fast_1_1(p, tile, epi, out, stream);
    return hipErrorInvalidValue;
}

}  // namespace sq8
