// sq8_wdirect_inst.hip — instantiates the weight-direct kernels for one weight type (SQ8_WT) and
// layout (SQ8_WL: 1 [N, K], 2 packed), compiled once per pair so the sets build in parallel.
#include "sq8_gemv_kernel.h"
#include "sq8_skinny_kernel.h"
#include "sq8_w256_kernel.h"

#if !defined(SQ8_WT) || !defined(SQ8_WL)
#error "compile with -DSQ8_WT=<0 int8 | 1 fp8> -DSQ8_WL=<1 [N,K] | 2 packed>"
#endif

#define SQ8_CAT2(a, b) a##b
#define SQ8_CAT(a, b) SQ8_CAT2(a, b)

namespace sq8 {

hipError_t SQ8_CAT(launch_wdirect_, SQ8_CAT(SQ8_WT, SQ8_CAT(_, SQ8_WL)))(const GemmArgs &p, int tile, int epi, int out,
                                                                       hipStream_t stream) {
    // 256 × 256 or 224 × 256 tiles where their kernel serves the product (whole slabs, aligned scales and
    // biases); else the two-workgroup 128-row tiles.
    if (tile == WD_256 || tile == WD_224) {
        if (wd::w256_fits(p, epi, out))
            return tile == WD_256 ? wd::launch_w256<SQ8_WT, SQ8_WL, 256>(p, epi, out, stream)
                                  : wd::launch_w256<SQ8_WT, SQ8_WL, 224>(p, epi, out, stream);
        tile = WD_128;
    }
    if (tile == WD_128) return wd::dispatch_wd<128, 4, 2, SQ8_WT, SQ8_WL>(p, epi, out, stream);
    if (tile >= WD_K32x32 && tile <= WD_K64x192) {
        // One-block waves whose K steps split over four or two wave groups (three activation stages a
        // group); not for the GLU epilogues, and K/64 a multiple of the groups — else the tile of the same
        // height without groups.
        const bool plain = p.glu_half == 0;
        switch (tile) {
        case WD_K32x32:
            if (plain && p.kt % 4 == 0) return wd::dispatch_wd<32, 1, 2, SQ8_WT, SQ8_WL, 3, 1, 4>(p, epi, out, stream);
            tile = WD_32;
            break;
        case WD_K32x64:
            if (plain && p.kt % 4 == 0) return wd::dispatch_wd<32, 2, 2, SQ8_WT, SQ8_WL, 3, 1, 4>(p, epi, out, stream);
            tile = WD_32;
            break;
        case WD_K64x64:
            if (plain && p.kt % 4 == 0) return wd::dispatch_wd<64, 2, 2, SQ8_WT, SQ8_WL, 3, 1, 4>(p, epi, out, stream);
            tile = WD_64N;
            break;
        case WD_K64x128:
            if (plain && p.kt % 2 == 0) return wd::dispatch_wd<64, 4, 2, SQ8_WT, SQ8_WL, 3, 1, 2>(p, epi, out, stream);
            tile = WD_64N;
            break;
        default:
            if (plain && p.kt % 2 == 0) return wd::dispatch_wd<64, 6, 2, SQ8_WT, SQ8_WL, 3, 1, 2>(p, epi, out, stream);
            tile = WD_64x192;
            break;
        }
    }
    if (tile == WD_64x192) {
        // Six waves of one 32-column block each: not for the GLU epilogues.
        // Four activation stages and weight buffers (C0: 28.8 against 29.1 µs with two).
        if (p.glu_half == 0) return wd::dispatch_wd<64, 6, 2, SQ8_WT, SQ8_WL, 4, 1>(p, epi, out, stream);
        tile = WD_64;
    }
    if (tile == WD_64) return wd::dispatch_wd<64, 4, 1, SQ8_WT, SQ8_WL>(p, epi, out, stream);
    if (tile == WD_64N) {
        // One 32-column block a wave: not for the GLU epilogues (a wave needs both halves' blocks).
        // Three activation stages and weight buffers (C2's text stream: 19.5 against 20.8 µs with two).
        if (p.glu_half == 0) return wd::dispatch_wd<64, 4, 2, SQ8_WT, SQ8_WL, 3, 1>(p, epi, out, stream);
        tile = WD_32;
    }
    if (tile == WD_32) return wd::dispatch_wd<32, 4, 2, SQ8_WT, SQ8_WL, 4>(p, epi, out, stream);
    if (tile == WD_GEMV) {
        // Up to 16 rows (one group of 16 × 16 MFMAs); more rows take the skinny kernel.
        if (p.M <= 16) return wd::dispatch_gemv<SQ8_WT, SQ8_WL>(p, epi, out, stream);
        tile = p.M <= 128 ? WD_SKINNY32 : WD_SKINNY64;
    }
    if (tile == WD_SKINNY64) return wd::dispatch_skinny<64, 4, 2, SQ8_WT, SQ8_WL>(p, epi, out, stream);
    if (tile == WD_SKINNY32) return wd::dispatch_skinny<32, 4, 2, SQ8_WT, SQ8_WL>(p, epi, out, stream);
    return hipErrorInvalidValue;
}

}  // namespace sq8
