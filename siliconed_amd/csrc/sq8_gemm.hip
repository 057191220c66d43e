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

// The tile before the K-group tiles are considered.
static int base_wd_tile(int M, int N, bool glu, int cus) {
    // Tiles of 256 columns (four 64-column slabs; GLU: 32 output columns a slab), as tall as keeps
    // at least 9/16 of the CUs' worth of them (144 on the 256 CUs of a whole MI355X) — the measured point
    // below which a shorter tile fills the CUs better than the taller one loses (K = 3072: M = 1024 at
    // N = 3072 runs 64-row tiles at one workgroup a CU in 28.5 µs against 42.8 in 128-row tiles; M = 512
    // 32-row tiles in 22.7 against 42.9). Below that in 32-row tiles, the skinny kernel (K split over four
    // waves): 32-row tiles to M = 128, 64-row above (M = 16: 8.3 µs against 20.2 for 32-row tiles of the
    // main kernel); up to 16 rows on narrow weights, the short-M kernel. `cus`: the device's compute units (a compute-partitioned MI355X has fewer than 256),
    // so a round is `cus` tiles of one workgroup a CU.
    if (cus <= 0) cus = 256;
    const long slabs = glu ? (N / 2 + 31) / 32 : (N + 63) / 64;
    const long tn = (slabs + 3) / 4;
    const long fill = (long)cus * 9 / 16;
    auto tiles = [&](int bm) { return (long)((M + bm - 1) / bm) * tn; };
    // 256 × 256 tiles (one workgroup a CU) once they occupy more than half the CUs: C1's
    // up-projection, 768 tiles, 243.6 µs against 265.1 in 128-row tiles (one process, medians); C3's fp8
    // gate-up (SiLU-GLU, 1280 tiles) 1353 against 1290 TFLOP/s; C1's down-projection, 192 tiles (one
    // partial round), 1208–1228 against 1105. With fewer, the 128-row tiles spread over more CUs.
    if (tiles(256) > cus / 2) {
        // 224-row tiles where their rounds on the CUs cover fewer rows than the 256-row tiles' (the
        // same work per row, one workgroup a CU): C1's down-projection (M = 4096, N = 3072) 228 tiles in
        // one round against 192 in one; C4's and C2's fused QKV (M = 4608, N = 9216) 756 tiles in three
        // rounds against 648 in three; never C1's up-projection (768 tiles, three full rounds).
        auto rows = [&](int bm) { return (tiles(bm) + cus - 1) / cus * bm; };
        return rows(224) < rows(256) ? WD_224 : WD_256;
    }
    if (tiles(128) >= fill) return WD_128;
    if (tiles(64) >= fill) {
        // 64 × 192 tiles of six one-block waves while they fit one round on the CUs (and not for the GLU
        // epilogues): less activation and weight per workgroup for the same rows. Measured against the 64-row
        // tiles at K = 3072 in one process: C0 (1024 × 3072) 29.7 against 30.9 µs, and 3–5 % faster on five
        // other shapes of one round (768 × 3072, 192 and 256 × 12288, 256 × 9216); past one round (1280 × 3072,
        // 384 × 9216) 1.6× slower, so not there.
        const long tiles64x192 = (long)((M + 63) / 64) * ((N + 191) / 192);
        return !glu && tiles64x192 <= cus ? WD_64x192 : WD_64;
    }
    if (tiles(32) >= fill) {
        // 64 × 128 tiles, a 32-column block a wave (half the codes widened per MFMA), where they add no tiles
        // to the 32-row ones (a ragged last row tile would): measured over 15 shapes at K = 3072 in one
        // process, C2's text stream (512 × 3072) 20.5 against 23.3 µs, the shapes whose 32-row tiles number
        // more than 256 (704 × 3072, 256 × 9216, 384 × 6144, 512 × 4608) 27.4–27.9 against 34.4–35.1 µs, the
        // others within 0–5 % slower; not for the GLU epilogues.
        const long tiles64n = (long)((M + 63) / 64) * ((N + 127) / 128);
        return !glu && tiles64n <= tiles(32) ? WD_64N : WD_32;
    }
    // Up to 16 rows, the 16-column groups of the short-M kernel where they fit one round on the CUs (N ≤ 4096
    // on 256 CUs; GLU: 2048 output columns): every K step's loads in flight, the activation read once per
    // workgroup. Kernel traces at K = 3072, N = 3072 (int8 packed, bias): M = 1 4.10 µs against the skinny
    // kernel's 7.44, M = 16 5.95 against 8.73; K = 12288, N = 3072: M = 1 10.1 against 19.4. Past one round
    // (N = 9216, 12288) the skinny kernel's 64-column slabs stream better (M = 8: 8.3 against 11.6 µs).
    // Without GLU also two groups a workgroup where one round holds them (N = 6144, M = 1: 7.4 against the
    // skinny kernel's 9.7 µs; M = 16: 9.6 against 10.9), and three for a single row (N = 9216: 8.9 against
    // 9.7; N = 12288: 10.6 against 11.4; at M = 16 the skinny kernel's 10.9 and 11.8 against 11.5 and 13.5).
    const long gemv_groups = glu ? (N / 2 + 7) / 8 : (N + 15) / 16;
    if (M <= 16 && gemv_groups <= cus) return WD_GEMV;
    if (M <= 16 && !glu && (gemv_groups <= 2L * cus || (M == 1 && gemv_groups <= 3L * cus))) return WD_GEMV;
    return M <= 128 ? WD_SKINNY32 : WD_SKINNY64;
}

int choose_wd_tile(int M, int N, bool glu, int cus, int kt) {
    if (cus <= 0) cus = 256;
    const int base = base_wd_tile(M, N, glu, cus);
    // Below the 128-row tiles and not for the GLU epilogues: tiles of one-block waves whose K
    // steps split over wave groups (each group its own activation stages; the CU holds two or four times
    // the waves and the loads in flight of the same tile). The largest of them whose tiles number between
    // 3/4 of the CUs and the CUs, else the one with the most tiles within one round. Measured against the
    // kernel taken without them (one process, medians of 140 launches, HIP events), M × N at K = 3072:
    // 64 × 3072 9.6 against 13.2 µs (32 × 32, four groups), 128 × 3072 11.4 against 13.6 (32 × 64), 256 ×
    // 3072 14.7 against 19.3 (64 × 64), C2's text stream 512 × 3072 18.6 against 20.0 (64 × 128, two
    // groups), C0 1024 × 3072 26.3 against 28.3 (64 × 192), 64 × 9216 14.4 against 20.8, 256 × 12288 26.3
    // against 28.2; at K = 12288, N = 3072: M = 64 19.4 against 33.8, M = 256 36.2 against 56.8.
    // Up to 16 rows only where the short-M kernel would read the activation from global memory (it does not
    // fit its LDS): 16 × 6144 × 3072 11.2 against 13.4 µs, 16 × 12288 × 3072 16.8 against 21.1 (M = 4 at K =
    // 12288 fits: 13.6 against 16.6 for the K-group tile). Past one round of 16-column groups the skinny kernel
    // stays (M = 16, K = 12288, N = 12288: 26.7 against 27.8).
    if (glu || base == WD_256 || base == WD_224 || base == WD_128) return base;
    if (M <= 16 && (base != WD_GEMV || gemv_x_in_lds(M, kt))) return base;
    // The short-M kernel's several groups a workgroup were measured with the activation in LDS only.
    if (M <= 16 && (N + 15) / 16 > cus) return WD_SKINNY32;
    struct Cand { int tile, bm, bn, groups; };
    static const Cand cands[] = {{WD_K64x192, 64, 192, 2}, {WD_K64x128, 64, 128, 2}, {WD_K64x64, 64, 64, 4},
                                 {WD_K32x64, 32, 64, 4}, {WD_K32x32, 32, 32, 4}};
    auto count = [&](const Cand &c) { return (long)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn); };
    for (const Cand &c : cands)
        if (kt % c.groups == 0 && count(c) >= (long)cus * 3 / 4 && count(c) <= cus) return c.tile;
    int best = base;
    long most = 0;
    for (const Cand &c : cands)
        if (kt % c.groups == 0 && count(c) <= cus && count(c) > most) {
            best = c.tile;
            most = count(c);
        }
    return best;
}

int64_t skinny_part_bytes(int M, int N, bool glu, int bm, int splits) {
    const long slabs = glu ? (N / 2 + 31) / 32 : (N + 63) / 64;
    const long tiles = (long)((M + bm - 1) / bm) * slabs;
    return (int64_t)splits * tiles * (2 * (bm / 32)) * 1024 * 4;
}

int choose_tile(int M, int N_out, bool glu, int cus) {
    // Tiles of 256 × 256 while they fill the CUs at least 3/4 of the way; 128 × 128 below.
    if (cus <= 0) cus = 256;
    const int n_virtual = glu ? 2 * N_out : N_out;
    const long big = (long)((M + 255) / 256) * ((n_virtual + 255) / 256);
    return big >= (long)cus * 3 / 4 ? TILE_256x256 : TILE_128x128;
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
