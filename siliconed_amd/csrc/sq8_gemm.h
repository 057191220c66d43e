// sq8_gemm.h — host/device interface of the gfx950 weight-quantized GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sq8_device.h"

namespace sq8 {

// One launch's operands; all pointers are device pointers.
struct GemmArgs {
    const uint16_t *a;      // bf16 [M, K], leading dimension lda (elements)
    int64_t lda;
    const uint8_t *w;       // codes: [K, N] (W_KN) or [N, K] (W_NK), leading dimension ldw
    int64_t ldw;
    const float *scale;     // fp32 [N] (scale_per_col) or [1]
    const float *bias;      // fp32 [N] or null
    void *c[3];             // outputs; c[1], c[2] only with `split`
    int64_t c_d1, c_d2;     // byte offsets of c[1], c[2] from c[0] (the device never indexes c[])
    int64_t ldc;
    int split;              // > 0: output columns [i·split, (i+1)·split) go to c[i]
    int head_dim;           // > 0: each output is [cols/head_dim, M, head_dim]
    int M, N, K;            // N: weight columns (2h for a GLU epilogue)
    int glu_half;           // h for GLU epilogues
    int scale_per_col;
    int a_vec, w_vec, c_vec; // 16-byte loads of A, wide loads of W, wide stores of C allowed
    int c_vec16;            // 16-byte stores of C allowed (aligned base, stride, split and head size)
    int sb_vec;             // 16-byte loads of 4 scales / biases allowed (aligned bases, GLU half % 4 == 0)
    int kt;                 // K steps of 64 (the packed layout's K extent); W8A8: K steps of 128
    int tiles_m, tiles_n;   // set by the launcher
    const float *gate;      // EPI_RESIDUAL: per-column gate fp32 [N], or null (1)
    const float *sx;        // W8A8: the activation's row scales fp32 [M] (`a` then holds int8 codes)
    int kt_w;               // W8A8: K steps of 64 of the packed weight; weight-direct kernels: the weight's
                            // K steps when the activation holds several parts along K (0: kt)
    float *part;            // the skinny kernel's K split: fp32 partial sums, skinny_part_bytes() of them
    int splits;             // > 1: the skinny kernel's K steps split over this many workgroups per tile, whose
                            // sums a second launch adds in split order before the epilogue
    int cus;                // the device's compute units (0: 256), for launch shapes chosen per product
};

enum Tile { TILE_256x256 = 0, TILE_128x128 = 1 };

int choose_tile(int M, int N_out, bool glu, int cus);
// `fast`: the branch-free kernels, valid when A rows and W rows/columns can be read with vector
// loads (alignment), K is a positive multiple of 64, and there are at least 4 weight columns (per
// GLU half) with a [K, N] weight's column count a multiple of 4.
hipError_t launch_gemm(const GemmArgs &p, bool fast, int tile, int wt, int wl, int epi, int out, hipStream_t stream);

// The weight-direct kernels (sq8_wdirect_inst.hip): [N, K] or packed weights, K a multiple of 64,
// A aligned for 16-byte loads. `tile`: WD_256 (256 × 256, one workgroup per CU), WD_224 (224 × 256, the
// same kernel), WD_128 (128 × 256, two workgroups per CU), WD_64 (64 × 256, one per CU), WD_32 (32 × 256,
// two per CU), WD_64N (64 × 128, a 32-column block a wave, two per CU; not GLU), WD_64x192 (64 × 192, six
// waves of one 32-column block; not GLU), or the skinny-M kernel with 64- or 32-row tiles of one 64-column
// slab and the K steps split over four waves (WD_SKINNY64, WD_SKINNY32), or M ≤ 64 in 16-column groups on
// 16 × 16 MFMAs, every K step's loads issued far ahead (WD_GEMV), or tiles of one-block waves whose K steps
// split over two or four wave groups (WD_K32x32, WD_K32x64, WD_K64x64: four groups; WD_K64x128, WD_K64x192:
// two; not GLU, K/64 a multiple of the groups).
enum WdTile { WD_256 = 0, WD_128 = 1, WD_SKINNY64 = 2, WD_SKINNY32 = 3, WD_64 = 4, WD_32 = 5, WD_224 = 6, WD_64N = 7, WD_64x192 = 8,
              WD_GEMV = 9, WD_K32x32 = 10, WD_K32x64 = 11, WD_K64x64 = 12, WD_K64x128 = 13, WD_K64x192 = 14 };
// The tile for an M × N product (GLU: N = 2h): 256 or 224 rows × 256 while those tiles occupy more than
// half the 256 CUs (the height whose rounds of 256 tiles cover the fewest rows; launch_wdirect takes
// 128-row tiles where that kernel cannot serve the product), else the tallest of 128, 64 and 32 rows
// whose tiles number at least 144 (enough to occupy the 256 CUs), else the skinny kernel; below the 128-row
// tiles the K-group tiles where one fits a round (up to 16 rows only where the short-M kernel would read the
// activation from global memory). `kt`: the product's K steps of 64.
int choose_wd_tile(int M, int N, bool glu, int cus, int kt);
// The short-M kernel (sq8_gemv_kernel.h): the activation staged in LDS (M rows of K' = kt · 64 bf16, rows
// gemv_xpitch bytes apart: 16 more than a row, so the 16 rows a fragment read touches start on different banks)
// when it fits GEMV_XLDS bytes and each row is whole 1 KB runs (K' a multiple of 512), the unit of a direct load.
constexpr int GEMV_XLDS = 100 * 1024;
__host__ __device__ constexpr int64_t gemv_xpitch(int kt) { return (int64_t)kt * 128 + 16; }
__host__ __device__ constexpr bool gemv_x_in_lds(int m, int kt) {
    return kt % 8 == 0 && (int64_t)m * gemv_xpitch(kt) <= GEMV_XLDS;
}
// Bytes of the partial sums of a split skinny product (tile height bm, `splits` splits).
int64_t skinny_part_bytes(int M, int N, bool glu, int bm, int splits);
hipError_t launch_wdirect(const GemmArgs &p, int tile, int wt, int wl, int epi, int out, hipStream_t stream);

// Bytes of the packed layout of a weight with k rows of K and n columns (GLU: n = 2h, packed in
// pairs of 32-column blocks of the two halves).
int64_t packed_bytes(int k, int n, bool glu);
// True when launch_pack has its LDS-transposing path for these [K, N] codes (k % 256 == 0, whole
// 64-column slabs, 16-byte aligned rows): a repack runs near the memory bandwidth.
bool pack_is_fast(const uint8_t *w, int wl, int64_t ldw, int k, int n, bool glu);
// Writes the packed layout of codes `w` (layout W_KN or W_NK, leading dimension ldw) into `out`.
hipError_t launch_pack(const uint8_t *w, int wl, int64_t ldw, int k, int n, bool glu, uint8_t *out,
                       hipStream_t stream);

// Codes with a scale per block of rows and column (GGUF Q8_0; sq8_blocks.hip): the packed Q8 layout
// (codes in block-aligned K order, then fp32 scales per step and column) and its product, int8
// codes, K a multiple of 64, A aligned for 16-byte loads. `tile`: BL_64x256 (two workgroups per CU),
// BL_64x512 (one), BL_128x256 / BL_128x128 (eight waves of one 32-column block each, one or two
// workgroups per CU; not for GLU epilogues, which then take BL_64x256). Scales [K/B, N] for W_KN codes, [N, K/B] for W_NK; B a multiple of 32
// dividing K; scale dtype numbered as the C ABI's (fp32, bf16, fp16).
enum BlocksTile { BL_64x256 = 0, BL_64x512 = 1, BL_128x256 = 2, BL_128x128 = 3 };
int64_t packed_blocks_bytes(int k, int n, bool glu);
hipError_t launch_pack_blocks(const uint8_t *w, int wl, int64_t ldw, const void *scale, int scale_dtype, int block,
                              int k, int n, bool glu, uint8_t *out, hipStream_t stream);
hipError_t launch_blocks_product(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream);

// Auxiliary kernels (sq8_aux.hip).
hipError_t launch_dequantize(const uint8_t *codes, int wt, int64_t rows, int64_t columns, const void *scale,
                             int scale_dtype, int scale_layout, int64_t block_rows, int64_t first_row, float *out,
                             hipStream_t stream);
hipError_t launch_round_bf16(const float *x, uint16_t *y, int64_t count, hipStream_t stream);
// rows × k values read ldx apart → rows × kp bf16 written kp apart (kp ≥ k, columns [k, kp) zero; one
// launch, any stride).
hipError_t launch_round_bf16_rows(const float *x, int64_t ldx, uint16_t *y, int64_t rows, int k, int kp,
                                  hipStream_t stream);
// bf16 rows × k read ldx apart → rows × kp written kp apart, columns [k, kp) zero.
hipError_t launch_pad_bf16_rows(const uint16_t *x, int64_t ldx, uint16_t *y, int64_t rows, int k, int kp,
                                hipStream_t stream);
// Columns [k, kp) of rows × ld bf16 set to zero.
hipError_t launch_zero_tail(uint16_t *y, int64_t ld, int64_t rows, int k, int kp, hipStream_t stream);
// fp32 [rows, k] (leading dimension ldx) → bf16 [rows, 3kp]: the three parts hi | mid | lo of each value
// (each the top 16 bits of what the one before leaves: hi + mid + lo = x, no part rounded), each part kp ≥ k
// wide with columns [k, kp) zero; the fp32 route's operand.
hipError_t launch_split3(const float *x, int64_t ldx, uint16_t *y, int64_t rows, int k, int kp, hipStream_t stream);

// ComfyUI's convrot (sq8_convrot.hip): the activation's rotation x·R by groups of `group` (4, 16,
// 64 or 256; k a multiple of it), fp32 or bf16 in, fp32 or bf16 (rounded to nearest even) out; and
// the rotated weight widened, Float(H·q)·(s/√G), codes [k, n] rotated along k.
bool is_rotation_group(int group);
hipError_t launch_rotate_groups(const void *x, bool x_bf16, int64_t ldx, void *y, bool y_bf16, int64_t ldy, int64_t rows,
                                int k, int group, hipStream_t stream);
hipError_t launch_dequantize_rotated(const int8_t *q, int64_t ldq, int k, int n, int group, const void *scale,
                                     int scale_dtype, bool per_column, float *out, int64_t ldo, hipStream_t stream);

// W8A8 (sq8_w8a8.hip, sq8_i8_inst.hip): the activation's per-row quantization (optionally rotated
// first) into int8 codes of rows k_pad ≥ k bytes (zero past k) and fp32 row scales; rows up to
// quantize_row_limit() values. The int8 × int8 product: `a` the codes (lda a multiple of 16,
// 16-byte aligned, kt = k_pad / 128 steps, zero past K), `sx` their scales, the weight packed
// (kt_w = its 64-steps) or [N, K] with K a multiple of 128.
int quantize_row_limit();
hipError_t launch_quantize_rows(const void *x, bool x_bf16, int64_t ldx, int rows, int k, int group, int8_t *codes,
                                int64_t ldq, int k_pad, float *scales, hipStream_t stream);
hipError_t launch_pad_codes(const int8_t *src, int64_t ld_src, int8_t *dst, int64_t ld_dst, int64_t rows, int k, int k_pad,
                            hipStream_t stream);
hipError_t launch_i8gemm(const GemmArgs &p, int wl, int epi, int out, hipStream_t stream);

// The DiT block's elementwise passes (sq8_block.hip).
hipError_t launch_norm_modulate(const float *x, int64_t ldx, const float *w, const float *scale, const float *shift,
                                float eps, uint16_t *out, int64_t ldo, int rows, int cols, hipStream_t stream);
// The modulated RMSNorm writing the next product's operand: y rotated by `group` (0: none) and
// rounded to bf16 into `out` (codes == nullptr), or quantized per row into codes (rows of k_pad) and
// scales; y itself into y_out when given. cols % 4 == 0, 16-byte aligned rows and vectors, cols ≤ 32 768.
hipError_t launch_norm_operand(const float *x, int64_t ldx, const float *w, const float *scale, const float *shift,
                               float eps, int rows, int cols, int group, float *y_out, int64_t ldy, uint16_t *out,
                               int64_t ldo, int8_t *codes, int64_t ldq, int k_pad, float *scales, hipStream_t stream);
hipError_t launch_rms_rows(uint16_t *t, int64_t ld, int64_t rows, int cols, const float *w, float eps, hipStream_t stream);
hipError_t launch_gated_residual(float *x, int64_t ldx, const void *y, bool y_bf16, int64_t ldy, const float *gate,
                                 int64_t rows, int cols, hipStream_t stream);

}  // namespace sq8
