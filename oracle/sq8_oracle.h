/*
 * sq8_oracle.h — CPU restatement of the reference's arithmetic for the weight-quantized linear
 * layer (gwenn-ha-dev/Siliconed). TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it as the checker. The product library never links or calls it.
 *
 * Every function names the reference file:line it restates (paths relative to the reference root).
 */
#ifndef SQ8_ORACLE_H
#define SQ8_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element kinds, numbered as the product library's `sq8_dtype`. */
enum { ORC_BF16 = 1, ORC_F32 = 2, ORC_INT8 = 3, ORC_FP8_E4M3 = 4, ORC_F16 = 5 };
/* Scale layouts of Widen.ScaleLayout (Sources/Siliconed/Widen.swift:100-110). */
enum { ORC_SCALE_TENSOR = 0, ORC_SCALE_COLUMNS = 1, ORC_SCALE_BLOCKS = 2, ORC_SCALE_ROWS = 3 };
/* Epilogues (bias is separate). */
enum { ORC_EPI_NONE = 0, ORC_EPI_GELU_TANH = 1, ORC_EPI_SILU_GLU = 2, ORC_EPI_SITU_GLU = 3 };

/* ---- reproducible synthetic inputs: Sources/Verification/KernelStages.swift:553-567 ---- */
uint64_t orc_splitmix_next(uint64_t *state);
double orc_splitmix_uniform(uint64_t *state);
double orc_splitmix_normal(uint64_t *state);
/* `count` draws mean + std·N(0,1) (Box–Muller of two uniforms each), rounded to fp32 then bf16 RNE. */
void orc_fill_normal_bf16(uint64_t seed, double mean, double std, uint16_t *out, size_t count);
void orc_fill_normal_f32(uint64_t seed, double mean, double std, float *out, size_t count);
/* `count` floats uniform in [lo, hi): lo + (hi − lo)·u, rounded to fp32. */
void orc_fill_uniform_f32(uint64_t seed, double lo, double hi, float *out, size_t count);
/* `count` integers uniform in [lo, hi] (inclusive) as int8: lo + floor(u·(hi − lo + 1)). */
void orc_fill_uniform_i8(uint64_t seed, int lo, int hi, int8_t *out, size_t count);

/* ---- conversions ---- */
/* fp32 → bf16 RNE, NaN kept quiet with its sign/payload: Sources/Siliconed/TensorGEMMBF16.swift:43-47. */
uint16_t orc_f32_to_bf16(float f);
/* bf16 → fp32, a shift: Sources/Siliconed/Widen.swift:25-49. */
float orc_bf16_to_f32(uint16_t b);
/* fp8 E4M3 "fn" → fp32 from the bit formula: Sources/Siliconed/Forge/Numerics.swift:48-55. */
float orc_e4m3_to_f32(uint8_t b);
/* fp16 → fp32 exactly (scales published in fp16: Widen.swift:273-281). */
float orc_f16_to_f32(uint16_t h);
/* fp32 → e4m3fn RNE, saturating at ±448 (the publishers' float8 quantizer cast, used to forge C3/C4 weights). */
uint8_t orc_f32_to_e4m3(float f);
void orc_quantize_e4m3(const float *x, uint8_t *out, size_t count);

/* ---- the dequantiser: Sources/Siliconed/Widen.swift:129-271 ----
 * out[i] = Float(q[i]) · s[layout(i)], one IEEE fp32 multiply, never fused, no scale → plain cast.
 * `columns`: row width for COLUMNS/BLOCKS layouts, K for ROWS; `block_rows`: rows per scale block;
 * `first_row`: the row of values[0] in the whole tensor (BLOCKS and ROWS). */
void orc_dequantize(const void *values, int kind, size_t count, const void *scale, int scale_type,
                    int layout, size_t columns, size_t block_rows, size_t first_row, float *out);

/* ---- ComfyUI's convrot (int8_tensorwise with a Hadamard rotation of the input) ---- */
/* Widen.isRotationGroup (Sources/Siliconed/Widen.swift:335-340): a power of 4, 4 to 256. */
int orc_is_rotation_group(int g);
/* 1/√G (Widen.swift:343). */
float orc_rotation_norm(int g);
/* y = x·R along each of `rows` rows of k values (k a multiple of `group`), R = H/√G block-diagonal:
 * the radix-4 butterflies of rotate_groups (Sources/Siliconed/TensorGEMM.swift:183-201) in fp32,
 * stage order and sums as there, then × 1/√G. x and y may not overlap. */
void orc_rotate_groups(const float *x, int64_t ldx, float *y, int64_t ldy, int rows, int k, int group);
/* Widen.dequantizeRotated (Widen.swift:374-428): codes q [k, n] (leading dimension ldq), rotated
 * along k by groups of `group` rows, exact integers H·q, then Float(m) · (s · 1/√G); scale of type
 * `scale_type` (F32/BF16/F16), one per column (COLUMNS) or one (TENSOR). out [k, n], leading ldo. */
void orc_dequantize_rotated(const int8_t *q, int64_t ldq, int k, int n, int group, const void *scale,
                            int scale_type, int layout, float *out, int64_t ldo);

/* ---- W8A8 (ComfyUI's int8_linear): Sources/Siliconed/TensorGEMMInt8.swift:4-37, 198-221 ---- */
/* Per row of x fp32 [rows, k]: rotated by groups of `group` (0: none) as orc_rotate_groups, then
 * s = max(max|y| / 127, 1e-30), q = clamp(rint(y / s), −128, 127); codes int8 [rows, ldq], scales [rows]. */
void orc_quantize_rows(const float *x, int64_t ldx, int rows, int k, int group, int8_t *codes, int64_t ldq,
                       float *scales);
/* C [m, n] = float(Σ codes·w) · (sx[row] · sw[col]), the sums exact; w int8 [k, n] (w_kn) or [n, k];
 * sw per column or one (sw_per_column 0). */
void orc_w8a8_product(const int8_t *codes, int64_t ldq, const float *sx, const int8_t *w, int w_kn, int64_t ldw,
                      const float *sw, int sw_per_column, int m, int k, int n, float *c, int64_t ldc);

/* ---- epilogues, in double (the definitions the GPU is judged against) ---- */
/* nn.GELU(approximate="tanh") in double: Sources/Siliconed/QwenImage21.swift:953-963. */
double orc_gelu_tanh(double x);
/* silu(g)·u = g / (1 + e^{−g}) · u: Sources/Verification/KernelStages.swift:128-132. */
double orc_silu_glu(double gate, double up);
/* SITU: 4·tanh(g/4)·σ(g) · 25·tanh(h/25): Sources/Siliconed/MossImage.swift:874-876. */
double orc_situ(double hidden, double gate);

/* ---- the truth: Sources/Siliconed/DiagnosticProbes.swift:74-178 ----
 * Midpoint rows of `count` equal slices of m: DiagnosticProbes.swift:75-77. */
void orc_sample_rows(int m, int count, int *rows);
/* fp64 product rows of A·W with W = dequantized weight (fp32, layout [K,N] if w_kn else [N,K]),
 * A bf16 [m, lda]; then scale per column (`scale` may be NULL: W already scaled), + bias (may be
 * NULL), then the epilogue (GLU epilogues read halves [0,h) and [h,2h) of the n = 2h columns and
 * write h). Output laid out row-major [nrows, n_out] in double. Threaded over rows. */
void orc_exact_rows(const int *rows, int nrows, const uint16_t *a, int64_t lda, const float *w,
                    int w_kn, int64_t ldw, int k, int n, const float *scale, const float *bias,
                    int epilogue, double *out);
/* As orc_exact_rows on an fp32 A [*, lda] taken whole. */
void orc_exact_rows_f32(const int *rows, int nrows, const float *a, int64_t lda, const float *w,
                        int w_kn, int64_t ldw, int k, int n, const float *scale, const float *bias,
                        int epilogue, double *out);
/* Per-channel relative error, floored at 1 % of the median norm, NaN = ∞:
 * Sources/Siliconed/DiagnosticJudgement.swift:39-71. got/expected row-major [rows, columns]. */
double orc_channel_error(const float *got, const double *expected, int rows, int columns,
                         int *worst_channel, double *median);

/* ---- the reference's CPU route (the timed baseline): WeightProducts.swift:698-709 + Ops.swift:400-407 ----
 * C[m, n_out] (fp32) = act(A_bf16 · W_f32 + bias) with W_f32 = dequantized weight [K, N]
 * (dequantized via orc_dequantize), A widened exactly; fp32 sums over K in blocks, multi-threaded.
 * Bias added after the product (one rounding), then the epilogue in fp32 (Ops.swift:386-398 for
 * GELU, Ops.swift:64-94 for SiLU). */
void orc_linear_f32(const uint16_t *a, int64_t lda, const float *w_kn, int64_t ldw, int m, int k,
                    int n, const float *bias, int epilogue, float *c, int64_t ldc, int threads);
/* Apply bias and epilogue in fp32 to an fp32 product P[m, n] (n = 2h for GLU) into C[m, n_out]. */
void orc_epilogue_f32(const float *p, int64_t ldp, int m, int n, const float *bias, int epilogue,
                      float *c, int64_t ldc, int threads);

int orc_version(void);

#ifdef __cplusplus
}
#endif
#endif
