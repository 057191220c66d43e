/*
 * sq8_oracle.c — CPU restatement of the reference's arithmetic for the weight-quantized linear
 * layer. TEST INFRASTRUCTURE ONLY (see sq8_oracle.h). Built with -ffp-contract=off: every product
 * below rounds once, as the reference's vDSP passes do (Sources/Siliconed/Widen.swift:94-97).
 */
#include "sq8_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int orc_version(void) { return 1; }

/* ---------------------------------------------------------------------------------------------
 * SplitMix64 and Box–Muller: Sources/Verification/KernelStages.swift:553-567.
 * uniform = (z >> 11) / 2^53; normal = sqrt(−2·log(max(u1, 1e−300)))·cos(2π·u2).
 * ------------------------------------------------------------------------------------------- */
uint64_t orc_splitmix_next(uint64_t *state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

double orc_splitmix_uniform(uint64_t *state) {
    return (double)(orc_splitmix_next(state) >> 11) / 9007199254740992.0; /* 2^53 */
}

double orc_splitmix_normal(uint64_t *state) {
    double u1 = orc_splitmix_uniform(state);
    double u2 = orc_splitmix_uniform(state);
    return sqrt(-2.0 * log(u1 > 1e-300 ? u1 : 1e-300)) * cos(2.0 * M_PI * u2);
}

/* Draw i of a stream depends on i only through the state after 2·i steps, so a long fill is
 * cut into chunks whose states are computed directly (state after j steps = seed + j·γ). */
#define ORC_CHUNK ((size_t)1 << 16)

void orc_fill_normal_f32(uint64_t seed, double mean, double std, float *out, size_t count) {
    long chunks = (long)((count + ORC_CHUNK - 1) / ORC_CHUNK);
#pragma omp parallel for schedule(static)
    for (long c = 0; c < chunks; ++c) {
        size_t first = (size_t)c * ORC_CHUNK, end = first + ORC_CHUNK < count ? first + ORC_CHUNK : count;
        uint64_t state = seed + (uint64_t)(2 * first) * 0x9E3779B97F4A7C15ull;
        for (size_t i = first; i < end; ++i) out[i] = (float)(mean + std * orc_splitmix_normal(&state));
    }
}

void orc_fill_normal_bf16(uint64_t seed, double mean, double std, uint16_t *out, size_t count) {
    long chunks = (long)((count + ORC_CHUNK - 1) / ORC_CHUNK);
#pragma omp parallel for schedule(static)
    for (long c = 0; c < chunks; ++c) {
        size_t first = (size_t)c * ORC_CHUNK, end = first + ORC_CHUNK < count ? first + ORC_CHUNK : count;
        uint64_t state = seed + (uint64_t)(2 * first) * 0x9E3779B97F4A7C15ull;
        for (size_t i = first; i < end; ++i)
            out[i] = orc_f32_to_bf16((float)(mean + std * orc_splitmix_normal(&state)));
    }
}

void orc_fill_uniform_f32(uint64_t seed, double lo, double hi, float *out, size_t count) {
    long chunks = (long)((count + ORC_CHUNK - 1) / ORC_CHUNK);
#pragma omp parallel for schedule(static)
    for (long c = 0; c < chunks; ++c) {
        size_t first = (size_t)c * ORC_CHUNK, end = first + ORC_CHUNK < count ? first + ORC_CHUNK : count;
        uint64_t state = seed + (uint64_t)first * 0x9E3779B97F4A7C15ull;
        for (size_t i = first; i < end; ++i) out[i] = (float)(lo + (hi - lo) * orc_splitmix_uniform(&state));
    }
}

void orc_fill_uniform_i8(uint64_t seed, int lo, int hi, int8_t *out, size_t count) {
    long chunks = (long)((count + ORC_CHUNK - 1) / ORC_CHUNK);
    double span = (double)(hi - lo + 1);
#pragma omp parallel for schedule(static)
    for (long c = 0; c < chunks; ++c) {
        size_t first = (size_t)c * ORC_CHUNK, end = first + ORC_CHUNK < count ? first + ORC_CHUNK : count;
        uint64_t state = seed + (uint64_t)first * 0x9E3779B97F4A7C15ull;
        for (size_t i = first; i < end; ++i) {
            int v = lo + (int)floor(orc_splitmix_uniform(&state) * span);
            out[i] = (int8_t)(v > hi ? hi : v);
        }
    }
}

/* ---------------------------------------------------------------------------------------------
 * Conversions.
 * ------------------------------------------------------------------------------------------- */
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Sources/Siliconed/TensorGEMMBF16.swift:43-47: a NaN stays a quiet NaN (sign and payload kept,
 * quiet bit set), else add 0x7FFF plus the lowest kept bit and shift — an overflow rounds to ∞. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* Sources/Siliconed/Widen.swift:25-49: the sixteen bits at the head of a 32-bit word. */
float orc_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* Sources/Siliconed/Forge/Numerics.swift:48-55: sign, e = bits 6..3, m = bits 2..0, bias 7;
 * e = 15 and m = 7 is NaN; e = 0 is m/8·2^−6; else (1 + m/8)·2^(e−7). No infinity. */
float orc_e4m3_to_f32(uint8_t b) {
    float sign = (b & 0x80) ? -1.0f : 1.0f;
    int e = (b >> 3) & 0xF, m = b & 0x7;
    if (e == 0xF && m == 0x7) return NAN;
    if (e == 0) return sign * (float)m / 8.0f * ldexpf(1.0f, -6);
    return sign * (1.0f + (float)m / 8.0f) * ldexpf(1.0f, e - 7);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1F) return bits_f32(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * ldexpf(1.0f, -24);
        return sign ? -v : v;
    }
    return bits_f32(sign | ((uint32_t)(e - 15 + 127) << 23) | (m << 13));
}

uint8_t orc_f32_to_e4m3(float f) {
    if (isnan(f)) return 0x7F;
    uint8_t sign = signbit(f) ? 0x80 : 0x00;
    double a = fabs((double)f);
    if (a >= 448.0) return sign | 0x7E;
    uint8_t code;
    if (a < 0.015625) {                                   /* below 2^−6: subnormal step 2^−9 */
        double q = nearbyint(a * 512.0);                  /* ties to even */
        code = (uint8_t)q;                                /* q == 8 is 2^−6, code 0x08 */
    } else {
        int e;
        double frac = frexp(a, &e);                       /* a = frac·2^e, frac in [0.5, 1) */
        e -= 1;                                           /* a = (2·frac)·2^e, 2·frac in [1, 2) */
        double q = nearbyint((2.0 * frac - 1.0) * 8.0);
        if (q == 8.0) { q = 0.0; e += 1; }
        int field = e + 7;
        code = (uint8_t)((field << 3) | (int)q);
        if (code > 0x7E) code = 0x7E;
    }
    return sign | code;
}

void orc_quantize_e4m3(const float *x, uint8_t *out, size_t count) {
    long n = (long)count;
#pragma omp parallel for schedule(static) if (n > (1L << 16))
    for (long i = 0; i < n; ++i) out[i] = orc_f32_to_e4m3(x[i]);
}

/* ---------------------------------------------------------------------------------------------
 * Dequantiser: Sources/Siliconed/Widen.swift:129-271.
 * ------------------------------------------------------------------------------------------- */
static inline float code_value(const void *values, int kind, size_t i) {
    if (kind == ORC_INT8) return (float)((const int8_t *)values)[i];
    return orc_e4m3_to_f32(((const uint8_t *)values)[i]);
}

static inline float scale_value(const void *scale, int scale_type, size_t i) {
    switch (scale_type) {
    case ORC_BF16: return orc_bf16_to_f32(((const uint16_t *)scale)[i]);
    case ORC_F16: return orc_f16_to_f32(((const uint16_t *)scale)[i]);
    default: return ((const float *)scale)[i];
    }
}

void orc_dequantize(const void *values, int kind, size_t count, const void *scale, int scale_type,
                    int layout, size_t columns, size_t block_rows, size_t first_row, float *out) {
    long n = (long)count;
    if (!scale) {
#pragma omp parallel for schedule(static) if (n > (1L << 17))
        for (long i = 0; i < n; ++i) out[i] = code_value(values, kind, (size_t)i);
        return;
    }
    switch (layout) {
    case ORC_SCALE_TENSOR: {
        float s = scale_value(scale, scale_type, 0);
#pragma omp parallel for schedule(static) if (n > (1L << 17))
        for (long i = 0; i < n; ++i) out[i] = code_value(values, kind, (size_t)i) * s;
        break;
    }
    case ORC_SCALE_COLUMNS:
#pragma omp parallel for schedule(static) if (n > (1L << 17))
        for (long i = 0; i < n; ++i)
            out[i] = code_value(values, kind, (size_t)i) * scale_value(scale, scale_type, (size_t)i % columns);
        break;
    case ORC_SCALE_BLOCKS:
#pragma omp parallel for schedule(static) if (n > (1L << 17))
        for (long i = 0; i < n; ++i) {
            size_t row = first_row + (size_t)i / columns, col = (size_t)i % columns;
            out[i] = code_value(values, kind, (size_t)i) * scale_value(scale, scale_type, (row / block_rows) * columns + col);
        }
        break;
    case ORC_SCALE_ROWS:
#pragma omp parallel for schedule(static) if (n > (1L << 17))
        for (long i = 0; i < n; ++i)
            out[i] = code_value(values, kind, (size_t)i) * scale_value(scale, scale_type, first_row + (size_t)i / columns);
        break;
    }
}

/* ---------------------------------------------------------------------------------------------
 * ComfyUI's convrot: Sources/Siliconed/Widen.swift:316-428 and the activation's rotation
 * Sources/Siliconed/TensorGEMM.swift:181-201.
 * ------------------------------------------------------------------------------------------- */
int orc_is_rotation_group(int g) {
    /* Widen.isRotationGroup (Widen.swift:335-340): a power of 4 from 4 to 256. */
    int p = 4;
    while (p < g) p *= 4;
    return p == g && g <= 256;
}

float orc_rotation_norm(int g) {
    /* Widen.rotationNorm (Widen.swift:343): 1 / √G, a power of two for a power of 4. */
    return 1.0f / sqrtf((float)g);
}

void orc_rotate_groups(const float *x, int64_t ldx, float *y, int64_t ldy, int rows, int k, int group) {
    /* rotate_groups (TensorGEMM.swift:183-201), one group at a time: spans 1, 4, 16, 64 below G;
     * the 4-point butterfly p = a + b, m = a − b, u = c + d, w = c − d → (p + w, p − w, m + u, u − m),
     * every sum rounded to fp32 on its own; then each value times 1/√G. */
    const float norm = orc_rotation_norm(group);
#pragma omp parallel for schedule(static) if ((int64_t)rows * k > (1L << 18))
    for (int r = 0; r < rows; ++r) {
        float v[256];
        for (int g0 = 0; g0 < k; g0 += group) {
            for (int i = 0; i < group; ++i) v[i] = x[(int64_t)r * ldx + g0 + i];
            for (int span = 1; span < group; span *= 4) {
                for (int t = 0; t < group / 4; ++t) {
                    const int j = (t / span) * 4 * span + t % span;
                    const float a = v[j], b = v[j + span], c = v[j + 2 * span], d = v[j + 3 * span];
                    const float p = a + b, m = a - b, u = c + d, w = c - d;
                    v[j] = p + w;
                    v[j + span] = p - w;
                    v[j + 2 * span] = m + u;
                    v[j + 3 * span] = u - m;
                }
            }
            for (int i = 0; i < group; ++i) y[(int64_t)r * ldy + g0 + i] = v[i] * norm;
        }
    }
}

void orc_dequantize_rotated(const int8_t *q, int64_t ldq, int k, int n, int group, const void *scale,
                            int scale_type, int layout, float *out, int64_t ldo) {
    /* Widen.dequantizeRotated (Widen.swift:374-428): per column c and group of G rows, the integer
     * m = H·q (H the unnormalized Kronecker power of H4, exact in int32: |m| ≤ 32 648 for G = 256),
     * then out = Float(m) · f_c with f_c = s_c · (1/√G) (one fp32 multiply each). Scales per column
     * (layout COLUMNS, n of them) or one for the tensor (TENSOR). */
    const float norm = orc_rotation_norm(group);
#pragma omp parallel for schedule(static) if ((int64_t)k * n > (1L << 18))
    for (int c = 0; c < n; ++c) {
        const float f = scale_value(scale, scale_type, layout == ORC_SCALE_TENSOR ? 0 : (size_t)c) * norm;
        int32_t v[256];
        for (int g0 = 0; g0 < k; g0 += group) {
            for (int i = 0; i < group; ++i) v[i] = q[(int64_t)(g0 + i) * ldq + c];
            for (int span = 1; span < group; span *= 4) {
                for (int t = 0; t < group / 4; ++t) {
                    const int j = (t / span) * 4 * span + t % span;
                    const int32_t a = v[j], b = v[j + span], cc = v[j + 2 * span], d = v[j + 3 * span];
                    v[j] = a + b + cc - d;
                    v[j + span] = a + b - cc + d;
                    v[j + 2 * span] = a - b + cc + d;
                    v[j + 3 * span] = -a + b + cc + d;
                }
            }
            for (int i = 0; i < group; ++i) out[(int64_t)(g0 + i) * ldo + c] = (float)v[i] * f;
        }
    }
}

/* ---------------------------------------------------------------------------------------------
 * W8A8: ComfyUI's int8_linear on a per-row quantized activation,
 * Sources/Siliconed/TensorGEMMInt8.swift:4-37 (the recipe), :198-221 (W8A8.quantize).
 * ------------------------------------------------------------------------------------------- */
void orc_quantize_rows(const float *x, int64_t ldx, int rows, int k, int group, int8_t *codes, int64_t ldq,
                       float *scales) {
    /* Per row: y = x rotated by groups of `group` (none when 0: TensorGEMMInt8.swift:200-216, the
     * butterflies of rotate_groups then × 1/√G), s = max(max|y| / 127, 1e-30) (an IEEE division),
     * q = clamp(rint(y / s), −128, 127) (IEEE division, rint half to even). */
#pragma omp parallel for schedule(static) if ((int64_t)rows * k > (1L << 18))
    for (int r = 0; r < rows; ++r) {
        float *y = (float *)malloc((size_t)(k > 0 ? k : 1) * sizeof(float));
        if (group > 0) orc_rotate_groups(x + (int64_t)r * ldx, ldx, y, k, 1, k, group);
        else memcpy(y, x + (int64_t)r * ldx, (size_t)k * sizeof(float));
        float top = 0.0f;
        for (int i = 0; i < k; ++i) top = fmaxf(top, fabsf(y[i]));
        const float q = top / 127.0f;
        const float scale = q > 1e-30f ? q : 1e-30f;
        for (int i = 0; i < k; ++i) {
            float c = rintf(y[i] / scale);
            c = c < -128.0f ? -128.0f : (c > 127.0f ? 127.0f : c);
            codes[(int64_t)r * ldq + i] = (int8_t)c;
        }
        scales[r] = scale;
        free(y);
    }
}

void orc_w8a8_product(const int8_t *codes, int64_t ldq, const float *sx, const int8_t *w, int w_kn, int64_t ldw,
                      const float *sw, int sw_per_column, int m, int k, int n, float *c, int64_t ldc) {
    /* acc = Σ codes·w exactly (int64 here; int32 in the kernel, exact for k < 2^17), then
     * C = float(acc) · (s_x[row] · s_w[col]): the scale product first (TensorGEMMInt8.swift:19-31,
     * `scale_products` :133-140). */
#pragma omp parallel for schedule(static) if ((int64_t)m * n > 4096)
    for (int r = 0; r < m; ++r) {
        for (int j = 0; j < n; ++j) {
            int64_t acc = 0;
            for (int i = 0; i < k; ++i) {
                const int8_t wv = w_kn ? w[(int64_t)i * ldw + j] : w[(int64_t)j * ldw + i];
                acc += (int64_t)codes[(int64_t)r * ldq + i] * wv;
            }
            const float f = sx[r] * sw[sw_per_column ? j : 0];
            c[(int64_t)r * ldc + j] = (float)(int32_t)acc * f;
        }
    }
}

/* ---------------------------------------------------------------------------------------------
 * Epilogues in double.
 * ------------------------------------------------------------------------------------------- */
/* GELU-tanh, ½x(1 + tanh u) with u = √(2/π)(x + 0.044715x³) (QwenImage21.swift:953-963, the double
 * form rounded once), evaluated as x / (1 + e^(−2u)): the identical function, since ½(1 + tanh u) =
 * 1 / (1 + e^(−2u)), without the cancellation of 1 + tanh u in the negative tail, where the literal form
 * returns −0 for x ≤ −8 although the value (about x·e^(2u), −3·10⁻²¹ at x = −8) is a normal fp32. */
double orc_gelu_tanh(double x) {
    const double c = sqrt(2.0 / M_PI);
    const double u = c * (x + 0.044715 * x * x * x);
    return x / (1.0 + exp(-2.0 * u));
}

double orc_silu_glu(double gate, double up) { return gate / (1.0 + exp(-gate)) * up; }

double orc_situ(double hidden, double gate) {
    return (4.0 * tanh(gate / 4.0) * (1.0 / (1.0 + exp(-gate)))) * (25.0 * tanh(hidden / 25.0));
}

/* ---------------------------------------------------------------------------------------------
 * The truth: Sources/Siliconed/DiagnosticProbes.swift:74-178.
 * ------------------------------------------------------------------------------------------- */
void orc_sample_rows(int m, int count, int *rows) {
    for (int i = 0; i < count; ++i) rows[i] = (int)(((int64_t)(2 * i + 1) * m) / (2 * count));
}

static double epilogue_one(int epilogue, const double *row, int j, int h) {
    switch (epilogue) {
    case ORC_EPI_GELU_TANH: return orc_gelu_tanh(row[j]);
    case ORC_EPI_SILU_GLU: return orc_silu_glu(row[j], row[h + j]);
    case ORC_EPI_SITU_GLU: return orc_situ(row[j], row[h + j]);
    default: return row[j];
    }
}

/* The sampled rows of A, widened to double ([nrows, k]), against W: the probe's sums in double. */
static void exact_from_rows(double *arow, int nrows, const float *w, int w_kn, int64_t ldw, int k, int n,
                            const float *scale, const float *bias, int epilogue, double *out) {
    int glu = epilogue == ORC_EPI_SILU_GLU || epilogue == ORC_EPI_SITU_GLU;
    int h = glu ? n / 2 : n;
    double *prod = (double *)calloc((size_t)nrows * n, sizeof(double));
    if (w_kn) {
        /* W [K, N]: each thread owns a block of columns and streams its K rows once. */
        const int CB = 256;
        int blocks = (n + CB - 1) / CB;
#pragma omp parallel for schedule(dynamic)
        for (int b = 0; b < blocks; ++b) {
            int j0 = b * CB, j1 = j0 + CB < n ? j0 + CB : n;
            for (int kk = 0; kk < k; ++kk) {
                const float *wr = w + (int64_t)kk * ldw;
                for (int r = 0; r < nrows; ++r) {
                    double av = arow[(size_t)r * k + kk];
                    double *pr = prod + (size_t)r * n;
                    for (int j = j0; j < j1; ++j) pr[j] += av * (double)wr[j];
                }
            }
        }
    } else {
#pragma omp parallel for schedule(dynamic)
        for (int j = 0; j < n; ++j) {
            const float *wr = w + (int64_t)j * ldw;
            for (int r = 0; r < nrows; ++r) {
                const double *ar = arow + (size_t)r * k;
                double s = 0.0;
                for (int kk = 0; kk < k; ++kk) s += ar[kk] * (double)wr[kk];
                prod[(size_t)r * n + j] = s;
            }
        }
    }
    for (int r = 0; r < nrows; ++r) {
        double *pr = prod + (size_t)r * n;
        for (int j = 0; j < n; ++j) {
            if (scale) pr[j] *= (double)scale[j];
            if (bias) pr[j] += (double)bias[j];
        }
        for (int j = 0; j < h; ++j) out[(size_t)r * h + j] = epilogue_one(epilogue, pr, j, h);
    }
    free(prod);
}

void orc_exact_rows(const int *rows, int nrows, const uint16_t *a, int64_t lda, const float *w,
                    int w_kn, int64_t ldw, int k, int n, const float *scale, const float *bias,
                    int epilogue, double *out) {
    double *arow = (double *)malloc((size_t)nrows * k * sizeof(double));
    for (int r = 0; r < nrows; ++r)
        for (int kk = 0; kk < k; ++kk) arow[(size_t)r * k + kk] = orc_bf16_to_f32(a[(int64_t)rows[r] * lda + kk]);
    exact_from_rows(arow, nrows, w, w_kn, ldw, k, n, scale, bias, epilogue, out);
    free(arow);
}

/* The same truth on an fp32 A taken whole (the reference's probe widens its fp32 operand to double,
 * DiagnosticProbes.swift:79-84): the truth of the fp32 route. */
void orc_exact_rows_f32(const int *rows, int nrows, const float *a, int64_t lda, const float *w,
                        int w_kn, int64_t ldw, int k, int n, const float *scale, const float *bias,
                        int epilogue, double *out) {
    double *arow = (double *)malloc((size_t)nrows * k * sizeof(double));
    for (int r = 0; r < nrows; ++r)
        for (int kk = 0; kk < k; ++kk) arow[(size_t)r * k + kk] = (double)a[(int64_t)rows[r] * lda + kk];
    exact_from_rows(arow, nrows, w, w_kn, ldw, k, n, scale, bias, epilogue, out);
    free(arow);
}

/* Sources/Siliconed/DiagnosticJudgement.swift:39-71. */
static int cmp_double(const void *x, const void *y) {
    double a = *(const double *)x, b = *(const double *)y;
    return (a > b) - (a < b);
}

double orc_channel_error(const float *got, const double *expected, int rows, int columns,
                         int *worst_channel, double *median) {
    double *num = (double *)calloc((size_t)columns, sizeof(double));
    double *den = (double *)calloc((size_t)columns, sizeof(double));
    double *norms = (double *)malloc((size_t)columns * sizeof(double));
    double *live = (double *)malloc((size_t)columns * sizeof(double));
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < columns; ++c) {
            size_t i = (size_t)r * columns + c;
            double e = expected[i], d = (double)got[i] - e;
            num[c] += d * d;
            den[c] += e * e;
        }
    int nn = 0;
    for (int c = 0; c < columns; ++c)
        if (den[c] > 0) norms[nn++] = sqrt(den[c]);
    double worst = 0.0, med = 0.0;
    int channel = 0;
    if (nn > 0) {
        qsort(norms, (size_t)nn, sizeof(double), cmp_double);
        double floor_ = 0.01 * norms[nn / 2];
        int nl = 0;
        for (int c = 0; c < columns; ++c) {
            if (!(den[c] > 0)) continue;
            double d = sqrt(den[c]);
            double r = sqrt(num[c]) / (d > floor_ ? d : floor_);
            if (isnan(r)) r = INFINITY;
            live[nl++] = r;
            if (r > worst) { worst = r; channel = c; }
        }
        qsort(live, (size_t)nl, sizeof(double), cmp_double);
        med = live[nl / 2];
    }
    if (worst_channel) *worst_channel = channel;
    if (median) *median = med;
    free(num); free(den); free(norms); free(live);
    return worst;
}

/* ---------------------------------------------------------------------------------------------
 * The reference's fp32 epilogue passes: bias (Ops.swift:400-407, vDSP_vadd after the product),
 * GELU-tanh in fp32 with tanhf (Ops.swift:386-398), SiLU gate (Ops.swift:64-94: −a, e^{−a},
 * 1 + e^{−a}, a / (1 + e^{−a}), · b, each rounded), SITU in fp32 (MossImage.swift:889-900).
 * ------------------------------------------------------------------------------------------- */
void orc_epilogue_f32(const float *p, int64_t ldp, int m, int n, const float *bias, int epilogue,
                      float *c, int64_t ldc, int threads) {
    int glu = epilogue == ORC_EPI_SILU_GLU || epilogue == ORC_EPI_SITU_GLU;
    int h = glu ? n / 2 : n;
    const float gc = (float)sqrt(2.0 / M_PI);
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (int i = 0; i < m; ++i) {
        const float *pr = p + (int64_t)i * ldp;
        float *cr = c + (int64_t)i * ldc;
        for (int j = 0; j < h; ++j) {
            float v = pr[j];
            if (bias) v = v + bias[j];
            switch (epilogue) {
            case ORC_EPI_GELU_TANH:
                v = 0.5f * v * (1.0f + tanhf(gc * (v + 0.044715f * v * v * v)));
                break;
            case ORC_EPI_SILU_GLU: {
                float u = pr[h + j];
                if (bias) u = u + bias[h + j];
                float e = expf(-v);
                float s = 1.0f + e;
                v = (v / s) * u;
                break;
            }
            case ORC_EPI_SITU_GLU: {
                float g = pr[h + j];
                if (bias) g = g + bias[h + j];
                float gate = 4.0f * tanhf(g / 4.0f) * (1.0f / (1.0f + expf(-g)));
                float value = 25.0f * tanhf(v / 25.0f);
                v = gate * value;
                break;
            }
            default: break;
            }
            cr[j] = v;
        }
    }
}
