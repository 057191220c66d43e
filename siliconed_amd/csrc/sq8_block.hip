// sq8_block.hip — the elementwise passes a DiT block runs between its weight-quantized products,
// each one pass over HBM: the modulated RMSNorm that writes the next product's bf16 operand, the
// per-head RMSNorm of q and k, and the gated residual update.
//
// Rounding as the reference's kernels: every product and sum rounded on its own (no contraction),
// the row's 1/sqrt(mean + eps) from an IEEE divide and square root.
#include <hip/hip_runtime.h>

#include "sq8_device.h"
#include "sq8_gemm.h"
#include "sq8_quant.h"
#include "sq8_rotate.h"

namespace sq8 {
namespace {

// Sum over a workgroup of 256 threads (4 waves): lane butterflies, then the waves' sums in wave
// order.
__device__ __forceinline__ float block_sum_256(float v, float *partial) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = __fadd_rn(v, __shfl_xor(v, o, 64));
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) partial[wave] = v;
    __syncthreads();
    const float total = __fadd_rn(__fadd_rn(__fadd_rn(partial[0], partial[1]), partial[2]), partial[3]);
    return total;
}

// One row per workgroup: out = bf16(((x·r)·w)·(1 + scale) + shift), r = 1/sqrt(mean(x²) + eps)
// (Sources/Siliconed/ElementwiseGPUMoss.swift:30-91, `norm_modulate_rounded`). VEC: four columns a
// thread and step (16-byte loads, 8-byte stores; cols % 4 == 0 and aligned rows).
template <bool VEC>
__global__ void __launch_bounds__(256) norm_modulate_kernel(const float *__restrict__ x, int64_t ldx,
                                                            const float *__restrict__ w, const float *__restrict__ scale,
                                                            const float *__restrict__ shift, float eps,
                                                            uint16_t *__restrict__ out, int64_t ldo, int cols) {
    __shared__ float partial[4];
    const float *src = x + (int64_t)blockIdx.x * ldx;
    uint16_t *dst = out + (int64_t)blockIdx.x * ldo;
    float ss = 0.0f;
    if constexpr (VEC) {
        for (int i = 4 * threadIdx.x; i < cols; i += 1024) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(src + i);
#pragma unroll
            for (int e = 0; e < 4; ++e) ss = __fadd_rn(ss, __fmul_rn(v[e], v[e]));
        }
    } else {
        for (int i = threadIdx.x; i < cols; i += 256) ss = __fadd_rn(ss, __fmul_rn(src[i], src[i]));
    }
    const float mean = __fdiv_rn(block_sum_256(ss, partial), (float)cols);
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
    auto one = [&](float xv, int i) {
        const float v = __fmul_rn(__fmul_rn(xv, r), w[i]);
        return __fadd_rn(__fmul_rn(v, __fadd_rn(scale[i], 1.0f)), shift[i]);
    };
    if constexpr (VEC) {
        for (int i = 4 * threadIdx.x; i < cols; i += 1024) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(src + i);
            const uint32_t lo = round_bf16(one(v[0], i)) | round_bf16(one(v[1], i + 1)) << 16;
            const uint32_t hi = round_bf16(one(v[2], i + 2)) | round_bf16(one(v[3], i + 3)) << 16;
            *reinterpret_cast<u32x2 *>(dst + i) = u32x2{lo, hi};
        }
    } else {
        for (int i = threadIdx.x; i < cols; i += 256) dst[i] = round_bf16(one(src[i], i));
    }
}

// The modulated RMSNorm writing the next product's operand itself (the reference's
// `norm_modulate_quantized`, ElementwiseGPUMoss.swift:94-130, and the operand contract of
// WeightProducts.swift:130-229): y — the fp32 row norm_modulate_kernel<true> computes, the same r
// (its summation order) and the same operations, hence the same bits — is rotated by `stages` stages
// (a convrot weight) and then rounded to bf16 (ROT: what sq8_rotate_groups writes from y) or
// quantized per row (Q8: what sq8_quantize_rows writes from y). y is also written where `y_out` is
// given. The row is held as rot::rotate_chunk holds it, wave w taking the quads w, w + 4, …
// (IT of them at most). cols % 4 == 0 and 16-byte aligned rows and vectors (the launcher checks).
constexpr int OP_ROT = 0, OP_Q8 = 1;

template <int MODE, int IT>
__global__ void __launch_bounds__(256) norm_operand_kernel(const float *__restrict__ x, int64_t ldx, const float *__restrict__ w,
                                                           const float *__restrict__ scale, const float *__restrict__ shift,
                                                           float eps, int cols, int stages, float norm, float *y_out,
                                                           int64_t ldy, uint16_t *out, int64_t ldo, int8_t *codes,
                                                           int64_t ldq, int k_pad, float *scales) {
    __shared__ float partial[4];
    __shared__ __attribute__((aligned(16))) float lds[4][4 * rot::PITCH];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cc = lane >> 4, l16 = lane & 15;
    float *mine = lds[wave] + cc * rot::PITCH;
    const int64_t row = blockIdx.x;
    const float *src = x + row * ldx;
    // r exactly as norm_modulate_kernel<true>: 16-byte loads at 4t + 1024j, then the block sum.
    float ss = 0.0f;
    for (int i = 4 * threadIdx.x; i < cols; i += 1024) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(src + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) ss = __fadd_rn(ss, __fmul_rn(v[e], v[e]));
    }
    const float mean = __fdiv_rn(block_sum_256(ss, partial), (float)cols);
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
    const int cpr = (cols + 255) / 256;
    float v[IT][16];
    float m = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int quad = it * 4 + wave;
        if (4 * quad >= cpr) break;  // wave-uniform
        const int chunk = 4 * quad + cc;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int col = chunk * 256 + 4 * l16 + 64 * u;
            if (chunk < cpr && col < cols) {
                const f32x4 xv = *reinterpret_cast<const f32x4 *>(src + col);
                const f32x4 wv = *reinterpret_cast<const f32x4 *>(w + col);
                const f32x4 sv = *reinterpret_cast<const f32x4 *>(scale + col);
                const f32x4 hv = *reinterpret_cast<const f32x4 *>(shift + col);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float t = __fmul_rn(__fmul_rn(xv[e], r), wv[e]);
                    v[it][4 * u + e] = __fadd_rn(__fmul_rn(t, __fadd_rn(sv[e], 1.0f)), hv[e]);
                }
                if (y_out)
                    *reinterpret_cast<f32x4 *>(y_out + row * ldy + col) =
                        f32x4{v[it][4 * u], v[it][4 * u + 1], v[it][4 * u + 2], v[it][4 * u + 3]};
            } else {
                v[it][4 * u] = v[it][4 * u + 1] = v[it][4 * u + 2] = v[it][4 * u + 3] = 0.0f;
            }
        }
        rot::rotate_chunk(v[it], mine, l16, stages);
        if constexpr (MODE == OP_ROT) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int col = chunk * 256 + 4 * l16 + 64 * u;
                if (chunk < cpr && col < cols) {
                    float t[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) t[e] = v[it][4 * u + e] * norm;
                    *reinterpret_cast<u32x2 *>(out + row * ldo + col) =
                        u32x2{round_bf16(t[0]) | round_bf16(t[1]) << 16, round_bf16(t[2]) | round_bf16(t[3]) << 16};
                }
            }
        } else {
            m = quant::scaled_max(v[it], norm, m);
        }
    }
    if constexpr (MODE == OP_Q8) {
        // The row's maximum (exact in any order), its scale, the codes (sq8_quantize_rows's code).
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        __syncthreads();  // every thread has read the sum out of partial[] before it is reused
        if (lane == 0) partial[wave] = m;
        __syncthreads();
        m = fmaxf(fmaxf(partial[0], partial[1]), fmaxf(partial[2], partial[3]));
        const float sc = quant::row_scale(m);
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int quad = it * 4 + wave;
            if (4 * quad >= cpr) break;
            quant::store_codes<true>(codes + row * ldq, cols, k_pad, 4 * quad + cc, cpr, l16, v[it], sc);
        }
        if (threadIdx.x == 0) scales[row] = sc;
    }
}

// One row of `cols` ≤ 256 bf16 values per wave, in place: t = bf16((t·r)·w), r as above — the
// per-head RMSNorm of q and k. Lane l holds the PER consecutive values [PER·l, PER·l + PER)
// (cols = 64·PER); a row of another width goes through the strided form (PER = 0).
template <int PER>
__global__ void __launch_bounds__(256) rms_rows_kernel(uint16_t *__restrict__ t, int64_t ld, int64_t rows, int cols,
                                                       const float *__restrict__ w, float eps) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    uint16_t *p = t + row * ld;
    constexpr int N = PER > 0 ? PER : 4;
    float v[N];
    if constexpr (PER == 2) {
        const uint32_t d = *reinterpret_cast<const uint32_t *>(p + 2 * lane);
        v[0] = __uint_as_float(d << 16);
        v[1] = __uint_as_float(d & 0xFFFF0000u);
    } else if constexpr (PER == 4) {
        const u32x2 d = *reinterpret_cast<const u32x2 *>(p + 4 * lane);
        v[0] = __uint_as_float(d[0] << 16);
        v[1] = __uint_as_float(d[0] & 0xFFFF0000u);
        v[2] = __uint_as_float(d[1] << 16);
        v[3] = __uint_as_float(d[1] & 0xFFFF0000u);
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int i = PER > 0 ? PER * lane + j : lane + 64 * j;
            v[j] = i < cols ? __uint_as_float((uint32_t)p[i] << 16) : 0.0f;
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < N; ++j) ss = __fadd_rn(ss, __fmul_rn(v[j], v[j]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, o, 64));
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)cols), eps)));
    uint32_t o[N];
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const int i = PER > 0 ? PER * lane + j : lane + 64 * j;
        o[j] = i < cols ? round_bf16(__fmul_rn(__fmul_rn(v[j], r), w[i])) : 0u;
    }
    if constexpr (PER == 2) {
        *reinterpret_cast<uint32_t *>(p + 2 * lane) = o[0] | o[1] << 16;
    } else if constexpr (PER == 4) {
        *reinterpret_cast<u32x2 *>(p + 4 * lane) = u32x2{o[0] | o[1] << 16, o[2] | o[3] << 16};
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int i = PER > 0 ? PER * lane + j : lane + 64 * j;
            if (i < cols) p[i] = (uint16_t)o[j];
        }
    }
}

// Rows of 128 (the heads of q and k): 16 lanes per row, 8 values (16 bytes) a lane, four rows per
// wave, sixteen per workgroup, rows looped over the grid. The same arithmetic as rms_rows_kernel (the
// sum of squares in another order).
__global__ void __launch_bounds__(256) rms_rows128_kernel(uint16_t *__restrict__ t, int64_t ld, int64_t rows,
                                                          const float *__restrict__ w, float eps) {
    const int lane = threadIdx.x & 63, sub = lane & 15;
    const int64_t slot = (int64_t)(threadIdx.x >> 4);  // 16 rows per workgroup
    float wv[8];
    {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(w + 8 * sub);
        const f32x4 b = *reinterpret_cast<const f32x4 *>(w + 8 * sub + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { wv[e] = a[e]; wv[4 + e] = b[e]; }
    }
    for (int64_t base = (int64_t)blockIdx.x * 16; base < rows; base += (int64_t)gridDim.x * 16) {
        const int64_t row = base + slot;
        const bool live = row < rows;  // the shuffles below run in every lane: the row's 16 lanes agree
        u32x4 d = u32x4{0, 0, 0, 0};
        uint16_t *p = t + row * ld + 8 * sub;
        if (live) d = *reinterpret_cast<const u32x4 *>(p);
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = __uint_as_float(d[e] << 16);
            v[2 * e + 1] = __uint_as_float(d[e] & 0xFFFF0000u);
        }
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = __fadd_rn(ss, __fmul_rn(v[e], v[e]));
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, o, 64));
        const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, 128.0f), eps)));
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = round_bf16(__fmul_rn(__fmul_rn(v[2 * e], r), wv[2 * e])) |
                   round_bf16(__fmul_rn(__fmul_rn(v[2 * e + 1], r), wv[2 * e + 1])) << 16;
        if (live) *reinterpret_cast<u32x4 *>(p) = u32x4{o[0], o[1], o[2], o[3]};
    }
}

// x += gate ⊙ y, the product rounded then the sum (ElementwiseGPUAnima.swift:47-62); y bf16 or fp32.
template <bool Y_BF16>
__global__ void __launch_bounds__(256) gated_residual_kernel(float *__restrict__ x, int64_t ldx, const void *__restrict__ y,
                                                             int64_t ldy, const float *__restrict__ gate, int64_t rows,
                                                             int cols) {
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        float *xr = x + r * ldx;
        for (int c = threadIdx.x; c < cols; c += 256) {
            float yv;
            if constexpr (Y_BF16) yv = __uint_as_float((uint32_t)static_cast<const uint16_t *>(y)[r * ldy + c] << 16);
            else yv = static_cast<const float *>(y)[r * ldy + c];
            xr[c] = __fadd_rn(xr[c], __fmul_rn(gate ? gate[c] : 1.0f, yv));
        }
    }
}

int grid_for_rows(int64_t rows) { return (int)(rows < 16384 ? rows : 16384); }

}  // namespace

hipError_t launch_norm_modulate(const float *x, int64_t ldx, const float *w, const float *scale, const float *shift,
                                float eps, uint16_t *out, int64_t ldo, int rows, int cols, hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    const bool vec = cols % 4 == 0 && ldx % 4 == 0 && ldo % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 7) == 0;
    auto a16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    // norm_operand_kernel without a rotation: the same operations in the same order, so the same bits (its
    // second pass over x finds the row in the caches). A version holding four rows a workgroup in registers,
    // x loaded once and the vectors once per four rows, ran the C4 block's 4608 × 3072 rows in the same
    // 21.8 µs (85 MB at 3.9 TB/s): not kept.
    if (vec && a16(w) && a16(scale) && a16(shift) && cols <= 8 * 4096)
        return launch_norm_operand(x, ldx, w, scale, shift, eps, rows, cols, 0, nullptr, 0, out, ldo, nullptr, 0, 0,
                                   nullptr, stream);
    if (vec)
        hipLaunchKernelGGL(norm_modulate_kernel<true>, dim3(rows), dim3(256), 0, stream, x, ldx, w, scale, shift, eps, out,
                           ldo, cols);
    else
        hipLaunchKernelGGL(norm_modulate_kernel<false>, dim3(rows), dim3(256), 0, stream, x, ldx, w, scale, shift, eps, out,
                           ldo, cols);
    return hipGetLastError();
}

hipError_t launch_norm_operand(const float *x, int64_t ldx, const float *w, const float *scale, const float *shift,
                               float eps, int rows, int cols, int group, float *y_out, int64_t ldy, uint16_t *out,
                               int64_t ldo, int8_t *codes, int64_t ldq, int k_pad, float *scales, hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    auto a16 = [](const void *q) { return q == nullptr || (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const bool q8 = codes != nullptr;
    if (cols % 4 || ldx % 4 || !a16(x) || !a16(w) || !a16(scale) || !a16(shift) || (y_out && (ldy % 4 || !a16(y_out))) ||
        (!q8 && (ldo % 4 || (reinterpret_cast<uintptr_t>(out) & 7))) ||
        (q8 && (ldq % 4 || (reinterpret_cast<uintptr_t>(codes) & 3) || k_pad % 4 || k_pad < cols)) ||
        cols > 8 * 4096)
        return hipErrorInvalidValue;
    const int stages = rot::stages_of(group);
    const float norm = group > 0 ? 1.0f / sqrtf((float)group) : 1.0f;
    const int quads = (cols + 1023) / 1024;
    const int it = quads <= 4 ? 1 : quads <= 8 ? 2 : quads <= 16 ? 4 : 8;
#define SQ8_NO(MD, I)                                                                                               \
    if ((q8 ? OP_Q8 : OP_ROT) == MD && it == I) {                                                                     \
        hipLaunchKernelGGL((norm_operand_kernel<MD, I>), dim3(rows), dim3(256), 0, stream, x, ldx, w, scale, shift, eps, \
                           cols, stages, norm, y_out, ldy, out, ldo, codes, ldq, k_pad, scales);                      \
        return hipGetLastError();                                                                                     \
    }
    SQ8_NO(OP_ROT, 1) SQ8_NO(OP_ROT, 2) SQ8_NO(OP_ROT, 4) SQ8_NO(OP_ROT, 8)
    SQ8_NO(OP_Q8, 1) SQ8_NO(OP_Q8, 2) SQ8_NO(OP_Q8, 4) SQ8_NO(OP_Q8, 8)
#undef SQ8_NO
    return hipErrorInvalidValue;
}

hipError_t launch_rms_rows(uint16_t *t, int64_t ld, int64_t rows, int cols, const float *w, float eps, hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    const dim3 grid((unsigned)((rows + 3) / 4));
    const bool aligned = ((uintptr_t)t & 7) == 0 && ld % 4 == 0;
    if (cols == 128 && ((uintptr_t)t & 15) == 0 && ld % 8 == 0 && ((uintptr_t)w & 15) == 0) {
        const int64_t want = (rows + 15) / 16;
        hipLaunchKernelGGL(rms_rows128_kernel, dim3((unsigned)(want < 65535 ? want : 65535)), dim3(256), 0, stream, t, ld,
                           rows, w, eps);
    } else if (!aligned) hipLaunchKernelGGL(rms_rows_kernel<0>, grid, dim3(256), 0, stream, t, ld, rows, cols, w, eps);
    else if (cols == 128) hipLaunchKernelGGL(rms_rows_kernel<2>, grid, dim3(256), 0, stream, t, ld, rows, cols, w, eps);
    else if (cols == 256) hipLaunchKernelGGL(rms_rows_kernel<4>, grid, dim3(256), 0, stream, t, ld, rows, cols, w, eps);
    else if (cols == 64) hipLaunchKernelGGL(rms_rows_kernel<1>, grid, dim3(256), 0, stream, t, ld, rows, cols, w, eps);
    else hipLaunchKernelGGL(rms_rows_kernel<0>, grid, dim3(256), 0, stream, t, ld, rows, cols, w, eps);
    return hipGetLastError();
}

hipError_t launch_gated_residual(float *x, int64_t ldx, const void *y, bool y_bf16, int64_t ldy, const float *gate,
                                 int64_t rows, int cols, hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    if (y_bf16)
        hipLaunchKernelGGL(gated_residual_kernel<true>, dim3(grid_for_rows(rows)), dim3(256), 0, stream, x, ldx, y, ldy,
                           gate, rows, cols);
    else
        hipLaunchKernelGGL(gated_residual_kernel<false>, dim3(grid_for_rows(rows)), dim3(256), 0, stream, x, ldx, y, ldy,
                           gate, rows, cols);
    return hipGetLastError();
}

}  // namespace sq8
