// sq8_block.hip — the elementwise passes a DiT block runs between its weight-quantized products,
// each one pass over HBM: the modulated RMSNorm that writes the next product's bf16 operand, the
// per-head RMSNorm of q and k, and the gated residual update.
//
// Rounding as the reference's kernels: every product and sum rounded on its own (no contraction),
// the row's 1/sqrt(mean + eps) from an IEEE divide and square root.
#include <hip/hip_runtime.h>

#include "sq8_device.h"
#include "sq8_gemm.h"

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
    if (vec)
        hipLaunchKernelGGL(norm_modulate_kernel<true>, dim3(rows), dim3(256), 0, stream, x, ldx, w, scale, shift, eps, out,
                           ldo, cols);
    else
        hipLaunchKernelGGL(norm_modulate_kernel<false>, dim3(rows), dim3(256), 0, stream, x, ldx, w, scale, shift, eps, out,
                           ldo, cols);
    return hipGetLastError();
}

hipError_t launch_rms_rows(uint16_t *t, int64_t ld, int64_t rows, int cols, const float *w, float eps, hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    const dim3 grid((unsigned)((rows + 3) / 4));
    const bool aligned = ((uintptr_t)t & 7) == 0 && ld % 4 == 0;
    if (!aligned) hipLaunchKernelGGL(rms_rows_kernel<0>, grid, dim3(256), 0, stream, t, ld, rows, cols, w, eps);
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
