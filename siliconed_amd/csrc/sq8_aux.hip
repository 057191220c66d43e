// sq8_aux.hip — the device dequantiser and the bf16 rounding pass.
//
// dequantize: out[i] = Float(code[i]) · s, one fp32 multiply, never fused
// (Sources/Siliconed/Widen.swift:81-97, :129-271). The code goes through the same widening the
// GEMM uses (sq8_device.h), so the bit-exact test of this kernel is the test of that conversion.
// round_bf16: fp32 → bf16 nearest-even, a NaN kept quiet (TensorGEMMBF16.swift:41-48, 67-73).
#include <hip/hip_fp16.h>

#include "sq8_gemm.h"

namespace sq8 {

namespace {

// Scale kinds, numbered as the C ABI's sq8_dtype.
constexpr int S_BF16 = 1, S_F32 = 2, S_F16 = 5;
constexpr int L_TENSOR = 0, L_COLUMNS = 1, L_BLOCKS = 2, L_ROWS = 3;

__device__ __forceinline__ float scale_at(const void *s, int kind, int64_t i) {
    if (kind == S_BF16) return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(s)[i] << 16);
    if (kind == S_F16) return __half2float(reinterpret_cast<const __half *>(s)[i]);
    return reinterpret_cast<const float *>(s)[i];
}

template <int WT>
__global__ void __launch_bounds__(256) dequantize_kernel(const uint8_t *__restrict__ codes, int64_t rows,
                                                         int64_t columns, const void *__restrict__ scale,
                                                         int scale_kind, int layout, int64_t block_rows,
                                                         int64_t first_row, float *__restrict__ out) {
    const int64_t count = rows * columns;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        const float v = widen1<WT>(codes[i]);
        if (!scale) {
            out[i] = v;
            continue;
        }
        const int64_t r = i / columns, c = i - r * columns;
        float s;
        switch (layout) {
        case L_TENSOR: s = scale_at(scale, scale_kind, 0); break;
        case L_COLUMNS: s = scale_at(scale, scale_kind, c); break;
        case L_BLOCKS: s = scale_at(scale, scale_kind, ((first_row + r) / block_rows) * columns + c); break;
        default: s = scale_at(scale, scale_kind, first_row + r); break;
        }
        out[i] = __fmul_rn(v, s);
    }
}

__global__ void __launch_bounds__(256) round_bf16_kernel(const float *__restrict__ x, uint16_t *__restrict__ y,
                                                         int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = (uint16_t)round_bf16(x[i]);
}

int grid_for(int64_t count) {
    const int64_t blocks = (count + 255) / 256;
    return (int)(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}

}  // namespace

hipError_t launch_dequantize(const uint8_t *codes, int wt, int64_t rows, int64_t columns, const void *scale,
                             int scale_dtype, int scale_layout, int64_t block_rows, int64_t first_row, float *out,
                             hipStream_t stream) {
    const int64_t count = rows * columns;
    if (count == 0) return hipSuccess;
    if (wt == W_INT8)
        hipLaunchKernelGGL(dequantize_kernel<W_INT8>, dim3(grid_for(count)), dim3(256), 0, stream, codes, rows, columns,
                           scale, scale_dtype, scale_layout, block_rows, first_row, out);
    else
        hipLaunchKernelGGL(dequantize_kernel<W_FP8>, dim3(grid_for(count)), dim3(256), 0, stream, codes, rows, columns,
                           scale, scale_dtype, scale_layout, block_rows, first_row, out);
    return hipGetLastError();
}

hipError_t launch_round_bf16(const float *x, uint16_t *y, int64_t count, hipStream_t stream) {
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(round_bf16_kernel, dim3(grid_for(count)), dim3(256), 0, stream, x, y, count);
    return hipGetLastError();
}

}  // namespace sq8
