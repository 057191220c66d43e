// sq8_w8a8.hip — W8A8's activation quantization (ComfyUI's int8_linear, the reference's
// QuantizedKernels: Sources/Siliconed/TensorGEMMInt8.swift:4-37, `quantize_rows` :109-131 and
// `quantize_held` :78-104): per row, the convrot rotation (optional), then
// s = max(max|y| / 127, 1e-30) and q = clamp(rint(y / s), −128, 127), both divisions correctly
// rounded, rint half to even. The product on the codes is gemm_i8_kernel (sq8_i8_kernel.h).
//
// One workgroup of four waves per row, the whole row in registers (the scale needs the row's
// maximum before any code is written): one read of the row, one write of its codes. The row's
// chunks of 256 are held and rotated as rot::rotate_chunk describes (the rotation pass's own code,
// so a rotated operand is bit for bit the one sq8_rotate_groups writes); wave w takes the quads
// (4 chunks) w, w + 4, …, IT of them at most. The codes go to rows of k_pad bytes (a multiple of
// 128, the product's K step), zero past k. (A wave per row, four rows a workgroup, measured 18.2 µs
// against this layout's 14.8 on C1's operand: every wave then loads, then computes, in one round.)
#include <hip/hip_runtime.h>

#include "sq8_device.h"
#include "sq8_gemm.h"
#include "sq8_quant.h"
#include "sq8_rotate.h"

namespace sq8 {
namespace {

using quant::row_scale;
using quant::scaled_max;
using quant::store_codes;

// The 16 values a lane holds of chunk `chunk` of a row starting at element `at` (positions
// 4·l16 + 64·u + e of the chunk, rot::rotate_chunk's arrangement); 0 past k and past the last chunk.
template <bool X_BF16, bool VEC>
__device__ __forceinline__ void load_chunk(const void *x, int64_t at, int k, int chunk, int cpr, int l16, float (&v)[16]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int col = chunk * 256 + 4 * l16 + 64 * u;
        if constexpr (VEC) {
            if (chunk < cpr && col < k) rot::load4<X_BF16, true>(x, at + col, &v[4 * u]);
            else v[4 * u] = v[4 * u + 1] = v[4 * u + 2] = v[4 * u + 3] = 0.0f;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float t = 0.0f;
                if (chunk < cpr && col + e < k) {
                    if constexpr (X_BF16) t = __uint_as_float((uint32_t) static_cast<const uint16_t *>(x)[at + col + e] << 16);
                    else t = static_cast<const float *>(x)[at + col + e];
                }
                v[4 * u + e] = t;
            }
        }
    }
}

template <bool X_BF16, bool VEC, int IT>
__global__ void __launch_bounds__(256) quantize_rows_kernel(const void *__restrict__ x, int64_t ldx, int k, int stages,
                                                            float norm, int8_t *__restrict__ codes, int64_t ldq, int k_pad,
                                                            float *__restrict__ scales) {
    __shared__ __attribute__((aligned(16))) float lds[4][4 * rot::PITCH];
    __shared__ float part[4];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cc = lane >> 4, l16 = lane & 15;
    float *mine = lds[wave] + cc * rot::PITCH;
    const int64_t row = blockIdx.x;
    const int cpr = (k + 255) / 256;
    float v[IT][16];
    // Every load of the row first (the rotations' LDS fences would otherwise hold the later ones back).
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int quad = it * 4 + wave;
        if (4 * quad >= cpr) break;  // wave-uniform
        load_chunk<X_BF16, VEC>(x, row * ldx, k, 4 * quad + cc, cpr, l16, v[it]);
    }
    float m = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        if (4 * (it * 4 + wave) >= cpr) break;
        rot::rotate_chunk(v[it], mine, l16, stages);
        m = scaled_max(v[it], norm, m);
    }
    // The row's maximum (exact in any order), then its scale.
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (lane == 0) part[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    const float scale = row_scale(m);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int quad = it * 4 + wave;
        if (4 * quad >= cpr) break;
        store_codes<VEC>(codes + row * ldq, k, k_pad, 4 * quad + cc, cpr, l16, v[it], scale);
    }
    if (threadIdx.x == 0) scales[row] = scale;
}

// Codes [rows, k] (leading dimension lds) copied to rows of k_pad bytes, zero past k: the
// product's K steps of 128 read whole rows.
__global__ void __launch_bounds__(256) pad_codes_kernel(const int8_t *__restrict__ src, int64_t ld_src,
                                                        int8_t *__restrict__ dst, int64_t ld_dst, int64_t rows, int k,
                                                        int k_pad) {
    const int64_t per_row = k_pad / 4;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < rows * per_row; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / per_row;
        const int c = (int)(i - r * per_row) * 4;
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (c + e < k) word |= (uint32_t)(uint8_t)src[r * ld_src + c + e] << (8 * e);
        *reinterpret_cast<uint32_t *>(dst + r * ld_dst + c) = word;
    }
}

}  // namespace

int quantize_row_limit() { return 8 * 4096; }

hipError_t launch_quantize_rows(const void *x, bool x_bf16, int64_t ldx, int rows, int k, int group, int8_t *codes,
                                int64_t ldq, int k_pad, float *scales, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    if (k > quantize_row_limit() || k_pad < k) return hipErrorInvalidValue;
    const int stages = rot::stages_of(group);
    const float norm = group > 0 ? 1.0f / sqrtf((float)group) : 1.0f;
    const size_t xa = x_bf16 ? 8 : 16;
    const bool vec = k % 4 == 0 && k_pad % 4 == 0 && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(x) % xa) == 0 &&
                     ldq % 4 == 0 && (reinterpret_cast<uintptr_t>(codes) % 4) == 0;
    const int quads = (k + 1023) / 1024;
    const int it = quads <= 4 ? 1 : quads <= 8 ? 2 : quads <= 16 ? 4 : 8;
#define SQ8_Q(XB, V, I)                                                                                          \
    if (x_bf16 == XB && vec == V && it == I) {                                                                   \
        hipLaunchKernelGGL((quantize_rows_kernel<XB, V, I>), dim3(rows), dim3(256), 0, stream, x, ldx, k, stages, \
                           norm, codes, ldq, k_pad, scales);                                                     \
        return hipGetLastError();                                                                                \
    }
#define SQ8_QI(XB, V) SQ8_Q(XB, V, 1) SQ8_Q(XB, V, 2) SQ8_Q(XB, V, 4) SQ8_Q(XB, V, 8)
    SQ8_QI(false, true)
    SQ8_QI(false, false)
    SQ8_QI(true, true)
    SQ8_QI(true, false)
#undef SQ8_QI
#undef SQ8_Q
    return hipErrorInvalidValue;
}

hipError_t launch_pad_codes(const int8_t *src, int64_t ld_src, int8_t *dst, int64_t ld_dst, int64_t rows, int k, int k_pad,
                            hipStream_t stream) {
    if (rows == 0 || k_pad == 0) return hipSuccess;
    const int64_t work = rows * (k_pad / 4);
    const int64_t want = (work + 255) / 256;
    hipLaunchKernelGGL(pad_codes_kernel, dim3((unsigned)(want < 16384 ? want : 16384)), dim3(256), 0, stream, src, ld_src,
                       dst, ld_dst, rows, k, k_pad);
    return hipGetLastError();
}

}  // namespace sq8
