// sq8_convrot.hip — ComfyUI's int8 `convrot` format on the GPU: the weight published rotated,
// W = (q·s)·R with R = H/√G block-diagonal along the input (groups of G = 4, 16, 64 or 256, H the
// Kronecker power of the regular Hadamard H4 = [[1,1,1,−1],[1,1,−1,1],[1,−1,1,1],[−1,1,1,1]]).
//
// Two routes, as the reference has them:
//  * the activation's rotation, x·R, before the plain 8-bit product (R is symmetric, so
//    x·Wᵀ = (x·R)·(q·s)ᵀ): `rotate_groups_kernel`, the butterflies of rotate_groups
//    (Sources/Siliconed/TensorGEMM.swift:181-201) in fp32, written as the product's bf16 operand
//    (the rounding of submitRounded, TensorGEMMBF16.swift:208-264) or in fp32;
//  * the weight widened with its rotation, Float(H·q)·(s/√G) (Widen.swift:316-428):
//    `dequantize_rotated_kernel`, the butterflies on the integers (exact), one multiply at the end.
//
// Both are one pass over HBM. A 256-value chunk (a group of 256, or 256/G whole groups of a
// smaller G) is four base-4 digits d0..d3 of the position p = d0 + 4·d1 + 16·d2 + 64·d3; the butterfly
// stage of span 4^s runs over digit s. A thread holds 16 values whose positions differ in two
// digits, so the stages on those run in its registers; a transposition through LDS brings the
// other two digits into the registers, one more takes them back.
#include <hip/hip_runtime.h>

#include "sq8_device.h"
#include "sq8_gemm.h"
#include "sq8_rotate.h"

namespace sq8 {
namespace {

using rot::butterfly;
using rot::load4;
using rot::PITCH;

template <bool Y_BF16, bool VEC>
__device__ __forceinline__ void store4(void *y, int64_t at, const float *v) {
    if constexpr (Y_BF16) {
        uint16_t *p = static_cast<uint16_t *>(y) + at;
        if constexpr (VEC) {
            *reinterpret_cast<u32x2 *>(p) = u32x2{round_bf16(v[0]) | round_bf16(v[1]) << 16,
                                                  round_bf16(v[2]) | round_bf16(v[3]) << 16};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) p[e] = (uint16_t)round_bf16(v[e]);
        }
    } else {
        float *p = static_cast<float *>(y) + at;
        if constexpr (VEC) {
            *reinterpret_cast<f32x4 *>(p) = f32x4{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) p[e] = v[e];
        }
    }
}

// y = x·R per row, `stages` = log4(G). Each wave takes four 256-value chunks of the rows (chunk c of
// row r: values [256c, 256c + 256), the last one of a row partial when k % 256 ≠ 0 — whole groups,
// since k % G == 0; its missing values read as 0 and are never stored), one per group of 16 lanes,
// held and rotated as rot::rotate_chunk describes. (An arrangement that keeps digits 0 and 1 in
// registers needs 64-byte-strided accesses per lane and ran at 4.4 TB/s against this one's 5.9 on
// the C1 operand.)
template <bool X_BF16, bool Y_BF16, bool VEC>
__global__ void __launch_bounds__(256) rotate_groups_kernel(const void *x, int64_t ldx, void *y,
                                                            int64_t ldy, int64_t rows, int k, int stages, float norm,
                                                            int64_t quads) {
    __shared__ __attribute__((aligned(16))) float lds[4][4 * PITCH];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cc = lane >> 4, l16 = lane & 15;
    float *mine = lds[wave] + cc * PITCH;
    const int64_t cpr = (k + 255) / 256;  // chunks per row
    for (int64_t qd = (int64_t)blockIdx.x * 4 + wave; qd < quads; qd += (int64_t)gridDim.x * 4) {
        const int64_t chunk = qd * 4 + cc;
        const int64_t row = chunk / cpr;
        const int base = (int)(chunk - row * cpr) * 256;
        const bool live = row < rows;
        float v[16];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int col = base + 4 * l16 + 64 * u;
            if (live && col < k) load4<X_BF16, VEC>(x, row * ldx + col, v + 4 * u);
            else v[4 * u] = v[4 * u + 1] = v[4 * u + 2] = v[4 * u + 3] = 0.0f;
        }
        rot::rotate_chunk(v, mine, l16, stages);
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = v[i] * norm;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int col = base + 4 * l16 + 64 * u;
            if (live && col < k) store4<Y_BF16, VEC>(y, row * ldy + col, v + 4 * u);
        }
    }
}

// Scale types, numbered as the C ABI's sq8_dtype: bf16 1, fp32 2, fp16 5 (widened exactly).
__device__ __forceinline__ float scale_at(const void *scale, int dtype, int64_t i) {
    if (dtype == 1) return __uint_as_float((uint32_t) static_cast<const uint16_t *>(scale)[i] << 16);
    if (dtype == 5) return (float)static_cast<const _Float16 *>(scale)[i];
    return static_cast<const float *>(scale)[i];
}

// out [k, n] = Float(H·q)·(s_c/√G) of codes q [k, n] rotated along k. A workgroup takes 256 rows
// (256/G whole groups; rows past k read as 0, never stored) × 64 columns. Thread t: columns
// 4·(t & 15) .. +3 of the tile; in the loaded arrangement rows 16·(t >> 4) + i (i = d0 + 4·d1 in
// registers); after the transposition through LDS (int32 [256][64]) rows (t >> 4) + 16·i
// (i = d2 + 4·d3). |partial sums| ≤ 32 648 (Widen.swift:326-329): int32 is exact.
template <bool VEC>
__global__ void __launch_bounds__(256) dequantize_rotated_kernel(const int8_t *__restrict__ q, int64_t ldq, int k, int n,
                                                                 int stages, const void *__restrict__ scale, int scale_dtype,
                                                                 int per_column, float norm, float *__restrict__ out,
                                                                 int64_t ldo, int tiles_n) {
    __shared__ __attribute__((aligned(16))) int lds[256 * 64];
    const int tk = blockIdx.x / tiles_n, tn = blockIdx.x - tk * tiles_n;
    const int row0 = tk * 256, cq = threadIdx.x & 15, rb = threadIdx.x >> 4;
    const int c0 = tn * 64 + 4 * cq;
    int v[16][4];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int row = row0 + 16 * rb + i;
        const int8_t *src = q + (int64_t)row * ldq + c0;
        if constexpr (VEC) {
            const uint32_t d = row < k && c0 < n ? *reinterpret_cast<const uint32_t *>(src) : 0u;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[i][e] = (int)(int8_t)(d >> (8 * e));
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[i][e] = row < k && c0 + e < n ? (int)src[e] : 0;
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int d1 = 0; d1 < 4; ++d1) butterfly(v[4 * d1][e], v[4 * d1 + 1][e], v[4 * d1 + 2][e], v[4 * d1 + 3][e]);
        if (stages > 1) {
#pragma unroll
            for (int d0 = 0; d0 < 4; ++d0) butterfly(v[d0][e], v[d0 + 4][e], v[d0 + 8][e], v[d0 + 12][e]);
        }
    }
    int first = row0 + 16 * rb, step = 1;  // row of v[i] = first + step·i
    if (stages > 2) {
        // The block-uniform branch: every thread of the workgroup reaches both barriers.
#pragma unroll
        for (int i = 0; i < 16; ++i)
            *reinterpret_cast<int4 *>(lds + (16 * rb + i) * 64 + 4 * cq) = int4{v[i][0], v[i][1], v[i][2], v[i][3]};
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int4 t = *reinterpret_cast<const int4 *>(lds + (rb + 16 * i) * 64 + 4 * cq);
            v[i][0] = t.x; v[i][1] = t.y; v[i][2] = t.z; v[i][3] = t.w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int d3 = 0; d3 < 4; ++d3) butterfly(v[4 * d3][e], v[4 * d3 + 1][e], v[4 * d3 + 2][e], v[4 * d3 + 3][e]);
            if (stages > 3) {
#pragma unroll
                for (int d2 = 0; d2 < 4; ++d2) butterfly(v[d2][e], v[d2 + 4][e], v[d2 + 8][e], v[d2 + 12][e]);
            }
        }
        first = row0 + rb;
        step = 16;
    }
    float f[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = c0 + e < n ? scale_at(scale, scale_dtype, per_column ? c0 + e : 0) * norm : 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int row = first + step * i;
        if (row >= k) continue;
        float *dst = out + (int64_t)row * ldo + c0;
        if constexpr (VEC) {
            if (c0 < n) *reinterpret_cast<f32x4 *>(dst) = f32x4{(float)v[i][0] * f[0], (float)v[i][1] * f[1],
                                                                (float)v[i][2] * f[2], (float)v[i][3] * f[3]};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (c0 + e < n) dst[e] = (float)v[i][e] * f[e];
        }
    }
}

}  // namespace

bool is_rotation_group(int group) { return group == 4 || group == 16 || group == 64 || group == 256; }

hipError_t launch_rotate_groups(const void *x, bool x_bf16, int64_t ldx, void *y, bool y_bf16, int64_t ldy, int64_t rows,
                                int k, int group, hipStream_t stream) {
    if (rows == 0 || k == 0) return hipSuccess;
    const int64_t chunks = rows * ((k + 255) / 256);
    const int64_t quads = (chunks + 3) / 4;
    const int64_t want = (quads + 3) / 4;
    const dim3 grid((unsigned)(want < 16384 ? want : 16384));
    const int stages = rot::stages_of(group);
    const float norm = 1.0f / sqrtf((float)group);
    const size_t xa = x_bf16 ? 8 : 16, ya = y_bf16 ? 8 : 16;
    const bool vec = (reinterpret_cast<uintptr_t>(x) % xa) == 0 && (reinterpret_cast<uintptr_t>(y) % ya) == 0 &&
                     ldx % 4 == 0 && ldy % 4 == 0;
#define SQ8_ROT(XB, YB, V)                                                                                           \
    if (x_bf16 == XB && y_bf16 == YB && vec == V) {                                                                  \
        hipLaunchKernelGGL((rotate_groups_kernel<XB, YB, V>), grid, dim3(256), 0, stream, x, ldx, y, ldy, rows, k,   \
                           stages, norm, quads);                                                                     \
        return hipGetLastError();                                                                                    \
    }
    SQ8_ROT(false, true, true)
    SQ8_ROT(false, true, false)
    SQ8_ROT(true, true, true)
    SQ8_ROT(true, true, false)
    SQ8_ROT(false, false, true)
    SQ8_ROT(false, false, false)
    SQ8_ROT(true, false, true)
    SQ8_ROT(true, false, false)
#undef SQ8_ROT
    return hipErrorInvalidValue;
}

hipError_t launch_dequantize_rotated(const int8_t *q, int64_t ldq, int k, int n, int group, const void *scale,
                                     int scale_dtype, bool per_column, float *out, int64_t ldo, hipStream_t stream) {
    if (k == 0 || n == 0) return hipSuccess;
    const int tiles_n = (n + 63) / 64, tiles_k = (k + 255) / 256;
    const dim3 grid((unsigned)((int64_t)tiles_n * tiles_k));
    const int stages = rot::stages_of(group);
    const float norm = 1.0f / sqrtf((float)group);
    const bool vec = n % 4 == 0 && ldq % 4 == 0 && ldo % 4 == 0 && (reinterpret_cast<uintptr_t>(q) % 4) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) % 16) == 0;
    if (vec)
        hipLaunchKernelGGL(dequantize_rotated_kernel<true>, grid, dim3(256), 0, stream, q, ldq, k, n, stages, scale,
                           scale_dtype, per_column ? 1 : 0, norm, out, ldo, tiles_n);
    else
        hipLaunchKernelGGL(dequantize_rotated_kernel<false>, grid, dim3(256), 0, stream, q, ldq, k, n, stages, scale,
                           scale_dtype, per_column ? 1 : 0, norm, out, ldo, tiles_n);
    return hipGetLastError();
}

}  // namespace sq8
