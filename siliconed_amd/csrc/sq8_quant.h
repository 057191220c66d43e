// sq8_quant.h — W8A8's per-row quantization of a row held in registers (ComfyUI's int8_linear,
// Sources/Siliconed/TensorGEMMInt8.swift:78-104, `quantize_held`), shared by the quantization pass
// (sq8_w8a8.hip) and the norms that write the quantized operand themselves (sq8_block.hip), so both
// give the same codes and scale for the same fp32 row. The row's values sit in rot::rotate_chunk's
// arrangement: a lane holds 16 values of one 256-value chunk, at positions 4·l16 + 64·u + e.
#pragma once

#include <hip/hip_runtime.h>

#include "sq8_device.h"

namespace sq8 {
namespace quant {

// v ← v · norm (the rotation's 1/√G; 1 without one, exact), and the running max|v|.
__device__ __forceinline__ float scaled_max(float (&v)[16], float norm, float m) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        v[i] = v[i] * norm;
        m = fmaxf(m, fabsf(v[i]));
    }
    return m;
}

// s = max(m / 127, 1e-30), the division correctly rounded (`precise::divide`).
__device__ __forceinline__ float row_scale(float m) {
    const float q = __fdiv_rn(m, 127.0f);
    return q > 1e-30f ? q : 1e-30f;
}

// The codes clamp(rint(v / s), −128, 127) of a lane's 16 values into the row `dst` (0 in [k, k_pad)),
// v / s correctly rounded. From the reciprocal's product where that gives the same integer:
// q' = fl(v · fl(1/s)) is within (2^-23 + 2^-48)·|v/s| ≤ 2^-16 of v/s (|v/s| ≤ 127.5 for every value of
// a row scaled by its own maximum), fl(v/s) within 2^-18 of it, so both round to the same integer
// unless q' lies within 2^-16 + 2^-18 of a half-integer, i.e. |q' − rint(q')| > 0.5 − 2^-14 covers
// every case that could differ. A lane with such a value (probability ~2^-13 a value) redoes its 16
// with the IEEE division; one branch per chunk.
template <bool VEC>
__device__ __forceinline__ void store_codes(int8_t *dst, int k, int k_pad, int chunk, int cpr, int l16, const float (&v)[16],
                                            float scale) {
    const float recip = __fdiv_rn(1.0f, scale);
    float c[16];
    bool hard = false;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float q = v[i] * recip;
        c[i] = rintf(q);
        hard |= fabsf(q - c[i]) > 0.5f - 0x1p-14f;
    }
    if (hard) {
#pragma unroll
        for (int i = 0; i < 16; ++i) c[i] = rintf(__fdiv_rn(v[i], scale));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int col = chunk * 256 + 4 * l16 + 64 * u;
        if (chunk >= cpr || col >= k_pad) continue;
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float cl = fminf(fmaxf(c[4 * u + e], -128.0f), 127.0f);
            const uint32_t b = col + e < k ? (uint32_t)(uint8_t)(int8_t)(int)cl : 0u;
            word |= b << (8 * e);
        }
        if constexpr (VEC) {
            *reinterpret_cast<uint32_t *>(dst + col) = word;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col + e < k_pad) dst[col + e] = (int8_t)(word >> (8 * e));
        }
    }
}

}  // namespace quant
}  // namespace sq8
