// sq8_device.h — device-side helpers shared by the gfx950 kernels of the weight-quantized linear:
// vector types, the exact 8-bit → bf16 widening, the bf16 rounding, the epilogue functions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace sq8 {

// Calls f(std::integral_constant<int, I>) for I in [B, E): indices the compiler cannot leave
// dynamic, so arrays indexed by them stay in registers.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum WType { W_INT8 = 0, W_FP8 = 1 };
enum WLayout { W_KN = 0, W_NK = 1, W_PACKED = 2 };
// EPI_RESIDUAL (fp32 output only): C += gate ⊙ (s·acc + b), C the caller's residual stream read and
// written in place (the product rounded, then the sum: the gated residual pass's arithmetic).
enum Epi { EPI_NONE = 0, EPI_GELU = 1, EPI_SILU_GLU = 2, EPI_SITU_GLU = 3, EPI_RESIDUAL = 4 };
enum OutT { OUT_BF16 = 0, OUT_F32 = 1 };

// Two fp32 values that are exactly bf16 values (every int8 and every e4m3 code is) packed into one
// bf16 pair by taking their high halves: truncation is the exact rounding here.
__device__ __forceinline__ uint32_t pack_exact_bf16(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Byte J of `d` as a signed int8, widened to fp32 (one v_cvt_f32_i32 with an SDWA byte select).
template <int J>
__device__ __forceinline__ float i8_byte(uint32_t d) {
    return (float)(int8_t)(uint8_t)(d >> (8 * J));
}

// Bytes (2W, 2W+1) of `d` as e4m3fn (gfx950's fp8 is the OCP "fn" format), widened to fp32.
template <int W>
__device__ __forceinline__ void fp8_pair(uint32_t d, float &lo, float &hi) {
    auto v = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, W != 0);
    lo = v[0];
    hi = v[1];
}

// Four consecutive codes (one dword) → four bf16 in two dwords, in order.
template <int WT>
__device__ __forceinline__ void widen4(uint32_t d, uint32_t &lo, uint32_t &hi) {
    if constexpr (WT == W_INT8) {
        lo = pack_exact_bf16(i8_byte<0>(d), i8_byte<1>(d));
        hi = pack_exact_bf16(i8_byte<2>(d), i8_byte<3>(d));
    } else {
        float a, b, c, e;
        fp8_pair<0>(d, a, b);
        fp8_pair<1>(d, c, e);
        lo = pack_exact_bf16(a, b);
        hi = pack_exact_bf16(c, e);
    }
}

// One code → fp32 exactly (scalar path for ragged edges and the dequantiser).
template <int WT>
__device__ __forceinline__ float widen1(uint8_t code) {
    if constexpr (WT == W_INT8) {
        return (float)(int8_t)code;
    } else {
        float a, b;
        fp8_pair<0>((uint32_t)code, a, b);
        return a;
    }
}

// fp32 → bf16, nearest-even; a NaN stays a quiet NaN with its sign (the reference's rounding).
__device__ __forceinline__ uint32_t round_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Two fp32 → a bf16 pair, nearest-even, by the hardware conversion (v_cvt_pk_bf16_f32). Finite
// values and infinities round exactly as round_bf16; a NaN stays a NaN (its payload is the
// hardware's). Used for the product's outputs; round_bf16 keeps the reference's NaN bits.
__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// tanh from exp: 1 − 2/(e^{2|y|} + 1), the sign restored. |error| ≲ 3e-7 absolute; overflow of
// the exponential gives exactly ±1.
__device__ __forceinline__ float tanh_fast(float y) {
    float e = __expf(2.0f * fabsf(y));
    float t = 1.0f - __fdividef(2.0f, e + 1.0f);
    return copysignf(t, y);
}

// GELU-tanh: ½·x·(1 + tanh(u)) with u = √(2/π)·(x + 0.044715·x³), computed as its identical form
// x·σ(2u) = x / (1 + e^{−2u}) — one exponential and one reciprocal; e^{−2u} overflowing gives
// x/∞ = −0 for large negative x, as the tanh form's ½·x·0. The exponent −2u·log2(e) is
// x·(k + k·0.044715·x²), k = −2·√(2/π)·log2(e), its constant folded into the polynomial (seven
// vector instructions a value).
constexpr float kGeluK = (float)(-2.0 * 0.7978845608028654 * 1.4426950408889634);
constexpr float kGeluK3 = (float)(-2.0 * 0.7978845608028654 * 1.4426950408889634 * 0.044715);
__device__ __forceinline__ float gelu_tanh(float x) {
    const float t = __builtin_fmaf(kGeluK3, x * x, kGeluK);
    const float e = __builtin_amdgcn_exp2f(x * t);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// silu(g)·u = g/(1 + e^{−g})·u; e^{−g} overflowing gives −0·u as the reference's.
__device__ __forceinline__ float silu_glu(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// tanh with a small relative error everywhere: below |y| = 1/4 the odd Taylor polynomial to y⁹
// (the first omitted term, 1382·y¹¹/155925, is under 1e-8 of y there), above it tanh_fast.
__device__ __forceinline__ float tanh_rel(float y) {
    const float y2 = y * y;
    float p = 62.0f / 2835.0f;
    p = p * y2 - 17.0f / 315.0f;
    p = p * y2 + 2.0f / 15.0f;
    p = p * y2 - 1.0f / 3.0f;
    const float small = y + y * y2 * p;
    return fabsf(y) < 0.25f ? small : tanh_fast(y);
}

// SITU: 4·tanh(g/4)·σ(g) · 25·tanh(h/25); both caps need tanh relatively exact near 0.
__device__ __forceinline__ float situ(float h, float g) {
    float gate = 4.0f * tanh_rel(0.25f * g) * __fdividef(1.0f, 1.0f + __expf(-g));
    float value = 25.0f * tanh_rel(h / 25.0f);
    return gate * value;
}

}  // namespace sq8
