// sq8_rotate.h — the convrot rotation of one 256-value chunk held by 16 lanes, shared by the
// rotation pass (sq8_convrot.hip) and the W8A8 activation quantization (sq8_w8a8.hip), so both
// compute the same bits.
//
// The rotation x·R, R = H/√G block-diagonal by groups of G = 4, 16, 64 or 256, H the Kronecker
// power of the regular Hadamard H4 = [[1,1,1,−1],[1,1,−1,1],[1,−1,1,1],[−1,1,1,1]]: the radix-4
// butterflies of rotate_groups (Sources/Siliconed/TensorGEMM.swift:181-201) in fp32, stage after
// stage (spans 1, 4, 16, 64 — the order matters, every sum is rounded), then × 1/√G (a power of two).
//
// A chunk's position p = d0 + 4·d1 + 16·d2 + 64·d3 (base-4 digits); the stage of span 4^s runs
// over digit s. The 16 lanes l16 = 0..15 of a lane group hold the chunk as loaded: lane l16, register
// r = e + 4u ↔ position 4·l16 + 64·u + e (r = d0 + 4·d3, l16 = d1 + 4·d2), so each load and store
// instruction covers 256 contiguous bytes of fp32 per chunk. Digit 0 is butterflied in registers; the
// chunk goes through LDS to the arrangement l16 = d0 + 4·d3, r = d1 + 4·d2 for digits 1 and 2, and
// back for digit 3. The LDS copy of position p sits at p + 4·(p >> 6), so both the 16-byte writes and
// the 4-byte reads of the transposition meet 64 different banks (four lane groups' chunks PITCH
// floats apart).
#pragma once

#include <hip/hip_runtime.h>

#include "sq8_device.h"

namespace sq8 {
namespace rot {

constexpr int PITCH = 272;  // floats per chunk in LDS: 256 + 4 per 64, so four chunks start 16 banks apart

// The 4-point butterfly of rotate_groups: p = a + b, m = a − b, u = c + d, w = c − d, then
// (p + w, p − w, m + u, u − m) — each sum rounded to fp32 on its own (the library is built without
// contraction).
__device__ __forceinline__ void butterfly(float &a, float &b, float &c, float &d) {
    const float p = a + b, m = a - b, u = c + d, w = c - d;
    a = p + w;
    b = p - w;
    c = m + u;
    d = u - m;
}

// The same on integers (exact).
__device__ __forceinline__ void butterfly(int &a, int &b, int &c, int &d) {
    const int p = a + b, m = a - b, u = c + d, w = c - d;
    a = p + w;
    b = p - w;
    c = m + u;
    d = u - m;
}

// Orders one wave's LDS writes before its later reads of other lanes' values. The LDS runs a
// wave's operations in issue order; these fences only keep the compiler from reordering them.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Four consecutive values of a row, widened to fp32. VEC: one 16-byte (fp32) or 8-byte (bf16) load.
template <bool X_BF16, bool VEC>
__device__ __forceinline__ void load4(const void *x, int64_t at, float *v) {
    if constexpr (X_BF16) {
        const uint16_t *p = static_cast<const uint16_t *>(x) + at;
        if constexpr (VEC) {
            const u32x2 d = *reinterpret_cast<const u32x2 *>(p);
            v[0] = __uint_as_float(d[0] << 16);
            v[1] = __uint_as_float(d[0] & 0xFFFF0000u);
            v[2] = __uint_as_float(d[1] << 16);
            v[3] = __uint_as_float(d[1] & 0xFFFF0000u);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __uint_as_float((uint32_t)p[e] << 16);
        }
    } else {
        const float *p = static_cast<const float *>(x) + at;
        if constexpr (VEC) {
            const f32x4 d = *reinterpret_cast<const f32x4 *>(p);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = d[e];
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = p[e];
        }
    }
}

// The rotation's `stages` (log4 G, 0 to 4) on the 16 values v a lane holds of its chunk, through
// the lane group's LDS chunk `mine` (PITCH floats, private to the 16 lanes). Wave-uniform `stages`.
// The scale 1/√G is the caller's.
__device__ __forceinline__ void rotate_chunk(float (&v)[16], float *mine, int l16, int stages) {
    if (stages < 1) return;
    // Span 1 (digit 0).
#pragma unroll
    for (int u = 0; u < 4; ++u) butterfly(v[4 * u], v[4 * u + 1], v[4 * u + 2], v[4 * u + 3]);
    if (stages < 2) return;
#pragma unroll
    for (int u = 0; u < 4; ++u)
        *reinterpret_cast<f32x4 *>(mine + 4 * l16 + 68 * u) = f32x4{v[4 * u], v[4 * u + 1], v[4 * u + 2], v[4 * u + 3]};
    wave_lds_sync();
    // Now l16 = d0 + 4·d3 and register r = d1 + 4·d2: position d0 + 4·r + 64·d3.
    const int d0 = l16 & 3, d3 = l16 >> 2;
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = mine[d0 + 4 * r + 68 * d3];
    // Span 4 (digit 1), then span 16 (digit 2).
#pragma unroll
    for (int d2 = 0; d2 < 4; ++d2) butterfly(v[4 * d2], v[4 * d2 + 1], v[4 * d2 + 2], v[4 * d2 + 3]);
    if (stages > 2) {
#pragma unroll
        for (int d1 = 0; d1 < 4; ++d1) butterfly(v[d1], v[d1 + 4], v[d1 + 8], v[d1 + 12]);
    }
    wave_lds_sync();
#pragma unroll
    for (int r = 0; r < 16; ++r) mine[d0 + 4 * r + 68 * d3] = v[r];
    wave_lds_sync();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const f32x4 t = *reinterpret_cast<const f32x4 *>(mine + 4 * l16 + 68 * u);
        v[4 * u] = t[0];
        v[4 * u + 1] = t[1];
        v[4 * u + 2] = t[2];
        v[4 * u + 3] = t[3];
    }
    wave_lds_sync();
    // Span 64 (digit 3).
    if (stages > 3) {
#pragma unroll
        for (int e = 0; e < 4; ++e) butterfly(v[e], v[e + 4], v[e + 8], v[e + 12]);
    }
}

// log4 of a rotation group (0 for none).
inline int stages_of(int group) {
    int s = 0;
    for (int g = 1; g < group; g *= 4) ++s;
    return s;
}

}  // namespace rot
}  // namespace sq8
