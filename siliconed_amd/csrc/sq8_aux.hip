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

// The same rounding of `rows` rows of k values read `ldx` apart, written kp ≥ k apart with columns
// [k, kp) zero (a strided fp32 operand into the bf16 copy the products read, padded to whole K steps).
__global__ void __launch_bounds__(256) round_bf16_rows_kernel(const float *__restrict__ x, int64_t ldx,
                                                              uint16_t *__restrict__ y, int64_t rows, int k, int kp) {
    const int64_t count = rows * kp;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / kp;
        const int c = (int)(i - r * kp);
        y[i] = c < k ? (uint16_t)round_bf16(x[r * ldx + c]) : (uint16_t)0;
    }
}

// bf16 rows copied as they are, k values read `ldx` apart, written kp ≥ k apart with columns [k, kp)
// zero: a bf16 operand whose K is not a whole number of 64-wide steps, padded for the step kernels.
__global__ void __launch_bounds__(256) pad_bf16_rows_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                            uint16_t *__restrict__ y, int64_t rows, int k, int kp) {
    const int64_t count = rows * kp;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / kp;
        const int c = (int)(i - r * kp);
        y[i] = c < k ? x[r * ldx + c] : (uint16_t)0;
    }
}

// Columns [k, kp) of `rows` bf16 rows `ld` apart set to zero (the padding after a pass that wrote
// only the first k).
__global__ void __launch_bounds__(256) zero_tail_kernel(uint16_t *__restrict__ y, int64_t ld, int64_t rows, int k,
                                                        int kp) {
    const int w = kp - k;
    const int64_t count = rows * w;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / w;
        y[r * ld + k + (i - r * w)] = 0;
    }
}

// fp32 → three bf16 parts along K: y[r, c] = hi, y[r, kp + c] = mid, y[r, 2kp + c] = lo (kp ≥ k; columns
// [k, kp) of each part zero, the padding to whole K steps), each part the top 16 bits of what the one
// before leaves (hi = x truncated to bf16, mid = (x − hi) truncated, lo = x − hi − mid): 24 significant
// bits in three parts of 8, every difference exact, no part rounded, so hi + mid + lo = x and every
// product of a part with a code is exact. Every part is a normal bf16 for |x| ≥ 2^−103; an infinity or
// NaN is its hi part alone. One thread per value of row r, column c.
__global__ void __launch_bounds__(256) split3_kernel(const float *__restrict__ x, int64_t ldx, uint16_t *__restrict__ y,
                                                     int64_t rows, int k, int kp) {
    const int64_t count = rows * kp;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / kp;
        const int c = (int)(i - r * kp);
        uint32_t u = 0, m = 0, l = 0;
        if (c < k) {
            const float v = x[r * ldx + c];
            u = __float_as_uint(v);
            if ((u & 0x7f800000u) != 0x7f800000u) {
                const float r1 = v - __uint_as_float(u & 0xffff0000u);  // the low 16 bits of x: exact
                m = __float_as_uint(r1) >> 16;
                l = __float_as_uint(r1 - __uint_as_float(m << 16)) >> 16;  // ≤ 8 bits left: a bf16 value
            }
        }
        uint16_t *row = y + r * 3 * (int64_t)kp;
        row[c] = (uint16_t)(u >> 16);
        row[kp + c] = (uint16_t)m;
        row[2 * kp + c] = (uint16_t)l;
    }
}

int grid_for(int64_t count) {
    const int64_t blocks = (count + 255) / 256;
    return (int)(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}

// One thread per 16-byte chunk of the packed layout: chunk c = ((slab·kt + t)·4 + j)·64 + lane holds
// codes k ∈ [64t + 32h + 16(j&1), +16) of virtual column 32·(j>>1) + (lane & 31) of the slab
// (h = lane >> 5); virtual columns are the weight's own, or for GLU the slab's 32 output columns of
// the first half then the same of the second. Zeros past K and past the columns.
__global__ void __launch_bounds__(256) pack_kernel(const uint8_t *__restrict__ w, int wl, int64_t ldw, int k, int n,
                                                   int glu, int kt, int64_t chunks, uint8_t *__restrict__ out) {
    for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(c & 63), j = (int)((c >> 6) & 3);
        const int64_t st = c >> 8;
        const int t = (int)(st % kt), slab = (int)(st / kt);
        const int b = j >> 1, h = lane >> 5, nl = lane & 31;
        int col;
        bool valid;
        if (glu) {
            const int half = n / 2, oc = slab * 32 + nl;
            valid = oc < half;
            col = oc + b * half;
        } else {
            col = slab * 64 + b * 32 + nl;
            valid = col < n;
        }
        const int k0 = 64 * t + 32 * h + 16 * (j & 1);
        u32x4 v = {0, 0, 0, 0};
        if (valid && wl == W_NK && k0 + 16 <= k && (ldw & 15) == 0 && ((uintptr_t)w & 15) == 0) {
            // [N, K]: the chunk is 16 contiguous codes of row `col`.
            v = *reinterpret_cast<const u32x4 *>(w + (int64_t)col * ldw + k0);
        } else {
            uint32_t d[4] = {0, 0, 0, 0};
            for (int e = 0; e < 16; ++e) {
                const int kk = k0 + e;
                uint32_t x = 0;
                if (valid && kk < k) x = wl == W_KN ? w[(int64_t)kk * ldw + col] : w[(int64_t)col * ldw + kk];
                d[e >> 2] |= x << (8 * (e & 3));
            }
            v = u32x4{d[0], d[1], d[2], d[3]};
        }
        *reinterpret_cast<u32x4 *>(out + c * 16) = v;
    }
}

// [K, N] codes, full tiles: one workgroup per (slab, 4 K steps) — 256 rows of K × the slab's 64
// (virtual) columns. Each thread loads 4 consecutive rows × 16 columns (four 16-byte loads),
// transposes the 4 × 16 bytes in registers into 16 words of 4 consecutive K of one column, and
// writes them to an LDS tile [column][K]; the packed chunks (16 consecutive K of one column) are then
// 16-byte LDS reads. Requires k % 256 == 0, whole slabs (n % 64 == 0, GLU: half % 32 == 0), ldw %
// 16 == 0 and a 16-byte aligned base.
constexpr int PK_KSTEPS = 4;
constexpr int PK_PITCH = 64 * PK_KSTEPS + 16;  // bytes per LDS column row (16-byte aligned, bank spread)

__device__ __forceinline__ uint32_t byte_of(const u32x4 &v, int e) { return (v[e >> 2] >> (8 * (e & 3))) & 0xFF; }

__global__ void __launch_bounds__(256) pack_kn_kernel(const uint8_t *__restrict__ w, int64_t ldw, int n, int glu, int kt,
                                                      uint8_t *__restrict__ out) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[64 * PK_PITCH];
    const int groups = kt / PK_KSTEPS;
    const int slab = blockIdx.x / groups, tq = blockIdx.x - slab * groups;
    const int tid = threadIdx.x;
    const int seg = tid & 3, kq = tid >> 2;  // columns [16·seg, +16) of the slab, rows 4·kq .. 4·kq + 3
    const int vc0 = 16 * seg, b = vc0 >> 5;
    const int col0 = glu ? slab * 32 + (vc0 & 31) + b * (n / 2) : slab * 64 + vc0;
    const uint8_t *src = w + (int64_t)(tq * 64 * PK_KSTEPS + 4 * kq) * ldw + col0;
    u32x4 r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = *reinterpret_cast<const u32x4 *>(src + i * ldw);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const uint32_t word = byte_of(r[0], e) | byte_of(r[1], e) << 8 | byte_of(r[2], e) << 16 | byte_of(r[3], e) << 24;
        *reinterpret_cast<uint32_t *>(tile + (vc0 + e) * PK_PITCH + 4 * kq) = word;
    }
    __syncthreads();
    // 4 K steps × 4 loads × 64 lanes = 1024 chunks, 4 per thread.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        const int lane = c & 63, j = (c >> 6) & 3, ts = c >> 8;
        const int vc = 32 * (j >> 1) + (lane & 31);
        const int kr = 64 * ts + 32 * (lane >> 5) + 16 * (j & 1);
        const u32x4 v = *reinterpret_cast<const u32x4 *>(tile + vc * PK_PITCH + kr);
        const int t = tq * PK_KSTEPS + ts;
        *reinterpret_cast<u32x4 *>(out + (((int64_t)slab * kt + t) * 4 + j) * 1024 + lane * 16) = v;
    }
}

}  // namespace

int64_t packed_bytes(int k, int n, bool glu) {
    const int64_t kt = (k + 63) / 64;
    const int64_t slabs = glu ? ((int64_t)n / 2 + 31) / 32 : ((int64_t)n + 63) / 64;
    return slabs * kt * 4096;
}

bool pack_is_fast(const uint8_t *w, int wl, int64_t ldw, int k, int n, bool glu) {
    const bool whole_slabs = glu ? (n % 2 == 0 && (n / 2) % 32 == 0) : n % 64 == 0;
    return wl == W_KN && k > 0 && k % (64 * PK_KSTEPS) == 0 && n > 0 && whole_slabs && ldw % 16 == 0 &&
           ((uintptr_t)w & 15) == 0;
}

hipError_t launch_pack(const uint8_t *w, int wl, int64_t ldw, int k, int n, bool glu, uint8_t *out, hipStream_t stream) {
    const int kt = (k + 63) / 64;
    const int64_t chunks = packed_bytes(k, n, glu) / 16;
    if (chunks == 0) return hipSuccess;
    if (pack_is_fast(w, wl, ldw, k, n, glu)) {
        const int64_t slabs = glu ? (n / 2) / 32 : n / 64;
        hipLaunchKernelGGL(pack_kn_kernel, dim3((unsigned)(slabs * (kt / PK_KSTEPS))), dim3(256), 0, stream, w, ldw, n,
                           glu ? 1 : 0, kt, out);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(pack_kernel, dim3(grid_for(chunks)), dim3(256), 0, stream, w, wl, ldw, k, n, glu ? 1 : 0, kt,
                       chunks, out);
    return hipGetLastError();
}

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

hipError_t launch_split3(const float *x, int64_t ldx, uint16_t *y, int64_t rows, int k, int kp, hipStream_t stream) {
    const int64_t count = rows * kp;
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(split3_kernel, dim3(grid_for(count)), dim3(256), 0, stream, x, ldx, y, rows, k, kp);
    return hipGetLastError();
}

hipError_t launch_round_bf16(const float *x, uint16_t *y, int64_t count, hipStream_t stream) {
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(round_bf16_kernel, dim3(grid_for(count)), dim3(256), 0, stream, x, y, count);
    return hipGetLastError();
}

hipError_t launch_round_bf16_rows(const float *x, int64_t ldx, uint16_t *y, int64_t rows, int k, int kp,
                                  hipStream_t stream) {
    if (rows == 0 || kp == 0) return hipSuccess;
    if (ldx == k && kp == k) return launch_round_bf16(x, y, rows * k, stream);
    hipLaunchKernelGGL(round_bf16_rows_kernel, dim3(grid_for(rows * kp)), dim3(256), 0, stream, x, ldx, y, rows, k, kp);
    return hipGetLastError();
}

hipError_t launch_pad_bf16_rows(const uint16_t *x, int64_t ldx, uint16_t *y, int64_t rows, int k, int kp,
                                hipStream_t stream) {
    if (rows == 0 || kp == 0) return hipSuccess;
    hipLaunchKernelGGL(pad_bf16_rows_kernel, dim3(grid_for(rows * kp)), dim3(256), 0, stream, x, ldx, y, rows, k, kp);
    return hipGetLastError();
}

hipError_t launch_zero_tail(uint16_t *y, int64_t ld, int64_t rows, int k, int kp, hipStream_t stream) {
    if (rows == 0 || kp <= k) return hipSuccess;
    hipLaunchKernelGGL(zero_tail_kernel, dim3(grid_for(rows * (kp - k))), dim3(256), 0, stream, y, ld, rows, k, kp);
    return hipGetLastError();
}

}  // namespace sq8
