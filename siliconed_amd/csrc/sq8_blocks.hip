// sq8_blocks.hip — codes with a scale per block of rows and column (GGUF Q8_0): the packing into the
// packed Q8 layout (codes in the block-aligned K order, then the scales per step and column, widened
// to fp32) and the product's instantiations (sq8_blocks_kernel.h).
#include <hip/hip_fp16.h>

#include "sq8_blocks_kernel.h"

namespace sq8 {

namespace {

constexpr int S_BF16 = 1, S_F32 = 2, S_F16 = 5;  // numbered as the C ABI's sq8_dtype

__device__ __forceinline__ float scale_value(const void *s, int kind, int64_t i) {
    if (kind == S_BF16) return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(s)[i] << 16);
    if (kind == S_F16) return __half2float(reinterpret_cast<const __half *>(s)[i]);
    return reinterpret_cast<const float *>(s)[i];
}

// Virtual column `vc` (0..63) of slab `slab` → the weight's column, or −1 past the columns.
__device__ __forceinline__ int weight_column(int slab, int vc, int n, int glu) {
    if (glu) {
        const int half = n / 2, oc = slab * 32 + (vc & 31);
        return oc < half ? oc + (vc >> 5) * half : -1;
    }
    const int col = slab * 64 + vc;
    return col < n ? col : -1;
}

// One thread per 16-byte chunk: the code chunks first (chunks of the packed layout, block-aligned K
// order), then the scale chunks ((slab·kt + t)·32 + nl). Codes [K, N] (wl W_KN) or [N, K] (W_NK);
// scales [K/B, ·] with the codes' row stride ldw for W_KN (n ≤ ldw: the first n columns of a wider
// weight), [N, K/B] for W_NK (each layout's own orientation: the map's blocks, GGUF's rows of blocks).
__global__ void __launch_bounds__(256) pack_blocks_kernel(const uint8_t *__restrict__ w, int wl, int64_t ldw,
                                                          const void *__restrict__ scale, int scale_kind, int block,
                                                          int k, int n, int glu, int kt, int64_t code_chunks,
                                                          int64_t chunks, uint8_t *__restrict__ out) {
    const int kb_count = k / block;
    for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += (int64_t)gridDim.x * blockDim.x) {
        if (c < code_chunks) {
            const int lane = (int)(c & 63), j = (int)((c >> 6) & 3);
            const int64_t st = c >> 8;
            const int t = (int)(st % kt), slab = (int)(st / kt);
            const int h = lane >> 5, col = weight_column(slab, 32 * (j >> 1) + (lane & 31), n, glu);
            uint32_t d[4] = {0, 0, 0, 0};
            for (int e = 0; e < 16; ++e) {
                const int kk = 64 * t + 32 * (j & 1) + 16 * (e >> 3) + 8 * h + (e & 7);
                uint32_t x = 0;
                if (col >= 0 && kk < k) x = wl == W_KN ? w[(int64_t)kk * ldw + col] : w[(int64_t)col * ldw + kk];
                d[e >> 2] |= x << (8 * (e & 3));
            }
            *reinterpret_cast<u32x4 *>(out + c * 16) = u32x4{d[0], d[1], d[2], d[3]};
        } else {
            const int64_t sc = c - code_chunks;
            const int nl = (int)(sc & 31);
            const int64_t st = sc >> 5;
            const int t = (int)(st % kt), slab = (int)(st / kt);
            float v[4];
            for (int q = 0; q < 4; ++q) {
                const int b = q >> 1, kb = q & 1;
                const int col = weight_column(slab, 32 * b + nl, n, glu);
                const int k0 = 64 * t + 32 * kb;
                float s = 0.0f;
                if (col >= 0 && k0 < k) {
                    const int blk = k0 / block;
                    s = scale_value(scale, scale_kind, wl == W_KN ? (int64_t)blk * ldw + col : (int64_t)col * kb_count + blk);
                }
                v[q] = s;
            }
            *reinterpret_cast<f32x4 *>(out + code_chunks * 16 + sc * 16) = f32x4{v[0], v[1], v[2], v[3]};
        }
    }
}

int grid_of(int64_t count) {
    const int64_t blocks = (count + 255) / 256;
    return (int)(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}

template <int BM, int NW, int OCC, int NB>
hipError_t dispatch(const GemmArgs &p, int epi, int out, hipStream_t stream) {
#define SQ8_CASE(E, O)                                                                            \
    if (epi == E && out == O) return blk::launch_blocks_product<BM, NW, OCC, NB, W_INT8, E, O>(p, stream);
    SQ8_CASE(EPI_NONE, OUT_BF16)
    SQ8_CASE(EPI_NONE, OUT_F32)
    SQ8_CASE(EPI_GELU, OUT_BF16)
    SQ8_CASE(EPI_GELU, OUT_F32)
    if constexpr (NB == 2) {
        SQ8_CASE(EPI_SILU_GLU, OUT_BF16)
        SQ8_CASE(EPI_SILU_GLU, OUT_F32)
        SQ8_CASE(EPI_SITU_GLU, OUT_BF16)
        SQ8_CASE(EPI_SITU_GLU, OUT_F32)
    }
#undef SQ8_CASE
    return hipErrorInvalidValue;
}

}  // namespace

int64_t packed_blocks_bytes(int k, int n, bool glu) {
    const int64_t kt = (k + 63) / 64;
    const int64_t slabs = glu ? ((int64_t)n / 2 + 31) / 32 : ((int64_t)n + 63) / 64;
    return slabs * kt * (4096 + 512);
}

hipError_t launch_pack_blocks(const uint8_t *w, int wl, int64_t ldw, const void *scale, int scale_dtype, int block,
                              int k, int n, bool glu, uint8_t *out, hipStream_t stream) {
    const int kt = (k + 63) / 64;
    const int64_t slabs = glu ? ((int64_t)n / 2 + 31) / 32 : ((int64_t)n + 63) / 64;
    const int64_t code_chunks = slabs * kt * 256, chunks = code_chunks + slabs * kt * 32;
    if (chunks == 0) return hipSuccess;
    hipLaunchKernelGGL(pack_blocks_kernel, dim3(grid_of(chunks)), dim3(256), 0, stream, w, wl, ldw, scale, scale_dtype,
                       block, k, n, glu ? 1 : 0, kt, code_chunks, chunks, out);
    return hipGetLastError();
}

hipError_t launch_blocks_product(const GemmArgs &p, int tile, int epi, int out, hipStream_t stream) {
    const bool glu = epi == EPI_SILU_GLU || epi == EPI_SITU_GLU;
    if (tile == BL_128x256 && !glu) return dispatch<128, 8, 1, 1>(p, epi, out, stream);
    if (tile == BL_128x128 && !glu) return dispatch<128, 4, 2, 1>(p, epi, out, stream);
    if (tile == BL_64x512) return dispatch<64, 8, 1, 2>(p, epi, out, stream);
    return dispatch<64, 4, 2, 2>(p, epi, out, stream);
}

}  // namespace sq8
