// sq8_skinny_kernel.h — the skinny-M variant of the weight-direct GEMM: short activation streams
// (text tokens, M up to a few hundred rows), where 128-row tiles leave most of the 256 CUs idle and
// the product turns bandwidth-bound on the weight.
//
// Arithmetic as the other kernels (Sources/Siliconed/TensorGEMM.swift:124-135, :173-179): exact
// bf16 × code products, fp32 sums, scale after the sum, bias after the scale, activation last.
//
// Tile BM × 64 (one 64-column weight slab; GLU: 32 output columns, both halves), BM = 32 or 64, and
// the K steps split over the workgroup's NWK waves: wave w takes steps w, w + NWK, w + 2·NWK, …
// Every wave streams its steps' codes and activation fragments straight from global memory into
// registers (PF steps in flight), widens the codes there and feeds the MFMAs: no LDS and no
// barrier in the K loop, so the waves run independently. The NWK partial sums then meet in LDS and
// are added in wave order (deterministic), one wave per 32 × 32 block, which runs the epilogue.
//
// K split (SPLIT, p.splits > 1; M up to a few tiles, where one workgroup per slab leaves most CUs
// idle): workgroup (tile, s) takes the s-th of p.splits contiguous ranges of K steps, its waves split
// those as above, and the wave-order sum of each 32 × 32 block goes to p.part as fp32 in the MFMA's
// register order ([split][tile][block][register][lane]: 256-byte rows, rows past M not written); a
// second launch (skinny_reduce_kernel) adds the splits in split order and runs the epilogue. Fixed
// order throughout, so the bits depend only on the split count, not on the tile height.
//
// Operand layouts as the weight-direct kernel: MFMA sub-step ks of lane half h (lanes 32h..32h+31)
// covers k ∈ [32h + 8ks, 32h + 8ks + 8) of the step, for codes and activations alike — a lane's
// activation bytes for the step are 64 contiguous bytes of its row.
#pragma once

#include "sq8_wdirect_kernel.h"

namespace sq8 {
namespace wd {

template <int BM, int NWK, int PF, int WT, int WL, int EPI, int OUT, bool SPLIT = false>
__global__ void __attribute__((amdgpu_flat_work_group_size(64 * NWK, 64 * NWK), amdgpu_waves_per_eu(2, 2)))
gemm_skinny_kernel(const GemmArgs p) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int FM = BM / 32;
    constexpr int NB = 2 * FM;                       // 32 × 32 blocks per wave
    constexpr int RED = NWK * NB * 1024 * 4;         // the partial sums of every wave, fp32
    constexpr int REGION = 32 * (32 * (OUT == OUT_BF16 ? 2 : 4) + 16);
    static_assert(NWK * REGION <= RED, "the epilogue regions fit in the reduction area");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[RED];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // This workgroup's K steps [k0, k0 + KT): all of them, or its split's contiguous range.
    int bid = blockIdx.x, split = 0, k0 = 0, KT = p.kt;
    if constexpr (SPLIT) {
        split = bid % p.splits;
        bid /= p.splits;
        k0 = (int)((int64_t)split * p.kt / p.splits);
        KT = (int)((int64_t)(split + 1) * p.kt / p.splits) - k0;
    }
    int tm, slab;
    kern::tile_of(bid, p.tiles_m, p.tiles_n, tm, slab);
    const int m0 = tm * BM;
    const kern::gbytes Ag = (kern::gbytes)p.a;
    const kern::gbytes Wg = (kern::gbytes)p.w;
    const int h = lane >> 5;

    // Activation fragments: row m0 + 32·bm + (lane & 31) (clamped: rows past M are computed on the
    // last row and never stored), bytes [64h, 64h + 64) of the step.
    uint32_t a_off[FM];
#pragma unroll
    for (int bm = 0; bm < FM; ++bm) {
        const int row = min(m0 + 32 * bm + (lane & 31), p.M - 1);
        a_off[bm] = (uint32_t)((int64_t)row * p.lda * 2) + 64 * h;
    }
    uint32_t w_off[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w_off[j] = w_offset<WL, GLU>(p, slab, j, lane);
    const uint32_t w_step = WL == W_PACKED ? 4096 : BK;

    u32x4 ra[PF][FM][4];  // [buffer][bm][ks]: 8 bf16 of the activation each
    u32x4 rw[PF][4];      // [buffer][load j]: 16 codes each
    // The loads of this wave's i-th step (clamped to the last step: prefetches past the wave's
    // last step are never used).
    auto issue = [&](int i, auto buf) {
        constexpr int B = decltype(buf)::value;
        const int t = k0 + min(wave + NWK * i, KT - 1);
        const kern::gbytes abase = Ag + (uint32_t)t * (BK * 2);
        const kern::gbytes wbase = Wg + (uint32_t)weight_step(p, t) * w_step;
#pragma unroll
        for (int j = 0; j < 4; ++j) rw[B][j] = kern::gld<u32x4>(wbase, w_off[j]);
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) ra[B][bm][ks] = kern::gld<u32x4>(abase, a_off[bm] + 16 * ks);
    };

    f32x16 acc[2][FM];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[b][bm][r] = 0.0f;

    auto compute = [&](auto buf) {
        constexpr int B = decltype(buf)::value;
        static_for<0, 4>([&](auto kc) {
            constexpr int ks = decltype(kc)::value;
            bf16x8 wk[2];
            static_for<0, 2>([&](auto bc) {
                constexpr int b = decltype(bc)::value;
                const u32x4 &r = rw[B][2 * b + (ks >> 1)];
                wk[b] = widen8<WT>(r[2 * (ks & 1)], r[2 * (ks & 1) + 1]);
            });
            static_for<0, 2>([&](auto bc) {
                constexpr int b = decltype(bc)::value;
                static_for<0, FM>([&](auto bmc) {
                    constexpr int bm = decltype(bmc)::value;
                    acc[b][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        wk[b], __builtin_bit_cast(bf16x8, ra[B][bm][ks]), acc[b][bm], 0, 0, 0);
                });
            });
        });
    };

    const int n = wave < KT ? (KT - wave + NWK - 1) / NWK : 0;  // this wave's steps
    // PF steps in flight: step i in buffer i % PF, its buffer refilled with step i + PF once used.
    static_for<0, PF>([&](auto bc) { issue(decltype(bc)::value, bc); });
    int i = 0;
    for (; i + PF - 1 < n; i += PF) {
        static_for<0, PF>([&](auto bc) {
            constexpr int B = decltype(bc)::value;
            compute(bc);
            issue(i + B + PF, bc);
        });
    }
    static_for<0, PF - 1>([&](auto bc) {
        if (i + decltype(bc)::value < n) compute(bc);
    });

    // ---- reduction: partial sums to LDS, [wave][block][register][lane], then block e summed by
    // wave e % NWK in wave order ---------------------------------------------------------------------
    float *red = reinterpret_cast<float *>(lds);
    static_for<0, 2>([&](auto bc) {
        constexpr int b = decltype(bc)::value;
        static_for<0, FM>([&](auto bmc) {
            constexpr int bm = decltype(bmc)::value;
            float *dst = red + ((wave * NB + b * FM + bm) * 16) * 64 + lane;
#pragma unroll
            for (int r = 0; r < 16; ++r) dst[r * 64] = acc[b][bm][r];
        });
    });
    __syncthreads();
    // Block e = b·FM + bm. GLU: wave bm sums both halves of row block bm (its epilogue needs both).
    f32x16 sum[2];
    int mine[2] = {-1, -1};
    if constexpr (GLU && !SPLIT) {
        if (wave < FM) { mine[0] = wave; mine[1] = FM + wave; }
    } else {
        if (wave < NB) mine[0] = wave;
        if (wave + NWK < NB) mine[1] = wave + NWK;
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sum[q][r] = 0.0f;
        if (mine[q] >= 0) {
#pragma unroll
            for (int w = 0; w < NWK; ++w) {
                const float *src = red + ((w * NB + mine[q]) * 16) * 64 + lane;
#pragma unroll
                for (int r = 0; r < 16; ++r) sum[q][r] += src[r * 64];
            }
        }
    }
    if constexpr (SPLIT) {
        // This split's sums of the wave's blocks, rows past M left out.
        const int tile = tm * p.tiles_n + slab;
        float *const part = p.part + ((int64_t)split * p.tiles_m * p.tiles_n + tile) * (NB * 1024) + lane;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if (mine[q] >= 0 && m0 + 32 * (mine[q] % FM) + (lane & 31) < p.M) {
#pragma unroll
                for (int r = 0; r < 16; ++r) part[(mine[q] * 16 + r) * 64] = sum[q][r];
            }
        }
        return;
    }
    __syncthreads();  // the reduction area becomes the epilogue regions

    // ---- epilogue --------------------------------------------------------------------------------
    const int n_out = GLU ? p.glu_half : p.N;
    const bool has_bias = p.bias != nullptr;
    uint8_t *region = lds + wave * REGION;
    if constexpr (GLU) {
        if (mine[0] >= 0) {
            const int col0 = slab * 32;
            ColParams cx, cu;
            load_col_params(p, cx, col0, 0, n_out, lane);
            load_col_params(p, cu, col0, p.glu_half, n_out, lane);
            if (col0 < n_out) store_block<EPI, OUT>(p, sum[0], cx, sum[1], cu, has_bias, col0, m0 + 32 * wave, n_out, region, lane);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if (mine[q] >= 0) {
                const int b = mine[q] / FM, bm = mine[q] % FM;
                const int col0 = slab * 64 + 32 * b;
                ColParams cx;
                load_col_params(p, cx, col0, 0, n_out, lane);
                if (col0 < n_out) store_block<EPI, OUT>(p, sum[q], cx, sum[q], cx, has_bias, col0, m0 + 32 * bm, n_out, region, lane);
            }
        }
    }
}

// The second launch of a split product: each 32 × 32 block's partial sums added in split order (from
// zero, as the unsplit kernel's wave sums), then the product's epilogue — one wave per block (GLU: per
// row block, both halves), four waves a workgroup, each with its own LDS region.
template <int BM, int EPI, int OUT>
__global__ void __launch_bounds__(256) skinny_reduce_kernel(const GemmArgs p) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int FM = BM / 32, NB = 2 * FM, UNITS = GLU ? FM : NB;
    constexpr int REGION = 32 * (32 * (OUT == OUT_BF16 ? 2 : 4) + 16);
    __shared__ __attribute__((aligned(16))) uint8_t lds[4 * REGION];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tiles = p.tiles_m * p.tiles_n;
    const int unit = blockIdx.x * 4 + wave;
    if (unit >= tiles * UNITS) return;
    const int tile = unit / UNITS, u = unit - tile * UNITS;
    const int tm = tile / p.tiles_n, slab = tile - tm * p.tiles_n;
    const int m0 = tm * BM, bm = u % FM;
    const int e0 = u, e1 = GLU ? FM + u : u;
    f32x16 x, y;
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = y[r] = 0.0f;
    if (m0 + 32 * bm + (lane & 31) < p.M) {
        // Four splits' loads in flight at once (each split a memory latency otherwise), then their sums
        // in split order.
        const int64_t stride = (int64_t)tiles * (NB * 1024);
        const float *src = p.part + (int64_t)tile * (NB * 1024) + lane;
        constexpr int G = 4;
        int s = 0;
        for (; s + G <= p.splits; s += G) {
            f32x16 vx[G], vy[G];
#pragma unroll
            for (int j = 0; j < G; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    vx[j][r] = src[(s + j) * stride + (e0 * 16 + r) * 64];
                    if constexpr (GLU) vy[j][r] = src[(s + j) * stride + (e1 * 16 + r) * 64];
                }
#pragma unroll
            for (int j = 0; j < G; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    x[r] += vx[j][r];
                    if constexpr (GLU) y[r] += vy[j][r];
                }
        }
        for (; s < p.splits; ++s) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                x[r] += src[s * stride + (e0 * 16 + r) * 64];
                if constexpr (GLU) y[r] += src[s * stride + (e1 * 16 + r) * 64];
            }
        }
    }
    const int n_out = GLU ? p.glu_half : p.N;
    const bool has_bias = p.bias != nullptr;
    uint8_t *region = lds + wave * REGION;
    if constexpr (GLU) {
        const int col0 = slab * 32;
        ColParams cx, cu;
        load_col_params(p, cx, col0, 0, n_out, lane);
        load_col_params(p, cu, col0, p.glu_half, n_out, lane);
        if (col0 < n_out) store_block<EPI, OUT>(p, x, cx, y, cu, has_bias, col0, m0 + 32 * bm, n_out, region, lane);
    } else {
        const int col0 = slab * 64 + 32 * (u / FM);
        ColParams cx;
        load_col_params(p, cx, col0, 0, n_out, lane);
        if (col0 < n_out) store_block<EPI, OUT>(p, x, cx, x, cx, has_bias, col0, m0 + 32 * bm, n_out, region, lane);
    }
}

template <int BM, int NWK, int PF, int WT, int WL, int EPI, int OUT>
hipError_t launch_skinny(const GemmArgs &args, hipStream_t stream) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    GemmArgs p = args;
    // tile_of's order: M tiles fastest inside a group, so the workgroups of one XCD share slabs.
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = GLU ? (p.glu_half + 31) / 32 : (p.N + 63) / 64;
    const int blocks = p.tiles_m * p.tiles_n;
    if (blocks == 0) return hipSuccess;
    if (p.splits > 1) {
        // Every split needs a step; the partial sums need their buffer (skinny_part_bytes).
        if (p.splits > p.kt || p.part == nullptr) return hipErrorInvalidValue;
        // The partial kernel has no epilogue: one instantiation per weight layout (GLU or not).
        constexpr int PE = GLU ? EPI_SILU_GLU : EPI_NONE;
        hipLaunchKernelGGL((gemm_skinny_kernel<BM, NWK, PF, WT, WL, PE, OUT_F32, true>), dim3(blocks * p.splits),
                           dim3(64 * NWK), 0, stream, p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        constexpr int UNITS = GLU ? BM / 32 : 2 * (BM / 32);
        hipLaunchKernelGGL((skinny_reduce_kernel<BM, EPI, OUT>), dim3((blocks * UNITS + 3) / 4), dim3(256), 0, stream, p);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((gemm_skinny_kernel<BM, NWK, PF, WT, WL, EPI, OUT>), dim3(blocks), dim3(64 * NWK), 0, stream, p);
    return hipGetLastError();
}

template <int BM, int NWK, int PF, int WT, int WL>
hipError_t dispatch_skinny(const GemmArgs &p, int epi, int out, hipStream_t stream) {
#define SQ8_CASE(E, O)                                                                            \
    if (epi == E && out == O) return launch_skinny<BM, NWK, PF, WT, WL, E, O>(p, stream);
    SQ8_CASE(EPI_NONE, OUT_BF16)
    SQ8_CASE(EPI_NONE, OUT_F32)
    SQ8_CASE(EPI_GELU, OUT_BF16)
    SQ8_CASE(EPI_GELU, OUT_F32)
    SQ8_CASE(EPI_SILU_GLU, OUT_BF16)
    SQ8_CASE(EPI_SILU_GLU, OUT_F32)
    SQ8_CASE(EPI_SITU_GLU, OUT_BF16)
    SQ8_CASE(EPI_SITU_GLU, OUT_F32)
    SQ8_CASE(EPI_RESIDUAL, OUT_F32)
#undef SQ8_CASE
    return hipErrorInvalidValue;
}

}  // namespace wd
}  // namespace sq8
