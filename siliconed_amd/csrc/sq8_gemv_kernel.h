// sq8_gemv_kernel.h — the short-M product (M up to 64 rows: a text-token stream, a decode-sized batch):
// narrow column groups so the weight stream spreads over every CU, and every K step's loads issued
// far ahead, so a workgroup's time is a few memory latencies, not one per step.
//
// Arithmetic as the other kernels (Sources/Siliconed/TensorGEMM.swift:124-135, :173-179): exact
// bf16 × code products, fp32 sums, scale after the sum, bias after the scale, activation last. The
// reference's own bandwidth-bound int8 path is a split-K GEMV (DecodeKernels.swift:66-110: columns a lane,
// rows strided over simdgroups, a fixed-order partial sum); this is its MI355X form on the matrix cores.
//
// A workgroup owns 16 virtual columns of the weight (GLU: 8 output columns, their gate and up halves)
// for all M (≤ 16·RM) rows, and its four waves split the K steps (wave w takes w, w + 4, …). Lane l of a
// wave holds, per K step, the 16 codes of virtual column l & 15 at k ∈ [16q, 16q + 16) of the step
// (q = l >> 4) — one 16-byte load, in the packed layout a chunk of the slab's step — and the matching
// 16 activation values of row l & 15 of each 16-row group, and feeds v_mfma_f32_16x16x32_bf16 twice a
// step (A: the activation, 16 rows × 32 K; B: the codes, 32 K × 16 columns; MFMA u takes k ∈ 16q + 8u +
// [0, 8) of every lane group q: a fixed permutation of the step's K, the same for both operands). PF
// steps of code loads are in flight; the activation is read from LDS where it fits there whole (staged
// once per workgroup), else loaded by each lane beside its codes; no barrier in the K loop. The four
// partial sums meet in LDS
// and are added in wave order (deterministic); wave 0 runs the epilogue on its 16·RM × 16 outputs (lane
// l: column l & 15, rows 4(l >> 4) + [0, 4) of each group).
#pragma once

#include "sq8_wdirect_kernel.h"

namespace sq8 {
namespace wd {

// The activation staged in LDS whole (XL: M rows of K' = p.kt · 64 bf16, rows XPITCH bytes apart) when it
// fits GEMV_XLDS bytes: the workgroup reads it from HBM once, with direct loads, and the K loop's only
// global loads are the codes. Else each lane loads its activation fragments itself.
constexpr int GEMV_XLDS = 64 * 1024;
__host__ __device__ constexpr int64_t gemv_xpitch(int kt) { return (int64_t)kt * 128 + 16; }

template <int RM, int PF, int WT, int WL, int EPI, int OUT, bool XL>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2, 2)))
gemm_gemv_kernel(const GemmArgs p) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int NWK = 4;
    constexpr int RED_BYTES = NWK * RM * 4 * 64 * 4;
    __shared__ __attribute__((aligned(16))) uint8_t lds[XL ? (GEMV_XLDS > RED_BYTES ? GEMV_XLDS : RED_BYTES) : RED_BYTES];
    float *const red = reinterpret_cast<float *>(lds);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, q = lane >> 4;
    // This workgroup's 16 virtual columns: slab `slab`, virtual column vc of lane column c.
    const int g = blockIdx.x;
    int slab, vc;
    if constexpr (GLU) {
        slab = g >> 2;
        vc = 8 * (g & 3) + (c & 7) + (c >> 3) * 32;  // lanes c < 8: gate columns, c ≥ 8: the same up columns
    } else {
        slab = g >> 2;
        vc = 16 * (g & 3) + c;
    }
    // The lane's 16 codes of a K step: byte offset at step 0 and the step's stride.
    uint32_t w_off;
    uint32_t w_step;
    const int h = q >> 1, j1 = q & 1;
    if constexpr (WL == W_PACKED) {
        const int slabs = GLU ? (p.glu_half + 31) / 32 : (p.N + 63) / 64;
        const int s = slab < slabs ? slab : slabs - 1;
        const int kt = p.kt_w > 0 ? p.kt_w : p.kt;
        const int j = 2 * (vc >> 5) + j1;
        w_off = (uint32_t)(((int64_t)s * kt * 4 + j) * 1024 + ((vc & 31) + 32 * h) * 16);
        w_step = 4096;
    } else {
        int n;
        if constexpr (GLU) {
            const int out = slab * 32 + (vc & 31);
            n = (out < p.glu_half ? out : p.glu_half - 1) + (vc >> 5) * p.glu_half;
        } else {
            n = slab * 64 + vc;
            n = n < p.N ? n : p.N - 1;
        }
        w_off = (uint32_t)((int64_t)n * p.ldw + 16 * q);
        w_step = BK;
    }
    // The activation: row (l & 15) of each 16-row group (clamped: rows past M are computed on the last
    // row and never stored), bytes [32q, 32q + 32) of the step.
    uint32_t a_off[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        const int row = min(16 * r + c, p.M - 1);
        a_off[r] = (uint32_t)((int64_t)row * p.lda * 2) + 32 * q;
    }
    const kern::gbytes Ag = (kern::gbytes)p.a;
    const kern::gbytes Wg = (kern::gbytes)p.w;
    const int KT = p.kt;

    u32x4 rw[PF];                      // 16 codes
    u32x4 ra[XL ? 1 : PF][RM][2];      // 16 activation values of each row group (global fragments)
    auto issue = [&](int i, auto buf) {
        constexpr int B = decltype(buf)::value;
        const int t = min(wave + NWK * i, KT - 1);  // past the wave's last step: never used
        rw[B] = kern::gld<u32x4>(Wg + (uint32_t)weight_step(p, t) * w_step, w_off);
        if constexpr (!XL) {
            const kern::gbytes abase = Ag + (uint32_t)t * (BK * 2);
#pragma unroll
            for (int r = 0; r < RM; ++r) {
                ra[B][r][0] = kern::gld<u32x4>(abase, a_off[r]);
                ra[B][r][1] = kern::gld<u32x4>(abase, a_off[r] + 16);
            }
        }
    };
    // XL: lane's fragment of row group r at step t: x_lds + row·XPITCH + t·128 + 32q.
    const int64_t xpitch = gemv_xpitch(KT);
    uint32_t x_off[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) x_off[r] = (uint32_t)(min(16 * r + c, p.M - 1) * xpitch) + 32 * q;
    f32x4 acc[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) acc[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](auto buf, int i) {
        constexpr int B = decltype(buf)::value;
        const bf16x8 w0 = widen8<WT>(rw[B][0], rw[B][1]);
        const bf16x8 w1 = widen8<WT>(rw[B][2], rw[B][3]);
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            bf16x8 a0, a1;
            if constexpr (XL) {
                const uint8_t *xr = lds + x_off[r] + (wave + NWK * i) * 128;
                a0 = *reinterpret_cast<const bf16x8 *>(xr);
                a1 = *reinterpret_cast<const bf16x8 *>(xr + 16);
            } else {
                a0 = __builtin_bit_cast(bf16x8, ra[B][r][0]);
                a1 = __builtin_bit_cast(bf16x8, ra[B][r][1]);
            }
            acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, w0, acc[r], 0, 0, 0);
            acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, w1, acc[r], 0, 0, 0);
        }
    };
    const int n = wave < KT ? (KT - wave + NWK - 1) / NWK : 0;  // this wave's steps
    static_for<0, PF>([&](auto bc) { issue(decltype(bc)::value, bc); });
    if constexpr (XL) {
        // The activation's M rows into LDS, 16 bytes a lane, while the codes' loads are in flight.
        const int chunks_row = KT * 8;  // 16-byte chunks per row
        const int total = p.M * chunks_row;
        for (int ch = threadIdx.x; ch < total; ch += 256) {
            const int row = ch / chunks_row, cr = ch - row * chunks_row;
            const u32x4 v = kern::gld<u32x4>(Ag, (uint32_t)((int64_t)row * p.lda * 2) + cr * 16);
            *reinterpret_cast<u32x4 *>(lds + row * xpitch + cr * 16) = v;
        }
        __syncthreads();
    }
    int i = 0;
    for (; i + PF - 1 < n; i += PF) {
        static_for<0, PF>([&](auto bc) {
            constexpr int B = decltype(bc)::value;
            compute(bc, i + B);
            issue(i + B + PF, bc);
        });
    }
    static_for<0, PF - 1>([&](auto bc) {
        if (i + decltype(bc)::value < n) compute(bc, i + decltype(bc)::value);
    });
    if constexpr (XL) __syncthreads();  // every wave's activation reads done before the reduction reuses LDS

    // ---- the four partial sums, added in wave order ----
#pragma unroll
    for (int r = 0; r < RM; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[((wave * RM + r) * 4 + e) * 64 + lane] = acc[r][e];
    __syncthreads();
    if (wave != 0) return;
    f32x4 sum[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < NWK; ++w) s += red[((w * RM + r) * 4 + e) * 64 + lane];
            sum[r][e] = s;
        }

    // ---- epilogue: lane column c, rows 16r + 4q + e ----
    const int n_out = GLU ? p.glu_half : p.N;
    int col;  // output column
    if constexpr (GLU)
        col = slab * 32 + 8 * (g & 3) + (c & 7);
    else
        col = slab * 64 + vc;
    const int wcol = col < n_out ? col : n_out - 1;  // the weight column whose scale and bias apply
    const float sc = p.scale[p.scale_per_col ? wcol : 0];
    const float bi = p.bias ? p.bias[wcol] : 0.0f;
    float su = 0.0f, bu = 0.0f;
    if constexpr (GLU) {
        su = p.scale[p.scale_per_col ? wcol + p.glu_half : 0];
        bu = p.bias ? p.bias[wcol + p.glu_half] : 0.0f;
    }
    const bool has_bias = p.bias != nullptr;
#pragma unroll
    for (int r = 0; r < RM; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float v = __fmul_rn(sum[r][e], sc);
            if (has_bias) v = __fadd_rn(v, bi);
            if constexpr (GLU) {
                // The up half's sum of the same output column: lane c + 8 (c < 8).
                float u = __shfl_down(sum[r][e], 8, 16);
                u = __fmul_rn(u, su);
                if (has_bias) u = __fadd_rn(u, bu);
                v = EPI == EPI_SILU_GLU ? silu_glu(v, u) : situ(v, u);
            } else if constexpr (EPI == EPI_GELU) {
                v = gelu_tanh(v);
            }
            const int m = 16 * r + 4 * q + e;
            if (m < p.M && col < n_out && (!GLU || c < 8)) {
                if constexpr (EPI == EPI_RESIDUAL) {
                    float *xr = reinterpret_cast<float *>(p.c[0]) + (int64_t)m * p.ldc + col;
                    *xr = __fadd_rn(*xr, __fmul_rn(p.gate ? p.gate[col] : 1.0f, v));
                } else {
                    int which;
                    const int64_t off = out_index(p, m, col, which);
                    uint8_t *o = kern::out_base(p, which);
                    if constexpr (OUT == OUT_BF16)
                        reinterpret_cast<uint16_t *>(o)[off] = (uint16_t)(pack_bf16_rne(v, 0.0f) & 0xFFFFu);
                    else
                        reinterpret_cast<float *>(o)[off] = v;
                }
            }
        }
}

template <int RM, int PF, int WT, int WL, int EPI, int OUT>
hipError_t launch_gemv(const GemmArgs &args, hipStream_t stream) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    GemmArgs p = args;
    if (p.M > 16 * RM) return hipErrorInvalidValue;
    const int groups = GLU ? (p.glu_half + 7) / 8 : (p.N + 15) / 16;
    if (groups == 0 || p.M == 0) return hipSuccess;
    if ((int64_t)p.M * gemv_xpitch(p.kt) <= GEMV_XLDS)
        hipLaunchKernelGGL((gemm_gemv_kernel<RM, PF, WT, WL, EPI, OUT, true>), dim3(groups), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((gemm_gemv_kernel<RM, PF, WT, WL, EPI, OUT, false>), dim3(groups), dim3(256), 0, stream, p);
    return hipGetLastError();
}

template <int RM, int PF, int WT, int WL>
hipError_t dispatch_gemv(const GemmArgs &p, int epi, int out, hipStream_t stream) {
#define SQ8_CASE(E, O)                                                                            \
    if (epi == E && out == O) return launch_gemv<RM, PF, WT, WL, E, O>(p, stream);
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
