// sq8_gemv_kernel.h — the short-M product (M up to 16 rows: a text-token stream, a decode-sized batch):
// narrow column groups so the weight stream spreads over every CU, and every K step's loads issued
// far ahead, so a workgroup's time is a few memory latencies, not one per step.
//
// Arithmetic as the other kernels (Sources/Siliconed/TensorGEMM.swift:124-135, :173-179): exact
// bf16 × code products, fp32 sums, scale after the sum, bias after the scale, activation last. The
// reference's own bandwidth-bound int8 path is a split-K GEMV (DecodeKernels.swift:66-110: columns a lane,
// rows strided over simdgroups, a fixed-order partial sum); this is its MI355X form on the matrix cores.
//
// A workgroup owns CG groups of 16 virtual columns of the weight (GLU: 8 output columns a group, their
// gate and up halves) for all M (≤ 16) rows, and its four waves split the K steps (wave w takes w, w + 4,
// …). Lane l of a wave holds, per K step and column group, the 16 codes of virtual column l & 15 at
// k ∈ [16q, 16q + 16) of the step (q = l >> 4) — one 16-byte load, in the packed layout a chunk of the
// slab's step — and the matching 16 activation values of row l & 15, and feeds v_mfma_f32_16x16x32_bf16
// twice a step and group (A: the activation, 16 rows × 32 K; B: the codes, 32 K × 16 columns; MFMA u takes
// k ∈ 16q + 8u + [0, 8) of every lane group q: a fixed permutation of the step's K, the same for both
// operands). PF steps of code loads are in flight. The activation is staged in LDS whole when it fits
// (direct global→LDS loads, once per workgroup), else each lane loads its fragments beside its codes.
// No barrier in the K loop. The four partial sums meet in LDS and are added in wave order
// (deterministic); wave 0 runs the epilogue (lane l: column l & 15 of each group, rows 4(l >> 4) + [0, 4)).
// More column groups a workgroup (CG = 2, 4) where the columns are many: each workgroup then reads the
// activation once for more columns.
#pragma once

#include "sq8_wdirect_kernel.h"

namespace sq8 {
namespace wd {


template <int CG, int PF, int WT, int WL, int EPI, int OUT, bool XL>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 2)))
gemm_gemv_kernel(const GemmArgs p) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int NWK = 4;
    constexpr int RED_BYTES = NWK * CG * 4 * 64 * 4;
    constexpr int LDS_BYTES = XL && GEMV_XLDS > RED_BYTES ? GEMV_XLDS : RED_BYTES;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
    float *const red = reinterpret_cast<float *>(lds);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, q = lane >> 4;
    const int h = q >> 1, j1 = q & 1;
    const int n_out = GLU ? p.glu_half : p.N;
    // Column group cg of this workgroup: output column out_col[cg] of lane column c, and the codes' byte
    // offset at step 0 (w_off[cg]); w_step the step's stride.
    uint32_t w_off[CG];
    int out_col[CG];
    const uint32_t w_step = WL == W_PACKED ? 4096 : BK;
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
        const int grp = blockIdx.x * CG + cg;  // the 16-column group
        int slab, vc;
        if constexpr (GLU) {
            const int oc = 8 * grp + (c & 7);  // lanes c < 8: the gate column, c ≥ 8: its up column
            slab = oc >> 5;
            vc = (oc & 31) + (c >> 3) * 32;
            out_col[cg] = oc;
        } else {
            const int v = 16 * grp + c;
            slab = v >> 6;
            vc = v & 63;
            out_col[cg] = v;
        }
        if constexpr (WL == W_PACKED) {
            const int slabs = GLU ? (p.glu_half + 31) / 32 : (p.N + 63) / 64;
            const int s = slab < slabs ? slab : slabs - 1;
            const int kt = p.kt_w > 0 ? p.kt_w : p.kt;
            const int j = 2 * (vc >> 5) + j1;
            w_off[cg] = (uint32_t)(((int64_t)s * kt * 4 + j) * 1024 + ((vc & 31) + 32 * h) * 16);
        } else {
            int n;
            if constexpr (GLU) {
                const int oc = min(out_col[cg], p.glu_half - 1);
                n = oc + (vc >> 5) * p.glu_half;
            } else {
                n = min(out_col[cg], p.N - 1);
            }
            w_off[cg] = (uint32_t)((int64_t)n * p.ldw + 16 * q);
        }
    }
    const int row = min(c, p.M - 1);  // rows past M are computed on the last row and never stored
    const kern::gbytes Ag = (kern::gbytes)p.a;
    const kern::gbytes Wg = (kern::gbytes)p.w;
    const int KT = p.kt;
    const uint32_t a_off = (uint32_t)((int64_t)row * p.lda * 2) + 32 * q;  // global fragment at step 0
    const uint32_t x_off = (uint32_t)(row * gemv_xpitch(KT)) + 32 * q;     // LDS fragment at step 0

    u32x4 rw[PF][CG];          // 16 codes of each column group
    u32x4 ra[XL ? 1 : PF][2];  // 16 activation values (global fragments)
    auto issue = [&](int i, auto buf) {
        constexpr int B = decltype(buf)::value;
        const int t = min(wave + NWK * i, KT - 1);  // past the wave's last step: never used
        const kern::gbytes wbase = Wg + (uint32_t)weight_step(p, t) * w_step;
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) rw[B][cg] = kern::gld<u32x4>(wbase, w_off[cg]);
        if constexpr (!XL) {
            const kern::gbytes abase = Ag + (uint32_t)t * (BK * 2);
            ra[B][0] = kern::gld<u32x4>(abase, a_off);
            ra[B][1] = kern::gld<u32x4>(abase, a_off + 16);
        }
    };
    f32x4 acc[CG];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) acc[cg] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](auto buf, int i) {
        constexpr int B = decltype(buf)::value;
        bf16x8 a0, a1;
        if constexpr (XL) {
            const uint8_t *xr = lds + x_off + (wave + NWK * i) * 128;
            a0 = *reinterpret_cast<const bf16x8 *>(xr);
            a1 = *reinterpret_cast<const bf16x8 *>(xr + 16);
        } else {
            a0 = __builtin_bit_cast(bf16x8, ra[B][0]);
            a1 = __builtin_bit_cast(bf16x8, ra[B][1]);
        }
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) {
            const bf16x8 w0 = widen8<WT>(rw[B][cg][0], rw[B][cg][1]);
            const bf16x8 w1 = widen8<WT>(rw[B][cg][2], rw[B][cg][3]);
            acc[cg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, w0, acc[cg], 0, 0, 0);
            acc[cg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, w1, acc[cg], 0, 0, 0);
        }
    };
    const int n = wave < KT ? (KT - wave + NWK - 1) / NWK : 0;  // this wave's steps
    if constexpr (XL) {
        // The activation's M rows into LDS by direct loads: one 1 KB run of a row (64 chunks of 16 bytes)
        // per instruction, the runs dealt over the waves; all in flight at once, ahead of the codes.
        const int runs_row = KT / 8;
        const int runs = p.M * runs_row;
        for (int r = wave; r < runs; r += NWK) {
            const int xr = r / runs_row, cr = r - xr * runs_row;
            __builtin_amdgcn_global_load_lds(
                (glb_ptr)(Ag + (uint32_t)((int64_t)xr * p.lda * 2) + (uint32_t)(cr * 1024 + lane * 16)),
                (lds_ptr)(lds + xr * gemv_xpitch(KT) + cr * 1024), 16, 0, 0);
        }
    }
    static_for<0, PF>([&](auto bc) { issue(decltype(bc)::value, bc); });
    if constexpr (XL) {
        wait_vmcnt<0>();
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
    // The loads past the wave's last step (never used) land before LDS is reused and the workgroup ends.
    wait_vmcnt<0>();
    __syncthreads();

    // ---- the four partial sums, added in wave order ----
#pragma unroll
    for (int cg = 0; cg < CG; ++cg)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[((wave * CG + cg) * 4 + e) * 64 + lane] = acc[cg][e];
    __syncthreads();
    if (wave != 0) return;
    const bool has_bias = p.bias != nullptr;
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
        f32x4 sum;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < NWK; ++w) s += red[((w * CG + cg) * 4 + e) * 64 + lane];
            sum[e] = s;
        }
        // ---- epilogue: lane column c of group cg, rows 4q + e ----
        const int col = out_col[cg];
        const int wcol = col < n_out ? col : n_out - 1;  // the weight column whose scale and bias apply
        const float sc = p.scale[p.scale_per_col ? wcol : 0];
        const float bi = has_bias ? p.bias[wcol] : 0.0f;
        float su = 0.0f, bu = 0.0f;
        if constexpr (GLU) {
            su = p.scale[p.scale_per_col ? wcol + p.glu_half : 0];
            bu = has_bias ? p.bias[wcol + p.glu_half] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float v = __fmul_rn(sum[e], sc);
            if (has_bias) v = __fadd_rn(v, bi);
            if constexpr (GLU) {
                // The up half's sum of the same output column: lane c + 8 (c < 8).
                float u = __shfl_down(sum[e], 8, 16);
                u = __fmul_rn(u, su);
                if (has_bias) u = __fadd_rn(u, bu);
                v = EPI == EPI_SILU_GLU ? silu_glu(v, u) : situ(v, u);
            } else if constexpr (EPI == EPI_GELU) {
                v = gelu_tanh(v);
            }
            const int m = 4 * q + e;
            if (m < p.M && col < n_out && (!GLU || c < 8)) {
                if constexpr (EPI == EPI_RESIDUAL) {
                    float *xo = reinterpret_cast<float *>(p.c[0]) + (int64_t)m * p.ldc + col;
                    *xo = __fadd_rn(*xo, __fmul_rn(p.gate ? p.gate[col] : 1.0f, v));
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
}

// Column groups of 16 a workgroup: the fewest that fit the groups in one round of workgroups on the CUs
// (1 … 4; more, four a workgroup in more rounds). Measured at K = 3072, M = 1 (one process, HIP events):
// N = 6144 two groups 7.4 µs against 8.2 with one (two rounds), N = 9216 three 8.9 against 11.8 with two,
// N = 12288 three 10.6 against 11.2 with four (192 workgroups).
inline int gemv_groups_per_wg(const GemmArgs &p, bool glu) {
    const int groups = glu ? (p.glu_half + 7) / 8 : (p.N + 15) / 16;
    const int cus = p.cus > 0 ? p.cus : 256;
    const int cg = (groups + cus - 1) / cus;
    return cg < 1 ? 1 : cg > 4 ? 4 : cg;
}

template <int CG, int PF, int WT, int WL, int EPI, int OUT>
hipError_t launch_gemv_cg(const GemmArgs &p, int groups, hipStream_t stream) {
    const int wgs = (groups + CG - 1) / CG;
    if (gemv_x_in_lds(p.M, p.kt))
        hipLaunchKernelGGL((gemm_gemv_kernel<CG, PF, WT, WL, EPI, OUT, true>), dim3(wgs), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((gemm_gemv_kernel<CG, PF, WT, WL, EPI, OUT, false>), dim3(wgs), dim3(256), 0, stream, p);
    return hipGetLastError();
}

template <int WT, int WL, int EPI, int OUT>
hipError_t launch_gemv(const GemmArgs &p, hipStream_t stream) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    if (p.M > 16) return hipErrorInvalidValue;
    const int groups = GLU ? (p.glu_half + 7) / 8 : (p.N + 15) / 16;
    if (groups == 0 || p.M == 0) return hipSuccess;
    // Steps of code loads in flight: eight of one group, six of two, five of three, four of four (the registers).
    switch (gemv_groups_per_wg(p, GLU)) {
    case 4: return launch_gemv_cg<4, 4, WT, WL, EPI, OUT>(p, groups, stream);
    case 3: return launch_gemv_cg<3, 5, WT, WL, EPI, OUT>(p, groups, stream);
    case 2: return launch_gemv_cg<2, 6, WT, WL, EPI, OUT>(p, groups, stream);
    default: return launch_gemv_cg<1, 8, WT, WL, EPI, OUT>(p, groups, stream);
    }
}

template <int WT, int WL>
hipError_t dispatch_gemv(const GemmArgs &p, int epi, int out, hipStream_t stream) {
#define SQ8_CASE(E, O)                                                                            \
    if (epi == E && out == O) return launch_gemv<WT, WL, E, O>(p, stream);
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
