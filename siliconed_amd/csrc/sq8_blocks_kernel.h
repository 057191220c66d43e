// sq8_blocks_kernel.h — the gfx950 product on codes with a scale per block of rows and column (GGUF
// Q8_0: int8 q [K, N], fp32 s [K/B, N], B = 32 or a multiple of it):
//
//     C = act(A · W + b),  W[k, n] = q[k, n] · s[k / B, n]
//
// (Sources/Siliconed/TensorGEMM.swift:137-171, `linear_q8`, which widens q · s into threadgroup
// memory and multiplies in fp32). Here the codes go to bf16 MFMAs as they are (exact), and each
// block's fp32 partial sum is scaled once it is complete:
//
//     C[m, n] = Σ_blocks s[blk, n] · (Σ_{k ∈ blk} a[m, k] · q[k, n])
//
// equal to the reference's sum in exact arithmetic, rounded differently: one fp32 product and sum
// per block instead of one fp32 product per weight.
//
// The weight-direct kernel's structure (sq8_wdirect_kernel.h: activation tiles through a 2-stage
// LDS ring, each wave streaming its 64-column slab of packed codes straight into registers) with
// three differences:
//   * the activation is the MFMA's first operand and the codes the second, so each lane's 16
//     results of a 32 × 32 block share one column (lane & 31) and one scale per block of K;
//   * a 64-step's K order keeps each block of 32 in two MFMA sub-steps: sub-step ks takes
//     k ∈ [16·ks, 16·ks + 16), lane half h the 8 at 16·ks + 8·h — the packed Q8 layout stores the
//     codes in that order, the activation fragment of (ks, h) is LDS chunk 2·ks + h;
//   * per block: P = MFMA(A, q) over its two sub-steps (from zero), then acc += P · s (fp32 FMA),
//     the scales of the step (two blocks × the lane's two 32-column blocks) one 16-byte load.
//
// Packed Q8 layout (sq8_pack_blocks): the codes as the packed layout's chunks — chunk c =
// ((slab·kt + t)·4 + j)·64 + lane, 16 bytes: k = 64t + 32(j&1) + 8h + [0, 8) then
// 64t + 32(j&1) + 16 + 8h + [0, 8) of virtual column 32(j>>1) + (lane & 31) — then, at byte
// slabs·kt·4096, the scales: per (slab, t), per column nl < 32, 16 bytes {s(block 0 of the step,
// column nl), s(block 1, nl), s(block 0, 32 + nl), s(block 1, 32 + nl)} (virtual columns; GLU:
// the slab's 32 output columns of each half). Zeros past K and past the columns.
#pragma once

#include "sq8_wdirect_kernel.h"

namespace sq8 {
namespace blk {

using wd::BK;
using wd::glb_ptr;
using wd::lds_ptr;
using wd::step_barrier;
using wd::swz;
using wd::wait_vmcnt;
using wd::widen8;

// Byte offset of the packed scales of a weight of kt steps and `slabs` slabs from the packed base.
__host__ __device__ inline int64_t scales_offset(int64_t slabs, int64_t kt) { return slabs * kt * 4096; }

// Bias, activation and store of one 32 × 32 block a wave holds in the transposed order (lane l,
// register r: row 8·(r >> 2) + 4·(l >> 5) + (r & 3), column l & 31): written value by value into the
// wave's LDS region, then stored as the weight-direct epilogue stores (flush_region).
template <int EPI, int OUT>
__device__ __forceinline__ void store_block_t(const GemmArgs &p, const f32x16 &x, float bx, const f32x16 &u, float bu,
                                              int col0, int m_first, int n_out, uint8_t *region, int lane) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int ESZ = OUT == OUT_BF16 ? 2 : 4;
    constexpr int PITCH = 32 * ESZ + 16;
    const int h = lane >> 5, c = lane & 31;
    wd::ResidualPre pre;
    if constexpr (EPI == EPI_RESIDUAL) wd::load_residual(p, col0, m_first, n_out, lane, pre);
    static_for<0, 16>([&](auto rc) {
        constexpr int r = decltype(rc)::value;
        float v = __fadd_rn(x[r], bx);
        if constexpr (EPI == EPI_GELU) {
            v = gelu_tanh(v);
        } else if constexpr (GLU) {
            const float w = __fadd_rn(u[r], bu);
            v = EPI == EPI_SILU_GLU ? silu_glu(v, w) : situ(v, w);
        }
        uint8_t *dst = region + (8 * (r >> 2) + 4 * h + (r & 3)) * PITCH + c * ESZ;
        if constexpr (OUT == OUT_BF16)
            *reinterpret_cast<uint16_t *>(dst) = (uint16_t)round_bf16(v);
        else
            *reinterpret_cast<float *>(dst) = v;
    });
    wd::flush_region<EPI, OUT>(p, col0, m_first, n_out, region, lane, EPI == EPI_RESIDUAL ? &pre : nullptr);
}

// NB: 32-column blocks per wave — 2 (the wave owns a 64-column slab) or 1 (waves in pairs share a
// slab, wave w taking block w & 1: half the registers per row block, so twice the rows fit).
template <int BM, int NW, int OCC, int NB, int WT, int EPI, int OUT>
__global__ void __attribute__((amdgpu_flat_work_group_size(64 * NW, 64 * NW), amdgpu_waves_per_eu(OCC, OCC)))
gemm_blocks_kernel(const GemmArgs p) {
    static_assert(NB == 1 || NB == 2, "one or two 32-column blocks a wave");
    static_assert(NB == 2 || NW % 2 == 0, "waves in pairs");
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int FM = BM / 32;
    constexpr int SA = BM * 128;
    constexpr int A_BLOCKS = BM / 8;
    constexpr int A_PER_WAVE = A_BLOCKS / NW;
    static_assert(A_BLOCKS % NW == 0, "the activation blocks split evenly over the waves");
    constexpr int WLOADS = 2 * NB + 1;  // code loads + the scale load per step
    static_assert(A_PER_WAVE + WLOADS < 64, "vmcnt budget");
    constexpr int REGION = 32 * (32 * (OUT == OUT_BF16 ? 2 : 4) + 16);
    constexpr int LDS_BYTES = NW * REGION > 2 * SA ? NW * REGION : 2 * SA;  // epilogue regions over the stages

    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tm, tn;
    kern::tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM;
    const int slabs = GLU ? (p.glu_half + 31) / 32 : (p.N + 63) / 64;
    constexpr int SLABS_PER_WG = NB == 2 ? NW : NW / 2;
    const int slab = tn * SLABS_PER_WG + (NB == 2 ? wave : wave >> 1);
    const int b0 = NB == 2 ? 0 : (wave & 1);  // the wave's first 32-column block in the slab
    const int rslab = slab < slabs ? slab : slabs - 1;  // a wave past the last slab reads the last
    const kern::gbytes Ag = (kern::gbytes)p.a;
    const kern::gbytes Wg = (kern::gbytes)p.w;
    const int KT = p.kt;

    uint32_t a_goff[A_PER_WAVE];
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i) {
        const int b = wave + NW * i;
        const int r = 8 * b + (lane >> 3);
        const int lc = (lane & 7) ^ ((r ^ (r >> 3)) & 7);
        const int row = min(m0 + r, p.M - 1);
        a_goff[i] = (uint32_t)((int64_t)row * p.lda * 2) + lc * 16;
    }
    auto issue_a = [&](int t, auto stage) {
        constexpr int S = decltype(stage)::value;
        const kern::gbytes base = Ag + (uint32_t)min(t, KT - 1) * (BK * 2);
#pragma unroll
        for (int i = 0; i < A_PER_WAVE; ++i)
            __builtin_amdgcn_global_load_lds((glb_ptr)(base + a_goff[i]), (lds_ptr)(lds + S * SA + (wave + NW * i) * 1024),
                                             16, 0, 0);
    };

    // Codes: 4 × 16 bytes per lane per step; scales: 16 bytes per lane per step (lanes l and l + 32
    // read the same).
    // The weight's K steps: KT, or kt_w when the activation holds several parts along K that each face
    // the whole weight (the fp32 route), the weight's step then t modulo kt_w.
    const int KW = p.kt_w > 0 ? p.kt_w : KT;
    const uint32_t w_base = (uint32_t)((int64_t)rslab * KW * 4096) + lane * 16;
    const uint32_t s_base = (uint32_t)(scales_offset(slabs, KW) + (int64_t)rslab * KW * 512) + (lane & 31) * 16;
    // raw[B][2·b + kb]: the codes of the wave's block b (0..NB−1 from b0), K block kb of the step.
    constexpr int NLOAD = 2 * NB;
    u32x4 raw[2][NLOAD];
    f32x4 sraw[2];
    auto issue_w = [&](int t, auto buf) {
        constexpr int B = decltype(buf)::value;
        const int tt = wd::weight_step(p, min(t, KT - 1));
        const kern::gbytes base = Wg + (uint32_t)tt * 4096;
#pragma unroll
        for (int j = 0; j < NLOAD; ++j) raw[B][j] = kern::gld<u32x4>(base, w_base + (2 * b0 + j) * 1024);
        sraw[B] = kern::gld<f32x4>(Wg + (uint32_t)tt * 512, s_base);
    };

    const int h = lane >> 5;
    int xo[2][4];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) xo[par][ks] = swz(32 * par + (lane & 31), 2 * ks + h) - 32 * 128 * par;

    f32x16 acc[NB][FM];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[b][bm][r] = 0.0f;

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;

    issue_a(0, I0{});
    issue_w(0, I0{});
    issue_w(1, I1{});
    wait_vmcnt<WLOADS>();
    step_barrier();

    auto step = [&](int t, auto par) {
        constexpr int P = decltype(par)::value;
        bf16x8 wk[2][NB];  // [ks & 1][block]
        bf16x8 xf[2][FM];
        f32x16 pp[NB][FM];
        const f32x4 sv = sraw[P];
        auto widen_ks = [&](auto kc) {
            constexpr int ks = decltype(kc)::value;
            static_for<0, NB>([&](auto bc) {
                constexpr int b = decltype(bc)::value;
                const u32x4 &r = raw[P][2 * b + (ks >> 1)];
                wk[ks & 1][b] = widen8<WT>(r[2 * (ks & 1)], r[2 * (ks & 1) + 1]);
            });
        };
        auto read_x = [&](auto kc) {
            constexpr int ks = decltype(kc)::value;
            static_for<0, FM>([&](auto bmc) {
                constexpr int bm = decltype(bmc)::value;
                xf[ks & 1][bm] = kern::lds_load_frag(lds + P * SA + 32 * 128 * bm, xo[bm & 1][ks]);
            });
        };
        __builtin_amdgcn_sched_barrier(0);
        read_x(I0{});
        widen_ks(I0{});
        issue_a(t + 1, std::integral_constant<int, 1 - P>{});
        static_for<0, 4>([&](auto kc) {
            constexpr int ks = decltype(kc)::value;
            if constexpr (ks < 3) {
                read_x(std::integral_constant<int, ks + 1>{});
                widen_ks(std::integral_constant<int, ks + 1>{});
            }
            if constexpr (ks == 2) {
                __builtin_amdgcn_sched_barrier(0);
                issue_w(t + 2, std::integral_constant<int, P>{});
                __builtin_amdgcn_sched_barrier(0);
            }
            static_for<0, NB>([&](auto bc) {
                constexpr int b = decltype(bc)::value;
                static_for<0, FM>([&](auto bmc) {
                    constexpr int bm = decltype(bmc)::value;
                    if constexpr ((ks & 1) == 0)
                        pp[b][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf[ks & 1][bm], wk[ks & 1][b],
                                                                            f32x16{}, 0, 0, 0);
                    else
                        pp[b][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf[ks & 1][bm], wk[ks & 1][b], pp[b][bm],
                                                                            0, 0, 0);
                });
            });
            if constexpr ((ks & 1) == 1) {
                // The block of K ends: its partial sums scaled into the totals.
                static_for<0, NB>([&](auto bc) {
                    constexpr int b = decltype(bc)::value;
                    const float s = NB == 2 ? sv[2 * b + (ks >> 1)] : (b0 ? sv[2 + (ks >> 1)] : sv[ks >> 1]);
                    static_for<0, FM>([&](auto bmc) {
                        constexpr int bm = decltype(bmc)::value;
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[b][bm][r] = __builtin_fmaf(pp[b][bm][r], s, acc[b][bm][r]);
                    });
                });
            }
        });
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<WLOADS>();
        step_barrier();
    };
    int t = 0;
    for (; t + 1 < KT; t += 2) {
        step(t, I0{});
        step(t + 1, I1{});
    }
    if (t < KT) step(t, I0{});

    const bool has_bias = p.bias != nullptr;
    const int n_out = GLU ? p.glu_half : p.N;
    float bias[NB];
    static_for<0, NB>([&](auto bc) {
        const int b = b0 + decltype(bc)::value;
        const int oc = GLU ? slab * 32 + (lane & 31) : slab * 64 + 32 * b + (lane & 31);
        const int col = GLU ? min(oc, n_out - 1) + b * p.glu_half : min(oc, n_out - 1);
        bias[decltype(bc)::value] = has_bias ? p.bias[col] : 0.0f;
    });
    wait_vmcnt<0>();
    step_barrier();

    uint8_t *region = lds + wave * REGION;
    if constexpr (NB == 2) {
        static_for<0, FM>([&](auto bmc) {
            constexpr int bm = decltype(bmc)::value;
            static_for<0, GLU ? 1 : 2>([&](auto bc) {
                constexpr int b = decltype(bc)::value;
                const int col0 = GLU ? slab * 32 : slab * 64 + 32 * b;
                if (col0 < n_out)
                    store_block_t<EPI, OUT>(p, acc[b][bm], bias[b], acc[GLU ? 1 : b][bm], bias[GLU ? 1 : b], col0,
                                            m0 + 32 * bm, n_out, region, lane);
            });
        });
    } else {
        static_assert(!GLU, "a GLU pair needs both blocks of the slab in one wave");
        const int col0 = slab * 64 + 32 * b0;
        static_for<0, FM>([&](auto bmc) {
            constexpr int bm = decltype(bmc)::value;
            if (col0 < n_out)
                store_block_t<EPI, OUT>(p, acc[0][bm], bias[0], acc[0][bm], bias[0], col0, m0 + 32 * bm, n_out, region,
                                        lane);
        });
    }
}

template <int BM, int NW, int OCC, int NB, int WT, int EPI, int OUT>
hipError_t launch_blocks_product(const GemmArgs &args, hipStream_t stream) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    GemmArgs p = args;
    p.tiles_m = (p.M + BM - 1) / BM;
    const int slabs = GLU ? (p.glu_half + 31) / 32 : (p.N + 63) / 64;
    constexpr int SLABS_PER_WG = NB == 2 ? NW : NW / 2;
    p.tiles_n = (slabs + SLABS_PER_WG - 1) / SLABS_PER_WG;
    const int blocks = p.tiles_m * p.tiles_n;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_blocks_kernel<BM, NW, OCC, NB, WT, EPI, OUT>), dim3(blocks), dim3(64 * NW), 0, stream, p);
    return hipGetLastError();
}

}  // namespace blk
}  // namespace sq8
