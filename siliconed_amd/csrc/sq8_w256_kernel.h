// sq8_w256_kernel.h — the weight-direct GEMM in 256 × 256 tiles, one workgroup of four waves per CU:
// the large-product kernel (C1's up-projection: 768 tiles, three rounds on 256 CUs). The same kernel in
// 224 × 256 tiles (BM = 224: 7 row blocks a wave) serves products whose 256-row tiles would leave the last
// round partly empty (C1's down-projection: 228 tiles in one round against 192).
//
// Arithmetic as the other kernels (Sources/Siliconed/TensorGEMM.swift:124-135, :173-179):
// C = act(s ⊙ (A·q) + b), exact bf16 × code products, fp32 sums, scale after the sum, bias after the
// scale, activation last; every output has the same bits as the 128-row kernel's (the same MFMA
// sequence over K for every sum).
//
// Why this shape. Each code is widened to bf16 once per tile row of the activation: 256-row tiles
// halve the widening (1.5 VALU operations per MFMA instead of 3) against the 128-row tiles of the
// two-workgroup kernel, and the single workgroup per CU owns the whole register file (accumulators
// in AGPRs: 2 × 8 blocks of 32 × 32 per wave). Nothing then covers a wave's stalls but its own
// pipelining, so everything is issued ahead:
//   * wave w owns weight slab w (64 columns) for all 256 rows; its codes go HBM → registers, four
//     K steps deep (4 × 16 bytes per lane per step), widened one MFMA sub-step ahead;
//   * the activation goes global → LDS by direct loads into a 4-stage ring of [256][64] bf16 tiles
//     (128-byte rows, 16-byte chunks XOR-swizzled by (r ^ r>>3) & 7), three steps ahead;
//   * both streams are issued a little per MFMA sub-step (two activation loads and one weight load
//     each), never in bursts: a burst of loads stalls the issuing wave once the address queue is
//     full, and with one wave per SIMD that stall is an idle matrix core;
//   * the fragments of step s+1's first sub-step are read during step s's last, so a step starts on
//     MFMAs; one barrier per step (stage reuse and the landed loads of all waves).
// Per step s (stage and raw buffer U = s mod 4), sub-step ks: read fragments (ks+1, or s+1's 0),
// widen its codes, issue activation rows 2ks, 2ks+1 of step s+3 and weight load ks of step s+3,
// 16 MFMAs; at the end: wait until step s+2's loads have landed (12 younger loads may fly), barrier.
//
// The tile's scales and biases are fetched into LDS by direct loads at the start (they land with
// the prologue); the epilogue reads them there. Epilogue: bf16 out with no activation or GELU through the
// wave's LDS region as full 128-byte row segments (slab_epilogue_bf16); the GLU epilogues (a slab is then
// 32 columns of each half: the packed GLU layout), fp32 outputs and the gated residual 32 × 32 block by
// block (store_block).
#pragma once

#include "sq8_wdirect_kernel.h"

namespace sq8 {
namespace wd {

template <int WT, int WL, int EPI, int OUT, int BM = 256>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
gemm_w256_kernel(const GemmArgs p) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr bool SLAB = (EPI == EPI_NONE || EPI == EPI_GELU) && OUT == OUT_BF16;
    static_assert(EPI != EPI_RESIDUAL || OUT == OUT_F32, "the residual stream is fp32");
    static_assert(BM == 256 || BM == 224, "256- or 224-row tiles");
    constexpr int NW = 4, FM = BM / 32, NAS = 4;
    constexpr int SA = BM * 128;             // bytes per activation stage
    constexpr int A_PER_WAVE = BM / 8 / NW;  // 1 KB direct loads per wave per step (8 or 7)
    constexpr int SB_OFF = NAS * SA;         // the tile's scales (1 KB) then biases (1 KB)
    constexpr int LDS_BYTES = SB_OFF + 2048;
    static_assert(NW * BM * 128 <= SB_OFF, "the epilogue regions lie over the stages");

    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
    // An AGPR operand: the compiler then places the accumulators in AGPRs (512 registers a wave).
    asm volatile("; accumulators in AGPRs %0" ::"a"(0.0f));

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tm, tn;
    kern::tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM;
    const int slab = tn * NW + wave;
    const kern::gbytes Ag = (kern::gbytes)p.a;
    const kern::gbytes Wg = (kern::gbytes)p.w;
    const int KT = p.kt;

    // Scales (wave 0) and biases (wave 1) of the tile's 256 weight columns, 16 bytes a lane, first in
    // issue order so that the prologue's wait covers them (GLU: lanes 0–31 the first half's 128
    // columns, lanes 32–63 the second half's). Columns past the end read the last four (never used).
    if (wave < 2) {
        const float *src = wave == 0 ? (p.scale_per_col ? p.scale : nullptr) : p.bias;
        if (src != nullptr) {
            const int col = GLU ? min(tn * 128 + (lane & 31) * 4, p.glu_half - 4) + (lane >> 5) * p.glu_half
                                : min(tn * 256 + lane * 4, p.N - 4);
            __builtin_amdgcn_global_load_lds((glb_ptr)(src + col), (lds_ptr)(lds + SB_OFF + wave * 1024), 16, 0, 0);
        }
    }

    // Activation direct loads: block b = wave + NW·i of 8 rows, lane → row 8b + lane/8, chunk lane%8.
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
    // In the K loop the same loads go through a buffer resource, the step's offset in a scalar register
    // (248.1 against 251.5 µs on C1 with the fragment offsets below, the same bits).
    const i32x4 a_rsrc = buffer_rsrc(p.a);
    auto issue_a2 = [&](int t, auto stage, auto part) {  // rows blocks 2·part, 2·part + 1 (those there are)
        constexpr int S = decltype(stage)::value, Q = decltype(part)::value;
        const int soff = __builtin_amdgcn_readfirstlane((int)((uint32_t)min(t, KT - 1) * (BK * 2)));
        static_for<2 * Q, 2 * Q + 2>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            if constexpr (i < A_PER_WAVE)
                raw_buffer_load_lds(a_rsrc, (lds_u32)(lds + S * SA + (wave + NW * i) * 1024), 16, (int)a_goff[i], soff, 0,
                                    0);
        });
    };

    uint32_t w_off[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w_off[j] = w_offset<WL, GLU>(p, slab, j, lane);
    const uint32_t w_step = WL == W_PACKED ? 4096 : BK;
    u32x4 raw[4][4];  // [K step mod 4][load j]
    auto issue_w = [&](int t, auto buf) {
        constexpr int B = decltype(buf)::value;
        const kern::gbytes base = Wg + (uint32_t)weight_step(p, min(t, KT - 1)) * w_step;
#pragma unroll
        for (int j = 0; j < 4; ++j) raw[B][j] = kern::gld<u32x4>(base, w_off[j]);
    };
    auto issue_w1 = [&](int t, auto buf, auto jc) {
        constexpr int B = decltype(buf)::value, J = decltype(jc)::value;
        const kern::gbytes base = Wg + (uint32_t)weight_step(p, min(t, KT - 1)) * w_step;
        raw[B][J] = kern::gld<u32x4>(base, w_off[J]);
    };

    const int h = lane >> 5;
    int xo[2][4];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) xo[par][ks] = swz(32 * par + (lane & 31), 4 * h + ks) - 32 * 128 * par;
    // The same offsets 64 KB up: fragments of the stages past 64 KB then take their stage and row-block
    // offset as the read's 16-bit immediate instead of a vector add each.
    int xoh[2][4];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            xoh[par][ks] = xo[par][ks] + 65536;
            asm volatile("" : "+v"(xoh[par][ks]));
        }

    f32x16 acc[2][FM];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[b][bm][r] = 0.0f;

    bf16x8 wk[2][2];   // widened codes [buffer][32-column block]
    bf16x8 xf[2][FM];  // activation fragments [buffer][32-row block]
    auto widen_ks = [&](auto rb, auto kc, auto dst) {
        constexpr int R = decltype(rb)::value, ks = decltype(kc)::value, D = decltype(dst)::value;
        static_for<0, 2>([&](auto bc) {
            constexpr int b = decltype(bc)::value;
            const u32x4 &r = raw[R][2 * b + (ks >> 1)];
            wk[D][b] = widen8<WT>(r[2 * (ks & 1)], r[2 * (ks & 1) + 1]);
        });
    };
    auto read_x = [&](auto stc, auto kc, auto dst) {
        constexpr int S = decltype(stc)::value, ks = decltype(kc)::value, D = decltype(dst)::value;
        static_for<0, FM>([&](auto bmc) {
            constexpr int bm = decltype(bmc)::value;
            if constexpr (S * SA + 32 * 128 * bm >= 65536)
                xf[D][bm] = kern::lds_load_frag(lds + S * SA + 32 * 128 * bm - 65536, xoh[bm & 1][ks]);
            else
                xf[D][bm] = kern::lds_load_frag(lds + S * SA + 32 * 128 * bm, xo[bm & 1][ks]);
        });
    };
    // Row block outer, column block inner: each activation fragment feeds two MFMAs back to back and is then
    // free (C1: 1.7 % fewer K-loop cycles than column block outer, same sums).
    auto mfma_ks = [&](auto src) {
        constexpr int D = decltype(src)::value;
        static_for<0, FM>([&](auto bmc) {
            constexpr int bm = decltype(bmc)::value;
            static_for<0, 2>([&](auto bc) {
                constexpr int b = decltype(bc)::value;
                acc[b][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wk[D][b], xf[D][bm], acc[b][bm], 0, 0, 0);
            });
        });
    };
    // Sub-step Q's schedule: 2·FM MFMAs, between them the next fragments' FM LDS reads, the next codes'
    // 24 widening operations and the sub-step's global loads (two activation rows blocks, those there
    // are, and one weight load).
    auto interleave = [&](auto part) {
        constexpr int Q = decltype(part)::value;
        constexpr int VMEM = (2 * Q < A_PER_WAVE) + (2 * Q + 1 < A_PER_WAVE) + 1;
        static_for<0, 2 * FM>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if constexpr (i < FM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if constexpr (i < 12) __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
            if constexpr ((i == 1 && VMEM > 0) || (i == 5 && VMEM > 1) || (i == 9 && VMEM > 2))
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        });
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;

    // Prologue: A(0..2), W(0..2); wait until all but step 2's loads (12) have landed.
    issue_a(0, I0{});
    issue_w(0, I0{});
    issue_a(1, I1{});
    issue_w(1, I1{});
    issue_a(2, I2{});
    issue_w(2, I2{});
    wait_vmcnt<A_PER_WAVE + 4>();
    step_barrier();
    read_x(I0{}, I0{}, I0{});
    widen_ks(I0{}, I0{}, I0{});

    auto step = [&](int s, auto uc) {
        constexpr int U = decltype(uc)::value;
        constexpr int N1 = (U + 1) % 4, N3 = (U + 3) % 4;
        using SU = std::integral_constant<int, U>;
        using S3 = std::integral_constant<int, N3>;
        static_for<0, 4>([&](auto kc) {
            constexpr int ks = decltype(kc)::value;
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (ks < 3) {
                read_x(SU{}, std::integral_constant<int, ks + 1>{}, std::integral_constant<int, (ks + 1) & 1>{});
                widen_ks(SU{}, std::integral_constant<int, ks + 1>{}, std::integral_constant<int, (ks + 1) & 1>{});
            } else {
                // Step s+1's first sub-step: its stage landed and was published by the previous barrier,
                // its codes by the previous step's wait.
                read_x(std::integral_constant<int, N1>{}, I0{}, I0{});
                widen_ks(std::integral_constant<int, N1>{}, I0{}, I0{});
            }
            // Stage (s+3) mod 4 was last read in step s−1 (before the previous barrier); raw buffer
            // (s+3) mod 4 was last widened in step s−1.
            issue_a2(s + 3, S3{}, kc);
            issue_w1(s + 3, S3{}, kc);
            mfma_ks(std::integral_constant<int, ks & 1>{});
            interleave(kc);
            __builtin_amdgcn_sched_barrier(0);
        });
        wait_vmcnt<A_PER_WAVE + 4>();
        step_barrier();
    };
    int s = 0;
    for (; s + 4 <= KT; s += 4) {
        step(s, I0{});
        step(s + 1, I1{});
        step(s + 2, I2{});
        step(s + 3, I3{});
    }
    if (s < KT) step(s, I0{});
    if (s + 1 < KT) step(s + 1, I1{});
    if (s + 2 < KT) step(s + 2, I2{});

    // Every wave's last (clamped) loads have landed before any wave writes its region over the stages.
    wait_vmcnt<0>();
    step_barrier();

    const int n_out = GLU ? p.glu_half : p.N;
    const int col0 = GLU ? slab * 32 : slab * 64;
    if (col0 >= n_out) return;  // a last tile's waves past the weight's columns
    const bool has_bias = p.bias != nullptr;
    ColParams cp[2];
    static_for<0, 2>([&](auto bc) {
        constexpr int b = decltype(bc)::value;
        static_for<0, 4>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            // Block b's columns in the LDS copy (GLU: block b is half b's 32 columns of the slab).
            const int lc = (GLU ? 128 * b + wave * 32 : wave * 64 + 32 * b) + 8 * g + 4 * h;
            const f32x4 sv = p.scale_per_col ? *reinterpret_cast<const f32x4 *>(lds + SB_OFF + lc * 4)
                                             : f32x4{p.scale[0], p.scale[0], p.scale[0], p.scale[0]};
            const f32x4 bv = has_bias ? *reinterpret_cast<const f32x4 *>(lds + SB_OFF + 1024 + lc * 4) : f32x4{0, 0, 0, 0};
            static_for<0, 4>([&](auto ec) {
                constexpr int e = decltype(ec)::value;
                cp[b].s[g][e] = sv[e];
                cp[b].b[g][e] = bv[e];
            });
        });
    });
    if constexpr (SLAB) {
        slab_epilogue_bf16<FM, EPI>(p, acc, cp, has_bias, m0, col0, lds + wave * (BM * 128), lane);
    } else {
        constexpr int REGION = 32 * (32 * (OUT == OUT_BF16 ? 2 : 4) + 16);
        uint8_t *region = lds + wave * REGION;
        ResidualPre pre[2];
        if constexpr (EPI == EPI_RESIDUAL && !GLU) load_residual(p, col0, m0, n_out, lane, pre[0]);
        static_for<0, FM>([&](auto bmc) {
            constexpr int bm = decltype(bmc)::value;
            if constexpr (GLU) {
                store_block<EPI, OUT>(p, acc[0][bm], cp[0], acc[1][bm], cp[1], has_bias, col0, m0 + 32 * bm, n_out,
                                      region, lane);
            } else if constexpr (EPI == EPI_RESIDUAL) {
                // The next block's residual operands load while this one is staged and stored.
                static_for<0, 2>([&](auto bc) {
                    constexpr int b = decltype(bc)::value, j = 2 * bm + b;
                    if constexpr (j + 1 < 2 * FM)
                        load_residual(p, col0 + 32 * ((j + 1) & 1), m0 + 32 * ((j + 1) >> 1), n_out, lane, pre[(j + 1) & 1]);
                    if (col0 + 32 * b < n_out)
                        store_block<EPI, OUT>(p, acc[b][bm], cp[b], acc[b][bm], cp[b], has_bias, col0 + 32 * b, m0 + 32 * bm,
                                              n_out, region, lane, &pre[j & 1]);
                });
            } else {
                static_for<0, 2>([&](auto bc) {
                    constexpr int b = decltype(bc)::value;
                    if (col0 + 32 * b < n_out)
                        store_block<EPI, OUT>(p, acc[b][bm], cp[b], acc[b][bm], cp[b], has_bias, col0 + 32 * b, m0 + 32 * bm,
                                              n_out, region, lane);
                });
            }
        });
    }
}

// True when the 256 × 256 kernel runs this product: whole 64-column slabs (GLU: whole 32-column
// slabs of each half) and 16-byte scale/bias loads; for the slab epilogue (bf16 out, no activation or
// GELU) also slabs that each lie in one output (and one head) and 16-byte stores. The fp32 route's three
// parts along K (kt_w > 0) face the weight's steps in turn (weight_step).
inline bool w256_fits(const GemmArgs &p, int epi, int out) {
    if (!p.sb_vec) return false;
    if (p.glu_half > 0 ? p.glu_half % 32 != 0 : p.N % 64 != 0) return false;
    if (epi == EPI_RESIDUAL && out != OUT_F32) return false;
    if ((epi == EPI_NONE || epi == EPI_GELU) && out == OUT_BF16)
        return p.split % 64 == 0 && p.head_dim % 64 == 0 && p.c_vec16;
    return true;
}

template <int WT, int WL, int BM = 256>
hipError_t launch_w256(const GemmArgs &args, int epi, int out, hipStream_t stream) {
    GemmArgs p = args;
    const bool glu = epi == EPI_SILU_GLU || epi == EPI_SITU_GLU;
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = glu ? (p.glu_half / 32 + 3) / 4 : (p.N + 255) / 256;
    const int blocks = p.tiles_m * p.tiles_n;
    if (blocks == 0) return hipSuccess;
#define SQ8_CASE(E, O)                                                                                   \
    if (epi == E && out == O) {                                                                          \
        hipLaunchKernelGGL((gemm_w256_kernel<WT, WL, E, O, BM>), dim3(blocks), dim3(256), 0, stream, p); \
        return hipGetLastError();                                                                        \
    }
    SQ8_CASE(EPI_NONE, OUT_BF16)
    SQ8_CASE(EPI_GELU, OUT_BF16)
    SQ8_CASE(EPI_NONE, OUT_F32)
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
