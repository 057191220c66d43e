// sq8_i8_kernel.h — the W8A8 product on gfx950: the activation's int8 codes (sq8_w8a8.hip) times
// the weight's int8 codes on v_mfma_i32_32x32x32_i8, int32 sums (exact: |Σ| < 2^31 for k < 2^17),
// then C = act(float(acc) · (s_x[row] · s_w[col]) + b) — ComfyUI's int8_linear as the reference
// runs it (Sources/Siliconed/TensorGEMMInt8.swift:4-37: `linear_i8i8`, then `scale_products`
// :133-140), the scale product formed first, the bias and the activation fused after it.
//
// The weight-direct structure (sq8_wdirect_kernel.h) with integer operands: each wave owns a
// 64-column slab and streams its codes from HBM straight into registers, where they are the MFMA's
// first operand as they are — no widening; the activation tile goes through LDS. A K step is 128
// codes: two steps of the packed layout (per lane and load j, 16 bytes = k ∈ [32h + 16·(j & 1), +16)
// of a 64-code step, h = lane ÷ 32), whose k sets the activation fragments match (row r of the A
// stage is 128 codes; sub-step s of lane half h reads its 16 bytes at 64·(s >> 1) + 32h + 16·(s & 1)).
//
// Activation: a 2- or 3-stage LDS ring of [BM][128] int8 tiles filled by direct global→LDS loads, rows
// XOR-swizzled as the bf16 kernel's. The activation rows must hold whole steps: k_pad = a multiple
// of 128 codes, zero past k (the quantization pass writes them so); the weight's last packed step is
// reused past its end when the packed steps are odd (times zero codes).
//
// Per step t (two workgroups per CU, ≤ 256 registers a wave): issue A(t+NA−1), the MFMAs of the four
// sub-steps with the fragments of s+1 read during s, W(t+2)'s first packed step into raw[t&1] once
// sub-step 1 has read it, its second once sub-step 3 has; wait until A(t+1) and W(t+1) landed;
// barrier.
#pragma once

#include "sq8_wdirect_kernel.h"

namespace sq8 {
namespace wd {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// Byte offset (packed step 0) of the 16 codes lane `lane`, load j (block j>>1, half j&1) reads for
// slab `slab`; [N, K]: the row of the column. Past the last column or slab: the last one (results
// never stored, reads kept inside the buffer).
template <int WL, bool GLU>
__device__ __forceinline__ uint32_t w_offset_i8(const GemmArgs &p, int slab, int j, int lane) {
    if constexpr (WL == W_PACKED) {
        const int slabs = GLU ? (p.glu_half + 31) / 32 : (p.N + 63) / 64;
        const int s = slab < slabs ? slab : slabs - 1;
        return (uint32_t)(((int64_t)s * p.kt_w * 4 + j) * 1024 + lane * 16);
    } else {
        const int b = j >> 1, c = j & 1, h = lane >> 5, nl = lane & 31;
        int n;
        if constexpr (GLU) {
            const int out = slab * 32 + nl;
            n = out < p.glu_half ? out + b * p.glu_half : (p.glu_half - 1) + b * p.glu_half;
        } else {
            n = slab * 64 + b * 32 + nl;
            n = n < p.N ? n : p.N - 1;
        }
        return (uint32_t)((int64_t)n * p.ldw + 32 * h + 16 * c);
    }
}

// NA: activation stages in the LDS ring (2: A(t+1) loads during step t; 3: A(t+2), one more step of
// memory latency covered, 3·BM·128 bytes of LDS).
template <int BM, int NW, int WL, int EPI, int OUT, int NA>
__global__ void __attribute__((amdgpu_flat_work_group_size(64 * NW, 64 * NW), amdgpu_waves_per_eu(2, 2)))
gemm_i8_kernel(const GemmArgs p) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int FM = BM / 32;
    constexpr int SA = BM * 128;          // bytes per A stage: BM rows of 128 codes
    constexpr int A_BLOCKS = BM / 8;      // 1 KB (8-row) blocks per stage
    constexpr int A_PER_WAVE = A_BLOCKS / NW;
    static_assert(NA == 2 || NA == 3, "two or three activation stages");
    static_assert(A_BLOCKS % NW == 0, "the activation blocks split evenly over the waves");
    static_assert(2 * A_PER_WAVE + 16 < 64, "vmcnt budget");
    constexpr int REGION = 32 * (32 * (OUT == OUT_BF16 ? 2 : 4) + 16);
    static_assert(NW * REGION <= 2 * SA, "the epilogue regions fit in the A stages");
    // Loads a wave may leave in flight at the end of step t, A(t+1) and W(t+1) landed: W(t+2), and with
    // three stages A(t+2) (issued in step t, before W(t+2)).
    constexpr int IN_FLIGHT = 8 + (NA == 3 ? A_PER_WAVE : 0);

    __shared__ __attribute__((aligned(1024))) uint8_t lds[NA * SA];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tm, tn;
    kern::tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM;
    const int slab = tn * NW + wave;
    const kern::gbytes Ag = (kern::gbytes)p.a;
    const kern::gbytes Wg = (kern::gbytes)p.w;
    const int KT = p.kt;     // steps of 128
    const int KW = p.kt_w;   // packed steps of 64

    // ---- activation loads: wave block b = wave + NW·i, lane → row 8b + (lane>>3), chunk lane&7 ----
    uint32_t a_goff[A_PER_WAVE];
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i) {
        const int b = wave + NW * i;
        const int r = 8 * b + (lane >> 3);
        const int lc = (lane & 7) ^ ((r ^ (r >> 3)) & 7);
        const int row = min(m0 + r, p.M - 1);
        a_goff[i] = (uint32_t)((int64_t)row * p.lda) + lc * 16;
    }
    auto issue_a = [&](int t, auto stage) {
        constexpr int S = decltype(stage)::value;
        const kern::gbytes base = Ag + (uint32_t)min(t, KT - 1) * 128;
#pragma unroll
        for (int i = 0; i < A_PER_WAVE; ++i)
            __builtin_amdgcn_global_load_lds((glb_ptr)(base + a_goff[i]), (lds_ptr)(lds + S * SA + (wave + NW * i) * 1024),
                                             16, 0, 0);
    };

    // ---- weight loads: per step, packed steps 2t and 2t+1, 4 × 16 bytes per lane each --------------
    uint32_t w_off[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w_off[j] = w_offset_i8<WL, GLU>(p, slab, j, lane);
    const uint32_t w_step = WL == W_PACKED ? 4096 : 64;
    u32x4 raw[2][8];
    auto issue_w = [&](int t, auto buf, auto half) {
        constexpr int B = decltype(buf)::value, H = decltype(half)::value;
        const kern::gbytes base = Wg + (uint32_t)min(2 * t + H, KW - 1) * w_step;
#pragma unroll
        for (int j = 0; j < 4; ++j) raw[B][4 * H + j] = kern::gld<u32x4>(base, w_off[j]);
    };

    // Fragment read offsets: sub-step s, row 32·bm + (lane & 31), logical chunk 4·(s >> 1) + 2h + (s & 1).
    const int h = lane >> 5;
    int xo[2][4];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
        for (int s = 0; s < 4; ++s) xo[par][s] = swz(32 * par + (lane & 31), 4 * (s >> 1) + 2 * h + (s & 1)) - 32 * 128 * par;

    i32x16 acc[2][FM];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[b][bm][r] = 0;

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;

    // Step t: the weight's register buffer P = t mod 2, the activation's stage S = t mod NA.
    auto step = [&](int t, auto par, auto stage) {
        constexpr int P = decltype(par)::value;
        constexpr int S = decltype(stage)::value;
        i32x4 xf[2][FM];
        auto read_x = [&](auto sc) {
            constexpr int s = decltype(sc)::value;
            static_for<0, FM>([&](auto bmc) {
                constexpr int bm = decltype(bmc)::value;
                xf[s & 1][bm] = __builtin_bit_cast(i32x4, kern::lds_load_frag(lds + S * SA + 32 * 128 * bm, xo[bm & 1][s]));
            });
        };
        __builtin_amdgcn_sched_barrier(0);
        read_x(I0{});
        // Into the stage read during step t − 1 (the barrier that ended it saw every wave's reads).
        issue_a(t + NA - 1, std::integral_constant<int, (S + NA - 1) % NA>{});
        static_for<0, 4>([&](auto sc) {
            constexpr int s = decltype(sc)::value;
            if constexpr (s < 3) read_x(std::integral_constant<int, s + 1>{});
            static_for<0, FM>([&](auto bmc) {  // row block outer: a fragment's MFMAs back to back
                constexpr int bm = decltype(bmc)::value;
                static_for<0, 2>([&](auto bc) {
                    constexpr int b = decltype(bc)::value;
                    const i32x4 w = __builtin_bit_cast(i32x4, raw[P][4 * (s >> 1) + 2 * b + (s & 1)]);
                    acc[b][bm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(w, xf[s & 1][bm], acc[b][bm], 0, 0, 0);
                });
            });
            if constexpr (s < 3) {
                static_for<0, 2 * FM>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if constexpr (i < FM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                });
            }
            __builtin_amdgcn_sched_barrier(0);
            // The first packed step of raw[P] is read by sub-steps 0 and 1, the second by 2 and 3; the
            // A loads stay ahead of these in issue order (the vmcnt counts rely on it).
            if constexpr (s == 1) issue_w(t + 2, par, I0{});
            if constexpr (s == 3) issue_w(t + 2, par, I1{});
            __builtin_amdgcn_sched_barrier(0);
        });
        wait_vmcnt<IN_FLIGHT>();
        step_barrier();
    };

    // Prologue: A(0) → stage 0, W(0) → raw[0], [A(1) → stage 1,] W(1) → raw[1]; A(0) and W(0) landed.
    issue_a(0, I0{});
    issue_w(0, I0{}, I0{});
    issue_w(0, I0{}, I1{});
    if constexpr (NA == 3) issue_a(1, I1{});
    issue_w(1, I1{}, I0{});
    issue_w(1, I1{}, I1{});
    wait_vmcnt<IN_FLIGHT>();
    step_barrier();

    using I2 = std::integral_constant<int, 2>;
    int t = 0;
    if constexpr (NA == 2) {
        for (; t + 1 < KT; t += 2) {
            step(t, I0{}, I0{});
            step(t + 1, I1{}, I1{});
        }
        if (t < KT) step(t, I0{}, I0{});
    } else {
        // (t mod 2, t mod 3) repeats every six steps.
        for (; t + 5 < KT; t += 6) {
            step(t, I0{}, I0{});
            step(t + 1, I1{}, I1{});
            step(t + 2, I0{}, I2{});
            step(t + 3, I1{}, I0{});
            step(t + 4, I0{}, I1{});
            step(t + 5, I1{}, I2{});
        }
        if (t < KT) step(t, I0{}, I0{});
        if (t + 1 < KT) step(t + 1, I1{}, I1{});
        if (t + 2 < KT) step(t + 2, I0{}, I2{});
        if (t + 3 < KT) step(t + 3, I1{}, I0{});
        if (t + 4 < KT) step(t + 4, I0{}, I1{});
    }

    const bool has_bias = p.bias != nullptr;
    const int n_out = GLU ? p.glu_half : p.N;
    ColParams cp[2];
    static_for<0, 2>([&](auto bc) {
        constexpr int b = decltype(bc)::value;
        load_col_params(p, cp[b], GLU ? slab * 32 : slab * 64 + 32 * b, GLU && b == 1 ? p.glu_half : 0, n_out, lane);
    });
    float sxr[FM];
#pragma unroll
    for (int bm = 0; bm < FM; ++bm) sxr[bm] = p.sx[min(m0 + 32 * bm + (lane & 31), p.M - 1)];
    wait_vmcnt<0>();
    step_barrier();

    // ---- epilogue: float(acc) · (s_x · s_w), then bias and activation (store_block) ----------------
    uint8_t *region = lds + wave * REGION;
    ResidualPre pre[2];
    if constexpr (EPI == EPI_RESIDUAL && !GLU) load_residual(p, slab * 64, m0, n_out, lane, pre[0]);
    static_for<0, FM>([&](auto bmc) {
        constexpr int bm = decltype(bmc)::value;
        ColParams cq[2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    cq[b].s[g][e] = sxr[bm] * cp[b].s[g][e];
                    cq[b].b[g][e] = cp[b].b[g][e];
                }
        f32x16 xf32[2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) xf32[b][r] = (float)acc[b][bm][r];
        static_for<0, GLU ? 1 : 2>([&](auto bc) {
            constexpr int b = decltype(bc)::value;
            const int col0 = GLU ? slab * 32 : slab * 64 + 32 * b;
            if constexpr (EPI == EPI_RESIDUAL && !GLU) {
                // The next block's residual operands load while this one is staged and stored.
                constexpr int j = 2 * bm + b;
                if constexpr (j + 1 < 2 * FM)
                    load_residual(p, slab * 64 + 32 * ((j + 1) & 1), m0 + 32 * ((j + 1) >> 1), n_out, lane, pre[(j + 1) & 1]);
                if (col0 < n_out)
                    store_block<EPI, OUT>(p, xf32[b], cq[b], xf32[b], cq[b], has_bias, col0, m0 + 32 * bm, n_out, region,
                                          lane, &pre[j & 1]);
            } else if (col0 < n_out) {
                store_block<EPI, OUT>(p, xf32[b], cq[b], xf32[GLU ? 1 : b], cq[GLU ? 1 : b], has_bias, col0, m0 + 32 * bm,
                                      n_out, region, lane);
            }
        });
    });
}

template <int BM, int NW, int WL, int EPI, int OUT, int NA>
hipError_t launch_i8(const GemmArgs &args, hipStream_t stream) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    GemmArgs p = args;
    p.tiles_m = (p.M + BM - 1) / BM;
    const int slabs = GLU ? (p.glu_half + 31) / 32 : (p.N + 63) / 64;
    p.tiles_n = (slabs + NW - 1) / NW;
    const int blocks = p.tiles_m * p.tiles_n;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_i8_kernel<BM, NW, WL, EPI, OUT, NA>), dim3(blocks), dim3(64 * NW), 0, stream, p);
    return hipGetLastError();
}

template <int BM, int NW, int WL, int NA>
hipError_t dispatch_i8(const GemmArgs &p, int epi, int out, hipStream_t stream) {
#define SQ8_CASE(E, O)                                                                            \
    if (epi == E && out == O) return launch_i8<BM, NW, WL, E, O, NA>(p, stream);
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
