// sq8_wdirect_kernel.h — the weight-direct gfx950 GEMM: each wave owns a 64-column slab of the
// weight and streams its 8-bit codes from HBM straight into registers, widening them to bf16 there
// while the previous K step's MFMAs run; only the activation tile goes through LDS.
//
// Arithmetic as the other kernels (Sources/Siliconed/TensorGEMM.swift:124-135, :173-179):
// C = act(s ⊙ (A·q) + b), exact bf16 × code products, fp32 sums, scale after the sum, bias after
// the scale, activation last.
//
// Tile BM × 64·NW, NW waves of 64 lanes; wave w computes all BM rows × its 64 virtual columns as
// 2 × (BM/32) blocks of v_mfma_f32_32x32x16_bf16 (the code the first operand, the activation the
// second: each lane ends with 4 consecutive output columns of a row).
//
// K order inside a 64-step: MFMA sub-step ks of lane half h (lanes 32h..32h+31) takes
// k ∈ [32h + 8ks, 32h + 8ks + 8). Any fixed permutation of K inside the step gives the same sums;
// this one makes a lane's codes for the whole step 32 contiguous bytes (two 16-byte loads per
// 32-column block), and its activation chunks 8-bf16 pieces of one LDS row.
//
// Activation: a 2-stage LDS ring of [BM][64] bf16 tiles filled by direct global→LDS loads
// (global_load_lds_dwordx4: each wave writes 1 KB = 8 rows per load, no VGPR, no ds_write), rows
// of 128 bytes whose 16-byte chunks are XOR-swizzled (chunk ^ ((r ^ r>>3) & 7)) so the fragment
// reads of 16 consecutive rows hit distinct banks.
//
// Pipeline per K step t (all loads issued ahead, the waits explicit):
//   issue A(t+1) → LDS stage (t+1)&1, issue W(t+2) → raw[t&1]        (clamped past the end)
//   wait W(t+1)                                                        vmcnt(A loads + 4)
//   MFMAs of step t  ∥  widen raw[(t+1)&1] → fragments of step t+1
//   wait A(t+1), barrier                                                vmcnt(4)
//
// Weight layouts: [N, K] (nn.Linear: row-strided 16-byte loads) or the packed layout of
// sq8_pack_weight — per 64-column slab, per K step, per load j, per lane, 16 bytes — in which each
// wave load is one contiguous kilobyte.
#pragma once

#include "sq8_gemm_kernel.h"

namespace sq8 {
namespace wd {

constexpr int BK = 64;

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef const __attribute__((address_space(1))) void *glb_ptr;

__device__ __forceinline__ int swz(int r, int lc) { return r * 128 + ((lc ^ ((r ^ (r >> 3)) & 7)) << 4); }

// s_waitcnt with only the vector-memory counter constrained (expcnt and lgkmcnt at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier ordering LDS only: the release/acquire fences are restricted to the local
// address space, so loads still in flight to registers (the weight prefetch) are not drained.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 8 codes (two dwords) → one MFMA operand of 8 bf16, exactly.
template <int WT>
__device__ __forceinline__ bf16x8 widen8(uint32_t d0, uint32_t d1) {
    uint32_t o0, o1, o2, o3;
    widen4<WT>(d0, o0, o1);
    widen4<WT>(d1, o2, o3);
    return __builtin_bit_cast(bf16x8, u32x4{o0, o1, o2, o3});
}

// Byte offset of the 16 bytes lane `lane`, load j (block j>>1, half j&1) of K step 0 reads for
// virtual 64-column slab `slab`, or −1 when the column is past the edge (zero-filled instead).
template <int WL, bool GLU>
__device__ __forceinline__ int64_t w_offset(const GemmArgs &p, int slab, int j, int lane) {
    if constexpr (WL == W_PACKED) {
        return ((int64_t)slab * p.kt * 4 + j) * 1024 + lane * 16;
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
        return (int64_t)n * p.ldw + 32 * h + 16 * c;
    }
}

template <int BM, int NW, int WT, int WL, int EPI, int OUT>
__global__ void __attribute__((amdgpu_flat_work_group_size(64 * NW, 64 * NW), amdgpu_waves_per_eu(1, 1)))
gemm_wd_kernel(const GemmArgs p) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int FM = BM / 32;                      // 32-row blocks per wave
    constexpr int SA = BM * 128;                     // bytes per A stage
    constexpr int A_BLOCKS = BM / 8;                 // 1 KB (8-row) blocks per A stage
    constexpr int A_PER_WAVE = (A_BLOCKS + NW - 1) / NW;
    constexpr bool A_EVEN = A_BLOCKS % NW == 0;
    // Every wave issues the same number of activation loads, so one vmcnt value fits them all.
    static_assert(A_EVEN, "the activation blocks split evenly over the waves");
    static_assert(A_PER_WAVE + 4 < 64, "vmcnt budget");

    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * SA];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tm, tn;
    kern::tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM;
    const int slab = tn * NW + wave;
    const kern::gbytes Ag = (kern::gbytes)p.a;
    const kern::gbytes Wg = (kern::gbytes)p.w;
    const int KT = p.kt;

    // ---- activation loads: wave block b = wave + NW·i, lane → row 8b + (lane>>3), chunk lane&7 ----
    uint32_t a_goff[A_PER_WAVE];
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i) {
        const int b = min(wave + NW * i, A_BLOCKS - 1);
        const int r = 8 * b + (lane >> 3);
        const int lc = (lane & 7) ^ ((r ^ (r >> 3)) & 7);
        const int row = min(m0 + r, p.M - 1);
        a_goff[i] = (uint32_t)((int64_t)row * p.lda * 2) + lc * 16;
    }
    auto issue_a = [&](int t, auto stage) {
        constexpr int S = decltype(stage)::value;
        const uint32_t k_bytes = (uint32_t)min(t, KT - 1) * (BK * 2);
#pragma unroll
        for (int i = 0; i < A_PER_WAVE; ++i) {
            if (A_EVEN || wave + NW * i < A_BLOCKS) {
                __builtin_amdgcn_global_load_lds((glb_ptr)(Ag + a_goff[i] + k_bytes),
                                                 (lds_ptr)(lds + S * SA + (wave + NW * i) * 1024), 16, 0, 0);
            }
        }
    };

    // ---- weight loads: 4 × 16 bytes per lane per K step --------------------------------------------
    int64_t w_off[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w_off[j] = w_offset<WL, GLU>(p, slab, j, lane);
    const int64_t w_step = WL == W_PACKED ? 4096 : BK;
    u32x4 raw[2][4];
    auto issue_w = [&](int t, auto buf) {
        constexpr int B = decltype(buf)::value;
        const int64_t k_off = (int64_t)min(t, KT - 1) * w_step;
#pragma unroll
        for (int j = 0; j < 4; ++j) raw[B][j] = *(const __attribute__((address_space(1))) u32x4 *)(Wg + w_off[j] + k_off);
    };

    // ---- fragments -----------------------------------------------------------------------------------
    bf16x8 wf[2][2][4];  // [buffer][block][ks]
    auto widen_w = [&](auto src, auto dst) {
        constexpr int S = decltype(src)::value, D = decltype(dst)::value;
        static_for<0, 2>([&](auto bc) {
            constexpr int b = decltype(bc)::value;
            static_for<0, 4>([&](auto kc) {
                constexpr int ks = decltype(kc)::value;
                const u32x4 &r = raw[S][2 * b + (ks >> 1)];
                wf[D][b][ks] = widen8<WT>(r[2 * (ks & 1)], r[2 * (ks & 1) + 1]);
            });
        });
    };

    // Fragment read offsets: row 32·bm + (lane & 31), logical chunk 4h + ks; the swizzle of row
    // r + 32·bm is r's with bit 2 flipped for odd bm.
    const int h = lane >> 5;
    int xo[2][4];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) xo[par][ks] = swz(32 * par + (lane & 31), 4 * h + ks) - 32 * 128 * par;

    f32x16 acc[2][FM];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[b][bm][r] = 0.0f;

    // One K step: the MFMAs on stage S with fragments F, the widening of raw[R] into fragments 1−F
    // interleaved with them.
    auto step = [&](auto stage, auto frag, auto rawbuf) {
        constexpr int S = decltype(stage)::value, F = decltype(frag)::value, R = decltype(rawbuf)::value;
        static_for<0, 4>([&](auto kc) {
            constexpr int ks = decltype(kc)::value;
            bf16x8 xf[FM];
            static_for<0, FM>([&](auto bmc) {
                constexpr int bm = decltype(bmc)::value;
                xf[bm] = kern::lds_load_frag(lds + S * SA + 32 * 128 * bm, xo[bm & 1][ks]);
            });
            // Widen the next step's block (ks & 1), half (ks >> 1) while these MFMAs run.
            {
                constexpr int b = ks >> 1;
                static_for<0, 2>([&](auto qc) {
                    constexpr int q = 2 * (ks & 1) + decltype(qc)::value;  // next-step ks index
                    const u32x4 &r = raw[R][2 * b + (q >> 1)];
                    wf[1 - F][b][q] = widen8<WT>(r[2 * (q & 1)], r[2 * (q & 1) + 1]);
                });
            }
            static_for<0, 2>([&](auto bc) {
                constexpr int b = decltype(bc)::value;
                static_for<0, FM>([&](auto bmc) {
                    constexpr int bm = decltype(bmc)::value;
                    acc[b][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[F][b][ks], xf[bm], acc[b][bm], 0, 0, 0);
                });
            });
        });
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    constexpr int A_LOADS = A_PER_WAVE;  // activation loads each wave issues per step

    // Prologue: A(0) → stage 0, W(0) → raw[0], W(1) → raw[1]; fragments of step 0.
    issue_a(0, I0{});
    issue_w(0, I0{});
    issue_w(1, I1{});
    wait_vmcnt<4>();
    widen_w(I0{}, I0{});
    lds_barrier();

    // Steps in pairs so every buffer index is a constant: step t uses stage t&1, fragments t&1,
    // and widens raw[(t+1)&1]; W(t+2) goes to raw[t&1].
    int t = 0;
    for (; t + 1 < KT; t += 2) {
        issue_a(t + 1, I1{});
        issue_w(t + 2, I0{});
        wait_vmcnt<A_LOADS + 4>();
        step(I0{}, I0{}, I1{});
        wait_vmcnt<4>();
        lds_barrier();
        issue_a(t + 2, I0{});
        issue_w(t + 3, I1{});
        wait_vmcnt<A_LOADS + 4>();
        step(I1{}, I1{}, I0{});
        wait_vmcnt<4>();
        lds_barrier();
    }
    if (t < KT) {  // odd KT: the last step on stage 0 (its widening works on a clamped copy)
        issue_a(t + 1, I1{});
        issue_w(t + 2, I0{});
        wait_vmcnt<A_LOADS + 4>();
        step(I0{}, I0{}, I1{});
    }
    wait_vmcnt<0>();

    // ---- epilogue ------------------------------------------------------------------------------
    // Lane l, register r of block (b, bm): row m0 + 32·bm + (l & 31), slab column
    // 32·b + 8·(r >> 2) + 4·(l >> 5) + (r & 3).
    const int n_out = GLU ? p.glu_half : p.N;
    constexpr int NB = GLU ? 1 : 2;
    static_for<0, NB>([&](auto bc) {
        constexpr int b = decltype(bc)::value;
        static_for<0, 4>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            const int nl = 8 * g + 4 * h;
            const int col = GLU ? slab * 32 + nl : slab * 64 + b * 32 + nl;
            if (col < n_out) {
                kern::epilogue_store<FM, EPI, OUT, g>(p, acc[b], acc[GLU ? 1 : b], col, n_out, m0 + (lane & 31));
            }
        });
    });
}

template <int BM, int NW, int WT, int WL, int EPI, int OUT>
hipError_t launch_wd(const GemmArgs &args, hipStream_t stream) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    GemmArgs p = args;
    p.tiles_m = (p.M + BM - 1) / BM;
    const int slabs = GLU ? (p.glu_half + 31) / 32 : (p.N + 63) / 64;
    p.tiles_n = (slabs + NW - 1) / NW;
    const int blocks = p.tiles_m * p.tiles_n;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_wd_kernel<BM, NW, WT, WL, EPI, OUT>), dim3(blocks), dim3(64 * NW), 0, stream, p);
    return hipGetLastError();
}

template <int BM, int NW, int WT, int WL>
hipError_t dispatch_wd(const GemmArgs &p, int epi, int out, hipStream_t stream) {
#define SQ8_CASE(E, O)                                                                            \
    if (epi == E && out == O) return launch_wd<BM, NW, WT, WL, E, O>(p, stream);
    SQ8_CASE(EPI_NONE, OUT_BF16)
    SQ8_CASE(EPI_NONE, OUT_F32)
    SQ8_CASE(EPI_GELU, OUT_BF16)
    SQ8_CASE(EPI_GELU, OUT_F32)
    SQ8_CASE(EPI_SILU_GLU, OUT_BF16)
    SQ8_CASE(EPI_SILU_GLU, OUT_F32)
    SQ8_CASE(EPI_SITU_GLU, OUT_BF16)
    SQ8_CASE(EPI_SITU_GLU, OUT_F32)
#undef SQ8_CASE
    return hipErrorInvalidValue;
}

}  // namespace wd
}  // namespace sq8
