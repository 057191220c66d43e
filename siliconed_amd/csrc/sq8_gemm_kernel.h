// sq8_gemm_kernel.h — the gfx950 weight-quantized GEMM kernel template: bf16 activations ×
// int8 / fp8-e4m3 weights, bf16 MFMA with fp32 sums, the per-channel scale, bias and activation
// fused in the epilogue. Included by the translation units that instantiate it (sq8_gemm_*.hip).
//
// Arithmetic (Sources/Siliconed/TensorGEMM.swift:124-135 then :173-179): C = act(s ⊙ (A·q) + b).
// Each product bf16 × code is exact in fp32 (8 + 8 significant bits), the sums are fp32 in the
// matrix cores, the scale multiplies the finished sum (one rounding), the bias is added after
// (one rounding, Ops.swift:400-407), the activation last.
//
// Tiling (one workgroup of 4 waves per tile, one tile per CU at a time):
//   * tile BM × BN of C, K in steps of 64; waves in a 2 × 2 grid, each (BM/2) × (BN/2) built from
//     32 × 32 blocks of v_mfma_f32_32x32x16_bf16;
//   * LDS holds two stages of A [BM][64] and W [BN][64] as bf16, K contiguous per row, 16-byte
//     chunks XOR-swizzled so the fragment reads and the tile writes spread over the banks;
//   * the next K step's global loads are in flight while the current step's MFMAs run; the 8-bit
//     codes are widened to bf16 in registers (v_cvt_f32_i32 SDWA / v_cvt_pk_f32_fp8 + v_perm,
//     exact) between the two, then written to the other stage;
//   * the weight is the MFMA's first operand and the activation its second, so each lane ends
//     with four consecutive output columns of one row: scale and bias are one 16-byte load, the
//     store one 8- (bf16) or 16-byte (fp32) write;
//   * workgroup ids are remapped so the tiles one XCD runs at once are neighbours (shared L2).
//
// FAST (aligned operands, K a multiple of 64): every load is an unconditional vector load; rows
// past M and columns past N read the last valid row / column instead (their results are computed
// and never stored), so the main loop has no branch. !FAST: every element is guarded, zeros past
// the edges — the ragged and unaligned shapes.
#pragma once

#include "sq8_gemm.h"

namespace sq8 {
namespace kern {

constexpr int BK = 64;
constexpr int THREADS = 256;

// Byte offset of logical 16-byte chunk `lc` (8 bf16 of K) of row `r` in a [rows][64] bf16 stage.
__device__ __forceinline__ int swz(int r, int lc) {
    return r * 128 + ((lc ^ ((r ^ (r >> 3)) & 7)) << 4);
}

__device__ __forceinline__ void lds_store16(uint8_t *base, int off, u32x4 v) {
    *reinterpret_cast<u32x4 *>(base + off) = v;
}

__device__ __forceinline__ bf16x8 lds_load_frag(const uint8_t *base, int off) {
    return *reinterpret_cast<const bf16x8 *>(base + off);
}

// Global memory seen as such (not through flat addressing, whose loads also count against the
// LDS wait counter): a uniform base plus a 32-bit byte offset.
typedef const __attribute__((address_space(1))) uint8_t *gbytes;

template <typename T>
__device__ __forceinline__ T gld(gbytes base, uint32_t off) {
    return *(const __attribute__((address_space(1))) T *)(base + off);
}

// Workgroup → tile. The dispatcher hands workgroup i to XCD i mod 8; consecutive logical tiles
// are given to one XCD, then ordered in groups of GROUP_M tile rows so an XCD's resident tiles
// share A rows and W columns in its L2. A bijection on [0, tiles) whatever the dispatch order.
// Base of output tensor `which` (0..2): c[0] plus a byte offset. Never p.c[which] (nor a select of
// c[1] / c[2], which the compiler folds back into one): a run-time index into the argument struct
// forces the whole struct into memory, a per-thread copy the compiler places in LDS.
__device__ __forceinline__ uint8_t *out_base(const GemmArgs &p, int which) {
    const int64_t d = (which == 1 ? p.c_d1 : 0) + (which == 2 ? p.c_d2 : 0);
    return reinterpret_cast<uint8_t *>(p.c[0]) + d;
}

__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int total = tiles_m * tiles_n;
    const int q = total >> 3, r = total & 7;
    const int xcd = bid & 7, local = bid >> 3;
    const int logical = xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
    constexpr int GROUP_M = 4;
    const int per_group = GROUP_M * tiles_n;
    const int group = logical / per_group;
    const int first_m = group * GROUP_M;
    const int gm = min(tiles_m - first_m, GROUP_M);
    const int in_group = logical - group * per_group;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

// Weight column of virtual column `v` of tile `tn` (GLU epilogues pair the 32-column blocks of a
// tile: block 2p holds output columns [32p, 32p+32) of the first half — gate / value —, block
// 2p+1 the same columns of the second half). `valid`: how many of the 4 virtual columns v..v+3
// (v a multiple of 4) are real columns of the same half. Past the edge: −1, or with `clamp` the
// last group of 4 valid columns of the same half (FAST; its results are never stored).
template <int BN, bool GLU>
__device__ __forceinline__ int weight_column(const GemmArgs &p, int tn, int v, bool clamp, int *valid = nullptr) {
    if constexpr (GLU) {
        const int b = v >> 5;
        int out = tn * (BN / 2) + (b >> 1) * 32 + (v & 31);
        if (valid) *valid = out < p.glu_half ? min(4, p.glu_half - out) : 0;
        if (out >= p.glu_half) {
            if (!clamp) return -1;
            out = p.glu_half - 4 + (v & 3);
        }
        return out + (b & 1) * p.glu_half;
    } else {
        int n = tn * BN + v;
        if (valid) *valid = n < p.N ? min(4, p.N - n) : 0;
        if (n >= p.N) {
            if (!clamp) return -1;
            n = p.N - 4 + (v & 3);
        }
        return n;
    }
}

// Scale, bias, activation and store of four consecutive output columns [col, col+4) for the FM
// rows m_first + 32·bm a lane holds: registers 4G..4G+3 of each block (`x` the first half of a
// GLU pair or the only product, `u` the second half).
template <int FM, int EPI, int OUT, int G>
__device__ __forceinline__ void epilogue_store(const GemmArgs &p, const f32x16 (&x)[FM], const f32x16 (&u)[FM],
                                               int col, int n_out, int m_first) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    const bool full = col + 4 <= n_out;
    float s1[4], b1[4], s2[4], b2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int c = col + (full ? e : min(e, n_out - 1 - col));
        const int n2 = c + (GLU ? p.glu_half : 0);
        s1[e] = p.scale_per_col ? p.scale[c] : p.scale[0];
        b1[e] = p.bias ? p.bias[c] : 0.0f;
        s2[e] = p.scale_per_col ? p.scale[n2] : p.scale[0];
        b2[e] = p.bias ? p.bias[n2] : 0.0f;
    }
    // Output tensor and column (the QKV split sends each third to its own tensor).
    int which = 0, ccol = col;
    if (p.split > 0) {
        which = col / p.split;
        ccol = col - which * p.split;
    }
    uint8_t *base = out_base(p, which);
    static_for<0, FM>([&](auto bmc) {
        constexpr int bm = decltype(bmc)::value;
        const int m = m_first + bm * 32;
        if (m < p.M) {
            float y[4];
            static_for<0, 4>([&](auto ec) {
                constexpr int e = decltype(ec)::value;
                float v = __fmul_rn(x[bm][4 * G + e], s1[e]);
                if (p.bias) v = __fadd_rn(v, b1[e]);
                if constexpr (EPI == EPI_GELU) {
                    v = gelu_tanh(v);
                } else if constexpr (GLU) {
                    float w = __fmul_rn(u[bm][4 * G + e], s2[e]);
                    if (p.bias) w = __fadd_rn(w, b2[e]);
                    v = EPI == EPI_SILU_GLU ? silu_glu(v, w) : situ(v, w);
                }
                y[e] = v;
            });
            int64_t off;
            if (p.head_dim > 0)
                off = ((int64_t)(ccol / p.head_dim) * p.M + m) * p.head_dim + ccol % p.head_dim;
            else
                off = (int64_t)m * p.ldc + ccol;
            if constexpr (OUT == OUT_BF16) {
                uint16_t *o = reinterpret_cast<uint16_t *>(base) + off;
                if (full && p.c_vec) {
                    *reinterpret_cast<u32x2 *>(o) = u32x2{pack_bf16_rne(y[0], y[1]), pack_bf16_rne(y[2], y[3])};
                } else {
                    const uint32_t lo = pack_bf16_rne(y[0], y[1]), hi = pack_bf16_rne(y[2], y[3]);
                    const uint16_t h[4] = {(uint16_t)lo, (uint16_t)(lo >> 16), (uint16_t)hi, (uint16_t)(hi >> 16)};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < n_out) o[e] = h[e];
                }
            } else {
                float *o = reinterpret_cast<float *>(base) + off;
                if (full && p.c_vec) {
                    *reinterpret_cast<f32x4 *>(o) = f32x4{y[0], y[1], y[2], y[3]};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < n_out) o[e] = y[e];
                }
            }
        }
    });
}

template <int BM, int BN, int WT, int WL, int EPI, int OUT, bool FAST>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
gemm_q8_kernel(const GemmArgs p) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int WM = BM / 2, WN = BN / 2;   // wave tile
    constexpr int FM = WM / 32, FN = WN / 32; // 32 × 32 blocks per wave
    constexpr int A_LOADS = BM / 32;          // 16-byte chunks of A per thread per K step
    constexpr int SA = BM * 128, SB = BN * 128; // bytes of one stage of A, of W
    constexpr int B0 = 2 * SA;                // W stages follow the two A stages
    static_assert(BN % 128 == 0 || WL == W_NK, "the [K,N] loader takes 128-column slabs");
    static_assert(!GLU || (FN % 2 == 0), "GLU pairs blocks inside a wave");

    // LDS: [A stage 0][A stage 1][W stage 0][W stage 1], each row 64 bf16 of K.
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * (SA + SB)];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM;
    const gbytes Ag = (gbytes)p.a;
    const gbytes Wg = (gbytes)p.w;

    // ---- A loader: thread t → chunk (t & 7) of rows (t >> 3) + 32·i -------------------------------
    // swz(r + 32i, c) = swz(r, c) + 4096·i with the chunk's bit 2 flipped for odd i: two offsets.
    const int a_chunk = tid & 7;
    const int a_row0 = tid >> 3;
    uint32_t a_goff[A_LOADS];
    int a_row[A_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        a_row[i] = m0 + a_row0 + 32 * i;
        const int r = FAST ? min(a_row[i], p.M - 1) : max(min(a_row[i], p.M - 1), 0);
        a_goff[i] = (uint32_t)((int64_t)r * p.lda * 2) + a_chunk * 16;
    }
    const int a_loff[2] = {swz(a_row0, a_chunk), swz(a_row0 + 32, a_chunk) - 32 * 128};

    // ---- W loader ----------------------------------------------------------------------------------
    // [N, K]: thread t → 16 bytes of K (chunk t & 3) of virtual rows (t >> 2) + 64·j.
    // [K, N]: thread t → items of 8 K-rows × 4 columns: item it = t + 256·j, column group
    //         it mod (BN/4), K group it / (BN/4).
    constexpr int W_ITEMS = WL == W_NK ? BN / 64 : BN / 128;
    int w_col[W_ITEMS], w_cnt[W_ITEMS];
    uint32_t w_goff[W_ITEMS];
#pragma unroll
    for (int j = 0; j < W_ITEMS; ++j) {
        if constexpr (WL == W_NK) {
            w_col[j] = weight_column<BN, GLU>(p, tn, (tid >> 2) + 64 * j, FAST);
            w_cnt[j] = 0;
            w_goff[j] = (uint32_t)((int64_t)max(w_col[j], 0) * p.ldw) + (tid & 3) * 16;
        } else {
            const int it = tid + 256 * j;
            w_col[j] = weight_column<BN, GLU>(p, tn, (it % (BN / 4)) * 4, FAST, &w_cnt[j]);
            w_goff[j] = (uint32_t)((int64_t)((it / (BN / 4)) * 8) * p.ldw) + max(w_col[j], 0);
        }
    }
    // LDS offsets of the W tile writes (stage 0, from the start of the W region).
    //   [N, K]: rows (t >> 2) + 64·j share swz's chunk permutation: chunks 2kq, 2kq + 1.
    //   [K, N]: item (cg, kg) writes chunk kg of rows 4cg + c, c < 4.
    int w_loff[WL == W_NK ? 2 : 4 * W_ITEMS];
    if constexpr (WL == W_NK) {
        w_loff[0] = swz(tid >> 2, 2 * (tid & 3));
        w_loff[1] = swz(tid >> 2, 2 * (tid & 3) + 1);
    } else {
#pragma unroll
        for (int j = 0; j < W_ITEMS; ++j) {
            const int it = tid + 256 * j;
#pragma unroll
            for (int c = 0; c < 4; ++c) w_loff[4 * j + c] = swz((it % (BN / 4)) * 4 + c, it / (BN / 4));
        }
    }

    u32x4 ra[A_LOADS];
    u32x4 rw_nk[WL == W_NK ? W_ITEMS : 1];
    uint32_t rw_kn[WL == W_KN ? W_ITEMS : 1][8];

    auto load_a = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            if constexpr (FAST) {
                ra[i] = gld<u32x4>(Ag, a_goff[i] + (uint32_t)k0 * 2);
            } else {
                const int k = k0 + a_chunk * 8;
                uint16_t e[8];
#pragma unroll
                for (int x = 0; x < 8; ++x)
                    e[x] = (a_row[i] < p.M && k + x < p.K) ? gld<uint16_t>(Ag, a_goff[i] + (uint32_t)(k0 + x) * 2)
                                                           : (uint16_t)0;
                ra[i] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                              e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
            }
        }
    };

    auto load_w = [&](int k0) {
#pragma unroll
        for (int j = 0; j < W_ITEMS; ++j) {
            if constexpr (WL == W_NK) {
                if constexpr (FAST) {
                    rw_nk[j] = gld<u32x4>(Wg, w_goff[j] + (uint32_t)k0);
                } else {
                    const int k = k0 + (tid & 3) * 16;
                    uint32_t d[4] = {0, 0, 0, 0};
#pragma unroll
                    for (int x = 0; x < 16; ++x) {
                        const uint32_t b =
                            (w_col[j] >= 0 && k + x < p.K) ? gld<uint8_t>(Wg, w_goff[j] + (uint32_t)(k0 + x)) : 0u;
                        d[x >> 2] |= b << (8 * (x & 3));
                    }
                    rw_nk[j] = u32x4{d[0], d[1], d[2], d[3]};
                }
            } else {
                const uint32_t base = w_goff[j] + (uint32_t)k0 * (uint32_t)p.ldw;
                if constexpr (FAST) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) rw_kn[j][i] = gld<uint32_t>(Wg, base + (uint32_t)i * (uint32_t)p.ldw);
                } else {
                    // Columns n..n+valid−1 are consecutive weight columns of one half (a 32-column
                    // block never splits); the rest of the 4 are zeros.
                    const int it = tid + 256 * j;
                    const int kr = k0 + (it / (BN / 4)) * 8;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        uint32_t d = 0;
#pragma unroll
                        for (int x = 0; x < 4; ++x)
                            if (x < w_cnt[j] && kr + i < p.K)
                                d |= (uint32_t)gld<uint8_t>(Wg, base + (uint32_t)i * (uint32_t)p.ldw + x) << (8 * x);
                        rw_kn[j][i] = d;
                    }
                }
            }
        }
    };

    auto store_stage = [&](auto stage) {
        constexpr int S = decltype(stage)::value;
        uint8_t *As = lds + S * SA;
        uint8_t *Bs = lds + B0 + S * SB;
        static_for<0, A_LOADS>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            lds_store16(As + 32 * 128 * i, a_loff[i & 1], ra[i]);
        });
#pragma unroll
        for (int j = 0; j < W_ITEMS; ++j) {
            if constexpr (WL == W_NK) {
                uint32_t o[8];
                widen4<WT>(rw_nk[j][0], o[0], o[1]);
                widen4<WT>(rw_nk[j][1], o[2], o[3]);
                widen4<WT>(rw_nk[j][2], o[4], o[5]);
                widen4<WT>(rw_nk[j][3], o[6], o[7]);
                lds_store16(Bs + 64 * 128 * j, w_loff[0], u32x4{o[0], o[1], o[2], o[3]});
                lds_store16(Bs + 64 * 128 * j, w_loff[1], u32x4{o[4], o[5], o[6], o[7]});
            } else {
                const uint32_t *d = rw_kn[j];
                // Column c of the item: byte c of each of the 8 K rows, widened and paired along K.
                if constexpr (WT == W_INT8) {
                    static_for<0, 4>([&](auto cc) {
                        constexpr int c = decltype(cc)::value;
                        lds_store16(Bs, w_loff[4 * j + c],
                                    u32x4{pack_exact_bf16(i8_byte<c>(d[0]), i8_byte<c>(d[1])),
                                          pack_exact_bf16(i8_byte<c>(d[2]), i8_byte<c>(d[3])),
                                          pack_exact_bf16(i8_byte<c>(d[4]), i8_byte<c>(d[5])),
                                          pack_exact_bf16(i8_byte<c>(d[6]), i8_byte<c>(d[7]))});
                    });
                } else {
                    float f[8][4];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        fp8_pair<0>(d[i], f[i][0], f[i][1]);
                        fp8_pair<1>(d[i], f[i][2], f[i][3]);
                    }
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        lds_store16(Bs, w_loff[4 * j + c],
                                    u32x4{pack_exact_bf16(f[0][c], f[1][c]), pack_exact_bf16(f[2][c], f[3][c]),
                                          pack_exact_bf16(f[4][c], f[5][c]), pack_exact_bf16(f[6][c], f[7][c])});
                }
            }
        }
    };

    f32x16 acc[FN][FM];
#pragma unroll
    for (int bn = 0; bn < FN; ++bn)
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[bn][bm][r] = 0.0f;

    // Fragment read offsets: rows wm·WM + bm·32 + (l & 31) (A) and wn·WN + bn·32 + (l & 31) (W);
    // swz's chunk permutation of row r + 32·bm is r's with bit 2 flipped for odd bm, so each lane
    // needs one offset per (bm parity, K sub-step) and the rest is an immediate.
    const int khalf = lane >> 5;
    int xo[2][4], wo[2][4];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            xo[par][ks] = swz(wm * WM + 32 * par + (lane & 31), 2 * ks + khalf) - 32 * 128 * par;
            wo[par][ks] = B0 + swz(wn * WN + 32 * par + (lane & 31), 2 * ks + khalf) - 32 * 128 * par;
        }

    auto compute = [&](auto stage) {
        constexpr int S = decltype(stage)::value;
        static_for<0, BK / 16>([&](auto ksc) {
            constexpr int ks = decltype(ksc)::value;
            bf16x8 xf[FM], wf[FN];
            static_for<0, FM>([&](auto bmc) {
                constexpr int bm = decltype(bmc)::value;
                xf[bm] = lds_load_frag(lds + S * SA + 32 * 128 * bm, xo[bm & 1][ks]);
            });
            static_for<0, FN>([&](auto bnc) {
                constexpr int bn = decltype(bnc)::value;
                wf[bn] = lds_load_frag(lds + S * SB + 32 * 128 * bn, wo[bn & 1][ks]);
            });
#pragma unroll
            for (int bn = 0; bn < FN; ++bn)
#pragma unroll
                for (int bm = 0; bm < FM; ++bm)
                    acc[bn][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[bn], xf[bm], acc[bn][bm], 0, 0, 0);
        });
    };

    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    const int KT = (p.K + BK - 1) / BK;
    load_a(0);
    load_w(0);
    store_stage(S0{});
    __syncthreads();
    // Pairs of steps, the stage a compile-time constant; stage 0 holds step kt at the top.
    int kt = 0;
    for (; kt + 2 < KT; kt += 2) {
        load_a((kt + 1) * BK);
        load_w((kt + 1) * BK);
        compute(S0{});
        store_stage(S1{});
        __syncthreads();
        load_a((kt + 2) * BK);
        load_w((kt + 2) * BK);
        compute(S1{});
        store_stage(S0{});
        __syncthreads();
    }
    if (kt + 1 < KT) {
        load_a((kt + 1) * BK);
        load_w((kt + 1) * BK);
        compute(S0{});
        store_stage(S1{});
        __syncthreads();
        compute(S1{});
    } else if (KT > 0) {
        compute(S0{});
    }

    // ---- epilogue ------------------------------------------------------------------------------
    // Lane l, register r of block (bn, bm): row m0 + wm·WM + bm·32 + (l & 31), virtual column
    // wn·WN + bn·32 + 8·(r >> 2) + 4·(l >> 5) + (r & 3).
    const int n_out = GLU ? p.glu_half : p.N;
    constexpr int NB = GLU ? FN / 2 : FN;  // output blocks per wave (GLU: pairs of blocks)
    static_for<0, NB>([&](auto bpc) {
        constexpr int bn = decltype(bpc)::value * (GLU ? 2 : 1);
        static_for<0, 4>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            const int vloc = wn * WN + bn * 32 + 8 * g + 4 * khalf;  // first of 4 virtual columns
            const int col = GLU ? tn * (BN / 2) + ((vloc >> 5) >> 1) * 32 + (vloc & 31) : tn * BN + vloc;
            if (col < n_out) {
                epilogue_store<FM, EPI, OUT, g>(p, acc[bn], acc[GLU ? bn + 1 : bn], col, n_out,
                                                m0 + wm * WM + (lane & 31));
            }
        });
    });
}

template <int BM, int BN, int WT, int WL, int EPI, int OUT, bool FAST>
hipError_t launch_tile(const GemmArgs &args, hipStream_t stream) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    GemmArgs p = args;
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = GLU ? (p.glu_half + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN;
    const int blocks = p.tiles_m * p.tiles_n;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_q8_kernel<BM, BN, WT, WL, EPI, OUT, FAST>), dim3(blocks), dim3(THREADS), 0, stream, p);
    return hipGetLastError();
}

template <int BM, int BN, int WT, int WL, bool FAST>
hipError_t dispatch_epi_out(const GemmArgs &p, int epi, int out, hipStream_t stream) {
#define SQ8_CASE(E, O)                                                                            \
    if (epi == E && out == O) return launch_tile<BM, BN, WT, WL, E, O, FAST>(p, stream);
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

}  // namespace kern
}  // namespace sq8
