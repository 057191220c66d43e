// sq8_gemm.hip — the gfx950 weight-quantized GEMM: bf16 activations × int8 / fp8-e4m3 weights,
// bf16 MFMA with fp32 sums, the per-channel scale, bias and activation fused in the epilogue.
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
#include "sq8_gemm.h"

namespace sq8 {

namespace {

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

// Workgroup → tile. The dispatcher hands workgroup i to XCD i mod 8; consecutive logical tiles
// are given to one XCD, then ordered in groups of GROUP_M tile rows so an XCD's resident tiles
// share A rows and W columns in its L2. A bijection on [0, tiles) whatever the dispatch order.
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

// Weight column of virtual column `v` of tile `tn`, or −1 past the edge; `valid` (when asked) is
// how many of the 4 virtual columns v..v+3 (v a multiple of 4) are real weight columns of the same
// half. GLU epilogues pair the 32-column blocks of a tile: block 2p holds output columns
// [32p, 32p+32) of the first half (gate / value), block 2p+1 the same columns of the second half.
template <int BN, bool GLU>
__device__ __forceinline__ int weight_column(const GemmArgs &p, int tn, int v, int *valid = nullptr) {
    if constexpr (GLU) {
        const int b = v >> 5, out = tn * (BN / 2) + (b >> 1) * 32 + (v & 31);
        if (valid) *valid = out < p.glu_half ? min(4, p.glu_half - out) : 0;
        return out < p.glu_half ? out + (b & 1) * p.glu_half : -1;
    } else {
        const int n = tn * BN + v;
        if (valid) *valid = n < p.N ? min(4, p.N - n) : 0;
        return n < p.N ? n : -1;
    }
}

// Scale, bias, activation and store of four consecutive output columns [col, col+4) for the FM
// rows m_first + 32·bm a lane holds: registers 4g..4g+3 of each block (`x` the first half of a
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
    uint8_t *base = reinterpret_cast<uint8_t *>(p.c[which]);
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

template <int BM, int BN, int WT, int WL, int EPI, int OUT>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
gemm_q8_kernel(const GemmArgs p) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int WM = BM / 2, WN = BN / 2;   // wave tile
    constexpr int FM = WM / 32, FN = WN / 32; // 32 × 32 blocks per wave
    constexpr int A_LOADS = BM / 32;          // 16-byte chunks of A per thread per K step
    constexpr int STAGE = (BM + BN) * 128;    // bytes per stage
    static_assert(BN % 128 == 0 || WL == W_NK, "the [K,N] loader takes 128-column slabs");
    static_assert(!GLU || (FN % 2 == 0), "GLU pairs blocks inside a wave");

    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM;

    const uint16_t *__restrict__ A = p.a;
    const uint8_t *__restrict__ W = p.w;

    // ---- A loader: thread t → chunk (t & 7) of rows (t >> 3) + 32·i -------------------------------
    const int a_chunk = tid & 7;
    const int a_row0 = tid >> 3;

    // ---- W loader ----------------------------------------------------------------------------------
    // [N, K]: thread t → 16 bytes of K (chunk t & 3) of virtual rows (t >> 2) + 64·j.
    // [K, N]: thread t → items of 8 K-rows × 4 columns: item it = t + 256·j, column group
    //         it mod (BN/4), K group it / (BN/4).
    constexpr int W_ITEMS = WL == W_NK ? BN / 64 : BN / 128;
    int w_col[W_ITEMS], w_cnt[W_ITEMS];
#pragma unroll
    for (int j = 0; j < W_ITEMS; ++j) {
        if constexpr (WL == W_NK) {
            w_col[j] = weight_column<BN, GLU>(p, tn, (tid >> 2) + 64 * j);
            w_cnt[j] = 0;
        } else {
            const int it = tid + 256 * j;
            w_col[j] = weight_column<BN, GLU>(p, tn, (it % (BN / 4)) * 4, &w_cnt[j]);
        }
    }

    u32x4 ra[A_LOADS];
    u32x4 rw_nk[WL == W_NK ? W_ITEMS : 1];
    uint32_t rw_kn[WL == W_KN ? W_ITEMS : 1][8];

    auto load_a = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int row = m0 + a_row0 + 32 * i;
            const int k = k0 + a_chunk * 8;
            if (p.a_vec && row < p.M && k + 8 <= p.K) {
                ra[i] = *reinterpret_cast<const u32x4 *>(A + (int64_t)row * p.lda + k);
            } else {
                uint16_t e[8];
#pragma unroll
                for (int x = 0; x < 8; ++x)
                    e[x] = (row < p.M && k + x < p.K) ? A[(int64_t)row * p.lda + k + x] : (uint16_t)0;
                ra[i] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                              e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
            }
        }
    };

    auto load_w = [&](int k0) {
#pragma unroll
        for (int j = 0; j < W_ITEMS; ++j) {
            const int n = w_col[j];
            if constexpr (WL == W_NK) {
                const int k = k0 + (tid & 3) * 16;
                if (p.w_vec && n >= 0 && k + 16 <= p.K) {
                    rw_nk[j] = *reinterpret_cast<const u32x4 *>(W + (int64_t)n * p.ldw + k);
                } else {
                    uint32_t d[4] = {0, 0, 0, 0};
#pragma unroll
                    for (int x = 0; x < 16; ++x) {
                        const uint32_t b = (n >= 0 && k + x < p.K) ? W[(int64_t)n * p.ldw + k + x] : 0u;
                        d[x >> 2] |= b << (8 * (x & 3));
                    }
                    rw_nk[j] = u32x4{d[0], d[1], d[2], d[3]};
                }
            } else {
                const int it = tid + 256 * j;
                const int kr = k0 + (it / (BN / 4)) * 8;
                // Columns n..n+ncols−1 are consecutive weight columns of one half (a 32-column block
                // never splits); the rest of the 4 are zeros.
                const int ncols = w_cnt[j];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int k = kr + i;
                    if (p.w_vec && ncols == 4 && k < p.K) {
                        rw_kn[j][i] = *reinterpret_cast<const uint32_t *>(W + (int64_t)k * p.ldw + n);
                    } else {
                        uint32_t d = 0;
#pragma unroll
                        for (int x = 0; x < 4; ++x)
                            if (x < ncols && k < p.K) d |= (uint32_t)W[(int64_t)k * p.ldw + n + x] << (8 * x);
                        rw_kn[j][i] = d;
                    }
                }
            }
        }
    };

    auto store_stage = [&](int s) {
        uint8_t *As = lds + s * STAGE;
        uint8_t *Bs = As + BM * 128;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) lds_store16(As, swz(a_row0 + 32 * i, a_chunk), ra[i]);
#pragma unroll
        for (int j = 0; j < W_ITEMS; ++j) {
            if constexpr (WL == W_NK) {
                const int v = (tid >> 2) + 64 * j, kq = tid & 3;
                uint32_t o[8];
                widen4<WT>(rw_nk[j][0], o[0], o[1]);
                widen4<WT>(rw_nk[j][1], o[2], o[3]);
                widen4<WT>(rw_nk[j][2], o[4], o[5]);
                widen4<WT>(rw_nk[j][3], o[6], o[7]);
                lds_store16(Bs, swz(v, 2 * kq), u32x4{o[0], o[1], o[2], o[3]});
                lds_store16(Bs, swz(v, 2 * kq + 1), u32x4{o[4], o[5], o[6], o[7]});
            } else {
                const int it = tid + 256 * j;
                const int v = (it % (BN / 4)) * 4, kg = it / (BN / 4);
                const uint32_t *d = rw_kn[j];
                // Column c of the item: byte c of each of the 8 K rows, widened and paired along K.
                if constexpr (WT == W_INT8) {
#define SQ8_KN_COL(C)                                                                              \
    lds_store16(Bs, swz(v + C, kg),                                                                \
                u32x4{pack_exact_bf16(i8_byte<C>(d[0]), i8_byte<C>(d[1])),                          \
                      pack_exact_bf16(i8_byte<C>(d[2]), i8_byte<C>(d[3])),                          \
                      pack_exact_bf16(i8_byte<C>(d[4]), i8_byte<C>(d[5])),                          \
                      pack_exact_bf16(i8_byte<C>(d[6]), i8_byte<C>(d[7]))});
                    SQ8_KN_COL(0) SQ8_KN_COL(1) SQ8_KN_COL(2) SQ8_KN_COL(3)
#undef SQ8_KN_COL
                } else {
                    float f[8][4];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        fp8_pair<0>(d[i], f[i][0], f[i][1]);
                        fp8_pair<1>(d[i], f[i][2], f[i][3]);
                    }
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        lds_store16(Bs, swz(v + c, kg),
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

    const int xrow = wm * WM + (lane & 31);
    const int wrow = wn * WN + (lane & 31);
    const int khalf = lane >> 5;

    auto compute = [&](int s) {
        const uint8_t *As = lds + s * STAGE;
        const uint8_t *Bs = As + BM * 128;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int lc = ks * 2 + khalf;
            bf16x8 xf[FM], wf[FN];
#pragma unroll
            for (int bm = 0; bm < FM; ++bm) xf[bm] = lds_load_frag(As, swz(xrow + bm * 32, lc));
#pragma unroll
            for (int bn = 0; bn < FN; ++bn) wf[bn] = lds_load_frag(Bs, swz(wrow + bn * 32, lc));
#pragma unroll
            for (int bn = 0; bn < FN; ++bn)
#pragma unroll
                for (int bm = 0; bm < FM; ++bm)
                    acc[bn][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[bn], xf[bm], acc[bn][bm], 0, 0, 0);
        }
    };

    const int KT = (p.K + BK - 1) / BK;
    load_a(0);
    load_w(0);
    store_stage(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int s = kt & 1;
        const bool more = kt + 1 < KT;
        if (more) {
            load_a((kt + 1) * BK);
            load_w((kt + 1) * BK);
        }
        compute(s);
        if (more) store_stage(s ^ 1);
        __syncthreads();
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

template <int BM, int BN, int WT, int WL, int EPI, int OUT>
hipError_t launch_tile(const GemmArgs &args, hipStream_t stream) {
    GemmArgs p = args;
    const int n_virtual = (EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU) ? 2 * p.glu_half : p.N;
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU) ? (p.glu_half + BN / 2 - 1) / (BN / 2)
                                                               : (n_virtual + BN - 1) / BN;
    const int blocks = p.tiles_m * p.tiles_n;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_q8_kernel<BM, BN, WT, WL, EPI, OUT>), dim3(blocks), dim3(THREADS), 0, stream, p);
    return hipGetLastError();
}

template <int BM, int BN, int WT, int WL>
hipError_t dispatch_epi_out(const GemmArgs &p, int epi, int out, hipStream_t stream) {
#define SQ8_CASE(E, O)                                                                            \
    if (epi == E && out == O) return launch_tile<BM, BN, WT, WL, E, O>(p, stream);
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

template <int BM, int BN>
hipError_t dispatch_weight(const GemmArgs &p, int wt, int wl, int epi, int out, hipStream_t stream) {
    if (wt == W_INT8 && wl == W_KN) return dispatch_epi_out<BM, BN, W_INT8, W_KN>(p, epi, out, stream);
    if (wt == W_INT8 && wl == W_NK) return dispatch_epi_out<BM, BN, W_INT8, W_NK>(p, epi, out, stream);
    if (wt == W_FP8 && wl == W_KN) return dispatch_epi_out<BM, BN, W_FP8, W_KN>(p, epi, out, stream);
    if (wt == W_FP8 && wl == W_NK) return dispatch_epi_out<BM, BN, W_FP8, W_NK>(p, epi, out, stream);
    return hipErrorInvalidValue;
}

}  // namespace

int choose_tile(int M, int N_out, bool glu) {
    // Tiles of 256 × 256 while they fill the 256 CUs at least once; 128 × 128 below.
    const int n_virtual = glu ? 2 * N_out : N_out;
    const long big = (long)((M + 255) / 256) * ((n_virtual + 255) / 256);
    return big >= 192 ? TILE_256x256 : TILE_128x128;
}

hipError_t launch_gemm(const GemmArgs &p, int tile, int wt, int wl, int epi, int out, hipStream_t stream) {
    switch (tile) {
    case TILE_256x256: return dispatch_weight<256, 256>(p, wt, wl, epi, out, stream);
    case TILE_128x128: return dispatch_weight<128, 128>(p, wt, wl, epi, out, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace sq8
