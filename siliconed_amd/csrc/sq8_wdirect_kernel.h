// sq8_wdirect_kernel.h — the weight-direct gfx950 GEMM: each wave owns a 64-column slab of the
// weight and streams its 8-bit codes from HBM straight into registers, widening them to bf16 there;
// only the activation tile goes through LDS.
//
// Arithmetic as the other kernels (Sources/Siliconed/TensorGEMM.swift:124-135, :173-179):
// C = act(s ⊙ (A·q) + b), exact bf16 × code products, fp32 sums, scale after the sum, bias after
// the scale, activation last.
//
// Tile BM × 64·NW, NW waves of 64 lanes; wave w computes all BM rows × its 64 virtual columns as
// 2 × (BM/32) blocks of v_mfma_f32_32x32x16_bf16 (the code the first operand, the activation the
// second: each lane ends with 4 consecutive output columns of a row). With CB = 1 a wave owns one
// 32-column block instead (tile BM × 32·NW): the activation rows then serve twice the columns per
// workgroup and each wave widens half the codes per MFMA (the short-M tiles of C2's text stream).
//
// K order inside a 64-step: MFMA sub-step ks of lane half h (lanes 32h..32h+31) takes
// k ∈ [32h + 8ks, 32h + 8ks + 8). Any fixed permutation of K inside the step gives the same sums;
// this one makes a lane's codes for the whole step 32 contiguous bytes (two 16-byte loads per
// 32-column block), and its activation chunks 8-bf16 pieces of one LDS row.
//
// Activation: a 2-stage LDS ring of [BM][64] bf16 tiles filled by direct global→LDS loads
// (global_load_lds_dwordx4: each wave writes 1 KB = 8 rows per load, no VGPR, no ds_write), rows
// of 128 bytes whose 16-byte chunks are XOR-swizzled (chunk ^ ((r ^ r>>3) & 7)) so the fragment
// reads of 16 consecutive rows hit distinct banks. Fragments of sub-step ks+1 are read while the
// MFMAs of ks run.
//
// Two pipelines, by occupancy:
//   OCC = 1 (one workgroup per CU): the codes of step t+1 are widened between the MFMAs of step t;
//     fragments double-buffered.
//   OCC = 2 (two workgroups per CU, ≤ 256 registers a wave): the codes of step t are widened at the
//     step's start — the other workgroup's MFMAs cover it — into one fragment buffer.
// Per step t, the loads issued ahead and the waits explicit (vmcnt counts in issue order):
//   [widen W(t)]  issue A(t+1) → LDS stage (t+1)&1, W(t+2) → raw[t&1]  MFMAs of t  wait vmcnt(4)
//   (A(t+1) and W(t+1) landed)  barrier (no fence: the W prefetch stays in flight)
//
// Weight layouts: [N, K] (nn.Linear: row-strided 16-byte loads) or the packed layout of
// sq8_pack_weight — per 64-column slab, per K step, per load j, per lane, 16 bytes — in which each
// wave load is one contiguous kilobyte.
//
// Epilogue: scale, bias, activation in registers; each 32 × 32 block goes through a wave-private
// LDS region and leaves as 16-byte row segments (coalesced rows instead of 8-byte pieces of 32).
#pragma once

#include "sq8_gemm_kernel.h"

namespace sq8 {
namespace wd {

constexpr int BK = 64;

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef const __attribute__((address_space(1))) void *glb_ptr;

// Direct loads through a buffer resource: the K step's byte offset rides in a scalar register (soffset) beside
// each lane's constant 32-bit offset, so a load needs no per-lane 64-bit address add. The resource spans the
// whole 32-bit offset range from `base` (raw, stride 0; the gfx9 family's word 3); every offset used here is
// the one the global load would have added to the same base.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint32_t *lds_u32;
__device__ void raw_buffer_load_lds(i32x4 rsrc, lds_u32 lds, int size, int voffset, int soffset, int offset,
                                    int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");
__device__ __forceinline__ i32x4 buffer_rsrc(const void *base) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    i32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)b);
    r[1] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)(b >> 32));
    r[2] = -1;
    r[3] = 0x00020000;
    return r;
}

__device__ __forceinline__ int swz(int r, int lc) { return r * 128 + ((lc ^ ((r ^ (r >> 3)) & 7)) << 4); }

// s_waitcnt with only the vector-memory counter constrained (expcnt and lgkmcnt at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// The K-loop's workgroup barrier: s_barrier, and a compiler barrier for memory operations — no
// fence. Across it, the LDS is written only by the direct global→LDS loads, which each wave has
// waited for (vmcnt) before arriving, and read only by fragment loads whose results the MFMAs
// already consumed; a fence would add vmcnt(0) for those LDS-bound loads, draining the weight
// prefetch the vmcnt counter holds behind them.
__device__ __forceinline__ void step_barrier() { asm volatile("s_barrier" ::: "memory"); }

// 8 codes (two dwords) → one MFMA operand of 8 bf16, exactly.
template <int WT>
__device__ __forceinline__ bf16x8 widen8(uint32_t d0, uint32_t d1) {
    uint32_t o0, o1, o2, o3;
    widen4<WT>(d0, o0, o1);
    widen4<WT>(d1, o2, o3);
    return __builtin_bit_cast(bf16x8, u32x4{o0, o1, o2, o3});
}

// The weight's K step under activation step t: t itself, or t modulo the weight's kt_w steps when
// the activation holds up to three parts along K that each face the whole weight (the fp32 route's
// three bf16 parts of every value, sq8_linear_f32: t < 3·kt_w). Two selects on a wave-uniform value,
// no branch: a loop here splits the main loop's blocks and the register allocation with them.
__device__ __forceinline__ int weight_step(const GemmArgs &p, int t) {
    const int kw = p.kt_w > 0 ? p.kt_w : 0x7fffffff;
    t -= t >= kw ? kw : 0;
    t -= t >= kw ? kw : 0;
    return t;
}

// Byte offset (K step 0) of the 16 bytes lane `lane`, load j (block j>>1, half j&1) reads for
// virtual 64-column slab `slab`. Past the edge of an [N, K] weight: the last column of the same half;
// past the last slab of a packed weight (a tile's waves outnumber the slabs left): the last slab —
// results never stored, reads kept inside the buffer.
template <int WL, bool GLU>
__device__ __forceinline__ uint32_t w_offset(const GemmArgs &p, int slab, int j, int lane) {
    if constexpr (WL == W_PACKED) {
        const int slabs = GLU ? (p.glu_half + 31) / 32 : (p.N + 63) / 64;
        const int s = slab < slabs ? slab : slabs - 1;
        const int kt = p.kt_w > 0 ? p.kt_w : p.kt;  // the weight's K steps
        return (uint32_t)(((int64_t)s * kt * 4 + j) * 1024 + lane * 16);
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

// Byte offset in output tensor `which` of row m, column col (the QKV split and head layout).
__device__ __forceinline__ int64_t out_index(const GemmArgs &p, int m, int col, int &which) {
    int cc = col;
    which = 0;
    if (p.split > 0) {
        which = col / p.split;
        cc = col - which * p.split;
    }
    return p.head_dim > 0 ? ((int64_t)(cc / p.head_dim) * p.M + m) * p.head_dim + cc % p.head_dim
                          : (int64_t)m * p.ldc + cc;
}

// Scales and biases of a lane's 16 columns of one 32-column block: group g holds columns
// col0 + 8g + 4h + [0, 4) (h = lane ÷ 32), the layout of the MFMA output registers. `off`: where the
// block's weight columns start relative to its output columns (the second half of a GLU weight).
struct ColParams {
    float s[4][4], b[4][4];
};

__device__ __forceinline__ void load_col_params(const GemmArgs &p, ColParams &cp, int col0, int off, int n_out,
                                                int lane) {
    const kern::gbytes S = (kern::gbytes)p.scale;
    const kern::gbytes B = (kern::gbytes)p.bias;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int col = col0 + 8 * g + 4 * (lane >> 5);
        if (p.sb_vec && col + 4 <= n_out) {
            const f32x4 sv = p.scale_per_col ? kern::gld<f32x4>(S, (uint32_t)(col + off) * 4) : f32x4{0, 0, 0, 0};
            const f32x4 bv = p.bias ? kern::gld<f32x4>(B, (uint32_t)(col + off) * 4) : f32x4{0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                cp.s[g][e] = p.scale_per_col ? sv[e] : p.scale[0];
                cp.b[g][e] = bv[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int cc = min(col + e, n_out - 1) + off;
                cp.s[g][e] = p.scale[p.scale_per_col ? cc : 0];
                cp.b[g][e] = p.bias ? p.bias[cc] : 0.0f;
            }
        }
    }
}

// The residual epilogue's operands of one 32 × 32 block, loaded before the block's values are staged so
// their memory latency overlaps the staging: the 16-byte segments of the fp32 stream this lane adds to
// (rows lane/8 + 8i, columns col0 + 4·(lane & 7) … + 3, as flush_region stores them) and the gate of those
// columns. Only whole, 16-byte-aligned segments inside the product (`vec`); the rest take the per-value path.
struct ResidualPre {
    f32x4 x[4];
    f32x4 g;
};
__device__ __forceinline__ void load_residual(const GemmArgs &p, int col0, int m_first, int n_out, int lane,
                                              ResidualPre &r) {
    const int col = col0 + 4 * (lane & 7);
    const bool vec = col + 4 <= n_out && p.c_vec16;
    r.g = vec && p.gate ? *reinterpret_cast<const f32x4 *>(p.gate + col) : f32x4{1.0f, 1.0f, 1.0f, 1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m_first + (lane >> 3) + 8 * i;
        r.x[i] = vec && m < p.M ? *reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(p.c[0]) +
                                                                 (int64_t)m * p.ldc + col)
                                : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

// The second half of an epilogue: a wave's LDS region of 32 rows × 32 finished values (row pitch
// 32·size + 16) read back as 16-byte row segments and stored (the residual epilogue adds them to
// the fp32 stream, whose segments `pre` holds when load_residual read them first). Output columns
// [col0, col0 + 32), rows [m_first, m_first + 32).
template <int EPI, int OUT>
__device__ __forceinline__ void flush_region(const GemmArgs &p, int col0, int m_first, int n_out, const uint8_t *region,
                                             int lane, const ResidualPre *pre = nullptr) {
    constexpr int ESZ = OUT == OUT_BF16 ? 2 : 4;
    constexpr int PITCH = 32 * ESZ + 16;
    // 16-byte row segments: CPR chunks per row, 64/CPR rows per pass. LDS operations
    // of one wave complete in order, so the wave reads back what it just wrote.
    constexpr int CPR = 32 * ESZ / 16;
    constexpr int ROWS = 64 / CPR;
    constexpr int PER = 16 / ESZ;  // values per chunk
    // The block's output tensor, head and column in it, once per block (wave-uniform): with the split
    // and the head size multiples of 32 a 32-column block lies in one output and one head, and the
    // 16-byte stores need no division per chunk.
    const bool whole = p.split % 32 == 0 && p.head_dim % 32 == 0;
    int which0 = 0, cc0 = col0, head0 = 0;
    if (whole) {
        if (p.split > 0) {
            which0 = col0 / p.split;
            cc0 = col0 - which0 * p.split;
        }
        if (p.head_dim > 0) {
            head0 = cc0 / p.head_dim;
            cc0 -= head0 * p.head_dim;
        }
    }
    uint8_t *const base0 = kern::out_base(p, which0);
    static_for<0, 32 / ROWS>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        const int row = lane / CPR + ROWS * i, chunk = lane % CPR;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(region + row * PITCH + chunk * 16);
        const int m = m_first + row;
        const int col = col0 + chunk * PER;
        if (m < p.M && col < n_out) {
            if constexpr (EPI == EPI_RESIDUAL) {
                // x = x + gate·y, y the fp32 sum scaled and biased (OUT_F32: 4 values a chunk).
                static_assert(OUT == OUT_F32, "the residual stream is fp32");
                float *xr = reinterpret_cast<float *>(p.c[0]) + (int64_t)m * p.ldc + col;
                if (col + PER <= n_out && p.c_vec16) {
                    const f32x4 xv = pre ? pre->x[i] : *reinterpret_cast<const f32x4 *>(xr);
                    const f32x4 gv = pre ? pre->g
                                         : p.gate ? *reinterpret_cast<const f32x4 *>(p.gate + col) : f32x4{1.0f, 1.0f, 1.0f, 1.0f};
                    f32x4 o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = __fadd_rn(xv[e], __fmul_rn(gv[e], __uint_as_float(v[e])));
                    *reinterpret_cast<f32x4 *>(xr) = o;
                } else {
#pragma unroll
                    for (int e = 0; e < PER; ++e)
                        if (col + e < n_out)
                            xr[e] = __fadd_rn(xr[e], __fmul_rn(p.gate ? p.gate[col + e] : 1.0f, __uint_as_float(v[e])));
                }
            } else if (col + PER <= n_out && p.c_vec16) {
                if (whole) {
                    const int cc = cc0 + chunk * PER;
                    const int64_t off = p.head_dim > 0 ? ((int64_t)head0 * p.M + m) * p.head_dim + cc : (int64_t)m * p.ldc + cc;
                    *reinterpret_cast<u32x4 *>(base0 + off * ESZ) = v;
                } else {
                    int which;
                    const int64_t off = out_index(p, m, col, which);
                    *reinterpret_cast<u32x4 *>(kern::out_base(p, which) + off * ESZ) = v;
                }
            } else {
                static_for<0, PER>([&](auto ec) {
                    constexpr int e = decltype(ec)::value;
                    if (col + e < n_out) {
                        int we;
                        const int64_t oe = out_index(p, m, col + e, we);
                        uint8_t *oo = kern::out_base(p, we) + oe * ESZ;
                        if constexpr (ESZ == 2)
                            *reinterpret_cast<uint16_t *>(oo) = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
                        else
                            *reinterpret_cast<uint32_t *>(oo) = v[e];
                    }
                });
            }
        }
    });
}


// Scale, bias and activation of the 16 values of one accumulator block (a lane's columns 8g + 4h + e,
// value 4g + e), GLU: with the 16 of the paired block `u` (scales and biases `cu`). Each operation is
// applied to all 16 values before the next one, so a single wave per SIMD issues 16 independent
// instructions back to back instead of stalling on each value's dependent chain (GELU's is seven
// instructions with two transcendental ones); the operations per value are exactly those of gelu_tanh,
// silu_glu and situ (sq8_device.h), after __fmul_rn by the scale and __fadd_rn of the bias.
template <int EPI, bool HB>
__device__ __forceinline__ void block_values(const f32x16 &x, const ColParams &cx, const f32x16 &u, const ColParams &cu,
                                             float (&v)[16]) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    float t[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = __fmul_rn(x[e], cx.s[e >> 2][e & 3]);
    if constexpr (HB) {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = __fadd_rn(v[e], cx.b[e >> 2][e & 3]);
    }
    if constexpr (EPI == EPI_GELU) {
        // gelu_tanh: x / (1 + 2^(x·(k + k3·x²))).
#pragma unroll
        for (int e = 0; e < 16; ++e) t[e] = v[e] * v[e];
#pragma unroll
        for (int e = 0; e < 16; ++e) t[e] = __builtin_fmaf(kGeluK3, t[e], kGeluK);
#pragma unroll
        for (int e = 0; e < 16; ++e) t[e] = v[e] * t[e];
#pragma unroll
        for (int e = 0; e < 16; ++e) t[e] = __builtin_amdgcn_exp2f(t[e]);
#pragma unroll
        for (int e = 0; e < 16; ++e) t[e] = 1.0f + t[e];
#pragma unroll
        for (int e = 0; e < 16; ++e) t[e] = __builtin_amdgcn_rcpf(t[e]);
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = v[e] * t[e];
    } else if constexpr (GLU) {
        float w[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) w[e] = __fmul_rn(u[e], cu.s[e >> 2][e & 3]);
        if constexpr (HB) {
#pragma unroll
            for (int e = 0; e < 16; ++e) w[e] = __fadd_rn(w[e], cu.b[e >> 2][e & 3]);
        }
        if constexpr (EPI == EPI_SILU_GLU) {
            // silu_glu: g · 1/(1 + 2^(−g·log2 e)) · u.
#pragma unroll
            for (int e = 0; e < 16; ++e) t[e] = v[e] * -1.4426950408889634f;
#pragma unroll
            for (int e = 0; e < 16; ++e) t[e] = __builtin_amdgcn_exp2f(t[e]);
#pragma unroll
            for (int e = 0; e < 16; ++e) t[e] = 1.0f + t[e];
#pragma unroll
            for (int e = 0; e < 16; ++e) t[e] = __builtin_amdgcn_rcpf(t[e]);
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = v[e] * t[e];
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = v[e] * w[e];
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = situ(v[e], w[e]);
        }
    }
}

// Scale, bias and activation of one 32 × 32 output block (GLU: the pair of blocks) a wave holds in
// `x` (and `u`, with `cu`), written to the wave's LDS region as rows of 32 values, then stored as
// 16-byte row segments. Output columns [col0, col0 + 32), rows [m_first, m_first + 32).
template <int EPI, int OUT, bool HB>
__device__ __forceinline__ void stage_block(const f32x16 &x, const ColParams &cx, const f32x16 &u, const ColParams &cu,
                                            uint8_t *region, int lane) {
    constexpr int ESZ = OUT == OUT_BF16 ? 2 : 4;
    constexpr int PITCH = 32 * ESZ + 16;  // row bytes + 16: keeps 16-byte alignment, spreads banks
    const int h = lane >> 5, r = lane & 31;
    float y[16];
    block_values<EPI, HB>(x, cx, u, cu, y);
    static_for<0, 4>([&](auto gc) {
        constexpr int g = decltype(gc)::value;
        const int c = 8 * g + 4 * h;  // first of this lane's 4 columns in the block
        uint8_t *dst = region + r * PITCH + c * ESZ;
        if constexpr (OUT == OUT_BF16)
            *reinterpret_cast<u32x2 *>(dst) = u32x2{pack_bf16_rne(y[4 * g], y[4 * g + 1]), pack_bf16_rne(y[4 * g + 2], y[4 * g + 3])};
        else
            *reinterpret_cast<f32x4 *>(dst) = f32x4{y[4 * g], y[4 * g + 1], y[4 * g + 2], y[4 * g + 3]};
    });
}

// (The bias test is one uniform branch around the whole block, not a select per value.) The residual
// epilogue's operands: `pre` when the caller loaded them ahead (a block earlier), else loaded here first.
template <int EPI, int OUT>
__device__ __forceinline__ void store_block(const GemmArgs &p, const f32x16 &x, const ColParams &cx, const f32x16 &u,
                                            const ColParams &cu, bool has_bias, int col0, int m_first, int n_out,
                                            uint8_t *region, int lane, const ResidualPre *pre = nullptr) {
    ResidualPre own;
    if constexpr (EPI == EPI_RESIDUAL) {
        if (!pre) {
            load_residual(p, col0, m_first, n_out, lane, own);
            pre = &own;
        }
    }
    if (has_bias)
        stage_block<EPI, OUT, true>(x, cx, u, cu, region, lane);
    else
        stage_block<EPI, OUT, false>(x, cx, u, cu, region, lane);
    flush_region<EPI, OUT>(p, col0, m_first, n_out, region, lane, EPI == EPI_RESIDUAL ? pre : nullptr);
}

// The 16 values of one accumulator block as 8 bf16 pairs (block_values, then nearest-even pairs).
template <int EPI, bool HB>
__device__ __forceinline__ void block_bf16_pairs(const f32x16 &a, const ColParams &c, uint32_t (&pk)[8]) {
    float v[16];
    block_values<EPI, HB>(a, c, a, c, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) pk[i] = pack_bf16_rne(v[2 * i], v[2 * i + 1]);
}

// The bf16 epilogue of one whole 64-column slab (columns [col0, col0 + 64) of the product, in one
// output and one head), 32 rows at a time: both 32-column blocks of a row block are scaled, biased and
// activated in registers (block_bf16_pairs), written to the wave's LDS region (rows of 128 bytes, 16-byte
// chunks XOR-swizzled by row & 7) and read back as 16-byte chunks, eight lanes a row, so each store
// instruction writes eight whole 128-byte row segments; the row block's stores are in flight while the
// next one is computed. Rows past M are not stored. `region`: 32·FM·128 bytes of the wave's own.
template <int FM, int EPI, bool HB>
__device__ __forceinline__ void slab_rows_bf16(const GemmArgs &p, const f32x16 (&acc)[2][FM], const ColParams (&cp)[2],
                                               int m0, uint8_t *out, int64_t pitch, uint8_t *region, int lane) {
    const int h = lane >> 5, r = lane & 31, chunk = lane & 7;
    static_for<0, FM>([&](auto bmc) {
        constexpr int bm = decltype(bmc)::value;
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, 2>([&](auto bc) {
            constexpr int b = decltype(bc)::value;
            uint32_t pk[8];
            block_bf16_pairs<EPI, HB>(acc[b][bm], cp[b], pk);
            const int row = 32 * bm + r;
            static_for<0, 4>([&](auto gc) {
                constexpr int g = decltype(gc)::value;
                const int ch = 4 * b + g;  // 8 columns: 8g + [0, 8) of block b; this lane's half h
                *reinterpret_cast<u32x2 *>(region + row * 128 + ((ch ^ (row & 7)) << 4) + 8 * h) =
                    u32x2{pk[2 * g], pk[2 * g + 1]};
            });
        });
        static_for<0, 4>([&](auto ic) {
            constexpr int i = 4 * bm + decltype(ic)::value;
            const int row = 8 * i + (lane >> 3);
            const u32x4 v = *reinterpret_cast<const u32x4 *>(region + row * 128 + ((chunk ^ (row & 7)) << 4));
            if (m0 + row < p.M) *reinterpret_cast<u32x4 *>(out + (int64_t)row * pitch * 2) = v;
        });
    });
}

template <int FM, int EPI>
__device__ __forceinline__ void slab_epilogue_bf16(const GemmArgs &p, const f32x16 (&acc)[2][FM], const ColParams (&cp)[2],
                                                   bool has_bias, int m0, int col0, uint8_t *region, int lane) {
    // Where the slab's rows go: output `which` of the QKV split, then row-major (ldc) or head-major
    // ([heads, M, head_dim]: consecutive rows of one head are head_dim apart).
    int which = 0, cc = col0;
    if (p.split > 0) {
        which = col0 / p.split;
        cc = col0 - which * p.split;
    }
    int64_t first, pitch;
    if (p.head_dim > 0) {
        const int head = cc / p.head_dim;
        first = ((int64_t)head * p.M + m0) * p.head_dim + (cc - head * p.head_dim);
        pitch = p.head_dim;
    } else {
        first = (int64_t)m0 * p.ldc + cc;
        pitch = p.ldc;
    }
    uint8_t *const out = kern::out_base(p, which) + (first + (lane & 7) * 8) * 2;
    // (The bias test is one uniform branch around the whole slab, not a select per value.)
    if (has_bias)
        slab_rows_bf16<FM, EPI, true>(p, acc, cp, m0, out, pitch, region, lane);
    else
        slab_rows_bf16<FM, EPI, false>(p, acc, cp, m0, out, pitch, region, lane);
}

// True when a kernel's slab epilogue serves this product: bf16 output, a plain or GELU epilogue,
// whole 64-column slabs that each lie in one output and one head, 16-byte stores.
inline bool slab_epilogue_fits(const GemmArgs &p, int epi, int out) {
    return (epi == EPI_NONE || epi == EPI_GELU) && out == OUT_BF16 && p.glu_half == 0 && p.N % 64 == 0 &&
           p.split % 64 == 0 && p.head_dim % 64 == 0 && p.c_vec16;
}

// LEAN: the slab epilogue (slab_epilogue_fits holds); else each 32 × 32 block through store_block.
// NAS: activation stages and weight register buffers (OCC = 2): A(t + NAS − 1) and W(t + NAS) are issued in
// step t (the 32-row tiles take four: C2's text stream, 512 × 3072 × 3072, 23.5 against 24.9 µs).
// CB: 32-column blocks a wave owns — 2 (a 64-column slab, tiles BM × 64·NW) or 1 (wave w: block w & 1 of
// slab w ÷ 2, tiles BM × 32·NW; no GLU, no slab epilogue, two workgroups a CU): half the codes a wave widens
// per MFMA.
// KS (one-block waves only): groups of NW waves that split the K steps — group g takes steps g, g + KS, …
// with its own activation stages, so a CU holds KS times the waves and loads in flight for the same tile;
// at the end the groups' sums meet in LDS and are added in group order (deterministic), then group 0 runs
// the epilogue. K/64 must be a multiple of KS.
constexpr int wd_waves_per_eu(int occ, int nw, int ks) { return ks == 1 ? occ : ((nw * ks + 3) / 4 > occ ? (nw * ks + 3) / 4 : occ); }

template <int BM, int NW, int OCC, int WT, int WL, int EPI, int OUT, bool LEAN = false, int NAS = 2, int CB = 2, int KS = 1>
__global__ void __attribute__((amdgpu_flat_work_group_size(64 * NW * KS, 64 * NW * KS),
                               amdgpu_waves_per_eu(wd_waves_per_eu(OCC, NW, KS), wd_waves_per_eu(OCC, NW, KS))))
gemm_wd_kernel(const GemmArgs p) {
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    constexpr int FM = BM / 32;                      // 32-row blocks per wave
    constexpr int SA = BM * 128;                     // bytes per A stage
    constexpr int A_BLOCKS = BM / 8;                 // 1 KB (8-row) blocks per A stage
    // Activation blocks a wave loads per stage; when the waves outnumber an even split (six waves, eight
    // blocks) the last loads of some waves repeat one of their own blocks, so every wave issues the same
    // count (one vmcnt value fits them all) and each LDS block is written with the same bytes.
    constexpr int A_PER_WAVE = (A_BLOCKS + NW - 1) / NW;
    constexpr int WLD = 2 * CB;                      // 16-byte weight loads per lane per K step
    static_assert(CB == 2 || (CB == 1 && !GLU && !LEAN && OCC == 2), "one-block waves: no GLU, block epilogue");
    // Every wave issues the same number of activation loads, so one vmcnt value fits them all.
    static_assert(A_PER_WAVE + WLD < 64, "vmcnt budget");
    constexpr int REGION = 32 * (32 * (OUT == OUT_BF16 ? 2 : 4) + 16);  // epilogue bytes per wave
    // The epilogue regions lie over the A stages (both idle by then); short tiles need more than the stages.
    static_assert(NAS == 2 || OCC == 2, "deeper pipelines on the two-workgroup path");
    constexpr int LDS_STAGES = NW * REGION > NAS * SA ? NW * REGION : NAS * SA;
    // Loads a wave may leave in flight at the end of step t, A(t+1) and W(t+1) landed: W(t+2) issued in
    // step t+2−NAS after A(t+1), then every load of the NAS − 2 steps after that one.
    constexpr int STEP_WAIT = WLD + (NAS - 2) * (A_PER_WAVE + WLD);
    static_assert(STEP_WAIT < 64, "vmcnt budget");
    // The slab epilogue stages the wave's whole BM × 64 bf16 outputs.
    constexpr int LDS_ONE = LEAN && NW * BM * 128 > LDS_STAGES ? NW * BM * 128 : LDS_STAGES;
    static_assert(!LEAN || (OUT == OUT_BF16 && (EPI == EPI_NONE || EPI == EPI_GELU)), "slab epilogue: bf16, plain or GELU");
    static_assert(KS == 1 || (CB == 1 && OCC == 2 && !LEAN), "K groups: one-block waves");
    // K groups: each group's stages side by side; the later groups' sums go past the epilogue regions.
    constexpr int RED_BYTES = (KS - 1) * NW * CB * FM * 16 * 64 * 4;
    constexpr int LDS_KS = KS * NAS * SA > NW * REGION + RED_BYTES ? KS * NAS * SA : NW * REGION + RED_BYTES;
    constexpr int LDS_BYTES = KS == 1 || LDS_ONE > LDS_KS ? LDS_ONE : LDS_KS;

    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = KS == 1 ? 0 : wave_all / NW;      // K group
    const int wave = KS == 1 ? wave_all : wave_all - grp * NW;
    uint8_t *const ldg = lds + grp * (NAS * SA);      // the group's activation stages
    int tm, tn;
    kern::tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM;
    // The wave's weight columns: slab `slab`, blocks [b0, b0 + CB) (one-block waves: the tile's 32-column
    // block tn·NW + wave).
    const int slab = CB == 2 ? tn * NW + wave : (tn * NW + wave) >> 1;
    const int b0 = CB == 2 ? 0 : ((tn * NW + wave) & 1);
    const kern::gbytes Wg = (kern::gbytes)p.w;
    const int KT = p.kt;

    // ---- activation loads: wave block b = wave + NW·i, lane → row 8b + (lane>>3), chunk lane&7 ----
    uint32_t a_goff[A_PER_WAVE];
    int a_blk[A_PER_WAVE];
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i) {
        int b = wave + NW * i;
        if constexpr (A_BLOCKS % NW != 0) b = b < A_BLOCKS ? b : b - NW;
        a_blk[i] = b;
        const int r = 8 * b + (lane >> 3);
        const int lc = (lane & 7) ^ ((r ^ (r >> 3)) & 7);
        const int row = min(m0 + r, p.M - 1);
        a_goff[i] = (uint32_t)((int64_t)row * p.lda * 2) + lc * 16;
    }
    // t: the group's own step count; its K step is t·KS + grp. Through a buffer resource: the step's offset
    // in a scalar register, no per-lane address add.
    const i32x4 a_rsrc = buffer_rsrc(p.a);
    auto issue_a = [&](int t, auto stage) {
        constexpr int S = decltype(stage)::value;
        const int soff = __builtin_amdgcn_readfirstlane((int)((uint32_t)min(t * KS + grp, KT - 1) * (BK * 2)));
#pragma unroll
        for (int i = 0; i < A_PER_WAVE; ++i)
            raw_buffer_load_lds(a_rsrc, (lds_u32)(ldg + S * SA + a_blk[i] * 1024), 16, (int)a_goff[i], soff, 0, 0);
    };

    // ---- weight loads: WLD × 16 bytes per lane per K step (load j: block b0 + j ÷ 2, half j & 1) ------
    uint32_t w_off[WLD];
#pragma unroll
    for (int j = 0; j < WLD; ++j) w_off[j] = w_offset<WL, GLU>(p, slab, 2 * b0 + j, lane);
    const uint32_t w_step = WL == W_PACKED ? 4096 : BK;
    u32x4 raw[NAS][WLD];
    auto issue_w = [&](int t, auto buf) {
        constexpr int B = decltype(buf)::value;
        const kern::gbytes base = Wg + (uint32_t)weight_step(p, min(t * KS + grp, KT - 1)) * w_step;
#pragma unroll
        for (int j = 0; j < WLD; ++j) raw[B][j] = kern::gld<u32x4>(base, w_off[j]);
    };

    // ---- fragments -----------------------------------------------------------------------------------
    bf16x8 wf[2][CB][4];  // OCC = 1: [buffer][block][ks]
    auto widen_all = [&](auto src, auto dst) {
        constexpr int S = decltype(src)::value, D = decltype(dst)::value;
        static_for<0, CB>([&](auto bc) {
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

    f32x16 acc[CB][FM];
#pragma unroll
    for (int b = 0; b < CB; ++b)
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[b][bm][r] = 0.0f;

    // The MFMAs of one step on stage S with fragments F; OCC = 1 widens raw[R] into fragments 1−F
    // between them. Activation fragments of sub-step ks+1 are read before the MFMAs of ks.
    auto mfmas = [&](auto stage, auto frag, auto rawbuf) {
        constexpr int S = decltype(stage)::value, F = decltype(frag)::value, R = decltype(rawbuf)::value;
        bf16x8 xf[2][FM];
        auto read_x = [&](auto kc, auto bufc) {
            constexpr int ks = decltype(kc)::value, B = decltype(bufc)::value;
            static_for<0, FM>([&](auto bmc) {
                constexpr int bm = decltype(bmc)::value;
                xf[B][bm] = kern::lds_load_frag(lds + S * SA + 32 * 128 * bm, xo[bm & 1][ks]);
            });
        };
        read_x(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
        static_for<0, 4>([&](auto kc) {
            constexpr int ks = decltype(kc)::value;
            if constexpr (ks < 3) read_x(std::integral_constant<int, ks + 1>{}, std::integral_constant<int, (ks + 1) & 1>{});
            if constexpr (OCC == 1 && CB == 2) {
                // Widen the next step's block ks >> 1, sub-steps 2(ks & 1) and 2(ks & 1) + 1.
                constexpr int b = ks >> 1;
                static_for<0, 2>([&](auto qc) {
                    constexpr int q = 2 * (ks & 1) + decltype(qc)::value;
                    const u32x4 &r = raw[R][2 * b + (q >> 1)];
                    wf[1 - F][b][q] = widen8<WT>(r[2 * (q & 1)], r[2 * (q & 1) + 1]);
                });
            }
            static_for<0, FM>([&](auto bmc) {  // row block outer: a fragment's MFMAs back to back
                constexpr int bm = decltype(bmc)::value;
                static_for<0, CB>([&](auto bc) {
                    constexpr int b = decltype(bc)::value;
                    acc[b][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[F][b][ks], xf[ks & 1][bm], acc[b][bm], 0, 0, 0);
                });
            });
        });
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;

    if constexpr (NAS == 2) {
        // Prologue: A(0) → stage 0, W(0) → raw[0], W(1) → raw[1]; A(0) and W(0) landed.
        issue_a(0, I0{});
        issue_w(0, I0{});
        issue_w(1, I1{});
        wait_vmcnt<WLD>();
        if constexpr (OCC == 1) widen_all(I0{}, I0{});
    } else {
        // Prologue in the steps' issue order: A(0 .. NAS−2) and W(0 .. NAS−1), all landed.
        static_for<0, NAS>([&](auto vc) {
            constexpr int v = decltype(vc)::value;
            if constexpr (v > 0) issue_a(v - 1, std::integral_constant<int, v - 1>{});
            issue_w(v, vc);
        });
        wait_vmcnt<0>();
    }
    step_barrier();

    // OCC = 2: the codes of W(t) are widened just in time, one sub-step ahead of the MFMAs that use
    // them, like the activation fragments: two sub-steps of fragments are live at a time (the
    // registers a full step of widened codes would take are what lets the fragment reads be
    // double-buffered). raw[P] is free once sub-step 3 is widened: W(t+2) is issued then.
    // Step t reads activation stage S and widens raw[P] (NAS = 2: S = P = t mod 2).
    auto step_jit = [&](int t, auto stc, auto par) {
        constexpr int S = decltype(stc)::value;
        constexpr int P = decltype(par)::value;
        bf16x8 wk[2][CB];  // [ks & 1][block]
        bf16x8 xf[2][FM];
        auto widen_ks = [&](auto kc) {
            constexpr int ks = decltype(kc)::value;
            static_for<0, CB>([&](auto bc) {
                constexpr int b = decltype(bc)::value;
                const u32x4 &r = raw[P][2 * b + (ks >> 1)];
                wk[ks & 1][b] = widen8<WT>(r[2 * (ks & 1)], r[2 * (ks & 1) + 1]);
            });
        };
        auto read_x = [&](auto kc) {
            constexpr int ks = decltype(kc)::value;
            static_for<0, FM>([&](auto bmc) {
                constexpr int bm = decltype(bmc)::value;
                xf[ks & 1][bm] = kern::lds_load_frag(ldg + S * SA + 32 * 128 * bm, xo[bm & 1][ks]);
            });
        };
        __builtin_amdgcn_sched_barrier(0);
        read_x(I0{});
        widen_ks(I0{});
        // Into the stage read in step t − 1 (the barrier that ended it saw every wave's reads).
        issue_a(t + NAS - 1, std::integral_constant<int, (S + NAS - 1) % NAS>{});
        static_for<0, 4>([&](auto kc) {
            constexpr int ks = decltype(kc)::value;
            if constexpr (ks < 3) {
                read_x(std::integral_constant<int, ks + 1>{});
                widen_ks(std::integral_constant<int, ks + 1>{});
            }
            if constexpr (ks == 2) {
                // The A loads stay ahead of these in issue order (the vmcnt counts rely on it).
                __builtin_amdgcn_sched_barrier(0);
                issue_w(t + NAS, std::integral_constant<int, P>{});
                __builtin_amdgcn_sched_barrier(0);
            }
            static_for<0, FM>([&](auto bmc) {  // row block outer: a fragment's MFMAs back to back
                constexpr int bm = decltype(bmc)::value;
                static_for<0, CB>([&](auto bc) {
                    constexpr int b = decltype(bc)::value;
                    acc[b][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wk[ks & 1][b], xf[ks & 1][bm], acc[b][bm], 0, 0, 0);
                });
            });
            if constexpr (ks < 3) {
                static_for<0, 8>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if constexpr (i < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    if constexpr (i < 6) __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
                });
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<STEP_WAIT>();
        // Groups of one wave share no LDS within the K loop (each reads only the stages it loads itself).
        if constexpr (NW > 1 || KS == 1) step_barrier();
    };

    // One step t of parity P: stage P, W(t) in raw[P]. OCC = 1 widened W(t) during step t−1 and
    // widens W(t+1) from raw[1−P] now.
    auto one_step = [&](int t, auto par) {
        constexpr int P = decltype(par)::value;
        if constexpr (OCC == 2) {
            step_jit(t, par, par);
        } else {
            issue_a(t + 1, std::integral_constant<int, 1 - P>{});
            issue_w(t + 2, std::integral_constant<int, P>{});
            __builtin_amdgcn_sched_barrier(0);
            // W(t+1) must have landed before it is widened: the loads after it are this step's.
            wait_vmcnt<A_PER_WAVE + WLD>();
            mfmas(std::integral_constant<int, P>{}, std::integral_constant<int, P>{}, std::integral_constant<int, 1 - P>{});
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<WLD>();
            step_barrier();
        }
    };
    const int KTG = KT / KS;  // the group's steps
    if constexpr (NAS == 2) {
        int t = 0;
        for (; t + 1 < KTG; t += 2) {
            one_step(t, I0{});
            one_step(t + 1, I1{});
        }
        if (t < KTG) one_step(t, I0{});
    } else {
        // Step t + u on stage and buffer u.
        int t = 0;
        for (; t + NAS <= KTG; t += NAS)
            static_for<0, NAS>([&](auto uc) { step_jit(t + decltype(uc)::value, uc, uc); });
        static_for<0, NAS - 1>([&](auto uc) {
            if (t + decltype(uc)::value < KTG) step_jit(t + decltype(uc)::value, uc, uc);
        });
    }
    // The scales and biases of the wave's columns, loaded once for all its row blocks; their latency
    // overlaps the wait below.
    const bool has_bias = p.bias != nullptr;
    ColParams cp[CB];
    {
        const int n_out = GLU ? p.glu_half : p.N;
        static_for<0, CB>([&](auto bc) {
            constexpr int b = decltype(bc)::value;
            load_col_params(p, cp[b], GLU ? slab * 32 : slab * 64 + 32 * (b0 + b), GLU && b == 1 ? p.glu_half : 0, n_out,
                            lane);
        });
    }
    // Every wave's last (clamped) activation load has landed before any wave writes its epilogue
    // region over the stages.
    wait_vmcnt<0>();
    step_barrier();
    if constexpr (KS > 1) {
        // Groups 1 … KS−1 leave their sums in LDS ([group][wave][block][register][lane]); group 0 adds
        // them in group order.
        constexpr int PER_WAVE = CB * FM * 16 * 64;
        float *red = reinterpret_cast<float *>(lds + NW * REGION);
        if (grp > 0) {
            float *dst = red + ((grp - 1) * NW + wave) * PER_WAVE + lane;
#pragma unroll
            for (int b = 0; b < CB; ++b)
#pragma unroll
                for (int bm = 0; bm < FM; ++bm)
#pragma unroll
                    for (int r = 0; r < 16; ++r) dst[((b * FM + bm) * 16 + r) * 64] = acc[b][bm][r];
        }
        __syncthreads();
        if (grp > 0) return;
#pragma unroll
        for (int g = 1; g < KS; ++g) {
            const float *src = red + ((g - 1) * NW + wave) * PER_WAVE + lane;
#pragma unroll
            for (int b = 0; b < CB; ++b)
#pragma unroll
                for (int bm = 0; bm < FM; ++bm)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[b][bm][r] += src[((b * FM + bm) * 16 + r) * 64];
        }
    }

    // ---- epilogue ------------------------------------------------------------------------------
    // Lane l, register r of block (b, bm): row m0 + 32·bm + (l & 31), slab column
    // 32·b + 8·(r >> 2) + 4·(l >> 5) + (r & 3). The A stages are free: every wave passed the last
    // barrier after its last fragment read and after its last load into them landed.
    const int n_out = GLU ? p.glu_half : p.N;
    if constexpr (LEAN) {
        if (slab * 64 < p.N)
            slab_epilogue_bf16<FM, EPI>(p, acc, cp, has_bias, m0, slab * 64, lds + wave * (BM * 128), lane);
        return;
    }
    uint8_t *region = lds + wave * REGION;
    static_for<0, FM>([&](auto bmc) {
        constexpr int bm = decltype(bmc)::value;
        static_for<0, GLU ? 1 : CB>([&](auto bc) {
            constexpr int b = decltype(bc)::value;
            const int col0 = GLU ? slab * 32 : slab * 64 + 32 * (b0 + b);
            if (col0 < n_out)
                store_block<EPI, OUT>(p, acc[b][bm], cp[b], acc[GLU ? CB - 1 : b][bm], cp[GLU ? CB - 1 : b], has_bias, col0,
                                      m0 + 32 * bm, n_out, region, lane);
        });
    });
}

template <int BM, int NW, int OCC, int WT, int WL, int EPI, int OUT, bool LEAN = false, int NAS = 2, int CB = 2, int KS = 1>
hipError_t launch_wd(const GemmArgs &args, hipStream_t stream) {
    if (KS > 1 && args.kt % KS != 0) return hipErrorInvalidValue;
    constexpr bool GLU = EPI == EPI_SILU_GLU || EPI == EPI_SITU_GLU;
    GemmArgs p = args;
    p.tiles_m = (p.M + BM - 1) / BM;
    const int slabs = GLU ? (p.glu_half + 31) / 32 : (p.N + 63) / 64;
    p.tiles_n = CB == 2 ? (slabs + NW - 1) / NW : (p.N + 32 * NW - 1) / (32 * NW);
    const int blocks = p.tiles_m * p.tiles_n;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_wd_kernel<BM, NW, OCC, WT, WL, EPI, OUT, LEAN, NAS, CB, KS>), dim3(blocks), dim3(64 * NW * KS), 0,
                       stream, p);
    return hipGetLastError();
}

template <int BM, int NW, int OCC, int WT, int WL, int NAS = 2, int CB = 2, int KS = 1>
hipError_t dispatch_wd(const GemmArgs &p, int epi, int out, hipStream_t stream) {
    if (CB == 1 && (epi == EPI_SILU_GLU || epi == EPI_SITU_GLU)) return hipErrorInvalidValue;
    if (CB == 2 && slab_epilogue_fits(p, epi, out))
        return epi == EPI_GELU ? launch_wd<BM, NW, OCC, WT, WL, EPI_GELU, OUT_BF16, true, NAS>(p, stream)
                               : launch_wd<BM, NW, OCC, WT, WL, EPI_NONE, OUT_BF16, true, NAS>(p, stream);
#define SQ8_CASE(E, O)                                                                            \
    if (epi == E && out == O) return launch_wd<BM, NW, OCC, WT, WL, E, O, false, NAS, CB, KS>(p, stream);
    SQ8_CASE(EPI_NONE, OUT_BF16)
    SQ8_CASE(EPI_NONE, OUT_F32)
    SQ8_CASE(EPI_GELU, OUT_BF16)
    SQ8_CASE(EPI_GELU, OUT_F32)
    if constexpr (CB == 2) {
        SQ8_CASE(EPI_SILU_GLU, OUT_BF16)
        SQ8_CASE(EPI_SILU_GLU, OUT_F32)
        SQ8_CASE(EPI_SITU_GLU, OUT_BF16)
        SQ8_CASE(EPI_SITU_GLU, OUT_F32)
    }
    SQ8_CASE(EPI_RESIDUAL, OUT_F32)
#undef SQ8_CASE
    return hipErrorInvalidValue;
}

}  // namespace wd
}  // namespace sq8
