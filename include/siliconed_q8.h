/*
 * siliconed_q8.h — C ABI of the MI355X (gfx950) weight-quantized linear layer.
 *
 * The drop-in boundary for Siliconed's weight-product path: the Swift host keeps its operator API
 * (`WeightProducts.linear`, Sources/Siliconed/WeightProducts.swift:278, and its planning) and calls
 * these entry points where it encoded Metal work through `TensorGEMM`
 * (Sources/Siliconed/TensorGEMM.swift:206-360, TensorGEMMBF16.swift:208-264). Plain pointers and
 * sizes only; every pointer to tensor data is a device pointer the caller allocated and owns.
 *
 * Arithmetic (the reference's, TensorGEMM.swift:124-135 then :173-179): C = act(s ⊙ (A · q) + b)
 * with q the 8-bit codes widened exactly, fp32 sums, the scale applied after the sum, the bias
 * added after the scale (Ops.swift:400-407), the activation last.
 *
 * Status codes: 0 = success; > 0 = the call was refused before any work (invalid argument or a
 * configuration this library does not run: the caller keeps its widened route, as it does when
 * `TensorGEMM.init?` returns nil); < 0 = a HIP error, negated. No entry point aborts.
 *
 * Threading: a context is used by one host thread at a time (no internal locks); contexts on
 * different streams may run concurrently (Sources/Siliconed/Engine.swift:19 runs one render at a
 * time; GEMM.swift:166-194 guards only counters).
 */
#ifndef SILICONED_Q8_H
#define SILICONED_Q8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SQ8_ABI_VERSION 1

/* ---- status ---- */
enum sq8_status {
    SQ8_OK = 0,
    SQ8_EINVAL = 1,        /* a null pointer, a negative size, a stride shorter than a row */
    SQ8_EUNSUPPORTED = 2,  /* a valid configuration this library does not run */
    SQ8_ENODEVICE = 3,     /* no gfx950 device at that ordinal */
    SQ8_ECAPACITY = 4,     /* the problem needs more than the static scratch holds
                              (sq8_linear_quantized_static only) */
};

/* ---- element types (Artifact.DType, Sources/Siliconed/Artifact.swift:65-113) ---- */
enum sq8_dtype {
    SQ8_BF16 = 1,
    SQ8_F32 = 2,
    SQ8_INT8 = 3,
    SQ8_FP8_E4M3 = 4,      /* "fn": bias 7, no infinity, 0x7F/0xFF NaN (Forge/Numerics.swift:48-55) */
    SQ8_F16 = 5,
};

/* ---- weight layouts ---- */
enum sq8_wlayout {
    SQ8_KN = 0,            /* [K, N] row-major, N contiguous: the map's layout
                              (`linear_weights_transposed`, Artifact.swift:655) */
    SQ8_NK = 1,            /* [N, K] row-major, K contiguous: a published nn.Linear */
    SQ8_PACKED = 2,        /* sq8_pack_weight's layout (glu = 0); `ldw` is ignored */
    SQ8_PACKED_GLU = 3,    /* sq8_pack_weight's layout of a [first half | second half] GLU weight
                              (glu = 1), for the GLU epilogues only */
};

/* ---- scale layouts (Widen.ScaleLayout, Sources/Siliconed/Widen.swift:100-110) ---- */
enum sq8_scale_layout {
    SQ8_SCALE_TENSOR = 0,  /* one scale: `perColumn` false (TensorGEMM.swift:264, :353) */
    SQ8_SCALE_COLUMNS = 1, /* one per output channel: `perColumn` true */
    SQ8_SCALE_BLOCKS = 2,  /* [K/b, N] (sq8_dequantize; the product: sq8_linear_blocks) */
    SQ8_SCALE_ROWS = 3,    /* one per row of [N, K] (dequantize only) */
};

/* ---- epilogues ---- */
enum sq8_epilogue {
    SQ8_EPI_NONE = 0,      /* C = s ⊙ (A·q) (+ b) */
    SQ8_EPI_GELU_TANH = 1, /* nn.GELU(approximate="tanh") (Ops.swift:386-398) */
    SQ8_EPI_SILU_GLU = 2,  /* n = 2h, output h: silu(gate)·up, gate = columns [0, h)
                              (ElementwiseGPU.swift:67-73 on Block.swift:499-504's w1/w3) */
    SQ8_EPI_SITU_GLU = 3,  /* n = 2h, output h: 4·tanh(g/4)·σ(g)·25·tanh(v/25), value = columns
                              [0, h), gate = [h, 2h) (MossImage.swift:874-876, 889-900) */
};

typedef struct sq8_ctx sq8_ctx;

/* Creates a context on HIP device `device`, launching on `stream` (a hipStream_t; NULL = the
 * device's null stream). Refuses (SQ8_ENODEVICE) a device that is not gfx950.
 * Three measurement knobs are read from the environment here, once per context: SQ8_TILE ("256",
 * "224", "128", "64", "32", "64n", "64x192", "s64", "s32", "gemv", "k32x32", "k32x64", "k64x64", "k64x128",
 * "k64x192": the weight-direct kernels' tile),
 * SQ8_Q8_TILE ("256", "512", "128x256", "128x128": the block-scale kernel's tile) and SQ8_SPLITS (a
 * count ≥ 1: the skinny
 * kernel's K split over workgroups, added by a second launch; 1, the default, none; at most the
 * product's K steps). A context created with
 * one set runs every product of that family on that tile (a tile that cannot serve a product falls
 * back to the nearest one that can); unset, the library chooses per product.
 * Replaces: TensorGEMM.init?(device:queue:roundingActivations:quantizingActivations:)
 * (Sources/Siliconed/TensorGEMM.swift:206-232). */
int sq8_create(int device, void *stream, sq8_ctx **out);

/* Releases the context and its scratch memory. Replaces: the TensorGEMM instance's release. */
int sq8_destroy(sq8_ctx *ctx);

/* Changes the stream later launches go to, after the work already queued on the previous stream has
 * finished (the context's scratch and packing buffer serve one stream at a time).
 * Replaces: the command queue passed at init (TensorGEMM.swift:206). */
int sq8_set_stream(sq8_ctx *ctx, void *stream);

/* 0 when `sq8_linear` runs this combination, else SQ8_EUNSUPPORTED / SQ8_EINVAL — the caller then
 * keeps the widened route. Replaces: the nil checks on `TensorGEMM.rounded`/`.int8`
 * (TensorGEMM.swift:218-229, `roundsActivations`, `readsBlocks`). */
int sq8_supports(const sq8_ctx *ctx, int a_dtype, int w_dtype, int w_layout, int scale_layout,
                 int c_dtype, int epilogue);

/* **The product**: C[m, n_out] = act(s ⊙ (A[m, k] · W) + b), W the 8-bit codes of `w_dtype` in
 * `w_layout` with leading dimension `ldw` (elements), `scale` fp32 ([n] per column or [1] per
 * tensor), `bias` fp32 [n] or NULL, A of `a_dtype` (SQ8_BF16, or SQ8_F32: rounded to bf16
 * nearest-even first, as `submitRounded` rounds its operand, TensorGEMMBF16.swift:41-48, 208-264),
 * C of `c_dtype` (SQ8_F32 as the reference writes it, or SQ8_BF16), written, not accumulated.
 * n_out = n, or n/2 for the GLU epilogues. A computes only the first `n` columns of a wider W when
 * `ldw`/`ldc` say so (the `columns` argument of `submit`, TensorGEMM.swift:296).
 * `gpu_seconds`: NULL → the launch is queued and the call returns at once (`settled`,
 * TensorGEMM.swift:261-263); non-NULL → the call waits and writes the kernel's GPU seconds
 * (TensorGEMM.swift:268-272, `Attention.verdict`). One exception to "at once": the context's
 * growable buffers — the bf16 copy (or, on the fp32 route, the three parts) of an fp32 A, the
 * repack of [K, N] codes read in place, and the fp32 partial sums of a short product whose K steps
 * are split over several workgroups (added by a second launch) — are sized by the largest product so far; a call that needs
 * more first synchronizes the context's stream (queued work may still read the old buffer), frees
 * and allocates. A caller that must never block runs one product of its largest shape first.
 * Replaces: TensorGEMM.linear(a:int8:weightOffset:scales:scalesOffset:perColumn:block:rotation:
 * rounding:quantizing:prequantized:c:m:k:n:settled:) -> Double (TensorGEMM.swift:264-290) and
 * its encoders submit (:296-360) / submitRounded (TensorGEMMBF16.swift:208-264), with the bias
 * (DiT.swift:403-413) and activation passes (Ops.swift:386-398, ElementwiseGPU.swift:67-73,
 * MossImage.swift:889-900) fused. */
int sq8_linear(sq8_ctx *ctx,
               const void *a, int a_dtype, int64_t lda,
               const void *w, int w_dtype, int w_layout, int64_t ldw,
               const float *scale, int scale_layout,
               const float *bias, int epilogue,
               void *c, int c_dtype, int64_t ldc,
               int m, int k, int n, double *gpu_seconds);

/* **The fp32 route**: the product on an fp32 activation used whole, not rounded — the reference's
 * `submit` on fp32 A (`linear_int8` and the `blocks` pipeline with fp32 operands, TensorGEMM.swift:125-135,
 * 296-360), judged by its fp32 bar (≤ 1e-5 per channel, Diagnostic.swift:105). Each value is split into three
 * bf16 parts hi + mid + lo = x along K (each the top 16 bits of what the one before leaves: 24 significant bits
 * in three parts of 8, none rounded; all normal for |x| ≥ 2^-103), so every product with a code is exact and
 * the sums are fp32: three times the MFMA work of the rounded route. Any K (the parts padded with zeros to
 * whole 64-wide steps, the weight packed with zero codes past K).
 *   `group` ≠ 0: convrot, A rotated by groups of `group` in fp32 first (TensorGEMM.swift:334-345), as
 *   sq8_linear_rotated; 0: none.
 *   `scale_layout` SQ8_SCALE_COLUMNS / SQ8_SCALE_TENSOR: fp32 scales (`scale_dtype` SQ8_F32, `block` 0),
 *   the weight int8 or fp8 as sq8_linear takes it (packed, [N, K], or [K, N] repacked);
 *   SQ8_SCALE_BLOCKS: int8 codes with one scale per `block` rows of K and column as sq8_linear_blocks
 *   takes them (no rotation).
 * Other arguments as sq8_linear. Replaces: TensorGEMM.linear(a:int8:…) with `rounding` nil
 * (TensorGEMM.swift:264-290). */
int sq8_linear_f32(sq8_ctx *ctx,
                   const float *a, int64_t lda, int group,
                   const void *w, int w_dtype, int w_layout, int64_t ldw,
                   const void *scale, int scale_dtype, int scale_layout, int block,
                   const float *bias, int epilogue,
                   void *c, int c_dtype, int64_t ldc,
                   int m, int k, int n, double *gpu_seconds);

/* **The bf16-weight product**: C fp32 [m, n] (leading dimension ldc) = A [m, k] · W, W bf16 [k, n]
 * (SQ8_KN: `weightIsTransposed`, the forge's layout) or [n, k] (SQ8_NK), no scale, no bias, C written. A fp32
 * (`a_dtype` SQ8_F32) is used whole — split into three exact bf16 parts as on the fp32 route, every product
 * exact, the sums fp32 — or bf16 (SQ8_BF16). A plain GEMM: the library GEMM (rocBLAS) runs it.
 * Replaces: TensorGEMM.linear(a:w:c:m:k:n:weightIsTransposed:) (TensorGEMM.swift:236-254). */
int sq8_linear_bf16_weight(sq8_ctx *ctx,
                           const void *a, int a_dtype, int64_t lda,
                           const void *w, int w_layout, int64_t ldw,
                           float *c, int64_t ldc,
                           int m, int k, int n, double *gpu_seconds);

/* Bytes of the packed layout of a weight of k × n codes (GLU: n = 2h, the halves paired).
 * Replaces: the reserve plan's size of the staged integers (WeightProducts.int8Plan,
 * Sources/Siliconed/WeightProducts.swift:535-600). */
int64_t sq8_packed_bytes(int k, int n, int glu);

/* **Staging**: rewrites the codes of a weight (`w_layout` SQ8_KN or SQ8_NK, leading dimension
 * `ldw`, k × n codes) into the layout the product streams fastest — per 64-column slab, per step
 * of 64 K, per lane, 16 contiguous bytes, zero-padded — into `out` (sq8_packed_bytes bytes, device
 * memory the caller owns). Once per weight, before its products; the bytes are the same codes
 * (no widening, the scales untouched). `glu` = 1 pairs the two halves of a gate-up weight for the
 * GLU epilogues. Queued on the context's stream.
 * Replaces: Artifact.stageInt8, the copy of q and its scales into the model's reserve
 * (Sources/Siliconed/Artifact.swift:755-774), for the packed route. */
int sq8_pack_weight(sq8_ctx *ctx, const void *w, int w_layout, int64_t ldw, int k, int n, int glu, void *out);

/* **The fused QKV product**: one product of n = 3·d columns whose output columns [0,d), [d,2d),
 * [2d,3d) go to `q`, `k`, `v`. `head_dim` = 0: each output is [m, d] row-major (leading
 * dimension `ldo`); `head_dim` > 0: each is [d/head_dim, m, head_dim] (heads outermost, the layout
 * an attention kernel reads), `ldo` ignored. Epilogue: none (bias added if given).
 * Replaces: the MOSS text block's fused qkv product, bias pass and row split
 * (MossImage.swift:548-560); the DiT blocks' three products on one operand (Block.swift:410-415). */
int sq8_linear_qkv(sq8_ctx *ctx,
                   const void *a, int a_dtype, int64_t lda,
                   const void *w, int w_dtype, int w_layout, int64_t ldw,
                   const float *scale, int scale_layout, const float *bias,
                   void *q, void *k_out, void *v, int c_dtype, int64_t ldo, int head_dim,
                   int m, int k, int d, double *gpu_seconds);

/* **The dequantiser on the device**: out[i] = Float(code[i]) · s[layout(i)], one fp32 multiply
 * (never fused), for `rows` × `columns` codes in row-major order; scale fp32/bf16/fp16
 * (`scale_dtype`), NULL → the plain conversion. `block_rows`: rows per scale (BLOCKS);
 * `first_row`: the row of codes[0] in the whole tensor (BLOCKS, ROWS). The codes go through the
 * same conversion the product uses, so this is the bit-exact check of it.
 * Replaces: Widen.dequantize (Sources/Siliconed/Widen.swift:129-271) as reached from
 * Artifact.materialize (Artifact.swift:670-713). */
int sq8_dequantize(sq8_ctx *ctx, const void *codes, int w_dtype, int64_t rows, int64_t columns,
                   const void *scale, int scale_dtype, int scale_layout, int64_t block_rows,
                   int64_t first_row, float *out);

/* fp32 → bf16, nearest-even, NaN kept quiet (2·count bytes written).
 * Replaces: the `round_bf16` pass (TensorGEMMBF16.swift:41-48, 67-73). */
int sq8_round_bf16(sq8_ctx *ctx, const float *x, uint16_t *y, int64_t count);

/* ---- ComfyUI's int8 convrot: the weight published rotated, W = (q·s)·R, R = H/√G block-diagonal
 * along the input, G ∈ {4, 16, 64, 256}, H the Kronecker power of the regular Hadamard
 * H4 = [[1,1,1,−1],[1,1,−1,1],[1,−1,1,1],[−1,1,1,1]] (Sources/Siliconed/Widen.swift:316-343).
 * A group that is not one of those, or k not a multiple of it, is SQ8_EINVAL (the reference's
 * precondition, Widen.swift:381). ---- */

/* **The product of a rotated weight**: `sq8_linear` on the activation rotated first, C = act(s ⊙
 * ((A·R) · q) + b), A·R computed in fp32 by the reference's butterflies then rounded to bf16 once
 * (A fp32 or bf16), into the context's scratch. Replaces: TensorGEMM.linear(…rotation:…) with
 * `rotation` set (TensorGEMM.swift:264-290), i.e. submitRounded's rotate_groups → round_bf16 →
 * product (TensorGEMMBF16.swift:208-264) and submit's rotate_groups → product (TensorGEMM.swift:335-346). */
int sq8_linear_rotated(sq8_ctx *ctx,
                       const void *a, int a_dtype, int64_t lda, int group,
                       const void *w, int w_dtype, int w_layout, int64_t ldw,
                       const float *scale, int scale_layout,
                       const float *bias, int epilogue,
                       void *c, int c_dtype, int64_t ldc,
                       int m, int k, int n, double *gpu_seconds);

/* **The activation's rotation**: y = x·R for `rows` rows of k values; x SQ8_F32 or SQ8_BF16 (leading
 * dimension ldx), y SQ8_F32 or SQ8_BF16 (rounded to nearest even; ldy). fp32 butterflies in the
 * reference's stage order (spans 1, 4, 16, 64), then × 1/√G. y may be x itself (same type and
 * leading dimension), no other overlap. Replaces: `rotate_groups` (TensorGEMM.swift:181-201) and,
 * with a bf16 y, the `round_bf16` after it (TensorGEMMBF16.swift:222-233); the rotation once per
 * input for several products on it (DecodeKernels.swift:19-21). */
int sq8_rotate_groups(sq8_ctx *ctx, const void *x, int x_dtype, int64_t ldx, void *y, int y_dtype, int64_t ldy,
                      int rows, int k, int group);

/* **The rotated weight widened**: out[r, c] = Float(m) · (s_c · 1/√G), m = H·q over each group of
 * `group` rows of column c (exact integers), for int8 codes [k, n] (leading dimension ldq) rotated
 * along k; scale SQ8_F32/SQ8_BF16/SQ8_F16, one per column (SQ8_SCALE_COLUMNS) or one
 * (SQ8_SCALE_TENSOR); out fp32 [k, n] (leading dimension ldo). A slice of columns is the same call
 * on codes + first, scale + first, with n = the slice's width. Replaces: Widen.dequantizeRotated
 * (Widen.swift:374-428), as reached from Artifact.materialize (Artifact.swift:694-706). */
int sq8_dequantize_rotated(sq8_ctx *ctx, const int8_t *codes, int64_t ldq, int k, int n, int group,
                           const void *scale, int scale_dtype, int scale_layout, float *out, int64_t ldo);

/* ---- W8A8: ComfyUI's int8_linear, the activation quantized per row (after its convrot rotation,
 * if any), int8 × int8 products summed exactly in int32, C = act(float(Σ) · (s_x · s_w) + b)
 * (Sources/Siliconed/TensorGEMMInt8.swift:4-37). Weights int8 only (w_dtype implied); k below 2^17
 * (the int32 sums exact). ---- */

/* **The activation's quantization**: per row of x (SQ8_F32 or SQ8_BF16, `rows` × k, leading
 * dimension ldx), rotated by groups of `group` first (0: none; else 4, 16, 64 or 256 dividing k),
 * s = max(max|y| / 127, 1e-30), codes = clamp(rint(y / s), −128, 127) — correctly rounded divisions,
 * rint half to even; codes int8 [rows, ldq], scales fp32 [rows]. k up to 32 768 (else
 * SQ8_EUNSUPPORTED). Replaces: `quantize_rows` / `quantize_held` (TensorGEMMInt8.swift:78-131),
 * whose CPU statement is W8A8.quantize (:198-221). */
int sq8_quantize_rows(sq8_ctx *ctx, const void *x, int x_dtype, int64_t ldx, int rows, int k, int group,
                      int8_t *codes, int64_t ldq, float *scales);

/* **The W8A8 product on a quantized activation**: codes int8 [m, ldq] with their row scales `sx`
 * (fp32 [m]) — as sq8_quantize_rows writes them —, the int8 weight in `w_layout` (SQ8_PACKED(_GLU)
 * as sq8_pack_weight stages it, SQ8_NK or SQ8_KN), `scale` fp32 per column or per tensor, `bias` fp32
 * [n] or NULL, the epilogue fused; C fp32 or bf16 [m, n_out]. Replaces: submitQuantized with
 * `prequantized` (TensorGEMMInt8.swift:237-281: the codes written by the operand's producer or the
 * product before) — `linear_i8i8` then `scale_products`, with the bias and activation passes fused. */
int sq8_linear_w8a8(sq8_ctx *ctx, const int8_t *codes, int64_t ldq, const float *sx,
                    const void *w, int w_layout, int64_t ldw,
                    const float *scale, int scale_layout, const float *bias, int epilogue,
                    void *c, int c_dtype, int64_t ldc, int m, int k, int n, double *gpu_seconds);

/* **The W8A8 route whole**: `a` (SQ8_F32 or SQ8_BF16) quantized per row (rotated by `group` first,
 * 0 for none) into the context's scratch, then the product as sq8_linear_w8a8. Replaces:
 * submitQuantized (TensorGEMMInt8.swift:237-281): quantize_rows → linear_i8i8 → scale_products. */
int sq8_linear_quantized(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, int group,
                         const void *w, int w_layout, int64_t ldw,
                         const float *scale, int scale_layout, const float *bias, int epilogue,
                         void *c, int c_dtype, int64_t ldc, int m, int k, int n, double *gpu_seconds);

/* **The W8A8 route whole, allocating nothing.** No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Arguments, arithmetic and results as sq8_linear_quantized (the same kernels, the
 * same bits), but the activation's codes and row scales go to a static scratch array of
 * SQ8_STATIC_SCRATCH_BYTES on each GPU, held from the library's load until the process ends, instead
 * of the context's growable scratch; nothing is allocated or freed and, with `gpu_seconds` NULL, the
 * stream is never synchronized by the call (a non-NULL `gpu_seconds` records two events and waits for
 * the second, which graph capture does not allow: pass NULL there). Limits: the codes (m rows of k rounded up to 128, the total rounded up to
 * 256 bytes) and 4·m bytes of row scales must fit (else SQ8_ECAPACITY), and the weight must be
 * packed (SQ8_PACKED / SQ8_PACKED_GLU) or [N, K] int8 with k % 128 == 0, ldw % 16 == 0 and a 16-byte
 * aligned base, the layouts the kernel reads in place (else SQ8_EUNSUPPORTED: a repack would need a
 * buffer). Every call on one GPU shares that GPU's array and leaves its codes there: calls that
 * overlap on one GPU (contexts on different streams) race and must be ordered by the caller. */
#define SQ8_STATIC_SCRATCH_BYTES (64ll << 20)
int sq8_linear_quantized_static(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, int group,
                                const void *w, int w_layout, int64_t ldw,
                                const float *scale, int scale_layout, const float *bias, int epilogue,
                                void *c, int c_dtype, int64_t ldc, int m, int k, int n,
                                double *gpu_seconds);

/* The static scratch's capacity in bytes (SQ8_STATIC_SCRATCH_BYTES). */
int64_t sq8_static_scratch_bytes(void);

/* **A product added into the residual stream**: x[m, n] += gate ⊙ (s ⊙ (A·W) + b), x fp32 (leading
 * dimension ldx) read and written in place, gate fp32 [n] or NULL (1), the sum in fp32 (not rounded
 * to bf16 first), then x + gate·y with each product and sum rounded on its own. Arguments otherwise
 * as sq8_linear (no activation); any K (a K that is not a multiple of 64 is padded with zeros in the
 * context's scratch, the weight repacked per product). Replaces: the Wo / W_down product and `x += gate · …` of a DiT block
 * (MossImage.swift:15-19; the residual loop of ElementwiseGPUAnima.swift:47-62), one pass. */
int sq8_linear_residual(sq8_ctx *ctx,
                        const void *a, int a_dtype, int64_t lda,
                        const void *w, int w_dtype, int w_layout, int64_t ldw,
                        const float *scale, int scale_layout, const float *bias, const float *gate,
                        float *x, int64_t ldx, int m, int k, int n, double *gpu_seconds);

/* The same on the W8A8 route: x += gate ⊙ (float(Σ codes·q) · (s_x · s_w) + b). */
int sq8_linear_w8a8_residual(sq8_ctx *ctx, const int8_t *codes, int64_t ldq, const float *sx,
                             const void *w, int w_layout, int64_t ldw,
                             const float *scale, int scale_layout, const float *bias, const float *gate,
                             float *x, int64_t ldx, int m, int k, int n, double *gpu_seconds);

/* **The W8A8 fused QKV product**: sq8_linear_w8a8 of n = 3·d columns whose outputs [0,d), [d,2d),
 * [2d,3d) go to q, k, v — row-major [m, d] (head_dim 0, leading dimension ldo) or head-major
 * [d/head_dim, m, head_dim]; bias if given, no activation. Replaces: the fused QKV of a block whose
 * weights take the W8A8 route (MossImage.swift:548-560, Block.swift:410-415, on submitQuantized). */
int sq8_linear_w8a8_qkv(sq8_ctx *ctx, const int8_t *codes, int64_t ldq, const float *sx,
                        const void *w, int w_layout, int64_t ldw,
                        const float *scale, int scale_layout, const float *bias,
                        void *q, void *k_out, void *v, int c_dtype, int64_t ldo, int head_dim,
                        int m, int k, int d, double *gpu_seconds);

/* ---- the elementwise passes of a DiT block around the products (all device pointers, queued) ---- */

/* **Modulated RMSNorm to the next product's operand**: for each of `rows` rows of fp32 x (leading
 * dimension `ldx`), out = bf16(((x·r)·w)·(1 + scale) + shift) with r = 1/sqrt(mean(x²) + eps), every
 * product and sum rounded on its own; w, scale, shift fp32 [cols]; out bf16, leading dimension `ldo`.
 * Replaces: `norm_modulate_rounded` (Sources/Siliconed/ElementwiseGPUMoss.swift:45-91), the
 * `modulatedNorm` of a MOSS block (MossImage.swift:399, :418). */
int sq8_norm_modulate(sq8_ctx *ctx, const float *x, int64_t ldx, const float *w, const float *scale,
                      const float *shift, float eps, uint16_t *out, int64_t ldo, int rows, int cols);

/* **The modulated RMSNorm writing a convrot product's operand**: y = ((x·r)·w)·(1 + scale) + shift as
 * sq8_norm_modulate computes it in fp32 (the same r, the same bits), then y·R by groups of `group`
 * (4, 16, 64 or 256 dividing cols) rounded to bf16 into `out` — what sq8_rotate_groups writes from y,
 * one pass instead of two; y itself into `y_out` (fp32, leading dimension ldy) unless NULL. cols a
 * multiple of 4 up to 32 768, rows and vectors 16-byte aligned (else SQ8_EUNSUPPORTED). Replaces:
 * the norm then rotate_groups and round_bf16 before a convrot product (ElementwiseGPUMoss.swift:45-91,
 * TensorGEMMBF16.swift:222-233); the producer-rounded operand (WeightProducts.swift:130-229). */
int sq8_norm_modulate_rotated(sq8_ctx *ctx, const float *x, int64_t ldx, const float *w, const float *scale,
                              const float *shift, float eps, int group, uint16_t *out, int64_t ldo,
                              float *y_out, int64_t ldy, int rows, int cols);

/* **The modulated RMSNorm writing a W8A8 product's operand**: y as above, rotated by `group` (0: none)
 * and quantized per row into codes int8 [rows, ldq] and scales fp32 [rows] — sq8_quantize_rows's bits
 * on y; y into `y_out` unless NULL. Same limits. Replaces: `norm_modulate_quantized`
 * (ElementwiseGPUMoss.swift:94-130) writing `RoundedOperand.int8` (WeightProducts.swift:144-229). */
int sq8_norm_modulate_quantized(sq8_ctx *ctx, const float *x, int64_t ldx, const float *w, const float *scale,
                                const float *shift, float eps, int group, int8_t *codes, int64_t ldq,
                                float *scales, float *y_out, int64_t ldy, int rows, int cols);

/* **Per-row RMSNorm in place** of bf16 rows of `cols` ≤ 256 values (the heads of q or k):
 * t = bf16((t·r)·w), r = 1/sqrt(mean(t²) + eps), w fp32 [cols]. Replaces: the per-head RMSNorm of
 * q and k (`RMS_h`, MossImage.swift:15-19). */
int sq8_rms_rows(sq8_ctx *ctx, uint16_t *t, int64_t ld, int64_t rows, int cols, const float *w, float eps);

/* **Gated residual update**: x[r, c] += gate[c] · y[r, c] (the product rounded, then the sum) over
 * `rows` × `cols`; x fp32 (leading dimension `ldx`), y `y_dtype` SQ8_BF16 or SQ8_F32 (`ldy`), gate
 * fp32 [cols] or NULL (1). Replaces: `x += gate · …` of a DiT block (MossImage.swift:15-19), the
 * residual loop of `residual_modulate` (ElementwiseGPUAnima.swift:47-62). */
int sq8_gated_residual(sq8_ctx *ctx, float *x, int64_t ldx, const void *y, int y_dtype, int64_t ldy,
                       const float *gate, int64_t rows, int cols);

/* ---- codes with a scale per block of rows and column: GGUF Q8_0 (w = q · d, one fp16 d per 32
 * consecutive K of an output; Sources/Siliconed/Forge/GGUF.swift, `deinterleaveQ8_0`) ---- */

/* **The product on block scales**: C[m, n_out] = act(A · W + b), W[k, c] = q[k, c] · s[k / block, c],
 * int8 codes q, `block` a multiple of 32 dividing k (Q8_0: 32), any k (A padded with zeros to whole 64-wide
 * steps against the packed copy's zero codes). Codes in
 * `w_layout` SQ8_KN ([k, n], scales [k/block, n] row-major with the codes' row stride `ldw` — the
 * map's `[K/b, N]`; n < ldw computes the first n columns, `submit(…columns:)`) or SQ8_NK
 * ([n, k], scales [n, k/block] — GGUF's rows of blocks), scales of `scale_dtype` SQ8_F32, SQ8_BF16
 * or SQ8_F16 (widened exactly); or SQ8_PACKED(_GLU): `w` written by sq8_pack_blocks, which holds the
 * scales (`scale`, `scale_dtype`, `ldw` ignored). Each block's fp32 partial sum of exact bf16 × code
 * products is scaled once complete (the reference widens q·s first; the two agree in exact
 * arithmetic). A, bias, epilogues, C, `gpu_seconds` as sq8_linear. Replaces: TensorGEMM.linear(…
 * block: B …) (TensorGEMM.swift:264-290) and its `linear_q8` encoder (TensorGEMM.swift:137-171,
 * :307-318), with its rounded-activation route (TensorGEMMBF16.swift, `roundsBlocks`). */
int sq8_linear_blocks(sq8_ctx *ctx,
                      const void *a, int a_dtype, int64_t lda,
                      const void *w, int w_layout, int64_t ldw,
                      const void *scale, int scale_dtype, int block,
                      const float *bias, int epilogue,
                      void *c, int c_dtype, int64_t ldc,
                      int m, int k, int n, double *gpu_seconds);

/* Bytes of sq8_pack_blocks' layout (codes, then fp32 scales per step and column), or −1. Replaces:
 * the reserve plan's size of a staged Q8_0 weight (WeightProducts.int8Plan, WeightProducts.swift:535-600). */
int64_t sq8_packed_blocks_bytes(int k, int n, int glu);

/* **Staging a block-scaled weight**: codes (`w_layout` SQ8_KN or SQ8_NK, `ldw`) and their scales (as
 * sq8_linear_blocks reads them) rewritten into the packed Q8 layout in `out` (16-byte aligned
 * device memory of sq8_packed_blocks_bytes bytes). `glu` pairs the halves of a gate-up weight.
 * Once per weight; queued on the context's stream. Replaces: Artifact.stageInt8's copy of q and
 * its block scales (Artifact.swift:755-774) for the Q8_0 route. */
int sq8_pack_blocks(sq8_ctx *ctx, const void *w, int w_layout, int64_t ldw, const void *scale, int scale_dtype,
                    int block, int k, int n, int glu, void *out);

/* Waits for everything queued on the context's stream. Replaces: waitUntilCompleted /
 * GPUStream.drain (GPUStream.swift). */
int sq8_synchronize(sq8_ctx *ctx);

/* A static English string for a status code (never NULL). */
const char *sq8_status_string(int status);

/* SQ8_ABI_VERSION of the library. */
int sq8_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif
