// sq8_api.hip — the C ABI (include/siliconed_q8.h) over the gfx950 kernels: argument checks,
// the launch choice, GPU timing, status codes. No entry point aborts; none allocates per call
// except the context's scratch for an fp32 activation, grown when a larger one arrives.
#include "siliconed_q8.h"

#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <initializer_list>
#include <mutex>
#include <new>

#include "sq8_gemm.h"

// The allocation-free entry point's device memory (sq8_linear_quantized_static): one array per GPU,
// held from the library's load until the process ends. Host code never names it in device work: the
// name is a host-side stand-in; its device address on each GPU comes from hipGetSymbolAddress, taken
// once per device (static_scratch_of) and used wherever a kernel or a copy needs the memory.
static __device__ __align__(256) uint8_t scratch[SQ8_STATIC_SCRATCH_BYTES];

struct sq8_ctx {
    int device;
    hipStream_t stream;
    hipEvent_t begin, end;
    void *scratch;          // bf16 copy of an fp32 activation (the reference's rounding scratch)
    size_t scratch_bytes;
    void *wpack;            // [K, N] codes repacked for the weight-direct kernels, per product
    size_t wpack_bytes;
    void *part;             // the skinny kernel's partial sums of a K split
    size_t part_bytes;
    rocblas_handle blas;    // the bf16-weight product's library GEMM (created on its first call)
    int wd_tile;            // measurement knobs, read once at sq8_create (SQ8_TILE, SQ8_Q8_TILE, SQ8_SPLITS): a
    int q8_tile;            // forced weight-direct / block-scale tile, or -1 (the product's own choice); the
    int splits;             // skinny kernel's K split count (1: none, the default)
    int cus;                // the device's compute units, read once here: the tile rules' rounds
};

namespace {

int hip_status(hipError_t e) { return e == hipSuccess ? SQ8_OK : -(int)e; }

// The static scratch's device address per device ordinal, looked up once with that device current.
constexpr int kMaxDevices = 64;
std::mutex g_static_mutex;
uint8_t *g_static_ptr[kMaxDevices];

// The address of `scratch` on `device` (the current device), looked up on the first call for it.
hipError_t static_scratch_of(int device, uint8_t **out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_static_mutex);
    if (!g_static_ptr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_static_ptr[device] = static_cast<uint8_t *>(p);
    }
    *out = g_static_ptr[device];
    return hipSuccess;
}

// Makes the context's device current for the scope, restoring the caller's afterwards.
struct DeviceScope {
    int previous = -1;
    hipError_t error = hipSuccess;
    explicit DeviceScope(int device) {
        error = hipGetDevice(&previous);
        if (error == hipSuccess && previous != device) error = hipSetDevice(device);
    }
    ~DeviceScope() {
        int now = -1;
        if (previous >= 0 && hipGetDevice(&now) == hipSuccess && now != previous) (void)hipSetDevice(previous);
    }
};

bool aligned(const void *p, size_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// A measurement knob's value (an environment variable read when a context is created): the tile named,
// or -1 when unset or unknown (the product's own choice).
struct KnobValue {
    const char *name;
    int tile;
};
int knob(const char *value, std::initializer_list<KnobValue> table) {
    if (!value) return -1;
    for (const KnobValue &v : table)
        if (strcmp(value, v.name) == 0) return v.tile;
    return -1;
}

bool is_glu(int epilogue) { return epilogue == SQ8_EPI_SILU_GLU || epilogue == SQ8_EPI_SITU_GLU; }

bool is_packed(int w_layout) { return w_layout == SQ8_PACKED || w_layout == SQ8_PACKED_GLU; }

int check_config(int a_dtype, int w_dtype, int w_layout, int scale_layout, int c_dtype, int epilogue) {
    if (a_dtype != SQ8_BF16 && a_dtype != SQ8_F32) return SQ8_EUNSUPPORTED;
    if (w_dtype != SQ8_INT8 && w_dtype != SQ8_FP8_E4M3) return SQ8_EUNSUPPORTED;
    if (w_layout < SQ8_KN || w_layout > SQ8_PACKED_GLU) return SQ8_EINVAL;
    if (is_packed(w_layout) && (w_layout == SQ8_PACKED_GLU) != is_glu(epilogue)) return SQ8_EINVAL;
    if (scale_layout != SQ8_SCALE_TENSOR && scale_layout != SQ8_SCALE_COLUMNS) return SQ8_EUNSUPPORTED;
    if (c_dtype != SQ8_BF16 && c_dtype != SQ8_F32) return SQ8_EUNSUPPORTED;
    if (epilogue < SQ8_EPI_NONE || epilogue > SQ8_EPI_SITU_GLU) return SQ8_EINVAL;
    return SQ8_OK;
}

// Grows the rounding scratch to `bytes` (never shrinks; freed with the context).
// Grows a context buffer (after the stream has finished with the old one).
int reserve_buffer(sq8_ctx *ctx, void **buf, size_t *have, size_t bytes) {
    if (*have >= bytes) return SQ8_OK;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_status(e);
    if (*buf) (void)hipFree(*buf);
    *buf = nullptr;
    *have = 0;
    e = hipMalloc(buf, bytes);
    if (e != hipSuccess) { *buf = nullptr; return hip_status(e); }
    *have = bytes;
    return SQ8_OK;
}

int reserve_scratch(sq8_ctx *ctx, size_t bytes) {
    if (ctx->scratch_bytes >= bytes) return SQ8_OK;
    if (ctx->scratch) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return hip_status(e);
        e = hipFree(ctx->scratch);
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
        if (e != hipSuccess) return hip_status(e);
    }
    hipError_t e = hipMalloc(&ctx->scratch, bytes);
    if (e != hipSuccess) {
        ctx->scratch = nullptr;
        return hip_status(e);
    }
    ctx->scratch_bytes = bytes;
    return SQ8_OK;
}

struct Product {
    const void *a; int a_dtype; int64_t lda;
    const void *w; int w_dtype; int w_layout; int64_t ldw;
    const float *scale; int scale_layout; const float *bias; int epilogue;
    void *c[3]; int c_dtype; int64_t ldc; int split; int head_dim;
    int m, k, n;
    int group;  // convrot: the operand rotated by groups of `group` first (0: none)
    bool residual; const float *gate;  // c (fp32) += gate ⊙ (s ⊙ (A·W) + b), in place
    bool exact;  // the fp32 route: A fp32 used whole, as three bf16 parts along K (every product exact)
};

// The fp32 route's operand (the reference's `submit` on an fp32 A, TensorGEMM.swift:296-360): A [m, k] —
// rotated first by `group` in fp32 when non-zero (rotate_groups, TensorGEMM.swift:334-345) — split into its
// three bf16 parts hi | mid | lo along K ([m, 3kp], hi + mid + lo = x, each part kp ≥ k wide with columns
// [k, kp) zero), in the context's scratch: the parts first, the rotated rows after them.
int stage_parts(sq8_ctx *ctx, const float *a, int64_t lda, int group, int m, int k, int kp, const uint16_t **out) {
    const size_t mk = (size_t)m * (size_t)k;
    const size_t parts = (size_t)m * (size_t)kp * 6;
    const size_t bytes = parts + (group != 0 ? mk * 4 : 0);
    int st = reserve_scratch(ctx, bytes > 0 ? bytes : 2);
    if (st != SQ8_OK) return st;
    uint16_t *y = static_cast<uint16_t *>(ctx->scratch);
    const float *src = a;
    int64_t lds = lda;
    if (group != 0) {
        // m·kp·6 bytes in: a multiple of 4 as kp is even.
        float *r = reinterpret_cast<float *>(static_cast<uint8_t *>(ctx->scratch) + parts);
        hipError_t e = sq8::launch_rotate_groups(a, false, lda, r, false, k, m, k, group, ctx->stream);
        if (e != hipSuccess) return hip_status(e);
        src = r;
        lds = k;
    }
    hipError_t e = sq8::launch_split3(src, lds, y, m, k, kp, ctx->stream);
    if (e != hipSuccess) return hip_status(e);
    *out = y;
    return SQ8_OK;
}

// A bf16 operand for the step kernels when K is not a whole number of 64-wide steps: rows copied into the
// context's scratch kp = ⌈k/64⌉·64 apart with columns [k, kp) zero (zero products with the packed
// weight's zero codes past K: every sum as over k alone).
int stage_padded_bf16(sq8_ctx *ctx, const uint16_t *a, int64_t lda, int m, int k, int kp, const uint16_t **out) {
    const size_t bytes = (size_t)m * (size_t)kp * 2;
    int st = reserve_scratch(ctx, bytes > 0 ? bytes : 2);
    if (st != SQ8_OK) return st;
    uint16_t *y = static_cast<uint16_t *>(ctx->scratch);
    hipError_t e = sq8::launch_pad_bf16_rows(a, lda, y, m, k, kp, ctx->stream);
    if (e != hipSuccess) return hip_status(e);
    *out = y;
    return SQ8_OK;
}

int run_product(sq8_ctx *ctx, const Product &q, double *gpu_seconds) {
    if (!ctx) return SQ8_EINVAL;
    int st = check_config(q.a_dtype, q.w_dtype, q.w_layout, q.scale_layout, q.c_dtype, q.epilogue);
    if (st != SQ8_OK) return st;
    if (q.m < 0 || q.k < 0 || q.n < 0) return SQ8_EINVAL;
    if (is_glu(q.epilogue) && (q.n % 2) != 0) return SQ8_EINVAL;
    const int n_out = is_glu(q.epilogue) ? q.n / 2 : q.n;
    if (gpu_seconds) *gpu_seconds = 0.0;
    if (q.m == 0 || n_out == 0) return SQ8_OK;
    if (!q.a || !q.w || !q.scale || !q.c[0]) return SQ8_EINVAL;
    if (q.lda < q.k) return SQ8_EINVAL;
    if (!is_packed(q.w_layout) && q.ldw < (q.w_layout == SQ8_KN ? q.n : q.k)) return SQ8_EINVAL;
    if (q.split == 0 && q.head_dim == 0 && q.ldc < n_out) return SQ8_EINVAL;
    if (q.group != 0 && (!sq8::is_rotation_group(q.group) || q.k % q.group != 0)) return SQ8_EINVAL;
    if (q.residual && (q.c_dtype != SQ8_F32 || is_glu(q.epilogue))) return SQ8_EUNSUPPORTED;
    if (q.exact && q.a_dtype != SQ8_F32) return SQ8_EINVAL;
    // K not a whole number of 64-wide steps on the step kernels (a packed weight, the fp32 route, the
    // residual epilogue): the operand is staged with its rows padded to kp (zeros past k) and the weight
    // packed (zero codes past k), so each sum is the one over k alone (TensorGEMM.swift:124-135 computes
    // any K). The bf16 route on codes as they lie keeps the guarded kernel for such K.
    const int kp = (q.k + 63) / 64 * 64;
    const bool pad_k = q.k % 64 != 0 && (q.exact || q.residual || is_packed(q.w_layout));
    // The kernels address A and W with 32-bit byte offsets from their bases.
    const int64_t a_row = q.exact ? 3 * (int64_t)kp : pad_k ? kp : q.a_dtype == SQ8_BF16 && q.group == 0 ? q.lda : q.k;
    if ((int64_t)q.m * a_row * 2 > (int64_t)UINT32_MAX ||
        std::max<int64_t>(sq8::packed_bytes(q.k, q.n, is_glu(q.epilogue)),
                          is_packed(q.w_layout) ? 0 : (int64_t)(q.w_layout == SQ8_KN ? q.k : q.n) * q.ldw) >
            (int64_t)UINT32_MAX)
        return SQ8_EUNSUPPORTED;

    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);

    sq8::GemmArgs p;
    memset(&p, 0, sizeof(p));
    p.lda = q.lda;
    p.a = static_cast<const uint16_t *>(q.a);
    if (gpu_seconds) {
        hipError_t e = hipEventRecord(ctx->begin, ctx->stream);
        if (e != hipSuccess) return hip_status(e);
    }
    if (q.exact) {
        // The fp32 route: the kernels run K' = 3K steps against the weight's K steps, each part facing
        // the whole weight, so every product is exact and the sums are fp32.
        const uint16_t *y = nullptr;
        st = stage_parts(ctx, static_cast<const float *>(q.a), q.lda, q.group, q.m, q.k, kp, &y);
        if (st != SQ8_OK) return st;
        p.a = y;
        p.lda = 3 * (int64_t)kp;
    } else if (q.group != 0) {
        // convrot: the operand rotated (fp32 butterflies) and rounded to bf16 in one pass, into the
        // context's scratch (TensorGEMMBF16.swift:222-233: rotate_groups, then round_bf16); rows kp apart
        // with zero columns past k when K is padded.
        const int ky = pad_k ? kp : q.k;
        const size_t bytes = (size_t)q.m * (size_t)ky * 2;
        st = reserve_scratch(ctx, bytes > 0 ? bytes : 2);
        if (st != SQ8_OK) return st;
        uint16_t *y = static_cast<uint16_t *>(ctx->scratch);
        hipError_t e = sq8::launch_rotate_groups(q.a, q.a_dtype == SQ8_BF16, q.lda, y, true, ky, q.m, q.k, q.group,
                                                 ctx->stream);
        if (e == hipSuccess) e = sq8::launch_zero_tail(y, ky, q.m, q.k, ky, ctx->stream);
        if (e != hipSuccess) return hip_status(e);
        p.a = y;
        p.lda = ky;
    } else if (q.a_dtype == SQ8_F32) {
        // The operand rounded to bf16 once, into the context's scratch (TensorGEMMBF16.swift:208-264).
        const int ky = pad_k ? kp : q.k;
        const size_t bytes = (size_t)q.m * (size_t)ky * 2;
        st = reserve_scratch(ctx, bytes > 0 ? bytes : 2);
        if (st != SQ8_OK) return st;
        const float *x = static_cast<const float *>(q.a);
        uint16_t *y = static_cast<uint16_t *>(ctx->scratch);
        hipError_t e = sq8::launch_round_bf16_rows(x, q.lda, y, q.m, q.k, ky, ctx->stream);
        if (e != hipSuccess) return hip_status(e);
        p.a = y;
        p.lda = ky;
    } else if (pad_k) {
        const uint16_t *y = nullptr;
        st = stage_padded_bf16(ctx, static_cast<const uint16_t *>(q.a), q.lda, q.m, q.k, kp, &y);
        if (st != SQ8_OK) return st;
        p.a = y;
        p.lda = kp;
    }
    p.w = static_cast<const uint8_t *>(q.w);
    p.ldw = q.ldw;
    p.scale = q.scale;
    p.bias = q.bias;
    p.c[0] = q.c[0];
    p.c[1] = q.c[1];
    p.c[2] = q.c[2];
    if (q.split > 0) {
        p.c_d1 = (int64_t)((uintptr_t)q.c[1] - (uintptr_t)q.c[0]);
        p.c_d2 = (int64_t)((uintptr_t)q.c[2] - (uintptr_t)q.c[0]);
    }
    p.ldc = q.ldc;
    p.split = q.split;
    p.head_dim = q.head_dim;
    p.M = q.m;
    p.N = q.n;
    p.K = q.k;
    p.glu_half = is_glu(q.epilogue) ? q.n / 2 : 0;
    p.scale_per_col = q.scale_layout == SQ8_SCALE_COLUMNS;
    p.a_vec = aligned(p.a, 16) && (p.lda % 8) == 0;
    // [N, K]: 16-byte loads along K. [K, N]: 4-byte loads of 4 columns, which also needs the second
    // half of a GLU weight to start on a multiple of 4.
    p.w_vec = q.w_layout == SQ8_NK ? (aligned(p.w, 16) && (p.ldw % 16) == 0)
                                   : (aligned(p.w, 4) && (p.ldw % 4) == 0 && (p.glu_half % 4) == 0);
    const size_t esz = q.c_dtype == SQ8_F32 ? 4 : 2;
    bool cv = true;
    for (int i = 0; i < (q.split > 0 ? 3 : 1); ++i) cv = cv && aligned(q.c[i], 4 * esz);
    if (q.head_dim > 0) cv = cv && (q.head_dim % 4) == 0;
    else cv = cv && (q.ldc % 4) == 0;
    p.c_vec = cv;
    // 16-byte stores: 8 bf16 / 4 fp32 columns that never straddle a split or a head.
    const int per16 = (int)(16 / esz);
    bool cv16 = true;
    for (int i = 0; i < (q.split > 0 ? 3 : 1); ++i) cv16 = cv16 && aligned(q.c[i], 16);
    if (q.split > 0) cv16 = cv16 && (q.split % per16) == 0;
    if (q.head_dim > 0) cv16 = cv16 && (q.head_dim % per16) == 0;
    else cv16 = cv16 && (q.ldc % per16) == 0;
    p.c_vec16 = cv16 && (!q.gate || aligned(q.gate, 16));
    p.gate = q.gate;
    p.sb_vec = aligned(p.scale, 16) && (!p.bias || aligned(p.bias, 16)) && (p.glu_half % 4) == 0;
    const int epi = q.residual ? sq8::EPI_RESIDUAL : q.epilogue;

    const int wt = q.w_dtype == SQ8_INT8 ? sq8::W_INT8 : sq8::W_FP8;
    const int out = q.c_dtype == SQ8_F32 ? sq8::OUT_F32 : sq8::OUT_BF16;
    const int cols_per_half = is_glu(q.epilogue) ? q.n / 2 : q.n;
    // Whole 64-wide K steps: K itself, or K padded in the staging above.
    const bool k_steps = q.k > 0 && ((q.k % 64) == 0 || pad_k);
    p.kt = (q.k + 63) / 64;
    if (q.exact) {
        p.kt_w = p.kt;  // the weight's steps; the activation has three parts of them
        p.kt = 3 * p.kt_w;
    }
    p.cus = ctx->cus;
    hipError_t e;
    // [K, N] codes in place: repacked per product into the context's buffer when the repack runs near
    // the memory bandwidth (the reference's in-place route, Artifact.swift:443-459, at the speed of
    // the staged one: 37.7 MB of C1 codes cost ~12 µs against ~230 µs saved).
    // The fp32 route and the residual epilogue run on the weight-direct kernels only: they repack any
    // [K, N] weight (the general pack where the fast one does not apply).
    int wl_run = q.w_layout;
    // A padded K takes the packed layout (its zero codes past k) whatever the weight's own layout.
    if (!is_packed(q.w_layout) && p.a_vec && k_steps &&
        (pad_k || (q.w_layout == SQ8_KN && (q.exact || q.residual ||
                                            sq8::pack_is_fast(p.w, sq8::W_KN, p.ldw, q.k, q.n, is_glu(q.epilogue)))))) {
        const int64_t bytes = sq8::packed_bytes(q.k, q.n, is_glu(q.epilogue));
        st = reserve_buffer(ctx, &ctx->wpack, &ctx->wpack_bytes, (size_t)bytes);
        if (st != SQ8_OK) return st;
        e = sq8::launch_pack(p.w, q.w_layout == SQ8_KN ? sq8::W_KN : sq8::W_NK, p.ldw, q.k, q.n, is_glu(q.epilogue),
                             static_cast<uint8_t *>(ctx->wpack), ctx->stream);
        if (e != hipSuccess) return hip_status(e);
        p.w = static_cast<const uint8_t *>(ctx->wpack);
        wl_run = is_glu(q.epilogue) ? SQ8_PACKED_GLU : SQ8_PACKED;
    }
    if (is_packed(wl_run) || (q.w_layout == SQ8_NK && p.a_vec && p.w_vec && k_steps && cols_per_half >= 1)) {
        // The weight-direct kernels: packed codes, or [N, K] rows read as they lie.
        if (!p.a_vec || !k_steps) return SQ8_EUNSUPPORTED;  // K = 0, or an activation not 16-byte aligned
        const int wl = is_packed(wl_run) ? sq8::W_PACKED : sq8::W_NK;
        const int tile = ctx->wd_tile >= 0 ? ctx->wd_tile : sq8::choose_wd_tile(q.m, q.n, is_glu(q.epilogue), ctx->cus, p.kt);
        if ((tile == sq8::WD_SKINNY32 || tile == sq8::WD_SKINNY64) && ctx->splits > 1) {
            // Short M with the SQ8_SPLITS knob: the K steps split over several workgroups per tile, partial
            // sums in the context's buffer, added in split order by a second launch. Not the default: the
            // second launch's fixed cost (~3.4 µs on this chip) exceeds what the split saves (M = 1 at
            // K = N = 3072: 7.5 µs unsplit, 5.0 + 4.5 in four splits).
            const int splits = std::min(ctx->splits, p.kt);
            if (splits > 1) {
                const int64_t bytes = sq8::skinny_part_bytes(q.m, q.n, is_glu(q.epilogue),
                                                             tile == sq8::WD_SKINNY32 ? 32 : 64, splits);
                st = reserve_buffer(ctx, &ctx->part, &ctx->part_bytes, (size_t)bytes);
                if (st != SQ8_OK) return st;
                p.part = static_cast<float *>(ctx->part);
                p.splits = splits;
            }
        }
        e = sq8::launch_wdirect(p, tile, wt, wl, epi, out, ctx->stream);
    } else if (q.residual || q.exact) {
        return SQ8_EUNSUPPORTED;  // the residual epilogue and the fp32 route run on the weight-direct kernels only
    } else {
        const int wl = q.w_layout == SQ8_KN ? sq8::W_KN : sq8::W_NK;
        const int tile = sq8::choose_tile(q.m, n_out, is_glu(q.epilogue), ctx->cus);
        const bool fast = p.a_vec && p.w_vec && k_steps && cols_per_half >= 4 &&
                          (q.w_layout == SQ8_NK || (cols_per_half % 4) == 0);
        e = sq8::launch_gemm(p, fast, tile, wt, wl, q.epilogue, out, ctx->stream);
    }
    if (e != hipSuccess) return hip_status(e);
    if (gpu_seconds) {
        e = hipEventRecord(ctx->end, ctx->stream);
        if (e == hipSuccess) e = hipEventSynchronize(ctx->end);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ctx->begin, ctx->end);
        if (e != hipSuccess) return hip_status(e);
        *gpu_seconds = (double)ms * 1e-3;
    }
    return SQ8_OK;
}

// The W8A8 product: codes [m, ldq] int8 with row scales sx (already quantized, or quantized here
// from `a` when `a` is non-null), the int8 weight packed or [N, K] (repacked into the context's
// buffer otherwise), C = act(float(Σ) · (s_x · s_w) + b).
struct W8A8 {
    const void *a; int a_dtype; int64_t lda; int group;     // quantized here when a != nullptr
    const int8_t *codes; int64_t ldq; const float *sx;       // else these
    const void *w; int w_layout; int64_t ldw;
    const float *scale; int scale_layout; const float *bias; int epilogue;
    void *c[3]; int c_dtype; int64_t ldc; int split; int head_dim;
    int m, k, n;
    bool residual; const float *gate;  // c (fp32) += gate ⊙ (…), in place
    bool no_alloc;  // the codes and row scales in the static scratch; no allocation, no repack
};

int run_w8a8(sq8_ctx *ctx, const W8A8 &q, double *gpu_seconds) {
    if (!ctx) return SQ8_EINVAL;
    int st = check_config(SQ8_BF16, SQ8_INT8, q.w_layout, q.scale_layout, q.c_dtype, q.epilogue);
    if (st != SQ8_OK) return st;
    if (q.a && q.a_dtype != SQ8_F32 && q.a_dtype != SQ8_BF16) return SQ8_EUNSUPPORTED;
    if (q.m < 0 || q.k < 0 || q.n < 0) return SQ8_EINVAL;
    if (is_glu(q.epilogue) && (q.n % 2) != 0) return SQ8_EINVAL;
    if (q.group != 0 && (!sq8::is_rotation_group(q.group) || q.k % q.group != 0)) return SQ8_EINVAL;
    if (q.k >= (1 << 17)) return SQ8_EUNSUPPORTED;  // the int32 sums stay exact below 2^17 terms
    if (q.residual && (q.c_dtype != SQ8_F32 || is_glu(q.epilogue))) return SQ8_EUNSUPPORTED;
    if (q.a && q.k > sq8::quantize_row_limit()) return SQ8_EUNSUPPORTED;
    const int n_out = is_glu(q.epilogue) ? q.n / 2 : q.n;
    if (gpu_seconds) *gpu_seconds = 0.0;
    if (q.m == 0 || n_out == 0) return SQ8_OK;
    if (q.k == 0) return SQ8_EUNSUPPORTED;
    if (!q.w || !q.scale || !q.c[0]) return SQ8_EINVAL;
    if (q.a ? q.lda < q.k : (!q.codes || !q.sx || q.ldq < q.k)) return SQ8_EINVAL;
    if (!is_packed(q.w_layout) && q.ldw < (q.w_layout == SQ8_KN ? q.n : q.k)) return SQ8_EINVAL;
    if (q.split == 0 && q.head_dim == 0 && q.ldc < n_out) return SQ8_EINVAL;
    const int k_pad = (q.k + 127) / 128 * 128;
    // The kernel addresses the codes and the weight with 32-bit byte offsets from their bases.
    if ((int64_t)q.m * std::max<int64_t>(k_pad, q.ldq) > (int64_t)UINT32_MAX ||
        std::max<int64_t>(sq8::packed_bytes(q.k, q.n, is_glu(q.epilogue)),
                          is_packed(q.w_layout) ? 0 : (int64_t)(q.w_layout == SQ8_KN ? q.k : q.n) * q.ldw) >
            (int64_t)UINT32_MAX)
        return SQ8_EUNSUPPORTED;

    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    // Scratch: codes [m, k_pad] (when quantized or padded here), then the row scales.
    const bool own_codes = q.a || q.k % 128 != 0 || q.ldq % 16 != 0 || !aligned(q.codes, 16);
    const size_t code_bytes = own_codes ? ((size_t)q.m * (size_t)k_pad + 255) / 256 * 256 : 0;
    const size_t bytes = code_bytes + (q.a ? (size_t)q.m * 4 : 0);
    uint8_t *scr = nullptr;
    if (q.no_alloc) {
        // The static scratch: its capacity is the limit, and the weight must be one the kernel reads
        // as it lies (packed, or [N, K] with whole 128-code rows), since a repack would need a buffer.
        if (bytes > (size_t)SQ8_STATIC_SCRATCH_BYTES) return SQ8_ECAPACITY;
        if (!(is_packed(q.w_layout) ||
              (q.w_layout == SQ8_NK && !is_glu(q.epilogue) && q.k % 128 == 0 && q.ldw % 16 == 0 && aligned(q.w, 16))))
            return SQ8_EUNSUPPORTED;
        const hipError_t e = static_scratch_of(ctx->device, &scr);
        if (e != hipSuccess) return hip_status(e);
    } else if (bytes > 0) {
        st = reserve_scratch(ctx, bytes);
        if (st != SQ8_OK) return st;
        scr = static_cast<uint8_t *>(ctx->scratch);
    }
    int8_t *codes = own_codes ? reinterpret_cast<int8_t *>(scr) : const_cast<int8_t *>(q.codes);
    const float *sx = q.a ? reinterpret_cast<float *>(scr + code_bytes) : q.sx;
    const int64_t ldq = own_codes ? k_pad : q.ldq;
    if (gpu_seconds) {
        hipError_t e = hipEventRecord(ctx->begin, ctx->stream);
        if (e != hipSuccess) return hip_status(e);
    }
    hipError_t e = hipSuccess;
    if (q.a)
        e = sq8::launch_quantize_rows(q.a, q.a_dtype == SQ8_BF16, q.lda, q.m, q.k, q.group, codes, ldq, k_pad,
                                      const_cast<float *>(sx), ctx->stream);
    else if (own_codes)
        e = sq8::launch_pad_codes(q.codes, q.ldq, codes, ldq, q.m, q.k, k_pad, ctx->stream);
    if (e != hipSuccess) return hip_status(e);

    sq8::GemmArgs p;
    memset(&p, 0, sizeof(p));
    p.a = reinterpret_cast<const uint16_t *>(codes);
    p.lda = ldq;
    p.sx = sx;
    p.scale = q.scale;
    p.bias = q.bias;
    p.c[0] = q.c[0];
    p.c[1] = q.c[1];
    p.c[2] = q.c[2];
    if (q.split > 0) {
        p.c_d1 = (int64_t)((uintptr_t)q.c[1] - (uintptr_t)q.c[0]);
        p.c_d2 = (int64_t)((uintptr_t)q.c[2] - (uintptr_t)q.c[0]);
    }
    p.ldc = q.ldc;
    p.split = q.split;
    p.head_dim = q.head_dim;
    p.M = q.m;
    p.N = q.n;
    p.K = q.k;
    p.glu_half = is_glu(q.epilogue) ? q.n / 2 : 0;
    p.scale_per_col = q.scale_layout == SQ8_SCALE_COLUMNS;
    const size_t esz = q.c_dtype == SQ8_F32 ? 4 : 2;
    // 16-byte stores: 8 bf16 / 4 fp32 columns that never straddle a split or a head.
    const int per16 = (int)(16 / esz);
    bool cv16 = true;
    for (int i = 0; i < (q.split > 0 ? 3 : 1); ++i) cv16 = cv16 && aligned(q.c[i], 16);
    if (q.split > 0) cv16 = cv16 && (q.split % per16) == 0;
    if (q.head_dim > 0) cv16 = cv16 && (q.head_dim % per16) == 0;
    else cv16 = cv16 && (q.ldc % per16) == 0;
    p.c_vec16 = cv16 && (!q.gate || aligned(q.gate, 16));
    p.c_vec = p.c_vec16;
    p.gate = q.gate;
    p.sb_vec = aligned(q.scale, 16) && (!q.bias || aligned(q.bias, 16)) && (p.glu_half % 4) == 0;
    p.kt = k_pad / 128;
    // The weight: packed as staged, [N, K] read in place when its rows hold whole steps, else
    // repacked per product into the context's buffer.
    int wl = sq8::W_PACKED;
    p.w = static_cast<const uint8_t *>(q.w);
    if (is_packed(q.w_layout)) {
        p.kt_w = (q.k + 63) / 64;
    } else if (q.w_layout == SQ8_NK && !is_glu(q.epilogue) && q.k % 128 == 0 && q.ldw % 16 == 0 && aligned(q.w, 16)) {
        wl = sq8::W_NK;
        p.ldw = q.ldw;
        p.kt_w = q.k / 64;
    } else {
        const int64_t wbytes = sq8::packed_bytes(q.k, q.n, is_glu(q.epilogue));
        st = reserve_buffer(ctx, &ctx->wpack, &ctx->wpack_bytes, (size_t)wbytes);
        if (st != SQ8_OK) return st;
        e = sq8::launch_pack(static_cast<const uint8_t *>(q.w), q.w_layout == SQ8_KN ? sq8::W_KN : sq8::W_NK, q.ldw, q.k,
                             q.n, is_glu(q.epilogue), static_cast<uint8_t *>(ctx->wpack), ctx->stream);
        if (e != hipSuccess) return hip_status(e);
        p.w = static_cast<const uint8_t *>(ctx->wpack);
        p.kt_w = (q.k + 63) / 64;
    }
    e = sq8::launch_i8gemm(p, wl, q.residual ? sq8::EPI_RESIDUAL : q.epilogue,
                           q.c_dtype == SQ8_F32 ? sq8::OUT_F32 : sq8::OUT_BF16, ctx->stream);
    if (e != hipSuccess) return hip_status(e);
    if (gpu_seconds) {
        e = hipEventRecord(ctx->end, ctx->stream);
        if (e == hipSuccess) e = hipEventSynchronize(ctx->end);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ctx->begin, ctx->end);
        if (e != hipSuccess) return hip_status(e);
        *gpu_seconds = (double)ms * 1e-3;
    }
    return SQ8_OK;
}

// ---- codes with a scale per block of rows and column (GGUF Q8_0) ----------------------------------

struct Blocks {
    const void *a; int a_dtype; int64_t lda;
    const void *w; int w_layout; int64_t ldw;
    const void *scale; int scale_dtype; int block;
    const float *bias; int epilogue;
    void *c; int c_dtype; int64_t ldc;
    int m, k, n;
    bool exact;  // the fp32 route: A fp32 used whole, as three bf16 parts along K
};

bool scale_dtype_ok(int t) { return t == SQ8_F32 || t == SQ8_BF16 || t == SQ8_F16; }

int run_blocks(sq8_ctx *ctx, const Blocks &q, double *gpu_seconds) {
    if (!ctx) return SQ8_EINVAL;
    if (q.a_dtype != SQ8_BF16 && q.a_dtype != SQ8_F32) return SQ8_EUNSUPPORTED;
    if (q.c_dtype != SQ8_BF16 && q.c_dtype != SQ8_F32) return SQ8_EUNSUPPORTED;
    if (q.w_layout < SQ8_KN || q.w_layout > SQ8_PACKED_GLU) return SQ8_EINVAL;
    if (q.epilogue < SQ8_EPI_NONE || q.epilogue > SQ8_EPI_SITU_GLU) return SQ8_EINVAL;
    if (is_packed(q.w_layout) && (q.w_layout == SQ8_PACKED_GLU) != is_glu(q.epilogue)) return SQ8_EINVAL;
    if (q.m < 0 || q.k < 0 || q.n < 0) return SQ8_EINVAL;
    if (is_glu(q.epilogue) && (q.n % 2) != 0) return SQ8_EINVAL;
    const bool packed = is_packed(q.w_layout);
    if (!packed && !scale_dtype_ok(q.scale_dtype)) return SQ8_EINVAL;
    if (q.block <= 0) return SQ8_EINVAL;
    const int n_out = is_glu(q.epilogue) ? q.n / 2 : q.n;
    if (gpu_seconds) *gpu_seconds = 0.0;
    if (q.m == 0 || n_out == 0) return SQ8_OK;
    if (!q.a || !q.w || !q.c || (!packed && !q.scale)) return SQ8_EINVAL;
    if (q.lda < q.k || q.ldc < n_out) return SQ8_EINVAL;
    if (!packed && q.ldw < (q.w_layout == SQ8_KN ? q.n : q.k)) return SQ8_EINVAL;
    // Blocks of whole MFMA sub-steps (32 rows of K), 32-bit offsets into A and the packed codes. K need not
    // be a whole number of 64-wide steps (the reference computes every block, TensorGEMM.swift:143-171,
    // `row < K` at :162): the operand is then staged with rows padded to kp, zeros past k, against the
    // packed layout's zero codes and zero scales past k.
    if (q.block % 32 != 0 || q.k % q.block != 0) return SQ8_EUNSUPPORTED;
    if (q.exact && q.a_dtype != SQ8_F32) return SQ8_EINVAL;
    const int kp = (q.k + 63) / 64 * 64;
    const bool pad_k = q.k % 64 != 0;
    const int64_t a_row = q.exact ? 3 * (int64_t)kp : pad_k ? kp : q.a_dtype == SQ8_BF16 ? q.lda : q.k;
    if ((int64_t)q.m * a_row * 2 > (int64_t)UINT32_MAX ||
        sq8::packed_blocks_bytes(q.k, q.n, is_glu(q.epilogue)) > (int64_t)UINT32_MAX)
        return SQ8_EUNSUPPORTED;
    if (packed && !aligned(q.w, 16)) return SQ8_EINVAL;

    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    sq8::GemmArgs p;
    memset(&p, 0, sizeof(p));
    p.a = static_cast<const uint16_t *>(q.a);
    p.lda = q.lda;
    if (gpu_seconds) {
        hipError_t e = hipEventRecord(ctx->begin, ctx->stream);
        if (e != hipSuccess) return hip_status(e);
    }
    if (q.exact) {
        // The fp32 route (the reference's `blocks` pipeline on an fp32 A, TensorGEMM.swift:307-320).
        const uint16_t *y = nullptr;
        int st = stage_parts(ctx, static_cast<const float *>(q.a), q.lda, 0, q.m, q.k, kp, &y);
        if (st != SQ8_OK) return st;
        p.a = y;
        p.lda = 3 * (int64_t)kp;
    } else if (q.a_dtype == SQ8_F32) {
        // The operand rounded to bf16 once, into the context's scratch (TensorGEMMBF16.swift:208-264).
        const size_t bytes = (size_t)q.m * (size_t)kp * 2;
        int st = reserve_scratch(ctx, bytes > 0 ? bytes : 2);
        if (st != SQ8_OK) return st;
        const float *x = static_cast<const float *>(q.a);
        uint16_t *y = static_cast<uint16_t *>(ctx->scratch);
        hipError_t e = sq8::launch_round_bf16_rows(x, q.lda, y, q.m, q.k, kp, ctx->stream);
        if (e != hipSuccess) return hip_status(e);
        p.a = y;
        p.lda = kp;
    } else if (pad_k) {
        const uint16_t *y = nullptr;
        int st = stage_padded_bf16(ctx, static_cast<const uint16_t *>(q.a), q.lda, q.m, q.k, kp, &y);
        if (st != SQ8_OK) return st;
        p.a = y;
        p.lda = kp;
    }
    if (!aligned(p.a, 16) || (p.lda % 8) != 0) return SQ8_EUNSUPPORTED;
    p.w = static_cast<const uint8_t *>(q.w);
    if (!packed) {
        // The codes and their scales packed per product into the context's buffer (the reference
        // reads the map's [K, N] codes and [K/B, N] scales in place, TensorGEMM.swift:307-318).
        const int64_t bytes = sq8::packed_blocks_bytes(q.k, q.n, is_glu(q.epilogue));
        int st = reserve_buffer(ctx, &ctx->wpack, &ctx->wpack_bytes, (size_t)bytes);
        if (st != SQ8_OK) return st;
        hipError_t e = sq8::launch_pack_blocks(p.w, q.w_layout == SQ8_KN ? sq8::W_KN : sq8::W_NK, q.ldw, q.scale,
                                               q.scale_dtype, q.block, q.k, q.n, is_glu(q.epilogue),
                                               static_cast<uint8_t *>(ctx->wpack), ctx->stream);
        if (e != hipSuccess) return hip_status(e);
        p.w = static_cast<const uint8_t *>(ctx->wpack);
    }
    p.bias = q.bias;
    p.c[0] = q.c;
    p.ldc = q.ldc;
    p.M = q.m;
    p.N = q.n;
    p.K = q.k;
    p.kt = kp / 64;
    if (q.exact) {
        p.kt_w = p.kt;  // the weight's steps; the activation has three parts of them
        p.kt = 3 * p.kt_w;
    }
    p.glu_half = is_glu(q.epilogue) ? q.n / 2 : 0;
    const size_t esz = q.c_dtype == SQ8_F32 ? 4 : 2;
    p.c_vec16 = aligned(q.c, 16) && (q.ldc % (int64_t)(16 / esz)) == 0;
    // 128-row tiles of one 32-column block per wave (the codes widened once for twice the rows);
    // the GLU epilogues pair both blocks of a slab in one wave: 64-row tiles.
    const int tile = ctx->q8_tile >= 0 ? ctx->q8_tile : is_glu(q.epilogue) ? sq8::BL_64x256 : sq8::BL_128x256;
    hipError_t e = sq8::launch_blocks_product(p, tile, q.epilogue, q.c_dtype == SQ8_F32 ? sq8::OUT_F32 : sq8::OUT_BF16,
                                  ctx->stream);
    if (e != hipSuccess) return hip_status(e);
    if (gpu_seconds) {
        e = hipEventRecord(ctx->end, ctx->stream);
        if (e == hipSuccess) e = hipEventSynchronize(ctx->end);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ctx->begin, ctx->end);
        if (e != hipSuccess) return hip_status(e);
        *gpu_seconds = (double)ms * 1e-3;
    }
    return SQ8_OK;
}

// The bf16-weight product (TensorGEMM.swift:236-254, `matmul2d` float × bfloat): C fp32 [m, n] = A · W,
// W bf16 [k, n] (SQ8_KN) or [n, k] (SQ8_NK). A plain GEMM, so the library GEMM (rocBLAS gemm_ex: bf16
// operands, fp32 sums) takes it; an fp32 A is split into its three bf16 parts first (stage_parts) and the
// three products summed into C (beta 0, 1, 1): every product exact, the sums fp32.
int blas_status(rocblas_status s) {
    switch (s) {
    case rocblas_status_success: return SQ8_OK;
    case rocblas_status_invalid_size:
    case rocblas_status_invalid_value:
    case rocblas_status_invalid_pointer:
    case rocblas_status_invalid_handle: return SQ8_EINVAL;
    case rocblas_status_not_implemented: return SQ8_EUNSUPPORTED;
    case rocblas_status_memory_error: return hip_status(hipErrorOutOfMemory);
    default: return hip_status(hipErrorLaunchFailure);
    }
}

int run_bf16_weight(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, const void *w, int w_layout, int64_t ldw,
                    float *c, int64_t ldc, int m, int k, int n, double *gpu_seconds) {
    if (!ctx) return SQ8_EINVAL;
    if (a_dtype != SQ8_BF16 && a_dtype != SQ8_F32) return SQ8_EUNSUPPORTED;
    if (w_layout != SQ8_KN && w_layout != SQ8_NK) return SQ8_EUNSUPPORTED;
    if (m < 0 || k < 0 || n < 0) return SQ8_EINVAL;
    if (gpu_seconds) *gpu_seconds = 0.0;
    if (m == 0 || n == 0) return SQ8_OK;
    if (!a || !w || !c) return SQ8_EINVAL;
    if (lda < k || ldw < (w_layout == SQ8_KN ? n : k) || ldc < n) return SQ8_EINVAL;
    // The library GEMM's sizes and leading dimensions are 32-bit.
    if (lda > INT32_MAX / 3 || ldw > INT32_MAX || ldc > INT32_MAX) return SQ8_EUNSUPPORTED;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    if (!ctx->blas) {
        rocblas_status bs = rocblas_create_handle(&ctx->blas);
        if (bs != rocblas_status_success) { ctx->blas = nullptr; return blas_status(bs); }
    }
    rocblas_status bs = rocblas_set_stream(ctx->blas, ctx->stream);
    if (bs != rocblas_status_success) return blas_status(bs);
    if (gpu_seconds) {
        hipError_t e = hipEventRecord(ctx->begin, ctx->stream);
        if (e != hipSuccess) return hip_status(e);
    }
    if (k == 0) {
        hipError_t e = hipMemset2DAsync(c, (size_t)ldc * 4, 0, (size_t)n * 4, (size_t)m, ctx->stream);
        if (e != hipSuccess) return hip_status(e);
    } else {
        const uint16_t *parts = static_cast<const uint16_t *>(a);
        int64_t ldp = lda;
        int count = 1;
        if (a_dtype == SQ8_F32) {
            int st = stage_parts(ctx, static_cast<const float *>(a), lda, 0, m, k, k, &parts);
            if (st != SQ8_OK) return st;
            ldp = 3 * (int64_t)k;
            count = 3;
        }
        // Row-major C [m, n] is column-major Cᵀ [n, m]: Cᵀ = op(W) · Aᵀ, W [k, n] row-major being the
        // column-major n × k matrix Wᵀ itself (no transpose), W [n, k] its transpose.
        const float one = 1.0f, zero = 0.0f;
        for (int part = 0; part < count; ++part) {
            bs = rocblas_gemm_ex(ctx->blas, w_layout == SQ8_KN ? rocblas_operation_none : rocblas_operation_transpose,
                                 rocblas_operation_none, n, m, k, &one, w, rocblas_datatype_bf16_r, (rocblas_int)ldw,
                                 parts + (int64_t)part * k, rocblas_datatype_bf16_r, (rocblas_int)ldp,
                                 part == 0 ? &zero : &one, c, rocblas_datatype_f32_r, (rocblas_int)ldc, c,
                                 rocblas_datatype_f32_r, (rocblas_int)ldc, rocblas_datatype_f32_r,
                                 rocblas_gemm_algo_standard, 0, 0);
            if (bs != rocblas_status_success) return blas_status(bs);
        }
    }
    if (gpu_seconds) {
        hipError_t e = hipEventRecord(ctx->end, ctx->stream);
        if (e == hipSuccess) e = hipEventSynchronize(ctx->end);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ctx->begin, ctx->end);
        if (e != hipSuccess) return hip_status(e);
        *gpu_seconds = (double)ms * 1e-3;
    }
    return SQ8_OK;
}

}  // namespace

extern "C" {

int sq8_abi_version(void) { return SQ8_ABI_VERSION; }

const char *sq8_status_string(int status) {
    switch (status) {
    case SQ8_OK: return "ok";
    case SQ8_EINVAL: return "invalid argument";
    case SQ8_EUNSUPPORTED: return "configuration not supported by this library";
    case SQ8_ENODEVICE: return "no gfx950 device at that ordinal";
    case SQ8_ECAPACITY: return "the problem exceeds the static scratch (SQ8_STATIC_SCRATCH_BYTES)";
    default: return status < 0 ? hipGetErrorString((hipError_t)(-status)) : "unknown status";
    }
}

int sq8_create(int device, void *stream, sq8_ctx **out) {
    if (!out) return SQ8_EINVAL;
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || device < 0 || device >= count) return SQ8_ENODEVICE;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_status(e);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return SQ8_ENODEVICE;
    DeviceScope scope(device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    sq8_ctx *ctx = new (std::nothrow) sq8_ctx;
    if (!ctx) return SQ8_EINVAL;
    memset(ctx, 0, sizeof(*ctx));
    ctx->device = device;
    ctx->stream = static_cast<hipStream_t>(stream);
    ctx->cus = prop.multiProcessorCount;
    ctx->wd_tile = knob(getenv("SQ8_TILE"), {{"256", sq8::WD_256}, {"224", sq8::WD_224}, {"128", sq8::WD_128}, {"64", sq8::WD_64},
                                             {"32", sq8::WD_32}, {"64n", sq8::WD_64N}, {"64x192", sq8::WD_64x192}, {"s64", sq8::WD_SKINNY64}, {"s32", sq8::WD_SKINNY32},
                                             {"gemv", sq8::WD_GEMV}, {"k32x32", sq8::WD_K32x32}, {"k32x64", sq8::WD_K32x64},
                                             {"k64x64", sq8::WD_K64x64}, {"k64x128", sq8::WD_K64x128}, {"k64x192", sq8::WD_K64x192}});
    ctx->q8_tile = knob(getenv("SQ8_Q8_TILE"), {{"256", sq8::BL_64x256}, {"512", sq8::BL_64x512},
                                                {"128x256", sq8::BL_128x256}, {"128x128", sq8::BL_128x128}});
    const char *splits = getenv("SQ8_SPLITS");
    ctx->splits = splits && atoi(splits) >= 1 ? atoi(splits) : 1;
    uint8_t *unused = nullptr;
    (void)static_scratch_of(device, &unused);  // set-up; sq8_linear_quantized_static retries and reports
    e = hipEventCreate(&ctx->begin);
    if (e == hipSuccess) e = hipEventCreate(&ctx->end);
    if (e != hipSuccess) {
        if (ctx->begin) (void)hipEventDestroy(ctx->begin);
        delete ctx;
        return hip_status(e);
    }
    *out = ctx;
    return SQ8_OK;
}

int sq8_destroy(sq8_ctx *ctx) {
    if (!ctx) return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    int st = SQ8_OK;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) st = hip_status(e);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->wpack) (void)hipFree(ctx->wpack);
    if (ctx->part) (void)hipFree(ctx->part);
    if (ctx->blas) (void)rocblas_destroy_handle(ctx->blas);
    (void)hipEventDestroy(ctx->begin);
    (void)hipEventDestroy(ctx->end);
    delete ctx;
    return st;
}

int sq8_set_stream(sq8_ctx *ctx, void *stream) {
    if (!ctx) return SQ8_EINVAL;
    if (static_cast<hipStream_t>(stream) != ctx->stream) {
        // The scratch and the packing buffer serve one stream at a time.
        DeviceScope scope(ctx->device);
        if (scope.error != hipSuccess) return hip_status(scope.error);
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return hip_status(e);
    }
    ctx->stream = static_cast<hipStream_t>(stream);
    return SQ8_OK;
}

int sq8_supports(const sq8_ctx *ctx, int a_dtype, int w_dtype, int w_layout, int scale_layout, int c_dtype,
                 int epilogue) {
    if (!ctx) return SQ8_EINVAL;
    return check_config(a_dtype, w_dtype, w_layout, scale_layout, c_dtype, epilogue);
}

int sq8_linear(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, const void *w, int w_dtype, int w_layout,
               int64_t ldw, const float *scale, int scale_layout, const float *bias, int epilogue, void *c,
               int c_dtype, int64_t ldc, int m, int k, int n, double *gpu_seconds) {
    Product q;
    memset(&q, 0, sizeof(q));
    q.a = a; q.a_dtype = a_dtype; q.lda = lda;
    q.w = w; q.w_dtype = w_dtype; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = scale; q.scale_layout = scale_layout; q.bias = bias; q.epilogue = epilogue;
    q.c[0] = c; q.c_dtype = c_dtype; q.ldc = ldc;
    q.m = m; q.k = k; q.n = n;
    return run_product(ctx, q, gpu_seconds);
}

int sq8_linear_qkv(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, const void *w, int w_dtype, int w_layout,
                   int64_t ldw, const float *scale, int scale_layout, const float *bias, void *q_out, void *k_out,
                   void *v_out, int c_dtype, int64_t ldo, int head_dim, int m, int k, int d, double *gpu_seconds) {
    if (d < 0 || (d % 4) != 0 || head_dim < 0) return SQ8_EINVAL;
    if (head_dim > 0 && ((d % head_dim) != 0 || (head_dim % 4) != 0)) return SQ8_EINVAL;
    if (head_dim == 0 && ldo < d) return SQ8_EINVAL;
    if (d > 0 && (!q_out || !k_out || !v_out)) return SQ8_EINVAL;
    if ((int64_t)3 * d > INT32_MAX) return SQ8_EINVAL;
    Product q;
    memset(&q, 0, sizeof(q));
    q.a = a; q.a_dtype = a_dtype; q.lda = lda;
    q.w = w; q.w_dtype = w_dtype; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = scale; q.scale_layout = scale_layout; q.bias = bias; q.epilogue = SQ8_EPI_NONE;
    q.c[0] = q_out; q.c[1] = k_out; q.c[2] = v_out; q.c_dtype = c_dtype; q.ldc = ldo;
    q.split = d; q.head_dim = head_dim;
    q.m = m; q.k = k; q.n = 3 * d;
    return run_product(ctx, q, gpu_seconds);
}

int sq8_linear_rotated(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, int group, const void *w, int w_dtype,
                       int w_layout, int64_t ldw, const float *scale, int scale_layout, const float *bias, int epilogue,
                       void *c, int c_dtype, int64_t ldc, int m, int k, int n, double *gpu_seconds) {
    if (group == 0) return SQ8_EINVAL;
    Product q;
    memset(&q, 0, sizeof(q));
    q.a = a; q.a_dtype = a_dtype; q.lda = lda; q.group = group;
    q.w = w; q.w_dtype = w_dtype; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = scale; q.scale_layout = scale_layout; q.bias = bias; q.epilogue = epilogue;
    q.c[0] = c; q.c_dtype = c_dtype; q.ldc = ldc;
    q.m = m; q.k = k; q.n = n;
    return run_product(ctx, q, gpu_seconds);
}

int sq8_rotate_groups(sq8_ctx *ctx, const void *x, int x_dtype, int64_t ldx, void *y, int y_dtype, int64_t ldy, int rows,
                      int k, int group) {
    if (!ctx || rows < 0 || k < 0) return SQ8_EINVAL;
    if ((x_dtype != SQ8_F32 && x_dtype != SQ8_BF16) || (y_dtype != SQ8_F32 && y_dtype != SQ8_BF16)) return SQ8_EUNSUPPORTED;
    if (!sq8::is_rotation_group(group) || k % group != 0) return SQ8_EINVAL;
    if (rows == 0 || k == 0) return SQ8_OK;
    if (!x || !y || ldx < k || ldy < k) return SQ8_EINVAL;
    // In place only as the same buffer read and written alike: each chunk is read whole before it is written.
    if (x == y && (x_dtype != y_dtype || ldx != ldy)) return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(sq8::launch_rotate_groups(x, x_dtype == SQ8_BF16, ldx, y, y_dtype == SQ8_BF16, ldy, rows, k, group,
                                                ctx->stream));
}

int sq8_dequantize_rotated(sq8_ctx *ctx, const int8_t *codes, int64_t ldq, int k, int n, int group, const void *scale,
                           int scale_dtype, int scale_layout, float *out, int64_t ldo) {
    if (!ctx || k < 0 || n < 0) return SQ8_EINVAL;
    if (scale_dtype != SQ8_F32 && scale_dtype != SQ8_BF16 && scale_dtype != SQ8_F16) return SQ8_EUNSUPPORTED;
    if (scale_layout != SQ8_SCALE_TENSOR && scale_layout != SQ8_SCALE_COLUMNS) return SQ8_EUNSUPPORTED;
    if (!sq8::is_rotation_group(group) || k % group != 0) return SQ8_EINVAL;
    if (k == 0 || n == 0) return SQ8_OK;
    if (!codes || !scale || !out || ldq < n || ldo < n) return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(sq8::launch_dequantize_rotated(codes, ldq, k, n, group, scale, scale_dtype,
                                                     scale_layout == SQ8_SCALE_COLUMNS, out, ldo, ctx->stream));
}

int sq8_quantize_rows(sq8_ctx *ctx, const void *x, int x_dtype, int64_t ldx, int rows, int k, int group, int8_t *codes,
                      int64_t ldq, float *scales) {
    if (!ctx || rows < 0 || k < 0) return SQ8_EINVAL;
    if (x_dtype != SQ8_F32 && x_dtype != SQ8_BF16) return SQ8_EUNSUPPORTED;
    if (group != 0 && (!sq8::is_rotation_group(group) || k % group != 0)) return SQ8_EINVAL;
    if (k > sq8::quantize_row_limit()) return SQ8_EUNSUPPORTED;
    if (rows == 0) return SQ8_OK;
    if (!x || !codes || !scales || ldx < k || ldq < k) return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(sq8::launch_quantize_rows(x, x_dtype == SQ8_BF16, ldx, rows, k, group, codes, ldq, k, scales,
                                                ctx->stream));
}

int sq8_linear_w8a8(sq8_ctx *ctx, const int8_t *codes, int64_t ldq, const float *sx, const void *w, int w_layout,
                    int64_t ldw, const float *scale, int scale_layout, const float *bias, int epilogue, void *c,
                    int c_dtype, int64_t ldc, int m, int k, int n, double *gpu_seconds) {
    W8A8 q;
    memset(&q, 0, sizeof(q));
    q.codes = codes; q.ldq = ldq; q.sx = sx;
    q.w = w; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = scale; q.scale_layout = scale_layout; q.bias = bias; q.epilogue = epilogue;
    q.c[0] = c; q.c_dtype = c_dtype; q.ldc = ldc;
    q.m = m; q.k = k; q.n = n;
    return run_w8a8(ctx, q, gpu_seconds);
}

int sq8_linear_residual(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, const void *w, int w_dtype, int w_layout,
                        int64_t ldw, const float *scale, int scale_layout, const float *bias, const float *gate, float *x,
                        int64_t ldx, int m, int k, int n, double *gpu_seconds) {
    Product q;
    memset(&q, 0, sizeof(q));
    q.a = a; q.a_dtype = a_dtype; q.lda = lda;
    q.w = w; q.w_dtype = w_dtype; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = scale; q.scale_layout = scale_layout; q.bias = bias; q.epilogue = SQ8_EPI_NONE;
    q.c[0] = x; q.c_dtype = SQ8_F32; q.ldc = ldx;
    q.m = m; q.k = k; q.n = n;
    q.residual = true; q.gate = gate;
    return run_product(ctx, q, gpu_seconds);
}

int sq8_linear_w8a8_residual(sq8_ctx *ctx, const int8_t *codes, int64_t ldq, const float *sx, const void *w, int w_layout,
                             int64_t ldw, const float *scale, int scale_layout, const float *bias, const float *gate,
                             float *x, int64_t ldx, int m, int k, int n, double *gpu_seconds) {
    W8A8 q;
    memset(&q, 0, sizeof(q));
    q.codes = codes; q.ldq = ldq; q.sx = sx;
    q.w = w; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = scale; q.scale_layout = scale_layout; q.bias = bias; q.epilogue = SQ8_EPI_NONE;
    q.c[0] = x; q.c_dtype = SQ8_F32; q.ldc = ldx;
    q.m = m; q.k = k; q.n = n;
    q.residual = true; q.gate = gate;
    return run_w8a8(ctx, q, gpu_seconds);
}

int sq8_linear_w8a8_qkv(sq8_ctx *ctx, const int8_t *codes, int64_t ldq, const float *sx, const void *w, int w_layout,
                        int64_t ldw, const float *scale, int scale_layout, const float *bias, void *q_out, void *k_out,
                        void *v_out, int c_dtype, int64_t ldo, int head_dim, int m, int k, int d, double *gpu_seconds) {
    if (d < 0 || (d % 4) != 0 || head_dim < 0) return SQ8_EINVAL;
    if (head_dim > 0 && ((d % head_dim) != 0 || (head_dim % 4) != 0)) return SQ8_EINVAL;
    if (head_dim == 0 && ldo < d) return SQ8_EINVAL;
    if (d > 0 && (!q_out || !k_out || !v_out)) return SQ8_EINVAL;
    if ((int64_t)3 * d > INT32_MAX) return SQ8_EINVAL;
    W8A8 q;
    memset(&q, 0, sizeof(q));
    q.codes = codes; q.ldq = ldq; q.sx = sx;
    q.w = w; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = scale; q.scale_layout = scale_layout; q.bias = bias; q.epilogue = SQ8_EPI_NONE;
    q.c[0] = q_out; q.c[1] = k_out; q.c[2] = v_out; q.c_dtype = c_dtype; q.ldc = ldo;
    q.split = d; q.head_dim = head_dim;
    q.m = m; q.k = k; q.n = 3 * d;
    return run_w8a8(ctx, q, gpu_seconds);
}

int sq8_norm_modulate_rotated(sq8_ctx *ctx, const float *x, int64_t ldx, const float *w, const float *scale,
                              const float *shift, float eps, int group, uint16_t *out, int64_t ldo, float *y_out,
                              int64_t ldy, int rows, int cols) {
    if (!ctx || rows < 0 || cols < 0) return SQ8_EINVAL;
    if (!sq8::is_rotation_group(group) || cols % group != 0) return SQ8_EINVAL;
    if (rows == 0 || cols == 0) return SQ8_OK;
    if (!x || !w || !scale || !shift || !out || ldx < cols || ldo < cols || (y_out && ldy < cols)) return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    const hipError_t e = sq8::launch_norm_operand(x, ldx, w, scale, shift, eps, rows, cols, group, y_out, ldy, out, ldo,
                                                  nullptr, 0, 0, nullptr, ctx->stream);
    return e == hipErrorInvalidValue ? SQ8_EUNSUPPORTED : hip_status(e);
}

int sq8_norm_modulate_quantized(sq8_ctx *ctx, const float *x, int64_t ldx, const float *w, const float *scale,
                                const float *shift, float eps, int group, int8_t *codes, int64_t ldq, float *scales,
                                float *y_out, int64_t ldy, int rows, int cols) {
    if (!ctx || rows < 0 || cols < 0) return SQ8_EINVAL;
    if (group != 0 && (!sq8::is_rotation_group(group) || cols % group != 0)) return SQ8_EINVAL;
    if (rows == 0 || cols == 0) return SQ8_OK;
    if (!x || !w || !scale || !shift || !codes || !scales || ldx < cols || ldq < cols || (y_out && ldy < cols))
        return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    const hipError_t e = sq8::launch_norm_operand(x, ldx, w, scale, shift, eps, rows, cols, group, y_out, ldy, nullptr, 0,
                                                  codes, ldq, cols, scales, ctx->stream);
    return e == hipErrorInvalidValue ? SQ8_EUNSUPPORTED : hip_status(e);
}

int sq8_linear_quantized(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, int group, const void *w, int w_layout,
                         int64_t ldw, const float *scale, int scale_layout, const float *bias, int epilogue, void *c,
                         int c_dtype, int64_t ldc, int m, int k, int n, double *gpu_seconds) {
    if (!a && m > 0) return SQ8_EINVAL;
    W8A8 q;
    memset(&q, 0, sizeof(q));
    q.a = a; q.a_dtype = a_dtype; q.lda = lda; q.group = group;
    q.w = w; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = scale; q.scale_layout = scale_layout; q.bias = bias; q.epilogue = epilogue;
    q.c[0] = c; q.c_dtype = c_dtype; q.ldc = ldc;
    q.m = m; q.k = k; q.n = n;
    if (!a) return m == 0 ? SQ8_OK : SQ8_EINVAL;
    return run_w8a8(ctx, q, gpu_seconds);
}

int sq8_linear_quantized_static(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, int group, const void *w,
                                int w_layout, int64_t ldw, const float *scale, int scale_layout, const float *bias,
                                int epilogue, void *c, int c_dtype, int64_t ldc, int m, int k, int n,
                                double *gpu_seconds) {
    if (!a && m > 0) return SQ8_EINVAL;
    W8A8 q;
    memset(&q, 0, sizeof(q));
    q.a = a; q.a_dtype = a_dtype; q.lda = lda; q.group = group;
    q.w = w; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = scale; q.scale_layout = scale_layout; q.bias = bias; q.epilogue = epilogue;
    q.c[0] = c; q.c_dtype = c_dtype; q.ldc = ldc;
    q.m = m; q.k = k; q.n = n;
    q.no_alloc = true;
    if (!a) return m == 0 ? SQ8_OK : SQ8_EINVAL;
    return run_w8a8(ctx, q, gpu_seconds);
}

int64_t sq8_static_scratch_bytes(void) { return (int64_t)SQ8_STATIC_SCRATCH_BYTES; }

int64_t sq8_packed_bytes(int k, int n, int glu) {
    if (k < 0 || n < 0 || (glu && (n % 2) != 0)) return -1;
    return sq8::packed_bytes(k, n, glu != 0);
}

int sq8_pack_weight(sq8_ctx *ctx, const void *w, int w_layout, int64_t ldw, int k, int n, int glu, void *out) {
    if (!ctx || k < 0 || n < 0 || (glu && (n % 2) != 0)) return SQ8_EINVAL;
    if (w_layout != SQ8_KN && w_layout != SQ8_NK) return SQ8_EINVAL;
    if (ldw < (w_layout == SQ8_KN ? n : k)) return SQ8_EINVAL;
    if (k == 0 || n == 0) return SQ8_OK;
    if (!w || !out) return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(sq8::launch_pack(static_cast<const uint8_t *>(w), w_layout == SQ8_KN ? sq8::W_KN : sq8::W_NK, ldw,
                                       k, n, glu != 0, static_cast<uint8_t *>(out), ctx->stream));
}

int sq8_dequantize(sq8_ctx *ctx, const void *codes, int w_dtype, int64_t rows, int64_t columns, const void *scale,
                   int scale_dtype, int scale_layout, int64_t block_rows, int64_t first_row, float *out) {
    if (!ctx) return SQ8_EINVAL;
    if (w_dtype != SQ8_INT8 && w_dtype != SQ8_FP8_E4M3) return SQ8_EUNSUPPORTED;
    if (rows < 0 || columns < 0 || first_row < 0) return SQ8_EINVAL;
    if (rows == 0 || columns == 0) return SQ8_OK;
    if (!codes || !out) return SQ8_EINVAL;
    if (scale) {
        if (scale_dtype != SQ8_F32 && scale_dtype != SQ8_BF16 && scale_dtype != SQ8_F16) return SQ8_EUNSUPPORTED;
        if (scale_layout < SQ8_SCALE_TENSOR || scale_layout > SQ8_SCALE_ROWS) return SQ8_EINVAL;
        if (scale_layout == SQ8_SCALE_BLOCKS && block_rows <= 0) return SQ8_EINVAL;
    }
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(sq8::launch_dequantize(static_cast<const uint8_t *>(codes),
                                             w_dtype == SQ8_INT8 ? sq8::W_INT8 : sq8::W_FP8, rows, columns, scale,
                                             scale_dtype, scale_layout, block_rows, first_row, out, ctx->stream));
}

int sq8_round_bf16(sq8_ctx *ctx, const float *x, uint16_t *y, int64_t count) {
    if (!ctx || count < 0) return SQ8_EINVAL;
    if (count == 0) return SQ8_OK;
    if (!x || !y) return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(sq8::launch_round_bf16(x, y, count, ctx->stream));
}

int sq8_norm_modulate(sq8_ctx *ctx, const float *x, int64_t ldx, const float *w, const float *scale,
                      const float *shift, float eps, uint16_t *out, int64_t ldo, int rows, int cols) {
    if (!ctx || rows < 0 || cols < 0) return SQ8_EINVAL;
    if (rows == 0 || cols == 0) return SQ8_OK;
    if (!x || !w || !scale || !shift || !out || ldx < cols || ldo < cols || !(eps >= 0.0f)) return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(sq8::launch_norm_modulate(x, ldx, w, scale, shift, eps, out, ldo, rows, cols, ctx->stream));
}

int sq8_rms_rows(sq8_ctx *ctx, uint16_t *t, int64_t ld, int64_t rows, int cols, const float *w, float eps) {
    if (!ctx || rows < 0 || cols < 0) return SQ8_EINVAL;
    if (rows == 0 || cols == 0) return SQ8_OK;
    if (!t || !w || ld < cols || !(eps >= 0.0f)) return SQ8_EINVAL;
    if (cols > 256) return SQ8_EUNSUPPORTED;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(sq8::launch_rms_rows(t, ld, rows, cols, w, eps, ctx->stream));
}

int sq8_gated_residual(sq8_ctx *ctx, float *x, int64_t ldx, const void *y, int y_dtype, int64_t ldy,
                       const float *gate, int64_t rows, int cols) {
    if (!ctx || rows < 0 || cols < 0) return SQ8_EINVAL;
    if (rows == 0 || cols == 0) return SQ8_OK;
    if (!x || !y || ldx < cols || ldy < cols) return SQ8_EINVAL;
    if (y_dtype != SQ8_BF16 && y_dtype != SQ8_F32) return SQ8_EUNSUPPORTED;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(sq8::launch_gated_residual(x, ldx, y, y_dtype == SQ8_BF16, ldy, gate, rows, cols, ctx->stream));
}

int sq8_synchronize(sq8_ctx *ctx) {
    if (!ctx) return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(hipStreamSynchronize(ctx->stream));
}


int64_t sq8_packed_blocks_bytes(int k, int n, int glu) {
    if (k < 0 || n < 0 || (glu && (n % 2) != 0)) return -1;
    return sq8::packed_blocks_bytes(k, n, glu != 0);
}

int sq8_pack_blocks(sq8_ctx *ctx, const void *w, int w_layout, int64_t ldw, const void *scale, int scale_dtype,
                    int block, int k, int n, int glu, void *out) {
    if (!ctx || k < 0 || n < 0 || (glu && (n % 2) != 0) || block <= 0) return SQ8_EINVAL;
    if (w_layout != SQ8_KN && w_layout != SQ8_NK) return SQ8_EINVAL;
    if (!scale_dtype_ok(scale_dtype)) return SQ8_EINVAL;
    if (ldw < (w_layout == SQ8_KN ? n : k)) return SQ8_EINVAL;
    if (block % 32 != 0 || k % block != 0) return SQ8_EUNSUPPORTED;
    if (k == 0 || n == 0) return SQ8_OK;
    if (!w || !scale || !out) return SQ8_EINVAL;
    if (!aligned(out, 16)) return SQ8_EINVAL;
    DeviceScope scope(ctx->device);
    if (scope.error != hipSuccess) return hip_status(scope.error);
    return hip_status(sq8::launch_pack_blocks(static_cast<const uint8_t *>(w), w_layout == SQ8_KN ? sq8::W_KN : sq8::W_NK,
                                              ldw, scale, scale_dtype, block, k, n, glu != 0,
                                              static_cast<uint8_t *>(out), ctx->stream));
}

int sq8_linear_blocks(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, const void *w, int w_layout, int64_t ldw,
                      const void *scale, int scale_dtype, int block, const float *bias, int epilogue, void *c,
                      int c_dtype, int64_t ldc, int m, int k, int n, double *gpu_seconds) {
    Blocks q;
    memset(&q, 0, sizeof(q));
    q.a = a; q.a_dtype = a_dtype; q.lda = lda;
    q.w = w; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = scale; q.scale_dtype = scale_dtype; q.block = block;
    q.bias = bias; q.epilogue = epilogue;
    q.c = c; q.c_dtype = c_dtype; q.ldc = ldc;
    q.m = m; q.k = k; q.n = n;
    return run_blocks(ctx, q, gpu_seconds);
}

int sq8_linear_f32(sq8_ctx *ctx, const float *a, int64_t lda, int group, const void *w, int w_dtype, int w_layout,
                   int64_t ldw, const void *scale, int scale_dtype, int scale_layout, int block, const float *bias,
                   int epilogue, void *c, int c_dtype, int64_t ldc, int m, int k, int n, double *gpu_seconds) {
    if (scale_layout == SQ8_SCALE_BLOCKS) {
        // Block scales take int8 codes and no rotation (the reference's Artifact refuses one there).
        if (w_dtype != SQ8_INT8 || group != 0) return SQ8_EUNSUPPORTED;
        Blocks q;
        memset(&q, 0, sizeof(q));
        q.a = a; q.a_dtype = SQ8_F32; q.lda = lda;
        q.w = w; q.w_layout = w_layout; q.ldw = ldw;
        q.scale = scale; q.scale_dtype = scale_dtype; q.block = block;
        q.bias = bias; q.epilogue = epilogue;
        q.c = c; q.c_dtype = c_dtype; q.ldc = ldc;
        q.m = m; q.k = k; q.n = n;
        q.exact = true;
        return run_blocks(ctx, q, gpu_seconds);
    }
    if (scale_dtype != SQ8_F32 || block != 0) return SQ8_EINVAL;
    Product q;
    memset(&q, 0, sizeof(q));
    q.a = a; q.a_dtype = SQ8_F32; q.lda = lda;
    q.w = w; q.w_dtype = w_dtype; q.w_layout = w_layout; q.ldw = ldw;
    q.scale = static_cast<const float *>(scale); q.scale_layout = scale_layout; q.bias = bias; q.epilogue = epilogue;
    q.c[0] = c; q.c_dtype = c_dtype; q.ldc = ldc;
    q.m = m; q.k = k; q.n = n;
    q.group = group;
    q.exact = true;
    return run_product(ctx, q, gpu_seconds);
}

int sq8_linear_bf16_weight(sq8_ctx *ctx, const void *a, int a_dtype, int64_t lda, const void *w, int w_layout,
                           int64_t ldw, float *c, int64_t ldc, int m, int k, int n, double *gpu_seconds) {
    return run_bf16_weight(ctx, a, a_dtype, lda, w, w_layout, ldw, c, ldc, m, k, n, gpu_seconds);
}

}  // extern "C"
