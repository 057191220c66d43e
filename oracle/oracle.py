"""ctypes view of the CPU oracle (oracle/libsq8_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, where it is the checker. The product path (siliconed_amd) never imports it.

Each wrapper names the reference file:line its C function restates (paths relative to the
reference root).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsq8_oracle.so")

BF16, F32, INT8, FP8_E4M3, F16 = 1, 2, 3, 4, 5
SCALE_TENSOR, SCALE_COLUMNS, SCALE_BLOCKS, SCALE_ROWS = 0, 1, 2, 3
EPI_NONE, EPI_GELU_TANH, EPI_SILU_GLU, EPI_SITU_GLU = 0, 1, 2, 3

_lib = None


def build() -> None:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(l: ctypes.CDLL) -> None:
    P, I, I64, U64, D, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_double, ctypes.c_size_t
    sig = {
        "orc_splitmix_next": (U64, [P]),
        "orc_splitmix_uniform": (D, [P]),
        "orc_splitmix_normal": (D, [P]),
        "orc_fill_normal_bf16": (None, [U64, D, D, P, SZ]),
        "orc_fill_normal_f32": (None, [U64, D, D, P, SZ]),
        "orc_fill_uniform_f32": (None, [U64, D, D, P, SZ]),
        "orc_fill_uniform_i8": (None, [U64, I, I, P, SZ]),
        "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_e4m3_to_f32": (ctypes.c_float, [ctypes.c_uint8]),
        "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_f32_to_e4m3": (ctypes.c_uint8, [ctypes.c_float]),
        "orc_quantize_e4m3": (None, [P, P, SZ]),
        "orc_dequantize": (None, [P, I, SZ, P, I, I, SZ, SZ, SZ, P]),
        "orc_is_rotation_group": (I, [I]),
        "orc_rotation_norm": (ctypes.c_float, [I]),
        "orc_rotate_groups": (None, [P, I64, P, I64, I, I, I]),
        "orc_dequantize_rotated": (None, [P, I64, I, I, I, P, I, I, P, I64]),
        "orc_quantize_rows": (None, [P, I64, I, I, I, P, I64, P]),
        "orc_w8a8_product": (None, [P, I64, P, P, I, I64, P, I, I, I, I, P, I64]),
        "orc_gelu_tanh": (D, [D]),
        "orc_silu_glu": (D, [D, D]),
        "orc_situ": (D, [D, D]),
        "orc_sample_rows": (None, [I, I, P]),
        "orc_exact_rows": (None, [P, I, P, I64, P, I, I64, I, I, P, P, I, P]),
        "orc_exact_rows_f32": (None, [P, I, P, I64, P, I, I64, I, I, P, P, I, P]),
        "orc_channel_error": (D, [P, P, I, I, P, P]),
        "orc_linear_f32": (None, [P, I64, P, I64, I, I, I, P, I, P, I64, I]),
        "orc_epilogue_f32": (None, [P, I64, I, I, P, I, P, I64, I]),
        "orc_version": (I, []),
    }
    for name, (res, args) in sig.items():
        f = getattr(l, name)
        f.restype = res
        f.argtypes = args


def _p(x):
    return None if x is None else ctypes.c_void_p(x.ctypes.data)


# ---- synthetic inputs: Sources/Verification/KernelStages.swift:553-567 ----------------------

def splitmix_stream(seed: int, count: int) -> np.ndarray:
    st = ctypes.c_uint64(seed)
    return np.array([lib().orc_splitmix_next(ctypes.byref(st)) for _ in range(count)], dtype=np.uint64)


def normal_bf16(seed: int, shape, mean=0.0, std=1.0) -> np.ndarray:
    """bf16 bits (uint16) of fp32 draws mean + std·N(0,1), rounded nearest-even."""
    out = np.empty(shape, dtype=np.uint16)
    lib().orc_fill_normal_bf16(seed, mean, std, _p(out), out.size)
    return out


def normal_f32(seed: int, shape, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().orc_fill_normal_f32(seed, mean, std, _p(out), out.size)
    return out


def uniform_f32(seed: int, shape, lo: float, hi: float) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().orc_fill_uniform_f32(seed, lo, hi, _p(out), out.size)
    return out


def uniform_i8(seed: int, shape, lo=-127, hi=127) -> np.ndarray:
    out = np.empty(shape, dtype=np.int8)
    lib().orc_fill_uniform_i8(seed, lo, hi, _p(out), out.size)
    return out


def quantize_int8_per_row(w: np.ndarray):
    """Per-output-channel int8: s = amax/127, q = clamp(rint(w/s), −127, 127) (nn.Linear [N, K])."""
    amax = np.abs(w).max(axis=1).astype(np.float32)
    s = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(w / s[:, None]), -127, 127).astype(np.int8)
    return q, s


def quantize_fp8_per_row(w: np.ndarray):
    """Per-output-channel e4m3fn: s = amax/448, q = e4m3fn(RNE(w/s)) saturating (nn.Linear [N, K])."""
    amax = np.abs(w).max(axis=1).astype(np.float32)
    s = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    q = f32_to_e4m3((w / s[:, None]).astype(np.float32))
    return q, s


# ---- conversions --------------------------------------------------------------------------

def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Sources/Siliconed/TensorGEMMBF16.swift:43-47, elementwise (vectorised restatement)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    q = ((u >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return np.where(nan, q, r)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    """Sources/Siliconed/Widen.swift:25-49."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def e4m3_table() -> np.ndarray:
    """All 256 codes decoded by the C restatement of Forge/Numerics.swift:48-55."""
    return np.array([lib().orc_e4m3_to_f32(b) for b in range(256)], dtype=np.float32)


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """fp32 → e4m3fn, nearest-even, saturating at ±448 (NaN → 0x7F)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().orc_quantize_e4m3(_p(x), _p(out), x.size)
    return out


def dequantize(values: np.ndarray, kind: int, scale: np.ndarray | None, scale_type: int = F32,
               layout: int = SCALE_COLUMNS, columns: int = 0, block_rows: int = 0,
               first_row: int = 0) -> np.ndarray:
    """Sources/Siliconed/Widen.swift:129-187: Float(q)·s, one fp32 multiply."""
    values = np.ascontiguousarray(values)
    out = np.empty(values.size, dtype=np.float32)
    sc = None if scale is None else np.ascontiguousarray(scale)
    lib().orc_dequantize(_p(values), kind, values.size, _p(sc), scale_type, layout, columns, block_rows,
                         first_row, _p(out))
    return out.reshape(values.shape)


# ---- convrot: Sources/Siliconed/Widen.swift:316-428, TensorGEMM.swift:181-201 -------------

def is_rotation_group(g: int) -> bool:
    """Widen.swift:335-340: a power of 4, 4 to 256."""
    return bool(lib().orc_is_rotation_group(int(g)))


def rotate_groups(x: np.ndarray, group: int) -> np.ndarray:
    """TensorGEMM.swift:183-201: fp32 rows [rows, k] times R = H/sqrt(G) by groups (fp32 butterflies)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    assert k % group == 0 and is_rotation_group(group)
    y = np.empty_like(x)
    lib().orc_rotate_groups(_p(x), k, _p(y), k, rows, k, group)
    return y


def dequantize_rotated(q: np.ndarray, group: int, scale: np.ndarray, scale_type: int = F32,
                       layout: int = SCALE_COLUMNS) -> np.ndarray:
    """Widen.swift:374-428: int8 [k, n] -> fp32 Float(H.q) * (s / sqrt(G)) per group of rows."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    k, n = q.shape
    assert k % group == 0 and is_rotation_group(group)
    out = np.empty((k, n), dtype=np.float32)
    sc = np.ascontiguousarray(scale)
    lib().orc_dequantize_rotated(_p(q), n, k, n, group, _p(sc), scale_type, layout, _p(out), n)
    return out


# ---- W8A8: Sources/Siliconed/TensorGEMMInt8.swift:4-37, 198-221 ------------------------------

def quantize_rows(x: np.ndarray, group: int = 0):
    """W8A8.quantize per row (TensorGEMMInt8.swift:198-221): int8 codes [rows, k], fp32 scales [rows]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    codes = np.empty((rows, k), dtype=np.int8)
    scales = np.empty(rows, dtype=np.float32)
    lib().orc_quantize_rows(_p(x), k, rows, k, int(group), _p(codes), k, _p(scales))
    return codes, scales


def w8a8_product(codes: np.ndarray, sx: np.ndarray, w: np.ndarray, w_kn: bool, sw: np.ndarray) -> np.ndarray:
    """float(Σ codes·w) · (s_x · s_w), the sums exact: fp32 [m, n]."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    m, k = codes.shape
    n = w.shape[1] if w_kn else w.shape[0]
    sx = np.ascontiguousarray(sx, dtype=np.float32)
    sw = np.ascontiguousarray(sw, dtype=np.float32)
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_w8a8_product(_p(codes), k, _p(sx), _p(w), int(w_kn), w.shape[1], _p(sw), int(sw.size != 1), m, k, n,
                           _p(c), n)
    return c


# ---- truth and judgement ------------------------------------------------------------------

def sample_rows(m: int, count: int = 64) -> np.ndarray:
    """Sources/Siliconed/DiagnosticProbes.swift:75-77."""
    count = min(count, m)
    out = np.empty(count, dtype=np.int32)
    lib().orc_sample_rows(m, count, _p(out))
    return out


def exact_rows(rows: np.ndarray, a_bf16: np.ndarray, w: np.ndarray, w_kn: bool, k: int, n: int,
               scale: np.ndarray | None = None, bias: np.ndarray | None = None,
               epilogue: int = EPI_NONE) -> np.ndarray:
    """fp64 rows of act(A·W·diag(s) + b): DiagnosticProbes.swift:82-178 (+ the epilogue in double).

    `a_bf16`: bf16 bits (uint16), or fp32 values taken whole. `w` fp32: [K, N] if w_kn else [N, K]
    (raw codes as floats with `scale`, or dequantized with scale None). Returns [len(rows), n_out]
    float64.
    """
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    f32 = a_bf16.dtype == np.float32      # an fp32 A taken whole (the fp32 route's truth)
    a_bf16 = np.ascontiguousarray(a_bf16, dtype=np.float32 if f32 else np.uint16)
    w = np.ascontiguousarray(w, dtype=np.float32)
    glu = epilogue in (EPI_SILU_GLU, EPI_SITU_GLU)
    n_out = n // 2 if glu else n
    out = np.empty((rows.size, n_out), dtype=np.float64)
    sc = None if scale is None else np.ascontiguousarray(scale, dtype=np.float32)
    bi = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    ldw = w.shape[1]
    (lib().orc_exact_rows_f32 if f32 else lib().orc_exact_rows)(
                         _p(rows), rows.size, _p(a_bf16), a_bf16.shape[1], _p(w), int(w_kn), ldw, k, n,
                         _p(sc), _p(bi), epilogue, _p(out))
    return out


def channel_error(got: np.ndarray, expected: np.ndarray):
    """DiagnosticJudgement.swift:39-71 → (worst, channel, median)."""
    got = np.ascontiguousarray(got, dtype=np.float32)
    expected = np.ascontiguousarray(expected, dtype=np.float64)
    rows, cols = expected.shape
    ch = ctypes.c_int(0)
    med = ctypes.c_double(0)
    worst = lib().orc_channel_error(_p(got), _p(expected), rows, cols, ctypes.byref(ch), ctypes.byref(med))
    return worst, ch.value, med.value


def linear_f32(a_bf16: np.ndarray, w_kn_f32: np.ndarray, bias=None, epilogue=EPI_NONE, threads=None) -> np.ndarray:
    """The reference's CPU route (WeightProducts.swift:698-709 + Ops.swift:386-407), fp32."""
    a_bf16 = np.ascontiguousarray(a_bf16, dtype=np.uint16)
    w = np.ascontiguousarray(w_kn_f32, dtype=np.float32)
    m, k = a_bf16.shape
    n = w.shape[1]
    glu = epilogue in (EPI_SILU_GLU, EPI_SITU_GLU)
    n_out = n // 2 if glu else n
    c = np.empty((m, n_out), dtype=np.float32)
    bi = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().orc_linear_f32(_p(a_bf16), k, _p(w), n, m, k, n, _p(bi), epilogue, _p(c), n_out,
                         threads or os.cpu_count() or 1)
    return c


def epilogue_f32(p: np.ndarray, bias=None, epilogue=EPI_NONE, threads=None) -> np.ndarray:
    p = np.ascontiguousarray(p, dtype=np.float32)
    m, n = p.shape
    glu = epilogue in (EPI_SILU_GLU, EPI_SITU_GLU)
    n_out = n // 2 if glu else n
    c = np.empty((m, n_out), dtype=np.float32)
    bi = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().orc_epilogue_f32(_p(p), n, m, n, _p(bi), epilogue, _p(c), n_out, threads or os.cpu_count() or 1)
    return c
