"""ctypes binding of the C ABI (include/siliconed_q8.h) in libsiliconed_q8.so.

The library is loaded from this package's directory only; a missing library is an error, never a
fallback: there is no CPU path behind these functions.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libsiliconed_q8.so")

# Values of include/siliconed_q8.h.
OK, EINVAL, EUNSUPPORTED, ENODEVICE, ECAPACITY = 0, 1, 2, 3, 4
BF16, F32, INT8, FP8_E4M3, F16 = 1, 2, 3, 4, 5
KN, NK, PACKED, PACKED_GLU = 0, 1, 2, 3
SCALE_TENSOR, SCALE_COLUMNS, SCALE_BLOCKS, SCALE_ROWS = 0, 1, 2, 3
EPI_NONE, EPI_GELU_TANH, EPI_SILU_GLU, EPI_SITU_GLU = 0, 1, 2, 3

# Every symbol the header declares, with (restype, argtypes).
_P, _I, _I64, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double
SIGNATURES = {
    "sq8_create": (_I, [_I, _P, ctypes.POINTER(_P)]),
    "sq8_destroy": (_I, [_P]),
    "sq8_set_stream": (_I, [_P, _P]),
    "sq8_supports": (_I, [_P, _I, _I, _I, _I, _I, _I]),
    "sq8_linear": (_I, [_P, _P, _I, _I64, _P, _I, _I, _I64, _P, _I, _P, _I, _P, _I, _I64, _I, _I, _I,
                        ctypes.POINTER(_D)]),
    "sq8_linear_qkv": (_I, [_P, _P, _I, _I64, _P, _I, _I, _I64, _P, _I, _P, _P, _P, _P, _I, _I64, _I, _I, _I, _I,
                            ctypes.POINTER(_D)]),
    "sq8_linear_rotated": (_I, [_P, _P, _I, _I64, _I, _P, _I, _I, _I64, _P, _I, _P, _I, _P, _I, _I64, _I, _I, _I,
                                ctypes.POINTER(_D)]),
    "sq8_rotate_groups": (_I, [_P, _P, _I, _I64, _P, _I, _I64, _I, _I, _I]),
    "sq8_dequantize_rotated": (_I, [_P, _P, _I64, _I, _I, _I, _P, _I, _I, _P, _I64]),
    "sq8_quantize_rows": (_I, [_P, _P, _I, _I64, _I, _I, _I, _P, _I64, _P]),
    "sq8_linear_w8a8": (_I, [_P, _P, _I64, _P, _P, _I, _I64, _P, _I, _P, _I, _P, _I, _I64, _I, _I, _I,
                             ctypes.POINTER(_D)]),
    "sq8_linear_quantized": (_I, [_P, _P, _I, _I64, _I, _P, _I, _I64, _P, _I, _P, _I, _P, _I, _I64, _I, _I, _I,
                                  ctypes.POINTER(_D)]),
    "sq8_linear_quantized_static": (_I, [_P, _P, _I, _I64, _I, _P, _I, _I64, _P, _I, _P, _I, _P, _I, _I64, _I, _I,
                                         _I, ctypes.POINTER(_D)]),
    "sq8_static_scratch_bytes": (_I64, []),
    "sq8_linear_w8a8_qkv": (_I, [_P, _P, _I64, _P, _P, _I, _I64, _P, _I, _P, _P, _P, _P, _I, _I64, _I, _I, _I, _I,
                                 ctypes.POINTER(_D)]),
    "sq8_norm_modulate_rotated": (_I, [_P, _P, _I64, _P, _P, _P, ctypes.c_float, _I, _P, _I64, _P, _I64, _I, _I]),
    "sq8_norm_modulate_quantized": (_I, [_P, _P, _I64, _P, _P, _P, ctypes.c_float, _I, _P, _I64, _P, _P, _I64, _I, _I]),
    "sq8_linear_residual": (_I, [_P, _P, _I, _I64, _P, _I, _I, _I64, _P, _I, _P, _P, _P, _I64, _I, _I, _I,
                                 ctypes.POINTER(_D)]),
    "sq8_linear_w8a8_residual": (_I, [_P, _P, _I64, _P, _P, _I, _I64, _P, _I, _P, _P, _P, _I64, _I, _I, _I,
                                      ctypes.POINTER(_D)]),
    "sq8_packed_bytes": (_I64, [_I, _I, _I]),
    "sq8_pack_weight": (_I, [_P, _P, _I, _I64, _I, _I, _I, _P]),
    "sq8_linear_f32": (_I, [_P, _P, _I64, _I, _P, _I, _I, _I64, _P, _I, _I, _I, _P, _I, _P, _I, _I64, _I, _I, _I,
                            ctypes.POINTER(ctypes.c_double)]),
    "sq8_linear_bf16_weight": (_I, [_P, _P, _I, _I64, _P, _I, _I64, _P, _I64, _I, _I, _I, ctypes.POINTER(_D)]),
    "sq8_linear_blocks": (_I, [_P, _P, _I, _I64, _P, _I, _I64, _P, _I, _I, _P, _I, _P, _I, _I64, _I, _I, _I,
                               ctypes.POINTER(ctypes.c_double)]),
    "sq8_packed_blocks_bytes": (_I64, [_I, _I, _I]),
    "sq8_pack_blocks": (_I, [_P, _P, _I, _I64, _P, _I, _I, _I, _I, _I, _P]),
    "sq8_dequantize": (_I, [_P, _P, _I, _I64, _I64, _P, _I, _I, _I64, _I64, _P]),
    "sq8_round_bf16": (_I, [_P, _P, _P, _I64]),
    "sq8_norm_modulate": (_I, [_P, _P, _I64, _P, _P, _P, ctypes.c_float, _P, _I64, _I, _I]),
    "sq8_rms_rows": (_I, [_P, _P, _I64, _I64, _I, _P, ctypes.c_float]),
    "sq8_gated_residual": (_I, [_P, _P, _I64, _P, _I, _I64, _P, _I64, _I]),
    "sq8_synchronize": (_I, [_P]),
    "sq8_status_string": (ctypes.c_char_p, [_I]),
    "sq8_abi_version": (_I, []),
}

_lib = None


class SQ8Error(RuntimeError):
    """A call the library refused (status > 0) or a HIP error (status < 0)."""

    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {status_string(status)} (status {status})")


class Unsupported(SQ8Error):
    """The library does not run this configuration: the caller keeps its widened route."""


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def status_string(status: int) -> str:
    return load().sq8_status_string(status).decode()


def check(status: int, what: str) -> None:
    if status == OK:
        return
    if status in (EUNSUPPORTED, ENODEVICE):
        raise Unsupported(status, what)
    raise SQ8Error(status, what)
