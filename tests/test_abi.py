"""The C ABI on the CPU: the library loads, exports every function include/*.h declares, and its
host-side checks answer without touching a GPU."""
import ctypes
import glob
import os
import re

import pytest

from conftest import ROOT


def _declared():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(sq8_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_abi():
    names = _declared()
    assert {"sq8_create", "sq8_destroy", "sq8_linear", "sq8_linear_qkv", "sq8_dequantize", "sq8_round_bf16"} <= set(names)


def test_library_exports_every_declared_symbol():
    from siliconed_amd import _abi
    lib = _abi.load()
    for name in _declared():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
        assert name in _abi.SIGNATURES, f"{name} has no ctypes signature"


def test_library_is_gfx950_code_object():
    from siliconed_amd import _abi
    data = open(_abi.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    assert b"gfx942" not in data and b"gfx90a" not in data


def test_status_strings_and_version():
    from siliconed_amd import _abi
    lib = _abi.load()
    assert lib.sq8_abi_version() == 1
    assert lib.sq8_status_string(0) == b"ok"
    assert b"not supported" in lib.sq8_status_string(2)
    assert b"static scratch" in lib.sq8_status_string(4)
    assert lib.sq8_static_scratch_bytes() == 64 << 20


def test_null_context_is_refused_not_crashed():
    from siliconed_amd import _abi
    lib = _abi.load()
    assert lib.sq8_destroy(None) == _abi.EINVAL
    assert lib.sq8_synchronize(None) == _abi.EINVAL
    assert lib.sq8_supports(None, 1, 3, 0, 1, 1, 0) == _abi.EINVAL
    assert lib.sq8_linear(None, None, 1, 0, None, 3, 0, 0, None, 1, None, 0, None, 1, 0, 0, 0, 0, None) == _abi.EINVAL
    assert lib.sq8_round_bf16(None, None, None, 0) == _abi.EINVAL
    # The fp32 route and the bf16-weight product refuse a null context before touching anything.
    assert lib.sq8_linear_f32(None, None, 64, 0, None, 3, 0, 64, None, 2, 1, 0, None, 0, None, 2, 64, 1, 64, 64,
                              None) == _abi.EINVAL
    assert lib.sq8_linear_bf16_weight(None, None, 2, 64, None, 0, 64, None, 64, 1, 64, 64, None) == _abi.EINVAL
    assert lib.sq8_create(0, None, None) == _abi.EINVAL
    assert lib.sq8_linear_quantized_static(None, None, 2, 64, 0, None, 1, 64, None, 1, None, 0, None, 1, 64, 1, 64,
                                           64, None) == _abi.EINVAL


def test_create_without_gfx950_says_no_device():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: covered by the GPU tests")
    from siliconed_amd import _abi
    h = ctypes.c_void_p()
    assert _abi.load().sq8_create(0, None, ctypes.byref(h)) == _abi.ENODEVICE
    assert not h.value
    import siliconed_amd as sq
    assert sq.TensorGEMM.make(0) is None  # init? → nil: the caller keeps its widened route
