"""The allocation-free W8A8 entry point (sq8_linear_quantized_static), through the C ABI, against the
allocating one it mirrors (sq8_linear_quantized): the same kernels on the same operands, so the same
bits. Two calls in a row, the second smaller, so the second reads the static scratch the first left
behind (codes past its own rows are the first call's): each must equal its allocating twin."""
import ctypes

import numpy as np
import pytest
import torch

from siliconed_amd import _abi as abi

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _static(gemm, x, w, s, b, group, epi, out):
    """`w`: a PackedWeight, or [N, K] int8 codes read in place (layout NK, ldw = its row stride)."""
    m, k = x.shape
    if isinstance(w, torch.Tensor):
        wptr, lay, ldw, n = w.data_ptr(), abi.NK, w.stride(0), w.shape[0]
    else:
        wptr, lay, ldw, n = w.data.data_ptr(), w.layout, w.k, w.n
    st = abi.load().sq8_linear_quantized_static(
        gemm._h, x.data_ptr(), abi.F32 if x.dtype == torch.float32 else abi.BF16, x.stride(0), group,
        wptr, lay, ldw, s.data_ptr(), abi.SCALE_COLUMNS, None if b is None else b.data_ptr(), epi,
        out.data_ptr(), abi.BF16 if out.dtype == torch.bfloat16 else abi.F32, out.stride(0), m, k, n, None)
    return st


@pytest.mark.parametrize("layout", ["packed", "nk"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_static_scratch_equals_the_allocating_route(gemm, orc, out_dtype, layout):
    """Packed weights, and [N, K] codes read in place (k % 128 == 0, 16-byte aligned rows)."""
    cases = [(2048, 3072, 3072, 256, abi.EPI_GELU_TANH, "gelu_tanh"),   # 6.3 MB of codes
             (37, 1024, 640, 0, abi.EPI_NONE, None)]                     # smaller: the first call's codes remain
    for i, (m, k, n, group, epi, name) in enumerate(cases):
        print(f"static scratch call {i}: {layout} m {m} k {k} n {n} group {group} out {out_dtype}", flush=True)
        x = torch.from_numpy(orc.normal_f32(40 + i, (m, k))).to(DEV)
        q = torch.from_numpy(orc.uniform_i8(41 + i, (n, k))).to(DEV)
        s = torch.from_numpy(orc.uniform_f32(42 + i, (n,), 1e-3, 2e-2)).to(DEV)
        b = torch.from_numpy(orc.normal_f32(43 + i, (n,), 0.0, 0.02)).to(DEV)
        w = gemm.pack(q, layout="nk") if layout == "packed" else q
        want = gemm.product_quantized(x, w, s, layout="nk", group=group, bias=b, epilogue=name, out_dtype=out_dtype)
        got = torch.full((m, n), float("nan"), dtype=out_dtype, device=DEV)
        assert _static(gemm, x, w, s, b, group, epi, got) == abi.OK
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32),
                           want.view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32))


def test_static_scratch_refuses_what_it_cannot_hold(gemm, orc):
    # Codes of 8192 rows × 8192 = 64 MiB plus the row scales: past the capacity, refused before any work.
    m, k, n = 8192, 8192, 128
    assert m * k + 4 * m > abi.load().sq8_static_scratch_bytes()
    x = torch.zeros((m, k), dtype=torch.bfloat16, device=DEV)
    q = torch.zeros((n, k), dtype=torch.int8, device=DEV)
    w = gemm.pack(q, layout="nk")
    s = torch.ones(n, dtype=torch.float32, device=DEV)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    assert _static(gemm, x, w, s, None, 0, abi.EPI_NONE, out) == abi.ECAPACITY
    # A [K, N] weight would need a repack buffer: refused (the allocating entry point repacks it).
    qkn = torch.zeros((256, n), dtype=torch.int8, device=DEV)
    x2 = torch.zeros((4, 256), dtype=torch.float32, device=DEV)
    out2 = torch.empty((4, n), dtype=torch.bfloat16, device=DEV)
    st = abi.load().sq8_linear_quantized_static(gemm._h, x2.data_ptr(), abi.F32, 256, 0, qkn.data_ptr(), abi.KN, n,
                                                 s.data_ptr(), abi.SCALE_COLUMNS, None, abi.EPI_NONE, out2.data_ptr(),
                                                 abi.BF16, n, 4, 256, n, None)
    assert st == abi.EUNSUPPORTED
    torch.cuda.synchronize()
