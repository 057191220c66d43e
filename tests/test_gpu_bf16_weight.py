"""The bf16-weight product (sq8_linear_bf16_weight: the reference's `linear(a:w:c:m:k:n:weightIsTransposed:)`,
TensorGEMM.swift:236-254, `matmul2d` float × bfloat) through the C ABI, against the fp64 truth of the fp32
(or bf16) activation and the bf16 weight's values (DiagnosticProbes.swift:79-84, the oracle's
orc_exact_rows / orc_exact_rows_f32) at the fp32 bar, channelError ≤ 1e-5 (Diagnostic.swift:105). Both
weight layouts, ragged and empty shapes, and an identity weight returning an fp32 activation bit for
bit."""
import numpy as np
import pytest
import torch

from test_gpu_parity import DEV, bf16_dev, dev, judge

pytestmark = pytest.mark.gpu


def weight(orc, n, k, seed):
    """bf16 W [n, k] ~ N(0, 1) (bits) and its fp32 values."""
    bits = orc.normal_bf16(seed, (n, k))
    return bits, orc.bf16_to_f32(bits)


def w_dev(bits, layout):
    b = bits if layout == "nk" else np.ascontiguousarray(bits.T)
    return torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).to(DEV)


def check(orc, got, x, wv, rows=None):
    n = wv.shape[0]
    return judge(orc, got, x, wv, None, np.ones(n, np.float32), None, "none", torch.float32, rows=rows, values=True)


@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("shape", [(200, 768, 320), (1, 64, 1), (37, 100, 75), (130, 3072, 520)],
                         ids=lambda s: "x".join(map(str, s)))
def test_fp32_activation(gemm, orc, layout, shape):
    m, k, n = shape
    x = orc.normal_f32(m + k, (m, k))
    bits, wv = weight(orc, n, k, n + 1)
    y = gemm.product_bf16_weight(dev(x), w_dev(bits, layout), layout=layout)
    torch.cuda.synchronize()
    check(orc, y.cpu().numpy(), x, wv)


@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_bf16_activation(gemm, orc, layout):
    m, k, n = 150, 512, 256
    xb = orc.normal_bf16(5, (m, k))
    bits, wv = weight(orc, n, k, 6)
    y = gemm.product_bf16_weight(bf16_dev(xb), w_dev(bits, layout), layout=layout)
    torch.cuda.synchronize()
    check(orc, y.cpu().numpy(), xb, wv)


def test_identity_weight_returns_the_activation(gemm, orc):
    """W = I: each output is hi + mid + lo of one fp32 value — the value, bit for bit."""
    m, k = 64, 128
    x = orc.normal_f32(9, (m, k))
    x[0, :4] = [1.0 + 2.0 ** -23, -(1.0 - 2.0 ** -24), 3.4028235e38, 2.0 ** -100]
    eye = orc.f32_to_bf16(np.eye(k, dtype=np.float32))
    for layout in ("nk", "kn"):
        y = gemm.product_bf16_weight(dev(x), w_dev(eye, layout), layout=layout)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), x.view(np.uint32)), layout


def test_reference_entry(gemm, orc):
    """`linear(a:w:c:m:k:n:weightIsTransposed:)` as the reference calls it: fp32 A, bf16 W from offset 0."""
    m, k, n = 96, 256, 192
    x = orc.normal_f32(11, (m, k))
    bits, wv = weight(orc, n, k, 12)
    for transposed in (True, False):
        c = torch.empty((m, n), dtype=torch.float32, device=DEV)
        secs = gemm.linear_bf16_weight(dev(x), w=w_dev(bits, "kn" if transposed else "nk"), c=c, m=m, k=k, n=n,
                                       weight_is_transposed=transposed)
        assert secs > 0
        check(orc, c.cpu().numpy(), x, wv)


def test_bench_size_sampled_rows(gemm, orc):
    m, k, n = 4096, 3072, 3072
    x = orc.normal_f32(13, (m, k))
    bits, wv = weight(orc, n, k, 14)
    y = gemm.product_bf16_weight(dev(x), w_dev(bits, "nk"))
    torch.cuda.synchronize()
    check(orc, y.cpu().numpy(), x, wv, rows=orc.sample_rows(m, 64))


def test_empty_and_refused(gemm, orc):
    from siliconed_amd import abi
    from siliconed_amd.tensor_gemm import _dev
    x = dev(orc.normal_f32(1, (8, 64)))
    w = w_dev(weight(orc, 16, 64, 2)[0], "nk")
    c = torch.full((8, 16), 7.0, device=DEV)
    lib = abi.load()
    call = lambda k=64, lay=abi.NK, ldc=16, adt=abi.F32: lib.sq8_linear_bf16_weight(
        gemm._h, _dev(x, "x"), adt, 64, _dev(w, "w"), lay, 64, _dev(c, "c"), ldc, 8, k, 16, None)
    assert call(k=0) == abi.OK                   # K = 0: C written with zeros
    torch.cuda.synchronize()
    assert (c == 0).all()
    assert call(lay=abi.PACKED) == abi.EUNSUPPORTED
    assert call(ldc=15) == abi.EINVAL
    assert call(adt=abi.INT8) == abi.EUNSUPPORTED
    assert gemm.product_bf16_weight(dev(np.zeros((0, 64), np.float32)), w).shape == (0, 16)
