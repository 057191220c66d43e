"""The short-M kernel (16-column groups on 16 × 16 MFMAs, one to four groups a workgroup, K split over four
waves, every step's loads issued far ahead, the activation staged in LDS where it fits; gemm_gemv_kernel)
forced through the SQ8_TILE knob, on every route and epilogue it serves, judged element by element against
the oracle's fp64 truth with the short-product bound of test_gpu_small_m (the per-channel metric is
ill-conditioned on a handful of rows). Rows 1 … 16 (more rows take the skinny kernel under the same knob),
column counts that give one, two, three and four groups a workgroup (ragged), packed and [N, K] codes, the
activation in LDS (K a multiple of 512) and not."""
import numpy as np
import pytest
import torch

from refgen import bitwise_equal
from test_gpu_parity import bf16_dev, dev, weight_tensor
from test_gpu_small_m import _bound_check

pytestmark = pytest.mark.gpu
K = 3072

# (epilogue, output columns): 1, 2, 3 and 4 column groups a workgroup on 256 CUs, each count ragged.
CASES = [("none", 200), ("gelu", 6160), ("none", 9232), ("none", 12304), ("silu", 136), ("silu", 3080),
         ("silu", 4616), ("silu", 6152)]


@pytest.mark.parametrize("m", [1, 5, 16])
@pytest.mark.parametrize("layout", ["packed", "nk"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}{c[1]}")
def test_gemv_products(gemm, orc, tile_gemm, m, layout, case):
    epi, n_out = case
    n = 2 * n_out if epi == "silu" else n_out
    i = 7 * m + 3 * ["packed", "nk"].index(layout) + CASES.index(case)
    out = torch.bfloat16 if i % 2 == 0 else torch.float32
    k = K + 64 if i % 3 == 0 else K   # K' not a multiple of 512: the activation read from global memory
    name = {"none": None, "gelu": "gelu_tanh", "silu": "silu_glu"}[epi]
    print(f"gemv: m {m} k {k} n {n} layout {layout} epilogue {epi} out {out}", flush=True)
    x = orc.normal_bf16(i, (m, k))
    q = orc.uniform_i8(i + 1, (n, k)).view(np.uint8)
    s = orc.uniform_f32(i + 2, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(i + 3, (n,), 0.0, 0.02)
    w = weight_tensor(q, False, "nk")
    if layout == "packed":
        w = gemm.pack(w, layout="nk", glu=epi == "silu")
    y = tile_gemm("gemv").product(bf16_dev(x), w, dev(s), layout="nk", bias=dev(b), epilogue=name, out_dtype=out)
    torch.cuda.synchronize()
    _bound_check(orc, y.float().cpu().numpy(), x, q.view(np.int8).astype(np.float32), s, b, epi, out, k)


@pytest.mark.parametrize("m", [1, 16, 40])
def test_gemv_fp8_fp32_route_and_qkv(gemm, orc, tile_gemm, m):
    """fp8 codes; the fp32 route (three bf16 parts along K against the weight's steps); the fused QKV split
    head-major — each against the truth, the QKV split bit-equal to the whole product's columns."""
    n = 384
    x32 = orc.normal_f32(50 + m, (m, K))
    q, s = orc.quantize_fp8_per_row(orc.normal_f32(51 + m, (n, K), 0.0, 0.02))
    b = orc.normal_f32(52 + m, (n,), 0.0, 0.02)
    from refgen import code_values
    wv = code_values(q, True)
    g = tile_gemm("gemv")
    w = g.pack(weight_tensor(q, True, "nk"), layout="nk", fp8=True)
    y = g.product(dev(x32), w, dev(s), bias=dev(b), epilogue="gelu_tanh", out_dtype=torch.float32, rounding=False)
    torch.cuda.synchronize()
    _bound_check(orc, y.cpu().numpy(), x32, wv, s, b, "gelu", torch.float32, 3 * K)
    xb = orc.f32_to_bf16(x32)
    whole = g.product(bf16_dev(xb), w, dev(s), bias=dev(b))
    qq, kk, vv = g.product_qkv(bf16_dev(xb), w, dev(s), bias=dev(b), head_dim=64)
    torch.cuda.synchronize()
    d = n // 3
    parts = [t.permute(1, 0, 2).reshape(m, d) for t in (qq, kk, vv)]
    assert bitwise_equal(torch.cat(parts, dim=1).float().cpu().numpy(), whole.float().cpu().numpy()) == 0
    _bound_check(orc, whole.float().cpu().numpy(), xb, wv, s, b, "none", torch.bfloat16, K)


def test_gemv_residual(gemm, orc, tile_gemm):
    """The gated residual on the short-M kernel: x + gate·(s·acc + b) equals its own fp32 product followed by
    the residual pass, bit for bit."""
    m, n = 9, 320
    x, q = orc.normal_bf16(60, (m, K)), orc.uniform_i8(61, (n, K)).view(np.uint8)
    s, b = orc.uniform_f32(62, (n,), 1e-3, 2e-2), orc.normal_f32(63, (n,), 0.0, 0.02)
    stream = orc.normal_f32(64, (m, n), 0.0, 1.0)
    gate = dev(orc.normal_f32(65, (n,), 0.0, 0.5))
    g = tile_gemm("gemv")
    w = g.pack(weight_tensor(q, False, "nk"), layout="nk")
    y = g.product(bf16_dev(x), w, dev(s), bias=dev(b), out_dtype=torch.float32)
    expect = dev(stream)
    g.gated_residual(expect, y, gate)
    got = dev(stream)
    g.product_residual(got, bf16_dev(x), w, dev(s), layout="nk", bias=dev(b), gate=gate)
    torch.cuda.synchronize()
    assert bitwise_equal(got.cpu().numpy(), expect.cpu().numpy()) == 0
    _bound_check(orc, y.cpu().numpy(), x, q.view(np.int8).astype(np.float32), s, b, "none", torch.float32, K)


@pytest.mark.parametrize("m", [5, 16])
def test_short_m_long_k_tile_choice(gemm, orc, tile_gemm, m):
    """Up to 16 rows the product keeps the short-M kernel while its activation fits the kernel's LDS (M = 5 at
    K = 6144) and takes a K-group tile where it would not (M = 16: 16 rows of 6144 bf16 exceed 100 KB): the
    default product equals the forced kernel's bits, judged against the truth."""
    k, n = 6144, 1024
    x = orc.normal_bf16(70 + m, (m, k))
    q = orc.uniform_i8(71 + m, (n, k)).view(np.uint8)
    s = orc.uniform_f32(72 + m, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(73 + m, (n,), 0.0, 0.02)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    ys = {}
    for name, g in (("default", gemm), ("gemv", tile_gemm("gemv")), ("k32x32", tile_gemm("k32x32"))):
        y = g.product(bf16_dev(x), w, dev(s), bias=dev(b), epilogue="gelu_tanh", out_dtype=torch.float32)
        torch.cuda.synchronize()
        ys[name] = y.cpu().numpy()
    assert bitwise_equal(ys["default"], ys["gemv" if m == 5 else "k32x32"]) == 0
    _bound_check(orc, ys["default"], x, q.view(np.int8).astype(np.float32), s, b, "gelu", torch.float32, k)


@pytest.mark.parametrize("m,n,kernel", [(1, 6144, "gemv"), (16, 6144, "gemv"), (1, 9216, "gemv"), (1, 12288, "gemv"),
                                        (8, 9216, "s32"), (16, 12288, "s32")])
def test_wide_short_m_tile_choice(gemm, orc, tile_gemm, m, n, kernel):
    """Past one round of 16-column groups the product keeps the short-M kernel with two groups a workgroup up to
    N = 8192, and with three for a single row up to N = 12288; more rows there take the skinny kernel. The default
    product equals the expected kernel's bits, judged against the truth."""
    x = orc.normal_bf16(80 + m, (m, K))
    q = orc.uniform_i8(81 + m, (n, K)).view(np.uint8)
    s = orc.uniform_f32(82 + m, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(83 + m, (n,), 0.0, 0.02)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    ys = {}
    for name, g in (("default", gemm), (kernel, tile_gemm(kernel))):
        y = g.product(bf16_dev(x), w, dev(s), bias=dev(b), epilogue="gelu_tanh", out_dtype=torch.float32)
        torch.cuda.synchronize()
        ys[name] = y.cpu().numpy()
    assert bitwise_equal(ys["default"], ys[kernel]) == 0
    _bound_check(orc, ys["default"], x, q.view(np.int8).astype(np.float32), s, b, "gelu", torch.float32, K)
