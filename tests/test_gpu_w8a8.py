"""W8A8 (ComfyUI's int8_linear) on the MI355X, through the C ABI, against the CPU oracle — bit for bit.

Every step of the route is a single rounding the oracle makes the same (the rotation's fp32 sums in
the reference's order, the correctly rounded divisions, rint half to even, int32 sums that are
exact, float(acc) · (s_x · s_w)), so codes, scales and outputs are compared for equality, as
W8A8KernelTests.swift:4-10 compares the reference's GPU with its CPU recipe. The cases follow that
file (:74-83, :164-168): rows in several tiles with a remainder, a row of 40 chunks of 256, a group
of 64 with one scale for the tensor, no rotation on a k that is no whole chunk, a row of zeros
(scale floor 1e-30), a massive column.
"""
import numpy as np
import pytest
import torch

from refgen import bitwise_equal
from test_gpu_parity import DEV, bf16_dev, dev

pytestmark = pytest.mark.gpu

EPIS = {"none": None, "gelu": "gelu_tanh", "silu": "silu_glu", "situ": "situ_glu"}


def inputs(orc, m, k, seed, zero_row=3, massive=True):
    x = orc.normal_f32(seed, (m, k), 0.0, 3.0)
    if zero_row is not None and zero_row < m:
        x[zero_row] = 0
    if massive:
        x[:, k // 3] *= 300
    return x


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


QUANT_CASES = [(150, 768, 256), (70, 10240, 0), (65, 448, 64), (33, 520, 0), (19, 520, 0), (8, 32768, 256),
               (300, 3072, 256), (5, 96, 16), (7, 20, 4), (2, 1, 0), (3, 4097, 0)]


@pytest.mark.parametrize("m,k,g", QUANT_CASES)
def test_quantize_rows_at_the_bit(gemm, orc, m, k, g):
    x = inputs(orc, m, k, m + k + g)
    codes, scales = gemm.quantize_rows(dev(x), g)
    ec, es = orc.quantize_rows(x, g)
    assert bitwise_equal(host(scales), es) == 0
    assert np.array_equal(host(codes), ec)
    if m > 3:
        assert host(scales)[3] == np.float32(1e-30) and not host(codes)[3].any()


def test_quantize_rows_known_answers(gemm, orc):
    # Ties of rint (scale exactly 1: 63.5 → 64, −0.5 → 0, 2.5 → 2, −126.5 → −126) and the quotient
    # whose reciprocal product rounds the other way (97 against the division's 96): the rows the
    # oracle's own tests work by hand, here through the kernel's exact-division branch.
    x = np.zeros((2, 8), np.float32)
    x[0] = [127.0, 63.5, -0.5, 1.5, 2.5, 0.0, -126.5, 3.49]
    x[1, :3] = [2.166764259338379, 1.646399736404419, -1.646399736404419]
    codes, scales = gemm.quantize_rows(dev(x))
    c = host(codes)
    assert c[0].tolist() == [127, 64, 0, 2, 2, 0, -126, 3] and host(scales)[0] == 1.0
    assert c[1, :3].tolist() == [127, 96, -96]


def test_quantize_rows_of_a_bf16_operand(gemm, orc):
    xb = orc.normal_bf16(77, (40, 3072))
    codes, scales = gemm.quantize_rows(bf16_dev(xb), 256)
    ec, es = orc.quantize_rows(orc.bf16_to_f32(xb), 256)
    assert np.array_equal(host(codes), ec) and bitwise_equal(host(scales), es) == 0


def test_quantize_rows_refusals(gemm):
    from siliconed_amd import abi
    x = torch.zeros((2, 96), device=DEV)
    with pytest.raises(abi.SQ8Error):
        gemm.quantize_rows(x, 64)             # 96 is no whole number of groups of 64
    with pytest.raises(abi.SQ8Error):
        gemm.quantize_rows(x, 8)
    with pytest.raises(abi.Unsupported):
        gemm.quantize_rows(torch.zeros((1, 32772), device=DEV))   # longer than a row the pass holds


PRODUCT_CASES = [  # (m, k, n, group, per-column scale, layout)
    (150, 768, 96, 256, True, "packed"),
    (70, 10240, 72, 0, True, "nk"),
    (65, 448, 130, 64, False, "kn"),
    (33, 520, 40, 0, True, "packed"),
    (256, 3072, 1024, 256, True, "packed"),
    (129, 1024, 384, 16, True, "nk"),
    (1, 256, 64, 256, True, "kn"),
]


def _weight(gemm, q_nk, layout, glu=False):
    if layout == "packed":
        return gemm.pack(dev(q_nk).view(torch.int8), layout="nk", glu=glu), "nk"
    if layout == "kn":
        return dev(np.ascontiguousarray(q_nk.T)).view(torch.int8), "kn"
    return dev(q_nk).view(torch.int8), "nk"


@pytest.mark.parametrize("m,k,n,g,per_col,layout", PRODUCT_CASES)
def test_w8a8_product_at_the_bit(gemm, orc, m, k, n, g, per_col, layout):
    seed = m * 3 + k + n
    x = inputs(orc, m, k, seed)
    q = orc.uniform_i8(seed + 1, (n, k))                          # the weight's codes [N, K]
    sw = orc.uniform_f32(seed + 2, (n if per_col else 1,), 1e-3, 2e-2)
    b = orc.normal_f32(seed + 3, (n,), 0.0, 0.02)
    codes, sx = orc.quantize_rows(x, g)
    expected = orc.w8a8_product(codes, sx, q, False, sw)
    w, lay = _weight(gemm, q, layout)
    # The whole route (quantized here) and the product on the oracle's codes: the same bits.
    got = host(gemm.product_quantized(dev(x), w, dev(sw), group=g, layout=lay, out_dtype=torch.float32))
    assert bitwise_equal(got, expected) == 0
    got_pre = host(gemm.product_w8a8(dev(codes), dev(sx), w, dev(sw), layout=lay, out_dtype=torch.float32))
    assert bitwise_equal(got_pre, expected) == 0
    # Bias after the scale (one rounding), bf16 out: the fp32 value rounded to nearest even.
    with_b = host(gemm.product_quantized(dev(x), w, dev(sw), group=g, layout=lay, bias=dev(b), out_dtype=torch.float32))
    assert bitwise_equal(with_b, expected + b[None, :]) == 0
    out16 = gemm.product_quantized(dev(x), w, dev(sw), group=g, layout=lay, bias=dev(b))
    torch.cuda.synchronize()
    assert np.array_equal(out16.cpu().view(torch.int16).numpy().view(np.uint16), orc.f32_to_bf16(expected + b[None, :]))


def test_w8a8_on_strided_and_unaligned_codes(gemm, orc):
    # Codes whose rows are not whole 128-code steps, or not 16-byte aligned: copied into padded
    # rows first, the same bits.
    m, k, n = 40, 200, 96
    x = inputs(orc, m, k, 5)
    q = orc.uniform_i8(6, (n, k))
    sw = orc.uniform_f32(7, (n,), 1e-3, 2e-2)
    codes, sx = orc.quantize_rows(x)
    expected = orc.w8a8_product(codes, sx, q, False, sw)
    big = np.zeros((m, k + 9), np.int8)
    big[:, 1:k + 1] = codes
    cd = dev(big)[:, 1:k + 1]
    got = host(gemm.product_w8a8(cd, dev(sx), dev(q).view(torch.int8), dev(sw), out_dtype=torch.float32))
    assert bitwise_equal(got, expected) == 0


@pytest.mark.parametrize("epi", ["gelu", "silu", "situ"])
def test_w8a8_epilogues(gemm, orc, epi):
    # The activation on the bit-exact scaled sum + bias: the same device functions as the bf16
    # route, compared with torch's on the oracle's fp32 value (fp32 out).
    m, k, n = 96, 1024, 256
    x = inputs(orc, m, k, 31)
    q = orc.uniform_i8(32, (n, k))
    sw = orc.uniform_f32(33, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(34, (n,), 0.0, 0.02)
    codes, sx = orc.quantize_rows(x, 256)
    pre = torch.from_numpy(orc.w8a8_product(codes, sx, q, False, sw) + b[None, :]).double()
    glu = epi != "gelu"
    w, lay = _weight(gemm, q, "packed", glu=glu)
    got = host(gemm.product_quantized(dev(x), w, dev(sw), group=256, layout=lay, bias=dev(b), epilogue=EPIS[epi],
                                      out_dtype=torch.float32))
    if epi == "gelu":
        ref = torch.nn.functional.gelu(pre, approximate="tanh")
    else:
        h = n // 2
        a_, g_ = pre[:, :h], pre[:, h:]
        if epi == "silu":
            ref = torch.nn.functional.silu(a_) * g_
        else:                       # value first, gate second: 4·tanh(g/4)·σ(g) · 25·tanh(v/25)
            ref = 4 * torch.tanh(g_ / 4) * torch.sigmoid(g_) * 25 * torch.tanh(a_ / 25)
    ref = ref.numpy()
    scale = np.sqrt((ref ** 2).mean(axis=0)) + 1e-30
    assert (np.abs(got - ref) / np.maximum(np.abs(ref), 0.01 * scale)).max() < 1e-4


def test_w8a8_at_the_bench_size(gemm, orc):
    # C1's shape, 4096 × 3072 × 12288, rotated by 256: every code and scale, and 64 sampled rows of
    # the product, bit for bit.
    m, k, n = 4096, 3072, 12288
    x = orc.normal_f32(8, (m, k))
    q = orc.uniform_i8(9, (n, k))
    sw = orc.uniform_f32(10, (n,), 1e-3, 2e-2)
    codes, sx = orc.quantize_rows(x, 256)
    w, lay = _weight(gemm, q, "packed")
    xd = dev(x)
    gc, gs = gemm.quantize_rows(xd, 256)
    assert np.array_equal(host(gc), codes) and bitwise_equal(host(gs), sx) == 0
    got = host(gemm.product_quantized(xd, w, dev(sw), group=256, layout=lay, out_dtype=torch.float32))
    rows = orc.sample_rows(m, 64)
    expected = orc.w8a8_product(codes[rows], sx[rows], q, False, sw)
    assert bitwise_equal(got[rows], expected) == 0


def test_linear_mirror_quantizing(gemm, orc):
    # TensorGEMM.linear(…quantizing:…) and (…prequantized:…) with the reference's argument names.
    m, k, n = 70, 512, 96
    x = inputs(orc, m, k, 41)
    q_kn = orc.uniform_i8(42, (k, n))
    sw = orc.uniform_f32(43, (n,), 1e-3, 2e-2)
    codes, sx = orc.quantize_rows(x, 256)
    expected = orc.w8a8_product(codes, sx, q_kn, True, sw)
    c = torch.empty((m, n), dtype=torch.float32, device=DEV)
    secs = gemm.linear(dev(x), int8=dev(q_kn).view(torch.int8), scales=dev(sw), per_column=True, c=c, m=m, k=k, n=n,
                       rotation=(256, None, 0, 64), quantizing=(None, 0, 0, 64))
    assert secs > 0 and bitwise_equal(host(c), expected) == 0
    c2 = torch.empty_like(c)
    gemm.linear(dev(x), int8=dev(q_kn).view(torch.int8), scales=dev(sw), per_column=True, c=c2, m=m, k=k, n=n,
                prequantized=(dev(codes), dev(sx)))
    assert bitwise_equal(host(c2), expected) == 0


# ---- the operand written by its producer (WeightProducts.swift:130-229, ElementwiseGPUMoss.swift:94-130) ----

def _norm_inputs(orc, rows, cols, seed):
    x = orc.normal_f32(seed, (rows, cols), 0.0, 2.0)
    w = (1.0 + 0.05 * orc.normal_f32(seed + 1, (cols,))).astype(np.float32)
    sc = (0.1 * orc.normal_f32(seed + 2, (cols,))).astype(np.float32)
    sh = (0.1 * orc.normal_f32(seed + 3, (cols,))).astype(np.float32)
    return x, w, sc, sh


@pytest.mark.parametrize("rows,cols,g", [(300, 3072, 256), (5, 1024, 0), (33, 5120, 64), (7, 12288, 256), (3, 20480, 16)])
def test_norm_writes_the_w8a8_operand(gemm, orc, rows, cols, g):
    # y is the fp32 row of sq8_norm_modulate (its bf16 rounding equals that pass's output, bit for bit);
    # the codes and scales are sq8_quantize_rows's on y (the oracle's, bit for bit); without y_out the same.
    x, w, sc, sh = _norm_inputs(orc, rows, cols, rows + cols + g)
    xd, wd, scd, shd = dev(x), dev(w), dev(sc), dev(sh)
    y = torch.empty((rows, cols), dtype=torch.float32, device=DEV)
    codes, scales = gemm.norm_modulate_quantized(xd, wd, scd, shd, 1e-6, g, y_out=y)
    yh = host(y)
    plain = gemm.norm_modulate(xd, wd, scd, shd, 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(plain.cpu().view(torch.int16).numpy().view(np.uint16), orc.f32_to_bf16(yh))
    ec, es = orc.quantize_rows(yh, g)
    assert np.array_equal(host(codes), ec) and bitwise_equal(host(scales), es) == 0
    c2, s2 = gemm.norm_modulate_quantized(xd, wd, scd, shd, 1e-6, g)
    assert np.array_equal(host(c2), ec) and bitwise_equal(host(s2), es) == 0


@pytest.mark.parametrize("rows,cols,g", [(300, 3072, 256), (9, 1024, 16), (4, 12288, 64)])
def test_norm_writes_the_convrot_operand(gemm, orc, rows, cols, g):
    # The rotated, rounded operand is the rotation pass's on y (the oracle's rotation, bit for bit).
    x, w, sc, sh = _norm_inputs(orc, rows, cols, rows * 7 + g)
    y = torch.empty((rows, cols), dtype=torch.float32, device=DEV)
    out = gemm.norm_modulate_rotated(dev(x), dev(w), dev(sc), dev(sh), 1e-6, g, y_out=y)
    torch.cuda.synchronize()
    got = out.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, orc.f32_to_bf16(orc.rotate_groups(host(y), g)))
    out2 = gemm.norm_modulate_rotated(dev(x), dev(w), dev(sc), dev(sh), 1e-6, g)
    torch.cuda.synchronize()
    assert np.array_equal(out2.cpu().view(torch.int16).numpy().view(np.uint16), got)


def test_norm_operand_refusals(gemm, orc):
    from siliconed_amd import abi
    x, w, sc, sh = (dev(a) for a in _norm_inputs(orc, 2, 96, 1))
    with pytest.raises(abi.SQ8Error):
        gemm.norm_modulate_quantized(x, w, sc, sh, 1e-6, 64)        # 96 is no whole number of groups of 64
    with pytest.raises(abi.SQ8Error):
        gemm.norm_modulate_rotated(x, w, sc, sh, 1e-6, 0)           # a rotation needs a group
    xs = torch.zeros((2, 98), device=DEV)
    with pytest.raises(abi.Unsupported):
        gemm.norm_modulate_quantized(xs, xs[0].contiguous(), xs[0].contiguous(), xs[0].contiguous(), 1e-6)  # cols % 4


@pytest.mark.parametrize("head_dim", [0, 128])
def test_w8a8_qkv_is_the_split_product(gemm, orc, head_dim):
    m, k, d = 300, 1024, 512
    x = inputs(orc, m, k, 61)
    q = orc.uniform_i8(62, (3 * d, k))
    sw = orc.uniform_f32(63, (3 * d,), 1e-3, 2e-2)
    b = orc.normal_f32(64, (3 * d,), 0.0, 0.02)
    codes, sx = orc.quantize_rows(x, 256)
    w = gemm.pack(dev(q).view(torch.int8), layout="nk")
    full = host(gemm.product_w8a8(dev(codes), dev(sx), w, dev(sw), bias=dev(b)).float())
    outs = gemm.product_w8a8_qkv(dev(codes), dev(sx), w, dev(sw), bias=dev(b), head_dim=head_dim)
    for i, t in enumerate(outs):
        part = host(t.float())
        if head_dim:
            part = part.transpose(1, 0, 2).reshape(m, d)
        assert np.array_equal(part, full[:, i * d:(i + 1) * d]), i


def test_w8a8_residual_product_is_product_then_residual(gemm, orc):
    m, k, n = 300, 1024, 768
    x = inputs(orc, m, k, 71)
    q = orc.uniform_i8(72, (n, k))
    sw = orc.uniform_f32(73, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(74, (n,), 0.0, 0.02)
    stream = orc.normal_f32(75, (m, n))
    gate = dev(orc.normal_f32(76, (n,), 0.0, 0.5))
    codes, sx = orc.quantize_rows(x, 256)
    w = gemm.pack(dev(q).view(torch.int8), layout="nk")
    y = dev(orc.w8a8_product(codes, sx, q, False, sw) + b[None, :])
    expect = dev(stream)
    gemm.gated_residual(expect, y, gate)
    got = dev(stream)
    gemm.product_w8a8_residual(got, dev(codes), dev(sx), w, dev(sw), bias=dev(b), gate=gate)
    assert bitwise_equal(host(got), host(expect)) == 0
