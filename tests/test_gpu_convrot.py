"""ComfyUI's int8 convrot on the MI355X, through the C ABI, against the CPU oracle.

The activation's rotation (rotate_groups, Sources/Siliconed/TensorGEMM.swift:181-201) and the
rotated weight's widening (Widen.dequantizeRotated, Widen.swift:374-428) are compared bit for bit:
both are fixed sequences of fp32 (or exact integer) operations. The product of a rotated weight is
judged as the reference judges it (CapacityProbes.swift:536-553): against the fp64 truth of the
rotated, rounded operand — here the oracle's, bit-identical to the GPU's — with the bars of the
plain products, and it must equal the plain product on that operand bit for bit. Its agreement with
the widened route (x · Float(H·q)·s/√G) is checked at the bar of a half-precision route.
"""
import math

import numpy as np
import pytest
import torch

from refgen import bitwise_equal
from test_gpu_parity import DEV, EPI, bf16_dev, dev, judge

pytestmark = pytest.mark.gpu

H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)


def hadamard(g):
    h = np.ones((1, 1))
    while h.shape[0] < g:
        h = np.kron(h, H4)
    return h


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()


# ---- the activation's rotation ------------------------------------------------------------------

ROT_CASES = [  # (rows, k, group): whole chunks, partial last chunks, a row of one group, many rows
    (5, 768, 256), (130, 3072, 256), (1, 256, 256), (3, 64 * 7, 64), (9, 16 * 13, 16), (4, 20, 4),
    (257, 1024, 64), (33, 4 * 67, 4),
]


@pytest.mark.parametrize("rows,k,g", ROT_CASES)
def test_rotation_is_the_oracles_at_the_bit(gemm, orc, rows, k, g):
    # fp32 → fp32 and fp32 → bf16 (the product's operand: rotate, then round to nearest even).
    x = orc.normal_f32(rows * 31 + k + g, (rows, k), 0.0, 2.0)
    x[0, :4] = [2.0 ** 24, 1.0, -(2.0 ** 24), 1.0]  # a tie inside the first butterfly
    expected = orc.rotate_groups(x, g)
    xd = dev(x)
    got32 = host(gemm.rotate(xd, g, out_dtype=torch.float32))
    assert bitwise_equal(got32, expected) == 0
    got16 = host(gemm.rotate(xd, g))
    assert np.array_equal(got16, orc.f32_to_bf16(expected))


@pytest.mark.parametrize("g", [4, 16, 64, 256])
def test_rotation_of_a_bf16_operand(gemm, orc, g):
    # bf16 in: widened exactly, rotated in fp32, rounded (or kept fp32).
    xb = orc.normal_bf16(g + 5, (17, 1280))
    expected = orc.rotate_groups(orc.bf16_to_f32(xb), g)
    got = host(gemm.rotate(bf16_dev(xb), g))
    assert np.array_equal(got, orc.f32_to_bf16(expected))
    got32 = host(gemm.rotate(bf16_dev(xb), g, out_dtype=torch.float32))
    assert bitwise_equal(got32, expected) == 0


def test_rotation_known_answers_on_the_device(gemm, orc):
    # The oracle's hand-worked cases: the tie drops the 1 in the first butterfly; span 1 runs first.
    T = 2.0 ** 24
    x = np.zeros((2, 16), np.float32)
    x[0, :4] = [T, 1, 1, 0]
    x[1, 0], x[1, 1], x[1, 4] = T, 1, 1
    got = host(gemm.rotate(dev(x), 16, out_dtype=torch.float32)).astype(np.float64)
    y1 = np.array([T, T, T, -T, T, T, T, -T, T - 1, T - 1, T - 2, -(T - 2), -(T - 1), -(T - 1), -(T - 2), T - 2]) / 4
    assert np.array_equal(got[1], y1)
    got4 = host(gemm.rotate(dev(x[:1, :4].copy()), 4, out_dtype=torch.float32)).astype(np.float64)
    assert np.array_equal(got4[0], [T / 2, (T - 1) / 2, T / 2, -(T - 2) / 2])


def test_rotation_strided_unaligned_and_in_place(gemm, orc):
    g, rows, k = 64, 7, 448
    x = orc.normal_f32(71, (rows, k + 3))
    expected = orc.rotate_groups(np.ascontiguousarray(x[:, 1:k + 1]), g)
    xd = dev(x)
    # Rows 4·(k+3) bytes apart, starting 4 bytes in: the element-wise path.
    got = host(gemm.rotate(xd[:, 1:k + 1], g, out_dtype=torch.float32))
    assert bitwise_equal(got, expected) == 0
    # Strided output rows.
    outb = torch.zeros((rows, k + 8), dtype=torch.bfloat16, device=DEV)
    gemm.rotate(xd[:, 1:k + 1], g, out=outb[:, :k])
    ob = host(outb)
    assert np.array_equal(ob[:, :k], orc.f32_to_bf16(expected)) and not ob[:, k:].any()
    # In place.
    y = dev(np.ascontiguousarray(x[:, :k]))
    gemm.rotate(y, g, out=y)
    assert bitwise_equal(host(y), orc.rotate_groups(np.ascontiguousarray(x[:, :k]), g)) == 0


def test_rotation_at_the_bench_size_is_exact_and_involutive(gemm, orc):
    # C1's operand, 4096 × 3072: the oracle's bits, and R·R = I within rounding.
    x = orc.normal_f32(4242, (4096, 3072))
    xd = dev(x)
    y = gemm.rotate(xd, 256, out_dtype=torch.float32)
    assert bitwise_equal(host(y), orc.rotate_groups(x, 256)) == 0
    back = host(gemm.rotate(y, 256, out_dtype=torch.float32))
    assert np.abs(back - x).max() <= 1e-5 * np.abs(x).max()


def test_rotation_refusals(gemm):
    from siliconed_amd import abi
    x = torch.zeros((2, 96), dtype=torch.float32, device=DEV)
    for g in (8, 32, 512, 0):
        with pytest.raises(abi.SQ8Error):
            gemm.rotate(x, g)
    with pytest.raises(abi.SQ8Error):
        gemm.rotate(x, 64)                       # 96 is no whole number of groups of 64
    gemm.rotate(torch.zeros((0, 256), device=DEV), 256)  # no rows: nothing to do


# ---- the rotated weight widened -------------------------------------------------------------------

DQ_CASES = [(256, 768, 328), (256, 256, 12), (64, 192, 136), (16, 64, 40), (4, 8, 20), (16, 32, 8200), (4, 8, 4100),
            (64, 320, 37)]


@pytest.mark.parametrize("g,k,n", DQ_CASES)
def test_dequantize_rotated_at_the_bit(gemm, orc, g, k, n):
    # DequantizeTests.swift:179-211's shapes (+ an odd width): the oracle's bits, which the CPU
    # suite pins to the fp64 Kronecker product; extremes of m in columns 0 and 1; bf16, fp32 and
    # fp16 scales per column and one fp32 scale for the tensor.
    rng = np.random.default_rng(g + k + n)
    q = rng.integers(-128, 128, (k, n)).astype(np.int8)
    h = hadamard(g)
    q[:g, 0] = np.where(h[0] > 0, 127, -128)
    q[:g, 1] = np.where(h[0] > 0, -128, 127)
    qd = dev(q)
    s = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    sb = orc.f32_to_bf16(s)
    sh = s.astype(np.float16)
    for scale_t, arr, stype, layout in ((bf16_dev(sb), sb, orc.BF16, orc.SCALE_COLUMNS),
                                        (dev(s), s, orc.F32, orc.SCALE_COLUMNS),
                                        (dev(sh), sh.view(np.uint16), orc.F16, orc.SCALE_COLUMNS),
                                        (dev(s[:1]), s[:1], orc.F32, orc.SCALE_TENSOR)):
        got = host(gemm.dequantize_rotated(qd, g, scale_t))
        expected = orc.dequantize_rotated(q, g, arr, stype, layout)
        assert bitwise_equal(got, expected) == 0, (stype, layout)


@pytest.mark.parametrize("g,k,n,lo,hi", [(256, 512, 328, 64, 328), (16, 64, 8200, 4096, 8200), (4, 8, 4100, 0, 12),
                                         (64, 192, 136, 64, 128)])
def test_dequantize_rotated_slice_is_the_wholes_columns(gemm, orc, g, k, n, lo, hi):
    # DequantizeTests.swift:216-238: a slice of columns (codes + lo, scales + lo, width hi − lo) is
    # those columns of the whole widening, nothing written past [k, width].
    rng = np.random.default_rng(n + lo)
    q = rng.integers(-128, 128, (k, n)).astype(np.int8)
    s = orc.f32_to_bf16(rng.uniform(1e-3, 2e-2, n).astype(np.float32))
    qd, sd = dev(q), bf16_dev(s)
    whole = host(gemm.dequantize_rotated(qd, g, sd))
    part = host(gemm.dequantize_rotated(qd[:, lo:hi], g, sd[lo:hi]))
    assert part.shape == (k, hi - lo)
    assert bitwise_equal(part, whole[:, lo:hi]) == 0


# ---- the product of a rotated weight --------------------------------------------------------------

PRODUCT_CASES = [  # (m, k, n, layout, epilogue, a fp32?, out dtype)
    (256, 3072, 1024, "packed", "none", True, torch.bfloat16),
    (300, 1024, 768, "nk", "gelu", False, torch.bfloat16),
    (64, 768, 512, "kn", "none", True, torch.float32),
    (16, 1024, 384, "nk", "none", False, torch.float32),   # fp32 judged on ≥ 16 rows: a column's error is a statistic
    (1, 2048, 256, "packed", "none", False, torch.bfloat16),  # one row: no GELU, whose saturated zeros
                                                               # leave a one-row column no error floor
    (600, 512, 640, "packed", "silu", True, torch.bfloat16),
    (37, 256, 200, "kn", "situ", False, torch.float32),
]


@pytest.mark.parametrize("m,k,n,layout,epi,a32,out_dtype", PRODUCT_CASES)
def test_rotated_product(gemm, orc, m, k, n, layout, epi, a32, out_dtype):
    g = 256 if k % 256 == 0 else 64
    seed = m * 7 + k + n
    x = orc.normal_f32(seed, (m, k))
    q = orc.uniform_i8(seed + 1, (n, k))                    # [N, K] codes, the weight W = (q·s)·R
    s = orc.uniform_f32(seed + 2, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(seed + 3, (n,), 0.0, 0.02)
    xr = orc.f32_to_bf16(orc.rotate_groups(x if a32 else orc.bf16_to_f32(orc.f32_to_bf16(x)), g))
    epilogue = None if epi == "none" else {"gelu": "gelu_tanh", "silu": "silu_glu", "situ": "situ_glu"}[epi]
    wq = dev(q).view(torch.int8)
    if layout == "packed":
        w, lay = gemm.pack(wq, layout="nk", glu=epi in ("silu", "situ")), "nk"
    elif layout == "kn":
        w, lay = dev(np.ascontiguousarray(q.T)).view(torch.int8), "kn"
    else:
        w, lay = wq, "nk"
    a = dev(x) if a32 else bf16_dev(orc.f32_to_bf16(x))
    got_t = gemm.product(a, w, dev(s), layout=lay, bias=dev(b), epilogue=epilogue, out_dtype=out_dtype, rotation=g)
    got = got_t.float().cpu().numpy()
    # The same kernel on the oracle's rotated operand: the same bits.
    plain = gemm.product(bf16_dev(xr), w, dev(s), layout=lay, bias=dev(b), epilogue=epilogue, out_dtype=out_dtype)
    assert bitwise_equal(got, plain.float().cpu().numpy()) == 0
    judge(orc, got, xr, q.view(np.uint8), False, s, b, epi, out_dtype, rows=orc.sample_rows(m, min(m, 64)))


def test_rotated_product_matches_the_widened_route(gemm, orc):
    # x · W with W = Float(H·q)·(s/√G) widened (the reference's CPU route), judged at a
    # half-precision route's bar, 1.25 × bf16's own error on the product (Diagnostic.swift:105-107):
    # the rotated operand's bf16 rounding is this route's error (≈ 1.0 × that floor here).
    m, k, n, g = 128, 1024, 512, 256
    x = orc.normal_bf16(11, (m, k))
    q_kn = orc.uniform_i8(12, (k, n))
    s = orc.uniform_f32(13, (n,), 1e-3, 2e-2)
    w_kn = orc.dequantize_rotated(q_kn, g, s)
    rows = orc.sample_rows(m, 64)
    exact = orc.exact_rows(rows, x, w_kn, True, k, n)
    got = gemm.product(bf16_dev(x), dev(q_kn).view(torch.int8), dev(s), layout="kn", out_dtype=torch.float32,
                       rotation=g).cpu().numpy()[rows]
    err = orc.channel_error(got, exact)[0]
    floor = orc.channel_error(orc.bf16_to_f32(orc.f32_to_bf16(exact.astype(np.float32))), exact)[0]
    assert err <= 1.25 * floor, (err, floor)


def test_linear_mirror_takes_the_rotation(gemm, orc):
    # TensorGEMM.linear(…rotation:…rounding:…) with the reference's (group, scratch, offset, chunk) and
    # (buffer, offset, rows) tuples: the rotated activation rounded to bf16, then the product.
    m, k, n = 70, 512, 96
    x = orc.normal_f32(21, (m, k))
    q_kn = orc.uniform_i8(22, (k, n))
    s = orc.uniform_f32(23, (n,), 1e-3, 2e-2)
    c = torch.empty((m, n), dtype=torch.float32, device=DEV)
    secs = gemm.linear(dev(x), int8=dev(q_kn).view(torch.int8), scales=dev(s), per_column=True, c=c, m=m, k=k, n=n,
                       rotation=(256, None, 0, 64), rounding=(None, 0, 64))
    assert secs > 0
    xr = orc.f32_to_bf16(orc.rotate_groups(x, 256))
    plain = gemm.product(bf16_dev(xr), dev(q_kn).view(torch.int8), dev(s), layout="kn", out_dtype=torch.float32)
    assert bitwise_equal(c.cpu().numpy(), plain.cpu().numpy()) == 0
