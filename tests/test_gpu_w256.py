"""The 256 × 256 kernel (one workgroup per CU) in 256- and 224-row tiles, its slab and block epilogues, on
an MI355X.

Every output of the weight-direct kernels is one MFMA sequence over K whatever the tile, and the slab
epilogue applies the same scale, bias and activation as the 32 × 32-block one: so the 256- and 224-row
tiles give the same bits as the 128-row tiles, and they are judged against the oracle's fp64 truth on
sampled rows at the reference's bars (DiagnosticProbes.swift:75-82, DiagnosticJudgement.swift:39-71).
Shapes cover a ragged last row tile, a last column tile with fewer slabs than waves, per-tensor scales,
no bias, fp8 codes, both weight layouts, the QKV split (row-major and head-major), the GLU epilogues,
fp32 outputs and the gated residual.
"""
import numpy as np
import pytest
import torch

from refgen import bitwise_equal
from test_gpu_parity import DEV, bf16_dev, dev, judge, problem, weight_tensor

pytestmark = pytest.mark.gpu


def product(tile_gemm, tile, x, w, s, b, layout, epi, out_dtype=torch.bfloat16):
    y = tile_gemm(tile).product(bf16_dev(x), w, dev(s), layout=layout, bias=None if b is None else dev(b),
                                epilogue="gelu_tanh" if epi == "gelu" else None, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


@pytest.mark.parametrize("m,k,n,fp8,layout,epi,bias,tensor_scale", [
    (1000, 512, 1344, False, "packed", "gelu", True, False),   # ragged rows; last column tile: 1 slab of 4
    (512, 1024, 1024, False, "nk", "none", False, False),       # [N, K] codes read in place, no bias
    (777, 768, 640, True, "packed", "none", True, False),       # fp8, ragged rows, 2 + 2 + 2... slabs
    (256, 2048, 768, True, "nk", "gelu", True, True),           # fp8 in place, one scale for the tensor
    (1, 512, 512, False, "packed", "gelu", True, False),        # one row
    # K steps not a multiple of four (the loop's leftover steps: 5, 7 and 9 steps leave 1, 3 and 1; 6 leaves
    # 2), at full row tiles and several column tiles, for both tile heights.
    (768, 320, 1024, False, "packed", "gelu", True, False),
    (600, 448, 1280, False, "nk", "none", True, False),
    (1024, 576, 768, True, "packed", "gelu", True, False),
    (512, 384, 1024, False, "packed", "none", True, False),
])
def test_w256_same_bits_as_128(gemm, orc, tile_gemm, m, k, n, fp8, layout, epi, bias, tensor_scale):
    x, q, s, b = problem(orc, m, k, n, fp8, 400 + m + n, bias=bias)
    if tensor_scale:
        s = np.array([float(np.median(s))], dtype=np.float32)
    w = weight_tensor(q, fp8, "nk")
    if layout == "packed":
        w = gemm.pack(w, layout="nk")
    y256 = product(tile_gemm, "256", x, w, s, b, "nk", epi)
    y224 = product(tile_gemm, "224", x, w, s, b, "nk", epi)
    y128 = product(tile_gemm, "128", x, w, s, b, "nk", epi)
    assert bitwise_equal(y256, y128) == 0
    assert bitwise_equal(y224, y128) == 0
    sj = np.full(n, s[0], dtype=np.float32) if tensor_scale else s
    judge(orc, y256, x, q, fp8, sj, b, epi, torch.bfloat16, rows=orc.sample_rows(m, 64))


def test_w256_fp32_output(gemm, orc, tile_gemm):
    """fp32 outputs on 256-row tiles (32 × 32 blocks through the epilogue regions): the same bits as the
    128-row tiles."""
    m, k, n = 600, 512, 768
    x, q, s, b = problem(orc, m, k, n, False, 91)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    y256 = product(tile_gemm, "256", x, w, s, b, "nk", "gelu", out_dtype=torch.float32)
    y224 = product(tile_gemm, "224", x, w, s, b, "nk", "gelu", out_dtype=torch.float32)
    y128 = product(tile_gemm, "128", x, w, s, b, "nk", "gelu", out_dtype=torch.float32)
    assert bitwise_equal(y256, y128) == 0
    assert bitwise_equal(y224, y128) == 0
    judge(orc, y256, x, q, False, s, b, "gelu", torch.float32, rows=orc.sample_rows(m, 64))


@pytest.mark.parametrize("head_dim", [0, 128, 64])
def test_w256_qkv(gemm, orc, tile_gemm, head_dim):
    """The fused QKV product on 256-row tiles: each 64-column slab lies in one output and one head, its
    rows stored row-major or head-major; the same bits as the 128-row tiles, each third judged."""
    m, k, d = 700, 512, 384
    x, q, s, b = problem(orc, m, k, 3 * d, False, 77 + head_dim)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    outs = {}
    for tile in ("256", "224", "128"):
        qq, kk, vv = tile_gemm(tile).product_qkv(bf16_dev(x), w, dev(s), bias=dev(b), head_dim=head_dim)
        torch.cuda.synchronize()
        parts = []
        for t in (qq, kk, vv):
            t = t.float()
            if head_dim:
                t = t.permute(1, 0, 2).reshape(m, d)  # [heads, m, hd] → [m, d]
            parts.append(t.cpu().numpy())
        outs[tile] = np.concatenate(parts, axis=1)
    assert bitwise_equal(outs["256"], outs["128"]) == 0
    assert bitwise_equal(outs["224"], outs["128"]) == 0
    judge(orc, outs["256"], x, q, False, s, b, "none", torch.bfloat16, rows=orc.sample_rows(m, 64))


def test_slab_epilogue_same_bits_as_block_epilogue(gemm, orc):
    """The slab epilogue (16-byte aligned bf16 rows) against the 32 × 32-block epilogue (the same product
    into rows whose stride is not a multiple of 8 bf16, which the slab epilogue does not take)."""
    m, k, n = 900, 1024, 1536
    x, q, s, b = problem(orc, m, k, n, False, 55)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    lean = gemm.product(bf16_dev(x), w, dev(s), bias=dev(b), epilogue="gelu_tanh")
    wide = torch.empty((m, n + 4), dtype=torch.bfloat16, device=DEV)
    block = gemm.product(bf16_dev(x), w, dev(s), bias=dev(b), epilogue="gelu_tanh", out=wide[:, :n])
    torch.cuda.synchronize()
    assert bitwise_equal(lean.float().cpu().numpy(), block.float().cpu().numpy()) == 0
    judge(orc, lean.float().cpu().numpy(), x, q, False, s, b, "gelu", torch.bfloat16, rows=orc.sample_rows(m, 64))


@pytest.mark.parametrize("blocks", [False, True], ids=["per_column", "q8_0"])
def test_strided_fp32_operand_rounded_in_one_pass(gemm, orc, blocks):
    """An fp32 A whose rows are further apart than k (lda > k) is rounded to bf16 by one strided pass: the
    product equals the product on the same rows made contiguous, bit for bit (per-column and Q8_0 scales)."""
    m, k, n = 300, 512, 640
    wide = orc.normal_f32(61, (m, k + 40))
    x = wide[:, :k]
    q = orc.uniform_i8(62, (n, k)).view(np.uint8)
    if blocks:
        d = orc.uniform_f32(63, (n, k // 32), 1e-3, 2e-2).astype(np.float16)
        w = weight_tensor(q, False, "nk")
        strided = gemm.product_blocks(dev(wide)[:, :k], w, dev(d), 32, layout="nk")
        packed = gemm.product_blocks(dev(np.ascontiguousarray(x)), w, dev(d), 32, layout="nk")
    else:
        s = orc.uniform_f32(63, (n,), 1e-3, 2e-2)
        w = weight_tensor(q, False, "nk")
        strided = gemm.product(dev(wide)[:, :k], w, dev(s), layout="nk")
        packed = gemm.product(dev(np.ascontiguousarray(x)), w, dev(s), layout="nk")
    torch.cuda.synchronize()
    assert bitwise_equal(strided.float().cpu().numpy(), packed.float().cpu().numpy()) == 0


def test_w256_on_the_fp32_route(gemm, orc, tile_gemm):
    """The fp32 route (an fp32 activation used whole: three exact bf16 parts along K, each facing the whole
    weight) on 256-row tiles, bf16 out: the same bits as the 128-row tiles, judged against the fp64 truth
    of the fp32 activation."""
    m, k, n = 520, 1024, 768
    x = orc.normal_f32(81, (m, k))
    q = orc.uniform_i8(82, (n, k)).view(np.uint8)
    s = orc.uniform_f32(83, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(84, (n,), 0.0, 0.02)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    outs = {}
    for tile in ("256", "224", "128"):
        y = tile_gemm(tile).product(dev(x), w, dev(s), bias=dev(b), epilogue="gelu_tanh", rounding=False)
        torch.cuda.synchronize()
        outs[tile] = y.float().cpu().numpy()
    assert bitwise_equal(outs["256"], outs["128"]) == 0
    assert bitwise_equal(outs["224"], outs["128"]) == 0
    judge(orc, outs["256"], x, q, False, s, b, "gelu", torch.bfloat16, rows=orc.sample_rows(m, 64))


@pytest.mark.parametrize("epi,h,fp8,layout", [("silu", 640, False, "packed"), ("situ", 160, True, "nk"),
                                              ("silu", 2048, True, "packed")])
def test_w256_glu(gemm, orc, tile_gemm, epi, h, fp8, layout):
    """The GLU epilogues on 256-row tiles (a slab: 32 columns of each half), bf16 and fp32 out: the same bits
    as the 128-row tiles, judged against the fp64 truth. h = 160: five slabs, the last tile one slab."""
    m, k = 600, 768
    x, q, s, b = problem(orc, m, k, 2 * h, fp8, 500 + h)
    w = weight_tensor(q, fp8, "nk")
    if layout == "packed":
        w = gemm.pack(w, layout="nk", glu=True)
    name = {"silu": "silu_glu", "situ": "situ_glu"}[epi]
    for out in (torch.bfloat16, torch.float32):
        ys = {}
        for tile in ("256", "224", "128"):
            y = tile_gemm(tile).product(bf16_dev(x), w, dev(s), layout="nk", bias=dev(b), epilogue=name, out_dtype=out)
            torch.cuda.synchronize()
            ys[tile] = y.float().cpu().numpy()
        assert bitwise_equal(ys["256"], ys["128"]) == 0
        assert bitwise_equal(ys["224"], ys["128"]) == 0
        judge(orc, ys["256"], x, q, fp8, s, b, epi, out, rows=orc.sample_rows(m, 64))


@pytest.mark.parametrize("gated", [True, False])
def test_w256_residual(gemm, orc, tile_gemm, gated):
    """x += gate ⊙ (s ⊙ (A·W) + b) on 256-row tiles: the same bits as on the 128-row tiles, and as the fp32
    product followed by the gated residual pass."""
    m, k, n = 700, 1024, 768
    x_, q, s, b = problem(orc, m, k, n, False, 81 + gated)
    stream = orc.normal_f32(83, (m, n), 0.0, 1.0)
    gate = dev(orc.normal_f32(84, (n,), 0.0, 0.5)) if gated else None
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    outs = {}
    for tile in ("256", "224", "128"):
        got = dev(stream)
        tile_gemm(tile).product_residual(got, bf16_dev(x_), w, dev(s), bias=dev(b), gate=gate)
        torch.cuda.synchronize()
        outs[tile] = got.cpu().numpy()
    assert bitwise_equal(outs["256"], outs["128"]) == 0
    assert bitwise_equal(outs["224"], outs["128"]) == 0
    y = tile_gemm("256").product(bf16_dev(x_), w, dev(s), bias=dev(b), out_dtype=torch.float32)
    expect = dev(stream)
    gemm.gated_residual(expect, y, gate)
    torch.cuda.synchronize()
    assert bitwise_equal(outs["256"], expect.cpu().numpy()) == 0

