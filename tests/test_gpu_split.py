"""The skinny kernel's K split over workgroups (short M, the SQ8_SPLITS knob), on an MI355X.

A split product runs two launches: each workgroup sums its contiguous range of K steps (its four waves
in wave order) into an fp32 partial buffer of the context, and a second kernel adds the splits in split
order and runs the product's epilogue. The order is fixed, so the bits depend on the split count only:
the 32- and 64-row tiles give the same bits at one count. Every result is judged against the oracle's
fp64 truth at the reference's bars (DiagnosticProbes.swift:75-82, DiagnosticJudgement.swift:39-71), and
the split's own counterpart in the reference is DecodeKernels.swift:66-110 (fixed-order partials).
"""
import numpy as np
import pytest
import torch

from refgen import bitwise_equal, code_values
from test_gpu_parity import bf16_dev, dev, judge, problem, weight_tensor
from test_gpu_small_m import _bound_check

pytestmark = pytest.mark.gpu


def check(orc, got, x, q, fp8, s, b, epi, out_dtype, k_eff=None):
    """The reference's per-channel judgement from 31 rows; below, where a column's few exact values can
    cancel, the magnitude-normalised bound of the short-product tests."""
    if x.shape[0] >= 31:
        judge(orc, got, x, q, fp8, s, b, epi, out_dtype)
    else:
        _bound_check(orc, got, x, code_values(q, fp8), s, b, epi, out_dtype, k_eff or x.shape[1])


SHAPES = [
    (1, 3072, 3072),   # one row: C2's text stream at decode
    (17, 1024, 520),   # ragged rows and a last slab of 8 columns
    (64, 3072, 768),   # two 32-row tiles
    (100, 2048, 1000),  # four 32-row tiles, the last ragged; ragged columns
]


@pytest.mark.parametrize("splits", [2, 5, 12])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_split_same_bits_both_heights(knob_gemm, orc, shape, splits):
    m, k, n = shape
    x, q, s, b = problem(orc, m, k, n, False, 700 + m + splits)
    w = knob_gemm().pack(weight_tensor(q, False, "nk"), layout="nk")
    print(f"split product: m {m} k {k} n {n} splits {splits}", flush=True)
    for out in (torch.bfloat16, torch.float32):
        ys = {}
        for tile in ("s32", "s64"):
            y = knob_gemm(tile, splits).product(bf16_dev(x), w, dev(s), bias=dev(b), epilogue="gelu_tanh",
                                                out_dtype=out)
            torch.cuda.synchronize()
            ys[tile] = y.float().cpu().numpy()
        assert bitwise_equal(ys["s32"], ys["s64"]) == 0
        check(orc, ys["s32"], x, q, False, s, b, "gelu", out)


def test_split_count_clamped_to_k_steps(knob_gemm, orc):
    """More splits than K steps: the library takes one step per split (K = 256: four splits)."""
    m, k, n = 9, 256, 384
    x, q, s, b = problem(orc, m, k, n, True, 51)
    w = weight_tensor(q, True, "nk")
    y4 = knob_gemm("s32", 4).product(bf16_dev(x), w, dev(s), layout="nk", bias=dev(b))
    y99 = knob_gemm("s32", 99).product(bf16_dev(x), w, dev(s), layout="nk", bias=dev(b))
    torch.cuda.synchronize()
    assert bitwise_equal(y4.float().cpu().numpy(), y99.float().cpu().numpy()) == 0
    check(orc, y99.float().cpu().numpy(), x, q, True, s, b, "none", torch.bfloat16)


@pytest.mark.parametrize("epi", ["silu", "situ"])
def test_split_glu(knob_gemm, orc, epi):
    """The GLU epilogues on split sums: each workgroup's slab holds 32 columns of both halves; the second
    launch adds the gate's and the value's splits and runs the epilogue on the pair."""
    m, k, n = 45, 1536, 2 * 200
    x, q, s, b = problem(orc, m, k, n, False, 61)
    g = knob_gemm("s32", 6)
    w = g.pack(weight_tensor(q, False, "kn"), layout="kn", glu=True)
    name = {"silu": "silu_glu", "situ": "situ_glu"}[epi]
    for out in (torch.float32, torch.bfloat16):
        y = g.product(bf16_dev(x), w, dev(s), bias=dev(b), epilogue=name, out_dtype=out)
        torch.cuda.synchronize()
        judge(orc, y.float().cpu().numpy(), x, q, False, s, b, epi, out)


@pytest.mark.parametrize("head_dim", [0, 64])
def test_split_qkv(knob_gemm, orc, head_dim):
    """The fused QKV product on split sums, row-major or head-major outputs."""
    m, k, d = 30, 1024, 256
    x, q, s, b = problem(orc, m, k, 3 * d, False, 67 + head_dim)
    qo, ko, vo = knob_gemm("s32", 4).product_qkv(bf16_dev(x), weight_tensor(q, False, "nk"), dev(s), layout="nk",
                                                  bias=dev(b), head_dim=head_dim, out_dtype=torch.float32)
    torch.cuda.synchronize()
    parts = [(t.permute(1, 0, 2).reshape(m, d) if head_dim else t).cpu().numpy() for t in (qo, ko, vo)]
    check(orc, np.concatenate(parts, axis=1), x, q, False, s, b, "none", torch.float32)


def test_split_residual(knob_gemm, orc):
    """x += gate ⊙ (s ⊙ (A·W) + b) on split sums equals the split fp32 product then the gated residual pass,
    bit for bit."""
    m, k, n = 24, 2048, 640
    x_, q, s, b = problem(orc, m, k, n, False, 71)
    g = knob_gemm("s32", 7)
    stream = orc.normal_f32(72, (m, n), 0.0, 1.0)
    gate = dev(orc.normal_f32(73, (n,), 0.0, 0.5))
    w = g.pack(weight_tensor(q, False, "nk"), layout="nk")
    y = g.product(bf16_dev(x_), w, dev(s), bias=dev(b), out_dtype=torch.float32)
    expect = dev(stream)
    g.gated_residual(expect, y, gate)
    got = dev(stream)
    g.product_residual(got, bf16_dev(x_), w, dev(s), bias=dev(b), gate=gate)
    torch.cuda.synchronize()
    assert bitwise_equal(got.cpu().numpy(), expect.cpu().numpy()) == 0
    check(orc, y.cpu().numpy(), x_, q, False, s, b, "none", torch.float32)


def test_split_fp32_route(knob_gemm, orc):
    """The fp32 route (three exact bf16 parts of the activation along K, 3× the steps) split over
    workgroups: judged against the fp64 truth of the fp32 activation."""
    m, k, n = 12, 1024, 512
    x = orc.normal_f32(81, (m, k))
    q = orc.uniform_i8(82, (n, k)).view(np.uint8)
    s = orc.uniform_f32(83, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(84, (n,), 0.0, 0.02)
    g = knob_gemm("s32", 5)
    w = g.pack(weight_tensor(q, False, "nk"), layout="nk")
    y = g.product(dev(x), w, dev(s), bias=dev(b), epilogue="gelu_tanh", rounding=False, out_dtype=torch.float32)
    torch.cuda.synchronize()
    check(orc, y.cpu().numpy(), x, q, False, s, b, "gelu", torch.float32, k_eff=3 * k)


def test_no_split_by_default(gemm, knob_gemm, orc):
    """Without the knob the product does not split (a second launch costs more than the split saves): the
    same bits as a context forced to one split."""
    m, k, n = 1, 3072, 3072
    x, q, s, b = problem(orc, m, k, n, False, 91)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    y = gemm.product(bf16_dev(x), w, dev(s), bias=dev(b))
    y1 = knob_gemm(None, 1).product(bf16_dev(x), w, dev(s), bias=dev(b))
    y11 = knob_gemm(None, 11).product(bf16_dev(x), w, dev(s), bias=dev(b))
    torch.cuda.synchronize()
    assert bitwise_equal(y.float().cpu().numpy(), y1.float().cpu().numpy()) == 0
    check(orc, y.float().cpu().numpy(), x, q, False, s, b, "none", torch.bfloat16)
    check(orc, y11.float().cpu().numpy(), x, q, False, s, b, "none", torch.bfloat16)
