"""The product on block scales (GGUF Q8_0: int8 codes, one fp16 scale per 32 consecutive K of an
output) through the C ABI, against the fp64 truth of the oracle's widened weight W = q · s
(orc_dequantize, SCALE_BLOCKS: Widen.swift:129-187, one fp32 multiply per weight) at the reference's
bars (Diagnostic.swift:105-107, CapacityProbes.swift:541-553; max-rel ≤ 2e-2 on bf16 outputs):
[N, K] codes with GGUF's [N, K/32] fp16 scales, the map's [K, N] with [K/B, N] fp32, the packed
layout, every epilogue, ragged shapes, and the reference's own entry `linear(…block:…)`."""
import numpy as np
import pytest
import torch

from test_gpu_parity import DEV, EPI, bf16_dev, dev, judge

pytestmark = pytest.mark.gpu

_EPI_NAMES = {"none": None, "gelu": "gelu_tanh", "silu": "silu_glu", "situ": "situ_glu"}


def q8_problem(orc, m, k, n, block, seed, bias=True):
    """bf16 X ~ N(0,1); int8 codes [N, K] uniform in [−127, 127]; scales per (output, block of K)
    U(1e−3, 2e−2) rounded to fp16 (GGUF's `d`); bias N(0, 0.02)."""
    x = orc.normal_bf16(seed, (m, k))
    q = orc.uniform_i8(seed + 1, (n, k))
    d = orc.uniform_f32(seed + 2, (n, k // block), 1e-3, 2e-2).astype(np.float16)
    b = orc.normal_f32(seed + 3, (n,), 0.0, 0.02) if bias else None
    return x, q, d, b


def widened(orc, q, d, block):
    """W [K, N] = q · s, the oracle's dequantiser on the map's layout (codes [K, N], scales [K/B, N])."""
    n, k = q.shape
    q_kn = np.ascontiguousarray(q.T)
    s_kn = np.ascontiguousarray(d.T)
    return orc.dequantize(q_kn.view(np.uint8), orc.INT8, s_kn.view(np.uint16), orc.F16, layout=orc.SCALE_BLOCKS,
                          columns=n, block_rows=block)


def judge_blocks(orc, got, x, q, d, block, b, epi, out_dtype, rows=None):
    n, k = q.shape
    w = widened(orc, q, d, block)
    # judge() widens codes with a per-column scale; here the weight is already q · s: codes = W
    # transposed to [N, K], scale 1.
    return judge(orc, got, x, np.ascontiguousarray(w.T), None, np.ones(n, np.float32), b, epi, out_dtype, rows=rows,
                 values=True)


@pytest.mark.parametrize("layout", ["nk", "kn", "packed"])
@pytest.mark.parametrize("epi", ["none", "gelu", "silu", "situ"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_block_scaled_product(gemm, orc, layout, epi, out_dtype):
    m, k, n, block = 200, 768, 320, 32
    x, q, d, b = q8_problem(orc, m, k, n, block, 11)
    if layout == "nk":
        w, s = dev(q).view(torch.int8), dev(d.view(np.int16)).view(torch.float16)
    elif layout == "kn":
        w, s = dev(np.ascontiguousarray(q.T)).view(torch.int8), dev(np.ascontiguousarray(d.T).astype(np.float32))
    else:
        w = gemm.pack_blocks(dev(q).view(torch.int8), dev(d.astype(np.float32)), block, layout="nk",
                             glu=epi in ("silu", "situ"))
        s = None
    y = gemm.product_blocks(bf16_dev(x), w, s, block, layout="kn" if layout == "kn" else "nk", bias=dev(b),
                            epilogue=_EPI_NAMES[epi], out_dtype=out_dtype)
    torch.cuda.synchronize()
    judge_blocks(orc, y.float().cpu().numpy(), x, q, d, block, b, epi, out_dtype)


@pytest.mark.parametrize("m,k,n,block", [(1, 64, 64, 32), (37, 1024, 100, 64), (130, 2048, 1000, 128),
                                         (64, 128, 8, 32), (512, 3072, 3072, 32)])
def test_block_scaled_shapes(gemm, orc, m, k, n, block):
    x, q, d, b = q8_problem(orc, m, k, n, block, 23 + m)
    y = gemm.product_blocks(bf16_dev(x), dev(q).view(torch.int8), dev(d.view(np.int16)).view(torch.float16), block,
                            bias=dev(b), out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = orc.sample_rows(m, 64) if m > 64 else None
    judge_blocks(orc, y.float().cpu().numpy(), x, q, d, block, b, "none", torch.float32, rows=rows)


def test_block_scaled_reference_entry(gemm, orc):
    """`linear(a:int8:…:scales:…:block:…)` as the reference calls it: fp32 activation (rounded to
    bf16 here), q [K, N] and fp32 scales [K/32, N] at offsets into larger buffers, fp32 C."""
    m, k, n, block = 96, 512, 192, 32
    x, q, d, b = q8_problem(orc, m, k, n, block, 5, bias=False)
    a = dev(orc.bf16_to_f32(x))
    q_kn = np.ascontiguousarray(q.T)
    buf = torch.zeros(64 + k * n, dtype=torch.int8, device=DEV)
    buf[64:] = dev(q_kn).view(torch.int8).reshape(-1)
    sbuf = torch.zeros(16 + (k // block) * n, dtype=torch.float32, device=DEV)
    sbuf[16:] = dev(np.ascontiguousarray(d.T).astype(np.float32)).reshape(-1)
    c = torch.empty((m, n), dtype=torch.float32, device=DEV)
    gemm.linear(a, int8=buf, scales=sbuf, per_column=False, c=c, m=m, k=k, n=n, weight_offset=64, scales_offset=64,
                block=block)
    judge_blocks(orc, c.cpu().numpy(), x, q, d, block, None, "none", torch.float32)


@pytest.mark.parametrize("k", [96, 160, 3072 + 32])
@pytest.mark.parametrize("layout", ["nk", "kn", "packed"])
def test_block_scaled_any_k(gemm, orc, k, layout):
    """Q8_0 with blocks of 32 at K = 32·odd — a valid GGUF shape (the reference computes every 64-row
    chunk under `row < K`, TensorGEMM.swift:143-171, :162): the activation padded to whole steps with
    zeros, the packed codes and scales zero past K; against the oracle's fp64 truth of q·d, GELU and
    SiLU-GLU, bf16 and fp32 out."""
    m, n, block = 130, 256, 32
    x, q, d, b = q8_problem(orc, m, k, n, block, 960 + k)
    for epi in ("none", "gelu", "silu"):
        glu = epi == "silu"
        if layout == "nk":
            w, sc = dev(q).view(torch.int8), dev(d.view(np.int16)).view(torch.float16)
        else:
            w, sc = dev(np.ascontiguousarray(q.T)).view(torch.int8), dev(np.ascontiguousarray(d.T).astype(np.float32))
        if layout == "packed":
            w, sc = gemm.pack_blocks(w, sc, block, layout="kn", glu=glu), None
        for out in (torch.bfloat16, torch.float32):
            y = gemm.product_blocks(bf16_dev(x), w, sc, block, layout="nk" if layout == "nk" else "kn", bias=dev(b),
                                    epilogue={"none": None, "gelu": "gelu_tanh", "silu": "silu_glu"}[epi],
                                    out_dtype=out)
            torch.cuda.synchronize()
            judge_blocks(orc, y.float().cpu().numpy(), x, q, d, block, b, epi, out)


def test_block_scaled_column_slice_kn(gemm, orc):
    """A column-sliced [K, N] Q8_0 weight (w_full[:, :n]) takes its scales as scale_full[:, :n], rows
    with the codes' stride: the same bits as the contiguous copy, direct and staged; a contiguous
    [K/B, n] scale with the wider codes is refused rather than read with the wrong stride."""
    m, k, n, wide, block = 96, 512, 192, 320, 32
    x, q, d, b = q8_problem(orc, m, k, wide, block, 77)
    w_full = dev(np.ascontiguousarray(q.T)).view(torch.int8)               # [K, wide]
    s_full = dev(np.ascontiguousarray(d.T).astype(np.float32))             # [K/B, wide]
    w_sl, s_sl = w_full[:, :n], s_full[:, :n]
    w_c, s_c = w_sl.contiguous(), s_sl.contiguous()
    a = bf16_dev(x)
    want = gemm.product_blocks(a, w_c, s_c, block, layout="kn", bias=dev(b[:n]), out_dtype=torch.float32)
    got = gemm.product_blocks(a, w_sl, s_sl, block, layout="kn", bias=dev(b[:n]), out_dtype=torch.float32)
    staged = gemm.product_blocks(a, gemm.pack_blocks(w_sl, s_sl, block, layout="kn"), bias=dev(b[:n]),
                                 out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(staged, want)
    judge_blocks(orc, got.cpu().numpy(), x, q[:n], d[:n], block, b[:n], "none", torch.float32)
    with pytest.raises(ValueError):
        gemm.product_blocks(a, w_sl, s_c, block, layout="kn")
    with pytest.raises(ValueError):
        gemm.pack_blocks(w_sl, s_c, block, layout="kn")


def test_block_scaled_refusals(gemm, orc):
    from siliconed_amd import abi
    x, q, d, b = q8_problem(orc, 8, 128, 64, 16, 3)
    with pytest.raises(abi.SQ8Error) as e:      # blocks of 16 split an MFMA sub-step
        gemm.product_blocks(bf16_dev(x), dev(q).view(torch.int8), dev(d.astype(np.float32)), 16)
    assert e.value.status == abi.EUNSUPPORTED


def test_block_scaled_bench_size(gemm, orc):
    """C1's up projection as a Q8_0 weight (4096 × 3072 × 12288, GELU, bf16 out) on 64 sampled rows."""
    m, k, n, block = 4096, 3072, 12288, 32
    x, q, d, b = q8_problem(orc, m, k, n, block, 41)
    w = gemm.pack_blocks(dev(q).view(torch.int8), dev(d.view(np.int16)).view(torch.float16), block)
    y = gemm.product_blocks(bf16_dev(x), w, bias=dev(b), epilogue="gelu_tanh")
    torch.cuda.synchronize()
    rows = orc.sample_rows(m, 64)
    judge_blocks(orc, y.float().cpu().numpy(), x, q, d, block, b, "gelu", torch.bfloat16, rows=rows)


def test_gguf_q8_0_weight_staged(gemm, orc, tmp_path):
    """A Q8_0 weight read from a GGUF file (siliconed_amd.gguf_q8) and staged: the same bits as the
    product on its codes and scales passed directly, and within the bars of the truth."""
    from siliconed_amd.gguf_q8 import GGUFFile, write
    m, k, n = 96, 512, 320
    x, q, d, b = q8_problem(orc, m, k, n, 32, 9)
    blocks = np.empty((n * k // 32, 34), np.uint8)
    blocks[:, :2] = d.reshape(-1, 1).view(np.uint8)
    blocks[:, 2:] = q.reshape(-1, 32).view(np.uint8)
    path = str(tmp_path / "w.gguf")
    write(path, {"general.architecture": ("string", "test")}, {"blk.0.w.weight": ("Q8_0", [k, n], blocks.tobytes())})
    with GGUFFile(path) as g:
        wp = g.stage("blk.0.w.weight", gemm)
    got = gemm.product_blocks(bf16_dev(x), wp, bias=dev(b), out_dtype=torch.float32)
    want = gemm.product_blocks(bf16_dev(x), dev(q).view(torch.int8), dev(d.view(np.int16)).view(torch.float16), 32,
                               bias=dev(b), out_dtype=torch.float32)
    torch.cuda.synchronize()
    from refgen import bitwise_equal
    assert bitwise_equal(got.cpu().numpy(), want.cpu().numpy()) == 0
    judge_blocks(orc, got.cpu().numpy(), x, q, d, 32, b, "none", torch.float32)


@pytest.mark.parametrize("cols", [192, 200])
def test_submit_first_columns_on_block_scales(gemm, orc, cols):
    """`submit(…columns:)` on a block-scaled [K, N] weight (the reference's Q8_0 submit dispatches
    ⌈columns/64⌉ threadgroups on the whole weight's scales, TensorGEMM.swift:292-318): the first `columns`
    of C written, the others untouched; each column the same bits as the whole product's (the codes and
    their [K/B, N] scales read with the whole weight's stride); within the bars of the truth."""
    m, k, n, block = 130, 512, 320, 32
    x, q, d, b = q8_problem(orc, m, k, n, block, 71)
    a = bf16_dev(x)
    w = dev(np.ascontiguousarray(q.T)).view(torch.int8)                 # [K, N]
    s = dev(np.ascontiguousarray(d.T).astype(np.float32))               # [K/B, N] fp32
    whole = torch.empty((m, n), dtype=torch.float32, device=DEV)
    gemm.linear(a, int8=w, scales=s, per_column=True, c=whole, m=m, k=k, n=n, block=block, bias=dev(b),
                epilogue="gelu_tanh")
    part = torch.full((m, n), 7.0, dtype=torch.float32, device=DEV)
    gemm.submit(a, int8=w, scales=s, per_column=True, c=part, m=m, k=k, n=n, columns=cols, block=block, bias=dev(b),
                epilogue="gelu_tanh")
    gemm.synchronize()
    assert (part[:, cols:] == 7.0).all()
    assert torch.equal(part[:, :cols], whole[:, :cols])
    judge_blocks(orc, part[:, :cols].cpu().numpy(), x, q[:cols], d[:cols], block, b[:cols], "gelu", torch.float32)
