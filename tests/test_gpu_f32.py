"""The fp32 route (sq8_linear_f32: the reference's `submit` on an fp32 activation, not rounded —
TensorGEMM.swift:125-135, 264-290) through the C ABI, against the fp64 truth of the fp32 activation
itself (DiagnosticProbes.swift:79-84, the oracle's orc_exact_rows_f32) at the reference's fp32 bar
(channelError ≤ 1e-5, Diagnostic.swift:105) — a bar the bf16-rounded route misses by two orders of
magnitude on the same problem, so these tests tell the routes apart. Every layout, epilogue, kernel
and ragged shape; an identity weight returns the activation bit for bit."""
import numpy as np
import pytest
import torch

from test_gpu_parity import DEV, bf16_dev, dev, judge, problem, weight_tensor

pytestmark = pytest.mark.gpu

_NAMES = {"none": None, "gelu": "gelu_tanh", "silu": "silu_glu", "situ": "situ_glu"}


def f32_problem(orc, m, k, n, fp8, seed):
    """fp32 X ~ N(0, 1) (24 significant bits, not bf16 values); codes, scales and bias as problem()."""
    _, q, s, b = problem(orc, m, k, n, fp8, seed)
    return orc.normal_f32(seed + 7, (m, k)), q, s, b


def test_identity_weight_returns_the_activation(gemm, orc):
    """Codes = I, scale 1: each output is hi + mid + lo of one value, summed in fp32 in that order —
    the value itself, bit for bit (a part lost, doubled or misplaced along K shows here)."""
    m, k = 100, 256
    x = orc.normal_f32(3, (m, k))
    x[0, :8] = [-0.0, 0.0, 1.0, -3.0e-30, 7.0e20, 1.0 + 2.0 ** -23, -(1.0 - 2.0 ** -24), 2.0 ** -100]
    eye = np.eye(k, dtype=np.int8)
    for layout in ("nk", "kn"):
        y = gemm.product(dev(x), weight_tensor(eye.view(np.uint8), False, layout),
                         dev(np.ones(k, np.float32)), layout=layout, out_dtype=torch.float32, rounding=False)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(got.view(np.uint32)[:, 1:], x.view(np.uint32)[:, 1:]), layout
        assert got[0, 0] == 0.0     # −0 · 1 summed from +0: a zero of either sign
    # The rounded route on the same weight returns bf16(x): the routes differ.
    r = gemm.product(dev(x), weight_tensor(eye.view(np.uint8), False, "nk"), dev(np.ones(k, np.float32)),
                     layout="nk", out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(r.cpu().numpy(), orc.bf16_to_f32(orc.f32_to_bf16(x)))


@pytest.mark.parametrize("layout", ["nk", "kn", "packed"])
@pytest.mark.parametrize("epi", ["none", "gelu", "silu", "situ"])
@pytest.mark.parametrize("fp8", [False, True], ids=["int8", "fp8"])
def test_fp32_route_products(gemm, orc, layout, epi, fp8):
    m, k, n = 200, 768, 320
    x, q, s, b = f32_problem(orc, m, k, n, fp8, 31 + n)
    w = weight_tensor(q, fp8, "nk" if layout == "nk" else "kn")
    if layout == "packed":
        w = gemm.pack(w, layout="kn", glu=epi in ("silu", "situ"), fp8=fp8 or None)
    for out in (torch.float32, torch.bfloat16):
        y = gemm.product(dev(x), w, dev(s), layout="nk" if layout == "nk" else "kn", bias=dev(b),
                         epilogue=_NAMES[epi], out_dtype=out, rounding=False)
        torch.cuda.synchronize()
        judge(orc, y.float().cpu().numpy(), x, q, fp8, s, b, epi, out)


def test_rounded_route_misses_the_fp32_bar(gemm, orc):
    """The same problem through the rounded route: its error against the fp32 activation's truth is
    the activation's bf16 rounding (~1e-3), far over 1e-5 — what the fp32 route exists for."""
    m, k, n = 128, 1024, 256
    x, q, s, b = f32_problem(orc, m, k, n, False, 77)
    w = weight_tensor(q, False, "nk")
    y = gemm.product(dev(x), w, dev(s), layout="nk", bias=dev(b), out_dtype=torch.float32)
    torch.cuda.synchronize()
    with pytest.raises(AssertionError, match="channelError"):
        judge(orc, y.cpu().numpy(), x, q, False, s, b, "none", torch.float32)
    e = gemm.product(dev(x), w, dev(s), layout="nk", bias=dev(b), out_dtype=torch.float32, rounding=False)
    torch.cuda.synchronize()
    assert judge(orc, e.cpu().numpy(), x, q, False, s, b, "none", torch.float32) <= 1e-6


KERNEL_KNOBS = {"main256": "256", "main224": "224", "main128": "128", "main64": "64", "main32": "32", "main64n": "64n",
                "main64x192": "64x192", "skinny64": "s64", "skinny32": "s32", "k32x32": "k32x32", "k64x64": "k64x64",
                "k64x192": "k64x192"}


@pytest.mark.parametrize("shape", [(1, 64, 64), (33, 320, 200), (130, 3072, 520), (300, 1024, 1000)],
                         ids=lambda s: "x".join(map(str, s)))
def test_every_kernel_on_the_fp32_route(gemm, orc, tile_gemm, shape):
    m, k, n = shape
    x, q, s, b = f32_problem(orc, m, k, n, False, 600 + n)
    pk = gemm.pack(weight_tensor(q, False, "kn"), layout="kn")
    wnk = weight_tensor(q, False, "nk")
    for name, knob in KERNEL_KNOBS.items():
        g = tile_gemm(knob)
        y = g.product(dev(x), pk, dev(s), bias=dev(b), epilogue="gelu_tanh", out_dtype=torch.float32,
                         rounding=False)
        d = g.product(dev(x), wnk, dev(s), layout="nk", bias=dev(b), epilogue="gelu_tanh",
                      out_dtype=torch.float32, rounding=False)
        torch.cuda.synchronize()
        assert torch.equal(y, d), name  # one kernel, one K order: packed and [N, K] give the same bits
        judge(orc, y.cpu().numpy(), x, q, False, s, b, "gelu", torch.float32)


def test_fp32_route_bench_size(gemm, orc):
    """C1's up projection on an fp32 activation (4096 × 3072 × 12288, GELU, fp32 out), 64 sampled rows."""
    m, k, n = 4096, 3072, 12288
    x, q, s, b = f32_problem(orc, m, k, n, False, 4242)
    pk = gemm.pack(weight_tensor(q, False, "kn"), layout="kn")
    y = gemm.product(dev(x), pk, dev(s), bias=dev(b), epilogue="gelu_tanh", out_dtype=torch.float32,
                     rounding=False)
    torch.cuda.synchronize()
    judge(orc, y.cpu().numpy(), x, q, False, s, b, "gelu", torch.float32, rows=orc.sample_rows(m, 64))


def test_reference_entry_without_rounding(gemm, orc):
    """`linear(a:int8:…:c:m:k:n:)` with `rounding` off, as the reference's fp32 callers make it: fp32
    A, q [K, N] and per-column scales at offsets into larger buffers, fp32 C."""
    m, k, n = 96, 512, 192
    x, q, s, b = f32_problem(orc, m, k, n, False, 5)
    buf = torch.zeros(64 + k * n, dtype=torch.int8, device=DEV)
    buf[64:] = weight_tensor(q, False, "kn").reshape(-1)
    sbuf = torch.zeros(16 + n, dtype=torch.float32, device=DEV)
    sbuf[16:] = dev(s)
    c = torch.empty((m, n), dtype=torch.float32, device=DEV)
    gemm.linear(dev(x), int8=buf, scales=sbuf, per_column=True, c=c, m=m, k=k, n=n, weight_offset=64,
                scales_offset=64, rounding=False)
    torch.cuda.synchronize()
    judge(orc, c.cpu().numpy(), x, q, False, s, None, "none", torch.float32)


@pytest.mark.parametrize("g", [4, 16, 64, 256])
def test_fp32_route_rotated(gemm, orc, g):
    """convrot on the fp32 route: x rotated in fp32 (the oracle's rotate_groups, bit for bit on the
    device) and used whole — judged against the fp64 truth of that rotated fp32 operand, as the reference
    judges a rotated product against its operand (CapacityProbes.swift:536-553)."""
    m, k, n = 130, 1024, 384
    x, q, s, b = f32_problem(orc, m, k, n, False, 70 + g)
    xr = orc.rotate_groups(x, g)
    w = weight_tensor(q, False, "nk")
    for out in (torch.float32, torch.bfloat16):
        y = gemm.product(dev(x), w, dev(s), layout="nk", bias=dev(b), epilogue="gelu_tanh", out_dtype=out,
                         rotation=g, rounding=False)
        torch.cuda.synchronize()
        judge(orc, y.float().cpu().numpy(), xr, q, False, s, b, "gelu", out)
    # The same as the fp32 route on the operand rotated beforehand, bit for bit.
    y = gemm.product(dev(x), w, dev(s), layout="nk", bias=dev(b), out_dtype=torch.float32, rotation=g,
                     rounding=False)
    r = gemm.product(dev(xr), w, dev(s), layout="nk", bias=dev(b), out_dtype=torch.float32, rounding=False)
    torch.cuda.synchronize()
    assert torch.equal(y, r)


def _q8(orc, m, k, n, block, seed):
    x = orc.normal_f32(seed, (m, k))
    q = orc.uniform_i8(seed + 1, (n, k))
    d = orc.uniform_f32(seed + 2, (n, k // block), 1e-3, 2e-2).astype(np.float16)
    b = orc.normal_f32(seed + 3, (n,), 0.0, 0.02)
    return x, q, d, b


def _q8_truth_weight(q, d, block):
    """W [N, K] = q · s (one fp32 product per weight, exact: 8 bits × an fp16)."""
    return q.astype(np.float32) * np.repeat(d.astype(np.float32), block, axis=1)


@pytest.mark.parametrize("layout", ["nk", "kn", "packed"])
@pytest.mark.parametrize("epi", ["none", "gelu", "silu"])
def test_fp32_route_block_scales(gemm, orc, layout, epi):
    """GGUF Q8_0 on the fp32 route (the reference's `blocks` pipeline takes fp32 A): against the fp64
    truth of the fp32 activation and W = q · s."""
    m, k, n, block = 200, 768, 320, 32
    x, q, d, b = _q8(orc, m, k, n, block, 13)
    if layout == "nk":
        w, sc = dev(q).view(torch.int8), dev(d.view(np.int16)).view(torch.float16)
    elif layout == "kn":
        w, sc = dev(np.ascontiguousarray(q.T)).view(torch.int8), dev(np.ascontiguousarray(d.T).astype(np.float32))
    else:
        w = gemm.pack_blocks(dev(q).view(torch.int8), dev(d.astype(np.float32)), block, layout="nk", glu=epi == "silu")
        sc = None
    wv = _q8_truth_weight(q, d, block)
    for out in (torch.float32, torch.bfloat16):
        y = gemm.product_blocks(dev(x), w, sc, block, layout="kn" if layout == "kn" else "nk", bias=dev(b),
                                epilogue=_NAMES[epi], out_dtype=out, rounding=False)
        torch.cuda.synchronize()
        judge(orc, y.float().cpu().numpy(), x, wv, None, np.ones(n, np.float32), b, epi, out, values=True)


def test_fp32_route_block_scales_reference_entry(gemm, orc):
    """`linear(a:int8:…:block:…)` with `rounding` off: q [K, N] and fp32 scales [K/32, N] at offsets."""
    m, k, n, block = 96, 512, 192, 32
    x, q, d, b = _q8(orc, m, k, n, block, 17)
    buf = torch.zeros(64 + k * n, dtype=torch.int8, device=DEV)
    buf[64:] = dev(np.ascontiguousarray(q.T)).view(torch.int8).reshape(-1)
    sbuf = torch.zeros(16 + (k // block) * n, dtype=torch.float32, device=DEV)
    sbuf[16:] = dev(np.ascontiguousarray(d.T).astype(np.float32)).reshape(-1)
    c = torch.empty((m, n), dtype=torch.float32, device=DEV)
    gemm.linear(dev(x), int8=buf, scales=sbuf, per_column=False, c=c, m=m, k=k, n=n, weight_offset=64,
                scales_offset=64, block=block, rounding=False)
    torch.cuda.synchronize()
    judge(orc, c.cpu().numpy(), x, _q8_truth_weight(q, d, block), None, np.ones(n, np.float32), None, "none",
          torch.float32, values=True)


@pytest.mark.parametrize("k", [96, 160, 3072 + 32])
@pytest.mark.parametrize("layout", ["nk", "kn", "packed"])
def test_fp32_route_any_k(gemm, orc, k, layout):
    """K not a multiple of 64 on the fp32 route (the reference's fp32 `linear_int8` has a dynamic K
    extent, TensorGEMM.swift:124-135): the parts padded to whole steps with zeros, the weight packed
    with zero codes past K; judged at the fp32 bar (1e-5), every epilogue, fp32 and bf16 outputs."""
    m, n = 150, 192
    for fp8 in (False, True):
        x, q, s, b = f32_problem(orc, m, k, n, fp8, 900 + k)
        for epi in ("none", "gelu", "silu"):
            w = weight_tensor(q, fp8, "nk" if layout == "nk" else "kn")
            if layout == "packed":
                w = gemm.pack(w, layout="kn", glu=epi == "silu", fp8=fp8 or None)
            for out in (torch.float32, torch.bfloat16):
                y = gemm.product(dev(x), w, dev(s), layout="nk" if layout == "nk" else "kn", bias=dev(b),
                                 epilogue=_NAMES[epi], out_dtype=out, rounding=False)
                torch.cuda.synchronize()
                judge(orc, y.float().cpu().numpy(), x, q, fp8, s, b, epi, out)


@pytest.mark.parametrize("k", [96, 160, 3072 + 32])
def test_fp32_route_block_scales_any_k(gemm, orc, k):
    """Q8_0 (blocks of 32) on the fp32 route at K = 32·odd (the reference's `linear_q8` computes every
    64-row chunk under `row < K`, TensorGEMM.swift:143-171, :162): against the fp64 truth at 1e-5."""
    m, n, block = 130, 192, 32
    x, q, d, b = _q8(orc, m, k, n, block, 950 + k)
    for layout in ("nk", "kn"):
        if layout == "nk":
            w, sc = dev(q).view(torch.int8), dev(d.view(np.int16)).view(torch.float16)
        else:
            w, sc = dev(np.ascontiguousarray(q.T)).view(torch.int8), dev(np.ascontiguousarray(d.T).astype(np.float32))
        for epi in ("none", "gelu"):
            y = gemm.product_blocks(dev(x), w, sc, block, layout=layout, bias=dev(b), epilogue=_NAMES[epi],
                                    out_dtype=torch.float32, rounding=False)
            torch.cuda.synchronize()
            judge(orc, y.cpu().numpy(), x, _q8_truth_weight(q, d, block), None, np.ones(n, np.float32), b, epi,
                  torch.float32, values=True)


def test_fp32_route_refusals(gemm, orc):
    from siliconed_amd import abi
    x, q, s, b = f32_problem(orc, 8, 128, 64, False, 3)
    lib = abi.load()
    w, sv, xt = weight_tensor(q, False, "nk"), dev(s), dev(x)
    from siliconed_amd.tensor_gemm import _dev
    def call(group=0, wd=abi.INT8, sdt=abi.F32, slay=abi.SCALE_COLUMNS, block=0, m=8):
        c = torch.empty((8, 64), dtype=torch.float32, device=DEV)
        return lib.sq8_linear_f32(gemm._h, _dev(xt, "x"), 128, group, _dev(w, "w"), wd, abi.NK, 128, _dev(sv, "s"),
                                  sdt, slay, block, None, 0, _dev(c, "c"), abi.F32, 64, m, 128, 64, None)
    assert call() == abi.OK
    assert call(sdt=abi.F16) == abi.EINVAL                   # per-column scales are fp32
    assert call(block=32) == abi.EINVAL                      # a block size without block scales
    assert call(slay=abi.SCALE_BLOCKS, block=32, group=16) == abi.EUNSUPPORTED  # block scales: no rotation
    assert call(m=-1) == abi.EINVAL
    torch.cuda.synchronize()
    # Empty M: nothing to do, no error.
    y = gemm.product(dev(np.zeros((0, 128), np.float32)), w, sv, layout="nk", out_dtype=torch.float32,
                     rounding=False)
    assert y.shape == (0, 64)
