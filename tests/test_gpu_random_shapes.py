"""A seeded sweep of random shapes through the product's routes — bf16-rounded, fp32 (used whole), convrot
(rounded or whole) and Q8_0 block scales — × layouts × epilogues × int8/fp8 × output types, each judged
on sampled rows against the oracle's fp64 truth at the reference's bars (Diagnostic.swift:105-107,
CapacityProbes.swift:541-553). Rows from 31 up: the per-channel metric averages over rows, and with a
handful of rows a column whose exact values cancel makes it ill-conditioned (the products' error
relative to Σ|x·w|·s stays at fp32's rounding there too)."""
import random

import numpy as np
import pytest
import torch

from test_gpu_parity import bf16_dev, dev, judge, problem, weight_tensor

pytestmark = pytest.mark.gpu

_NAMES = {"none": None, "gelu": "gelu_tanh", "silu": "silu_glu", "situ": "situ_glu"}


def _case(i):
    rng = random.Random(9000 + i)
    route = rng.choice(["bf16", "bf16", "fp32", "rot", "q8"])
    m = rng.choice([31, 64, 100, 257, 513, 1000])
    n = rng.choice([64, 96, 130, 320, 1000, 2048])
    layout = rng.choice(["nk", "kn", "packed"])
    k = 64 * rng.randint(1, 40)
    if route == "bf16" and layout != "packed" and rng.random() < 0.4:
        k = rng.randint(8, 700)                    # ragged K: the general kernel
    epi = rng.choice(["none", "gelu", "silu", "situ"] if route != "q8" else ["none", "gelu", "silu"])
    if epi in ("silu", "situ") and n % 2:
        n += 1
    fp8 = route in ("bf16", "fp32") and rng.random() < 0.3
    out = rng.choice([torch.float32, torch.bfloat16])
    grp = rng.choice([g for g in (4, 16, 64, 256) if k % g == 0]) if route == "rot" else 0
    rounding = rng.random() < 0.5
    return route, m, k, n, layout, epi, fp8, out, grp, rounding


@pytest.mark.parametrize("i", range(60))
def test_random_shape(gemm, orc, i):
    route, m, k, n, layout, epi, fp8, out, grp, rounding = _case(i)
    rows = orc.sample_rows(m, 48)
    if route == "q8":
        x = orc.normal_bf16(i, (m, k))
        q = orc.uniform_i8(i + 1, (n, k))
        d = orc.uniform_f32(i + 2, (n, k // 32), 1e-3, 2e-2).astype(np.float16)
        b = orc.normal_f32(i + 3, (n,), 0.0, 0.02)
        if layout == "packed":
            w, s, lay = gemm.pack_blocks(dev(q).view(torch.int8), dev(d.astype(np.float32)), 32, layout="nk",
                                         glu=epi in ("silu", "situ")), None, "nk"
        elif layout == "kn":
            w, s, lay = (dev(np.ascontiguousarray(q.T)).view(torch.int8),
                         dev(np.ascontiguousarray(d.T).astype(np.float32)), "kn")
        else:
            w, s, lay = dev(q).view(torch.int8), dev(d.view(np.int16)).view(torch.float16), "nk"
        y = gemm.product_blocks(bf16_dev(x), w, s, 32, layout=lay, bias=dev(b), epilogue=_NAMES[epi], out_dtype=out)
        torch.cuda.synchronize()
        wv = q.astype(np.float32) * np.repeat(d.astype(np.float32), 32, axis=1)
        judge(orc, y.float().cpu().numpy(), x, wv, None, np.ones(n, np.float32), b, epi, out, rows=rows, values=True)
        return
    x32 = orc.normal_f32(i, (m, k))
    _, q, s, b = problem(orc, m, k, n, fp8, i + 1)
    w = weight_tensor(q, fp8, "nk" if layout == "nk" else "kn")
    if layout == "packed":
        w = gemm.pack(w, layout="kn", glu=epi in ("silu", "situ"), fp8=fp8 or None)
    lay = "nk" if layout == "nk" else "kn"
    kw = dict(layout=lay, bias=dev(b), epilogue=_NAMES[epi], out_dtype=out)
    if route == "rot":
        y = gemm.product(dev(x32), w, dev(s), rotation=grp, rounding=rounding, **kw)
        xr = orc.rotate_groups(x32, grp)
        truth_x = orc.f32_to_bf16(xr) if rounding else xr
    elif route == "fp32":
        y = gemm.product(dev(x32), w, dev(s), rounding=False, **kw)
        truth_x = x32
    else:
        truth_x = orc.f32_to_bf16(x32)
        y = gemm.product(bf16_dev(truth_x), w, dev(s), **kw)
    torch.cuda.synchronize()
    judge(orc, y.float().cpu().numpy(), truth_x, q, fp8, s, b, epi, out, rows=rows)


def _w8a8_case(i):
    rng = random.Random(7000 + i)
    m = rng.choice([1, 2, 7, 31, 100, 257, 1000])
    layout = rng.choice(["nk", "kn", "packed"])
    k = 64 * rng.randint(1, 48) if layout == "packed" else rng.randint(8, 3000)
    n = rng.choice([8, 64, 130, 320, 1000, 2048])
    groups = [g for g in (0, 4, 16, 64, 256) if g == 0 or k % g == 0]
    return m, k, n, layout, rng.choice(groups), rng.random() < 0.7


@pytest.mark.parametrize("i", range(30))
def test_random_shape_w8a8_at_the_bit(gemm, orc, i):
    """The W8A8 route on random shapes, one row up: the same bits as the oracle's recipe (codes and row
    scales of W8A8.quantize, the integer sums exact, float(Σ) · (s_x · s_w))."""
    m, k, n, layout, g, per_col = _w8a8_case(i)
    x = orc.normal_f32(500 + i, (m, k))
    q = orc.uniform_i8(501 + i, (n, k))
    sw = orc.uniform_f32(502 + i, (n if per_col else 1,), 1e-3, 2e-2)
    codes, sx = orc.quantize_rows(x, g)
    expected = orc.w8a8_product(codes, sx, q, False, sw)
    if layout == "packed":
        w, lay = gemm.pack(dev(q).view(torch.int8), layout="nk"), "nk"
    elif layout == "kn":
        w, lay = dev(np.ascontiguousarray(q.T)).view(torch.int8), "kn"
    else:
        w, lay = dev(q).view(torch.int8), "nk"
    got = gemm.product_quantized(dev(x), w, dev(sw), group=g, layout=lay, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), expected.view(np.uint32))


def _exact_case(i):
    rng = random.Random(5000 + i)
    m = rng.choice([1, 2, 3, 7, 16, 33, 130, 600])
    layout = rng.choice(["nk", "kn", "packed"])
    route = rng.choice(["bf16", "fp32"])
    # Ragged K (the general kernel) on the rounded route; the fp32 route takes whole steps of 64.
    k = 64 * rng.randint(1, 60) if layout == "packed" or route == "fp32" or rng.random() < 0.6 else rng.randint(8, 2000)
    n = rng.choice([8, 64, 96, 130, 320, 1000, 3072])
    return m, k, n, layout, route, rng.choice([torch.float32, torch.bfloat16])


@pytest.mark.parametrize("i", range(30))
def test_random_shape_exact_sums_at_the_bit(gemm, orc, i):
    """Integer activations in [−5, 5] and codes: every product and every fp32 sum exact in any order
    (|Σ| ≤ 5·127·K < 2^24), so from one row up, on whichever kernel the shape takes (skinny, short or
    main tiles, the general kernel for ragged K), the output is the reference's two roundings bit for bit:
    the scale after the sum (TensorGEMM.swift:175-179), then the bias (Ops.swift:400-407)."""
    m, k, n, layout, route, out = _exact_case(i)
    rng = np.random.default_rng(4000 + i)
    xi = rng.integers(-5, 6, (m, k)).astype(np.float32)
    q = orc.uniform_i8(4100 + i, (n, k)).view(np.uint8)
    s = orc.uniform_f32(4200 + i, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(4300 + i, (n,), 0.0, 0.02)
    w = weight_tensor(q, False, "nk" if layout == "nk" else "kn")
    if layout == "packed":
        w = gemm.pack(w, layout="kn")
    lay = "nk" if layout == "nk" else "kn"
    x = dev(xi) if route == "fp32" else bf16_dev(orc.f32_to_bf16(xi))
    y = gemm.product(x, w, dev(s), layout=lay, bias=dev(b), out_dtype=out, rounding=route != "fp32")
    torch.cuda.synchronize()
    total = (xi.astype(np.float64) @ q.view(np.int8).astype(np.float64).T).astype(np.float32)   # exact
    want = (total * s[None, :]).astype(np.float32) + b[None, :]
    if out == torch.float32:
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.astype(np.float32).view(np.uint32))
    else:
        assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), orc.f32_to_bf16(want.astype(np.float32)))


@pytest.mark.parametrize("i", range(20))
def test_random_shape_block_scales_at_the_bit(gemm, orc, i):
    """GGUF Q8_0 block scales on integer activations: each block's sum Σ a·q is exact, so the product's
    arithmetic is fixed — per block of 32, in K order, acc = fl(P·d + acc) (one fused rounding), then
    the bias — and restated in numpy (float64 holds P·d + acc exactly) it gives the same bits, from one
    row up, on every layout."""
    rng = random.Random(3000 + i)
    m = rng.choice([1, 2, 5, 33, 130, 600])
    k = 64 * rng.randint(1, 40)
    n = rng.choice([8, 64, 130, 320, 1000])
    layout = rng.choice(["nk", "kn", "packed"])
    r = np.random.default_rng(3100 + i)
    xi = r.integers(-5, 6, (m, k)).astype(np.float32)
    q = orc.uniform_i8(3200 + i, (n, k))
    d = orc.uniform_f32(3300 + i, (n, k // 32), 1e-3, 2e-2).astype(np.float16)
    b = orc.normal_f32(3400 + i, (n,), 0.0, 0.02)
    if layout == "packed":
        w, s, lay = gemm.pack_blocks(dev(q).view(torch.int8), dev(d.astype(np.float32)), 32, layout="nk"), None, "nk"
    elif layout == "kn":
        w, s, lay = dev(np.ascontiguousarray(q.T)).view(torch.int8), dev(np.ascontiguousarray(d.T).astype(np.float32)), "kn"
    else:
        w, s, lay = dev(q).view(torch.int8), dev(d.view(np.int16)).view(torch.float16), "nk"
    y = gemm.product_blocks(bf16_dev(orc.f32_to_bf16(xi)), w, s, 32, layout=lay, bias=dev(b), out_dtype=torch.float32)
    torch.cuda.synchronize()
    acc = np.zeros((m, n), np.float32)
    qf = q.astype(np.float64)
    for blk in range(k // 32):
        p = xi[:, 32 * blk:32 * blk + 32].astype(np.float64) @ qf[:, 32 * blk:32 * blk + 32].T     # exact
        acc = (p * d[:, blk].astype(np.float64)[None, :] + acc.astype(np.float64)).astype(np.float32)
    want = (acc + b[None, :]).astype(np.float32)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("i", range(12))
def test_random_shape_fp8_exact_sums_at_the_bit(gemm, orc, i):
    """fp8-e4m3 codes of values in [−1, 1] (multiples of 2^−9) times integer activations in [−5, 5]:
    every partial sum is a multiple of 2^−9 below 2^15, exact in fp32 in any order (K ≤ 6400), so the
    output is the reference's two roundings bit for bit, from one row up, on every layout."""
    rng = random.Random(6000 + i)
    m = rng.choice([1, 3, 17, 64, 300])
    k = 64 * rng.randint(1, 50)
    n = rng.choice([8, 64, 130, 1000])
    layout = rng.choice(["nk", "kn", "packed"])
    r = np.random.default_rng(6100 + i)
    xi = r.integers(-5, 6, (m, k)).astype(np.float32)
    q = orc.f32_to_e4m3(r.uniform(-1.0, 1.0, (n, k)).astype(np.float32))       # [N, K] codes
    from refgen import code_values
    wv = code_values(q, True).astype(np.float64)
    s = orc.uniform_f32(6200 + i, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(6300 + i, (n,), 0.0, 0.02)
    w = weight_tensor(q, True, "nk" if layout == "nk" else "kn")
    if layout == "packed":
        w = gemm.pack(w, layout="kn", fp8=True)
    y = gemm.product(bf16_dev(orc.f32_to_bf16(xi)), w, dev(s), layout="nk" if layout == "nk" else "kn", bias=dev(b),
                     out_dtype=torch.float32)
    torch.cuda.synchronize()
    total = (xi.astype(np.float64) @ wv.T).astype(np.float32)                     # exact
    want = (total * s[None, :]).astype(np.float32) + b[None, :]
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.astype(np.float32).view(np.uint32))
