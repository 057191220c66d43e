"""Short products (M = 1 … 30 rows: the text-token streams and decode-sized batches) with the GELU-tanh
and SiLU-GLU epilogues on every route — bf16-rounded, fp32 (used whole), convrot and Q8_0 block scales —
judged element by element against the oracle's fp64 truth.

With a handful of rows the per-channel metric (DiagnosticJudgement.swift:39-71) is ill-conditioned: a
column whose few exact values cancel has a floor near zero. The bound here is normalised by magnitude
instead: before the activation, |y − t| ≤ ε·(Σ_k |x_k·w_k|·|s| + |b|) with ε = max(2⁻²⁰, 2·√(K′/16)·2⁻²⁴)
(K′ = K, or 3K on the fp32 route's three parts; the MFMA rounds once per 16 terms), carried through the
activation by its slope (|GELU′| ≤ 1.13; SiLU-GLU by the product rule with |SiLU′| ≤ 1.1), plus 2⁻¹⁸ of
the value for the activation's evaluation in fp32 and one unit in the last place of the output type.
The truth's GELU is evaluated without cancellation in its negative tail (values near −3·10⁻²¹ at
x = −8 stay normal fp32 numbers; oracle/sq8_oracle.c `orc_gelu_tanh`)."""
import math

import numpy as np
import pytest
import torch

from test_gpu_parity import bf16_dev, dev, weight_tensor

pytestmark = pytest.mark.gpu

MS = [1, 2, 7, 16, 30]
ROUTES = ["bf16", "fp32", "rot", "q8"]
EPIS = ["gelu", "silu"]
K, N_OUT = 3072, 512


def _bound_check(orc, got, xt, wv, s, b, epi, out_dtype, k_eff):
    """`xt`: the truth's activation (bf16 bits, or fp32 values taken whole), `wv`: the weight's values
    [N, K] fp32 (codes with scales `s`, or q·d with s = 1), `b` bias."""
    m, k = xt.shape
    n = wv.shape[0]
    rows = np.arange(m, dtype=np.int32)
    pre = orc.exact_rows(rows, xt, wv, False, k, n, scale=s, bias=b, epilogue=orc.EPI_NONE)
    xf = orc.bf16_to_f32(xt).astype(np.float64) if xt.dtype == np.uint16 else xt.astype(np.float64)
    mag = (np.abs(xf) @ np.abs(wv.astype(np.float64)).T) * np.abs(s.astype(np.float64)) + np.abs(b.astype(np.float64))
    eps = max(2.0 ** -20, 2.0 * math.sqrt(k_eff / 16) * 2.0 ** -24)
    e = eps * mag
    ulp = 2.0 ** -7 if out_dtype == torch.bfloat16 else 2.0 ** -23
    tiny = 2.0 ** -126
    if epi == "none":
        f = pre
        bound = e + ulp * np.abs(f) + tiny
    elif epi == "gelu":
        f = orc.exact_rows(rows, xt, wv, False, k, n, scale=s, bias=b, epilogue=orc.EPI_GELU_TANH)
        bound = 1.13 * e + (2.0 ** -18 + ulp) * np.abs(f) + tiny
    else:
        h = n // 2
        f = orc.exact_rows(rows, xt, wv, False, k, n, scale=s, bias=b, epilogue=orc.EPI_SILU_GLU)
        g, u, eg, eu = pre[:, :h], pre[:, h:], e[:, :h], e[:, h:]
        silu = g / (1.0 + np.exp(-np.clip(g, -700, 700)))
        bound = 1.1 * eg * np.abs(u) + np.abs(silu) * eu + 1.1 * eg * eu + (2.0 ** -18 + ulp) * np.abs(f) + tiny
    assert np.isfinite(got).all(), "non-finite outputs"
    err = np.abs(got.astype(np.float64) - f)
    worst = np.unravel_index(np.argmax(err / bound), err.shape)
    assert np.all(err <= bound), (f"row {worst[0]} column {worst[1]}: got {got[worst]:.6e}, truth {f[worst]:.6e}, "
                                  f"bound {bound[worst]:.3e}")
    # The negative tail is in the sample: outputs below 1e-12 in magnitude that are not zero.
    return int(((np.abs(f) < 1e-12) & (f != 0)).sum())


@pytest.mark.parametrize("epi", EPIS)
@pytest.mark.parametrize("route", ROUTES)
@pytest.mark.parametrize("m", MS)
def test_short_products_with_epilogues(gemm, orc, m, route, epi):
    i = 100 * m + 10 * ROUTES.index(route) + EPIS.index(epi)
    out = torch.bfloat16 if i % 2 == 0 else torch.float32
    n = 2 * N_OUT if epi == "silu" else N_OUT
    name = "gelu_tanh" if epi == "gelu" else "silu_glu"
    glu = epi == "silu"
    print(f"short product: m {m} route {route} epilogue {name} out {out}", flush=True)
    b = orc.normal_f32(i + 3, (n,), 0.0, 0.02)
    if route == "q8":
        x = orc.normal_bf16(i, (m, K))
        q = orc.uniform_i8(i + 1, (n, K))
        d = orc.uniform_f32(i + 2, (n, K // 32), 1e-3, 2e-2).astype(np.float16)
        w = gemm.pack_blocks(dev(q).view(torch.int8), dev(d.astype(np.float32)), 32, layout="nk", glu=glu)
        y = gemm.product_blocks(bf16_dev(x), w, None, 32, layout="nk", bias=dev(b), epilogue=name, out_dtype=out)
        torch.cuda.synchronize()
        wv = q.astype(np.float32) * np.repeat(d.astype(np.float32), 32, axis=1)
        _bound_check(orc, y.float().cpu().numpy(), x, wv, np.ones(n, np.float32), b, epi, out, K)
        return
    x32 = orc.normal_f32(i, (m, K))
    q = orc.uniform_i8(i + 1, (n, K)).view(np.uint8)
    s = orc.uniform_f32(i + 2, (n,), 1e-3, 2e-2)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk", glu=glu)
    kw = dict(bias=dev(b), epilogue=name, out_dtype=out)
    k_eff = K
    if route == "rot":
        y = gemm.product(dev(x32), w, dev(s), rotation=256, rounding=True, **kw)
        xt = orc.f32_to_bf16(orc.rotate_groups(x32, 256))
    elif route == "fp32":
        y = gemm.product(dev(x32), w, dev(s), rounding=False, **kw)
        xt, k_eff = x32, 3 * K
    else:
        xt = orc.f32_to_bf16(x32)
        y = gemm.product(bf16_dev(xt), w, dev(s), **kw)
    torch.cuda.synchronize()
    _bound_check(orc, y.float().cpu().numpy(), xt, q.view(np.int8).astype(np.float32), s, b, epi, out, k_eff)


def test_gelu_tail_reaches_the_sample(gemm, orc):
    # The sweep's pre-activations (|Σ x·q·s| up to ~10² at K = 3072) reach GELU's negative tail, where the
    # double form ½x(1 + tanh u) gave −0: outputs near −10⁻²¹ are judged, not skipped.
    m = 7
    x = orc.normal_bf16(5, (m, K))
    q = orc.uniform_i8(6, (N_OUT, K)).view(np.uint8)
    s = orc.uniform_f32(7, (N_OUT,), 1e-3, 2e-2)
    b = orc.normal_f32(8, (N_OUT,), 0.0, 0.02)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    y = gemm.product(bf16_dev(x), w, dev(s), bias=dev(b), epilogue="gelu_tanh", out_dtype=torch.float32)
    torch.cuda.synchronize()
    tail = _bound_check(orc, y.float().cpu().numpy(), x, q.view(np.int8).astype(np.float32), s, b, "gelu",
                        torch.float32, K)
    assert tail > 0
