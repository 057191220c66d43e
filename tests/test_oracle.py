"""The CPU oracle pinned before it is trusted: against published known answers, the reference's own
test vectors, torch's independent conversions, float64 products and closed forms. Each test names
the mistake it would catch."""
import json
import math
import os

import numpy as np
import pytest
import torch

from refgen import DequantizeGen, bitwise_equal, code_values, e4m3_torch_table, GOLDEN


# ---- SplitMix64 + Box–Muller (Sources/Verification/KernelStages.swift:553-567) -------------------

def test_splitmix_known_answers(orc):
    # SplitMix64 from state 0: the published first outputs (Steele, Lea & Flood's generator).
    assert [int(x) for x in orc.splitmix_stream(0, 3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_fills_equal_the_sequential_stream(orc):
    # The parallel fills jump the state to each chunk: a wrong jump breaks values past 65 536.
    import ctypes
    n = 70_000
    f = orc.normal_f32(99, (n,))
    st = ctypes.c_uint64(99)
    seq = [orc.lib().orc_splitmix_normal(ctypes.byref(st)) for _ in range(n)]
    assert np.array_equal(f, np.array(seq, dtype=np.float32))
    u = orc.uniform_f32(5, (n,), 1e-3, 2e-2)
    st = ctypes.c_uint64(5)
    seq = [1e-3 + (2e-2 - 1e-3) * orc.lib().orc_splitmix_uniform(ctypes.byref(st)) for _ in range(n)]
    assert np.array_equal(u, np.array(seq, dtype=np.float32))
    q = orc.uniform_i8(3, (n,), -127, 127)
    assert q.min() == -127 and q.max() == 127


def test_normal_draws_are_normal(orc):
    x = orc.normal_f32(1, (200_000,)).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01


# ---- conversions ------------------------------------------------------------------------------

def test_e4m3_decode_matches_torch_and_the_fp16_route(orc):
    table = orc.e4m3_table()
    # torch's float8_e4m3fn (an independent decoder): every code, NaN at 0x7F / 0xFF only.
    assert bitwise_equal(table, e4m3_torch_table()) == 0
    assert [c for c in range(256) if np.isnan(table[c])] == [0x7F, 0xFF]
    # The reference's own route (Widen.swift:283-313): the bits moved into an fp16, read ×256.
    codes = np.arange(256, dtype=np.uint16)
    half = (((codes & 0x80) << 8) | ((codes & 0x7F) << 7)).astype(np.uint16).view(np.float16)
    via16 = half.astype(np.float32) * np.float32(256)
    via16[(codes & 0x7F) == 0x7F] = np.nan
    assert bitwise_equal(table, via16) == 0


def test_e4m3_quantizer_round_trips_and_rounds_to_even(orc):
    table = orc.e4m3_table()
    finite = [c for c in range(256) if not np.isnan(table[c])]
    # Every finite code is a fixed point (−0 included).
    assert np.array_equal(orc.f32_to_e4m3(table[finite]), np.array(finite, dtype=np.uint8))
    # Midpoints go to the even code; values past 448 saturate; agree with torch below 448.
    x = np.array([1.0625, 1.1875, 0.0009765625, 0.0029296875, 464.0, -1000.0, 447.9], dtype=np.float32)
    assert list(orc.f32_to_e4m3(x)) == [0x38, 0x3A, 0x00, 0x02, 0x7E, 0xFE, 0x7E]
    r = np.random.default_rng(0).normal(0, 100, 5000).astype(np.float32)
    r = r[np.abs(r) < 448]
    t = torch.from_numpy(r).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(orc.f32_to_e4m3(r), t)


def test_bf16_rounding_matches_torch(orc):
    with open(os.path.join(GOLDEN, "bf16_rne.json")) as f:
        d = json.load(f)
    x = np.array([int(v, 16) for v in d["f32_bits"]], dtype=np.uint32).view(np.float32)
    want = np.array([int(v, 16) for v in d["bf16_bits"]], dtype=np.uint16)
    assert np.array_equal(orc.f32_to_bf16(x), want)                      # numpy restatement
    assert np.array_equal(np.array([orc.lib().orc_f32_to_bf16(float(v)) for v in x], dtype=np.uint16), want)


def test_bf16_nan_rule(orc):
    # TensorGEMMBF16.swift:45: a NaN keeps its sign and payload, quiet bit set.
    x = np.array([0x7F800001, 0xFF800001, 0x7FC00000, 0x7FFFFFFF], dtype=np.uint32).view(np.float32)
    assert list(orc.f32_to_bf16(x)) == [0x7FC0, 0xFFC0, 0x7FC0, 0x7FFF]


def test_bf16_widen_specials_and_round_trip(orc):
    # Sources/Verification/KernelStages.swift:24-31, 39-46.
    cases = [(0x0000, 0x00000000), (0x8000, 0x80000000), (0x3F80, 0x3F800000), (0xBF80, 0xBF800000),
             (0x4049, 0x40490000), (0x7F80, 0x7F800000), (0xFF80, 0xFF800000), (0x7F7F, 0x7F7F0000),
             (0x0080, 0x00800000), (0x0001, 0x00010000)]
    got = orc.bf16_to_f32(np.array([c[0] for c in cases], dtype=np.uint16)).view(np.uint32)
    assert list(got) == [c[1] for c in cases]
    assert float(orc.bf16_to_f32(np.array([0x4049], dtype=np.uint16))[0]) == 3.140625
    src = ((np.arange(4096, dtype=np.uint64) * 2654435761) & 0x7F7F0000).astype(np.uint32).view(np.float32)
    assert np.array_equal(orc.bf16_to_f32(orc.f32_to_bf16(src)).view(np.uint32), src.view(np.uint32))


# ---- the dequantiser: Tests/SiliconedTests/DequantizeTests.swift:79-133 ----------------------------

@pytest.mark.parametrize("fp8", [False, True])
def test_dequantize_column_scales(orc, fp8):
    g = DequantizeGen()
    k, n = 300, 500
    q = g.codes(k * n)
    for kind in ["bf16", "f32"]:
        raw, s = g.scales(n, kind)
        st = orc.BF16 if kind == "bf16" else orc.F32
        got = orc.dequantize(q, orc.FP8_E4M3 if fp8 else orc.INT8, raw, st, orc.SCALE_COLUMNS, columns=n)
        want = code_values(q, fp8) * np.tile(s, k)
        assert bitwise_equal(got, want) == 0
        one = orc.dequantize(q[:n], orc.FP8_E4M3 if fp8 else orc.INT8, raw, st, orc.SCALE_COLUMNS, columns=n)
        assert bitwise_equal(one, code_values(q[:n], fp8) * s) == 0


def test_dequantize_tensor_scale_and_plain_cast(orc):
    g = DequantizeGen()
    count = 140_001
    q = g.codes(count)
    raw, s = g.scales(4, "f32")
    for fp8 in [False, True]:
        kind = orc.FP8_E4M3 if fp8 else orc.INT8
        got = orc.dequantize(q, kind, raw[:1], orc.F32, orc.SCALE_TENSOR)
        assert bitwise_equal(got, code_values(q, fp8) * s[0]) == 0
    assert bitwise_equal(orc.dequantize(q, orc.FP8_E4M3, None), code_values(q, True)) == 0


def test_dequantize_block_scales_from_mid_block(orc):
    g = DequantizeGen()
    k, n, b = 100, 2052, 32
    q = g.codes(k * n)
    for kind, st in [("f16", orc.F16), ("bf16", orc.BF16), ("f32", orc.F32)]:
        raw, s = g.scales((k + b - 1) // b * n, kind)
        for fp8 in [False, True]:
            wk = orc.FP8_E4M3 if fp8 else orc.INT8
            got = orc.dequantize(q, wk, raw, st, orc.SCALE_BLOCKS, columns=n, block_rows=b)
            idx = np.arange(k * n)
            want = code_values(q, fp8) * s[(idx // n // b) * n + idx % n]
            assert bitwise_equal(got, want) == 0
            first, rows = 45, 50
            got = orc.dequantize(q[first * n:(first + rows) * n], wk, raw, st, orc.SCALE_BLOCKS, columns=n,
                                 block_rows=b, first_row=first)
            idx = np.arange(rows * n)
            want = code_values(q[first * n:(first + rows) * n], fp8) * s[((first + idx // n) // b) * n + idx % n]
            assert bitwise_equal(got, want) == 0


def test_dequantize_row_scales(orc):
    g = DequantizeGen()
    rows, k = 250, 600
    q = g.codes(rows * k)
    raw, s = g.scales(rows + 7, "bf16")
    got = orc.dequantize(q, orc.INT8, raw, orc.BF16, orc.SCALE_ROWS, columns=k, first_row=7)
    want = code_values(q, False) * s[7 + np.arange(rows * k) // k]
    assert bitwise_equal(got, want) == 0


def test_dequantize_is_one_rounding_not_fused(orc):
    # A fused or double-rounded product would differ from numpy's single multiply somewhere here.
    q = np.arange(-128, 128, dtype=np.int8)
    s = np.float32(0.0123456789)
    got = orc.dequantize(q.view(np.uint8), orc.INT8, np.array([s]), orc.F32, orc.SCALE_TENSOR)
    assert bitwise_equal(got, q.astype(np.float32) * s) == 0
    assert bitwise_equal(got, (q.astype(np.float64) * np.float64(s)).astype(np.float32)) == 0


# ---- the truth and its judge -----------------------------------------------------------------------

def _tiny():
    d = np.load(os.path.join(GOLDEN, "tiny_products.npz"))
    for i in range(4):
        yield i, d[f"a_bf16_{i}"], d[f"q_{i}"], d[f"s_{i}"], d[f"b_{i}"], d


def test_exact_rows_match_float64_products(orc):
    for i, a, q, s, b, d in _tiny():
        m, k = a.shape
        n = q.shape[0]
        rows = np.arange(m, dtype=np.int32)
        # [N, K] and [K, N] layouts; scale after the sum; bias; bitwise in float64 (every sum exact).
        y = orc.exact_rows(rows, a, q.astype(np.float32), False, k, n, scale=s, bias=b)
        assert np.array_equal(y, d[f"y_none_{i}"])
        y = orc.exact_rows(rows, a, np.ascontiguousarray(q.T).astype(np.float32), True, k, n, scale=s, bias=b)
        assert np.array_equal(y, d[f"y_none_{i}"])
        g = orc.exact_rows(rows, a, q.astype(np.float32), False, k, n, scale=s, bias=b, epilogue=orc.EPI_GELU_TANH)
        np.testing.assert_allclose(g, d[f"y_gelu_{i}"], rtol=1e-14, atol=1e-300)
        h = orc.exact_rows(rows, a, q.astype(np.float32), False, k, n, scale=s, bias=b, epilogue=orc.EPI_SILU_GLU)
        np.testing.assert_allclose(h, d[f"y_silu_glu_{i}"], rtol=1e-14, atol=1e-300)


def test_exact_rows_sampled_are_those_rows(orc):
    m, k, n = 300, 40, 24
    a = orc.normal_bf16(3, (m, k))
    q = orc.uniform_i8(4, (n, k)).astype(np.float32)
    full = orc.exact_rows(np.arange(m, dtype=np.int32), a, q, False, k, n)
    rows = orc.sample_rows(m, 64)
    assert np.array_equal(orc.exact_rows(rows, a, q, False, k, n), full[rows])


def test_sample_rows_visit_every_slice(orc):
    for m, c in [(4096, 64), (65, 64), (64, 64), (1000, 7)]:
        r = orc.sample_rows(m, c)
        assert len(r) == c and np.all(np.diff(r) > 0)
        for i, row in enumerate(r):
            assert i * m // c <= row < (i + 1) * m // c + (1 if (i + 1) * m % c else 0)


def test_situ_closed_forms(orc):
    f = orc.lib().orc_situ
    assert f(3.0, 0.0) == 0.0 and f(0.0, 2.0) == 0.0
    assert math.isclose(f(7.0, 80.0), 4 * 25 * math.tanh(7 / 25), rel_tol=1e-15)  # σ(g) → 1, tanh(g/4) → 1
    assert f(-2.5, 1.5) == -f(2.5, 1.5)
    assert math.isclose(f(1.0, 1.0), 4 * math.tanh(0.25) / (1 + math.exp(-1)) * 25 * math.tanh(0.04), rel_tol=1e-15)


def test_activations_match_torch_float64(orc):
    x = torch.linspace(-12, 12, 4001, dtype=torch.float64)
    g = np.array([orc.lib().orc_gelu_tanh(float(v)) for v in x])
    np.testing.assert_allclose(g, torch.nn.functional.gelu(x, approximate="tanh").numpy(), rtol=1e-13, atol=1e-15)
    s = np.array([orc.lib().orc_silu_glu(float(v), 1.5) for v in x])
    np.testing.assert_allclose(s, (torch.nn.functional.silu(x) * 1.5).numpy(), rtol=1e-13, atol=1e-15)


def test_channel_error_closed_forms(orc):
    rng = np.random.default_rng(1)
    e = rng.normal(size=(64, 50))
    # got = e·(1 + ε) on every value: each channel's error is exactly ε.
    worst, _, med = orc.channel_error((e * (1 + 1e-3)).astype(np.float32), e)
    assert abs(worst - 1e-3) < 1e-6 and abs(med - 1e-3) < 1e-6
    # One channel off by 10 %: it is the worst one, at 0.1.
    g = e.copy()
    g[:, 17] *= 1.1
    worst, ch, _ = orc.channel_error(g.astype(np.float32), e)
    assert ch == 17 and abs(worst - 0.1) < 1e-6
    # A NaN is infinite error (DiagnosticJudgement.swift:58-65).
    g = e.copy()
    g[3, 5] = np.nan
    assert orc.channel_error(g.astype(np.float32), e)[0] == math.inf
    # A near-silent channel is floored at 1 % of the median norm: absolute 1e-6 on a 1e-9 column.
    e2 = e.copy()
    e2[:, 9] = 1e-9
    g = e2.copy()
    g[:, 9] += 1e-6
    norms = np.sort(np.sqrt((e2 ** 2).sum(axis=0)))
    med_norm = norms[len(norms) // 2]  # the upper median, as the reference indexes count / 2
    worst, ch, _ = orc.channel_error(g.astype(np.float32), e2)
    assert ch == 9 and abs(worst - np.sqrt(64) * 1e-6 / (0.01 * med_norm)) / worst < 1e-3


# ---- the CPU route (the timed baseline) ------------------------------------------------------------

@pytest.mark.parametrize("epi", ["none", "gelu", "silu"])
def test_linear_f32_is_the_fp32_product(orc, epi):
    m, k, n = 37, 300, 64
    a = orc.normal_bf16(8, (m, k))
    q = orc.uniform_i8(9, (n, k))
    s = orc.uniform_f32(10, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(11, (n,), 0, 0.02)
    w_kn = orc.dequantize(np.ascontiguousarray(q.T).view(np.uint8), orc.INT8, s, orc.F32, orc.SCALE_COLUMNS, columns=n)
    e = {"none": orc.EPI_NONE, "gelu": orc.EPI_GELU_TANH, "silu": orc.EPI_SILU_GLU}[epi]
    c = orc.linear_f32(a, w_kn, bias=b, epilogue=e, threads=4)
    exact = orc.exact_rows(np.arange(m, dtype=np.int32), a, q.astype(np.float32), False, k, n, scale=s, bias=b, epilogue=e)
    assert orc.channel_error(c, exact)[0] < 1e-5  # the reference's fp32 bar (Diagnostic.swift:105)
    # And numpy's float32 BLAS on the same widened operands agrees to fp32 accuracy.
    p = orc.bf16_to_f32(a) @ w_kn
    ref = orc.epilogue_f32(p, bias=b, epilogue=e, threads=2)
    np.testing.assert_allclose(c, ref, rtol=2e-4, atol=2e-5)
