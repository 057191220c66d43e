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
        # The fixture is torch's float64 ½x(1 + tanh u), whose 1 + tanh u cancels for negative x: its own
        # error there is a few units of 2⁻⁵³ times ½|x|, which bounds the difference beside 1e-14 relative.
        pre = d[f"y_none_{i}"]
        assert np.all(np.abs(g - d[f"y_gelu_{i}"]) <= 1e-14 * np.abs(d[f"y_gelu_{i}"]) + 4 * 2.0 ** -53 * 0.5 * np.abs(pre))
        h = orc.exact_rows(rows, a, q.astype(np.float32), False, k, n, scale=s, bias=b, epilogue=orc.EPI_SILU_GLU)
        np.testing.assert_allclose(h, d[f"y_silu_glu_{i}"], rtol=1e-14, atol=1e-300)


def test_exact_rows_sampled_are_those_rows(orc):
    m, k, n = 300, 40, 24
    a = orc.normal_bf16(3, (m, k))
    q = orc.uniform_i8(4, (n, k)).astype(np.float32)
    full = orc.exact_rows(np.arange(m, dtype=np.int32), a, q, False, k, n)
    rows = orc.sample_rows(m, 64)
    assert np.array_equal(orc.exact_rows(rows, a, q, False, k, n), full[rows])


def test_exact_rows_of_an_fp32_activation(orc):
    """The truth on fp32 A taken whole (DiagnosticProbes.swift:79-84 widens A to double): against numpy's
    float64 product (each term exact, sums within a few ulp of double), and on fp32 values that are bf16
    values, the same doubles as the bf16 truth."""
    m, k, n = 40, 96, 24
    a = orc.normal_f32(8, (m, k))
    q = orc.uniform_i8(9, (n, k)).astype(np.float32)
    s = orc.uniform_f32(10, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(11, (n,), 0.0, 0.02)
    rows = np.arange(m, dtype=np.int32)
    y = orc.exact_rows(rows, a, q, False, k, n, scale=s, bias=b)
    want = (a.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64) + b.astype(np.float64)
    np.testing.assert_allclose(y, want, rtol=1e-13, atol=1e-15)
    assert np.abs(y - orc.exact_rows(rows, orc.f32_to_bf16(a), q, False, k, n, scale=s, bias=b)).max() > 1e-4
    bits = orc.f32_to_bf16(a)
    assert np.array_equal(orc.exact_rows(rows, orc.bf16_to_f32(bits), q, False, k, n, scale=s, bias=b),
                          orc.exact_rows(rows, bits, q, False, k, n, scale=s, bias=b))


def _parts(x):
    """hi, mid, lo: each the top 16 bits of what the part before leaves (truncation, no rounding)."""
    top = lambda v: (v.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    hi = top(x)
    r1 = (x - hi).astype(np.float32)
    mid = top(r1)
    r2 = (r1 - mid).astype(np.float32)
    return hi, mid, top(r2), r1, r2


def test_three_bf16_parts_are_exact():
    """The fp32 route's operand: three bf16 parts whose sum is x exactly (24 significant bits in three
    parts of 8): every fp32 difference exact, the last remainder already a bf16 value, every part a
    normal number for |x| ≥ 2^−103, and fp32's largest values kept (rounding hi to nearest would
    carry 3.4e38 to infinity)."""
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32),
                        (rng.standard_normal(20000) * 2.0 ** rng.integers(-103, 127, 20000)).astype(np.float32),
                        np.float32([1 + 2 ** -23, -(1 - 2 ** -24), 2 ** -103, 3.4028235e38, -3.4e38, 0.0])])
    x = x[np.isfinite(x)]
    hi, mid, lo, r1, r2 = _parts(x)
    d = lambda v: v.astype(np.float64)
    assert np.array_equal(d(r1), d(x) - d(hi)) and np.array_equal(d(r2), d(r1) - d(mid))
    assert np.array_equal(lo, r2)                            # the remainder is a bf16 value already
    assert np.array_equal(d(hi) + d(mid) + d(lo), d(x))
    tiny, big_enough = np.finfo(np.float32).tiny, np.abs(x) >= 2.0 ** -103
    assert (~big_enough).sum() > 10                          # the draw reaches below the bound too
    for part in (mid, lo):
        nz = part[big_enough & (part != 0)]
        assert (np.abs(nz) >= tiny).all()                    # no subnormal part for |x| ≥ 2^−103
    assert np.isfinite(hi).all()
    # Rounded to nearest even instead, fp32's largest value would carry into infinity.
    u = np.uint32(np.float32(3.4028235e38).view(np.uint32))
    rne = np.uint32((int(u) + 0x7FFF + ((int(u) >> 16) & 1)) & 0xFFFF0000).view(np.float32)
    assert np.isinf(rne) and np.isfinite(_parts(np.float32([3.4028235e38]))[0]).all()


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


def _gelu_tanh_decimal(x: float) -> float:
    """½x(1 + tanh u), u = √(2/π)(x + 0.044715x³), the reference's formula evaluated in 420-digit
    decimal arithmetic (tanh u = (e^(2u) − 1)/(e^(2u) + 1)): 1 + tanh u keeps more than 60 digits down
    to e^(2u) = 10⁻³⁵⁰, past double's range."""
    import decimal
    with decimal.localcontext() as c:
        c.prec = 420
        pi = decimal.Decimal("3.14159265358979323846264338327950288419716939937510582097494")
        d = decimal.Decimal(x)
        u = (decimal.Decimal(2) / pi).sqrt() * (d + decimal.Decimal("0.044715") * d * d * d)
        e = (2 * u).exp()
        return float(decimal.Decimal("0.5") * d * (1 + (e - 1) / (e + 1)))


def test_activations_match_torch_float64(orc):
    x = torch.linspace(-12, 12, 4001, dtype=torch.float64)
    g = np.array([orc.lib().orc_gelu_tanh(float(v)) for v in x])
    np.testing.assert_allclose(g, torch.nn.functional.gelu(x, approximate="tanh").numpy(), rtol=1e-13, atol=1e-15)
    s = np.array([orc.lib().orc_silu_glu(float(v), 1.5) for v in x])
    np.testing.assert_allclose(s, (torch.nn.functional.silu(x) * 1.5).numpy(), rtol=1e-13, atol=1e-15)


def test_gelu_truth_holds_in_the_tail(orc):
    # Relative accuracy on [−30, 12] against the reference's formula in 420-digit arithmetic: the truth
    # keeps its relative precision where the double form ½x(1 + tanh u) cancels to −0 (x ≤ −8), down to
    # values below double's normal range (x < −21: e^(2u) < 10⁻³⁰⁸), where both are below 1e-300.
    xs = np.concatenate([np.linspace(-30, 12, 2101), [-8.0, -9.5, -10.0, -20.0]])
    got = np.array([orc.lib().orc_gelu_tanh(float(v)) for v in xs])
    want = np.array([_gelu_tanh_decimal(float(v)) for v in xs])
    # e^(−2u) carries the relative rounding of its argument times |2u| (the function's own conditioning).
    u = math.sqrt(2 / math.pi) * (xs + 0.044715 * xs ** 3)
    assert np.all(np.abs(got - want) <= 1e-15 * (1 + 2 * np.abs(u)) * np.abs(want) + 1e-300)
    assert np.all(np.signbit(got[xs < 0])) and np.all(got[(xs < 0) & (xs > -21)] < 0)
    # The double literal form gives −0 at −8; the value there is a normal number, about x·e^(2u).
    x = -8.0
    u = math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)
    assert 0.5 * x * (1 + math.tanh(u)) == 0.0
    assert math.isclose(orc.lib().orc_gelu_tanh(x), x * math.exp(2 * u), rel_tol=1e-15)
    assert -4e-21 < orc.lib().orc_gelu_tanh(x) < -2e-21


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


# ---- convrot: Sources/Siliconed/Widen.swift:316-428, TensorGEMM.swift:181-201 ----------------------

H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)


def hadamard(g: int) -> np.ndarray:
    """The unnormalized rotation of a group, built independently of the oracle's butterflies: the
    Kronecker power of the regular H4 (Widen.swift:319-323)."""
    h = np.ones((1, 1))
    while h.shape[0] < g:
        h = np.kron(h, H4)
    return h


def test_rotation_groups_and_the_matrix(orc):
    # A power of 4 from 4 to 256, nothing else; H symmetric with H·H = G·I (R = H/√G orthogonal).
    assert [g for g in range(0, 1100) if orc.is_rotation_group(g)] == [4, 16, 64, 256]
    for g in (4, 16, 64, 256):
        h = hadamard(g)
        assert np.array_equal(h, h.T) and np.array_equal(h @ h, g * np.eye(g))
        assert float(orc.lib().orc_rotation_norm(g)) == 1 / math.sqrt(g)


def _bf16_scales(orc, n, rng):
    s = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    b = orc.f32_to_bf16(s)
    return b, orc.bf16_to_f32(b)


@pytest.mark.parametrize("g,k,n", [(256, 768, 328), (256, 256, 12), (64, 192, 136), (16, 64, 40), (4, 8, 20),
                                   (16, 32, 8200), (4, 8, 4100)])
def test_dequantize_rotated_is_the_exact_hadamard_product(orc, g, k, n):
    # DequantizeTests.swift:179-211, same shapes: Float(H·q)·(s/√G) at the bit, H·q as an fp64 matrix
    # product of the Kronecker-built H (integers under 2^53: exact), the extremes of m in columns 0
    # and 1 (±127/−128 following H's first row), bf16 and fp32 scales per column, one fp32 scale for
    # the tensor. Catches a wrong sign or digit in the butterflies, a scale applied before the sum,
    # a missing 1/√G, a transposed walk of the [k, n] codes.
    rng = np.random.default_rng(g * 7 + k + n)
    q = rng.integers(-128, 128, (k, n)).astype(np.int8)
    h = hadamard(g)
    q[:g, 0] = np.where(h[0] > 0, 127, -128)
    q[:g, 1] = np.where(h[0] > 0, -128, 127)
    m = np.concatenate([h @ q[g0:g0 + g].astype(np.float64) for g0 in range(0, k, g)])
    assert np.abs(m).max() <= 32648
    norm = np.float32(1 / math.sqrt(g))
    bits, sb = _bf16_scales(orc, n, rng)
    sf = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    for scale, stype, layout, s32 in ((bits, orc.BF16, orc.SCALE_COLUMNS, sb), (sf, orc.F32, orc.SCALE_COLUMNS, sf),
                                      (sf[:1], orc.F32, orc.SCALE_TENSOR, np.full(n, sf[0], np.float32))):
        got = orc.dequantize_rotated(q, g, scale, stype, layout)
        expected = m.astype(np.float32) * (s32 * norm)
        assert bitwise_equal(got, expected) == 0, (g, k, n, stype, layout)


def test_dequantize_rotated_extreme_columns_reach_the_bound(orc):
    # H's rows sum to +16 at G = 256: 136 plus and 120 minus signs. Codes following the first row
    # give m = 136·127 + 120·128 = 32 632; the opposite signs (−128 on the plus) give −(136·128 +
    # 120·127) = −32 648, the Int16 bound the reference states (Widen.swift:327-329).
    g = 256
    h = hadamard(g)
    assert (h[0] > 0).sum() == 136 and h.sum(axis=1).tolist() == [16.0] * g
    q = np.zeros((g, 4), np.int8)
    q[:, 0] = np.where(h[0] > 0, 127, -128)
    q[:, 1] = np.where(h[0] > 0, -128, 127)
    out = orc.dequantize_rotated(q, g, np.ones(4, np.float32) * 16, orc.F32)
    assert out[0, 0] == 32632.0 and out[0, 1] == -32648.0


@pytest.mark.parametrize("g", [4, 16, 64, 256])
def test_rotate_groups_is_the_exact_product_on_integers(orc, g):
    # Integers |x| ≤ 1024: every partial sum (≤ 2^18) is exact in fp32, so the rotation must equal
    # x·H/√G from the Kronecker-built H whatever the order of the sums. Catches a wrong sign, a wrong
    # span-to-digit mapping, a transposed group, a missing norm, groups that straddle rows.
    rng = np.random.default_rng(g)
    k = 3 * 256
    x = rng.integers(-1024, 1025, (5, k)).astype(np.float32)
    h = hadamard(g)
    expected = np.concatenate([x[:, g0:g0 + g].astype(np.float64) @ h for g0 in range(0, k, g)], axis=1) / math.sqrt(g)
    assert np.array_equal(orc.rotate_groups(x, g).astype(np.float64), expected)


def test_rotate_groups_rounds_the_pairwise_sums(orc):
    # Known answers worked by hand, fp32 round-to-nearest-even (ulp 2 at 2^24):
    # (2^24, 1, −2^24, 1): p = 2^24+1 → 2^24 (tie), m = 2^24−1, u = −(2^24−1), w = −2^24−1 → −2^24;
    #   out = (p+w, p−w, m+u, u−m)/2 = (0, 2^25, 0, −(2^25−2))/2. Left-to-right a+b+c−d gives −1 first.
    # (2^24, 1, 1, 0): p → 2^24, m = 2^24−1, u = w = 1: p+w = 2^24+1 → 2^24 (the correctly rounded
    #   a+b+c−d is 2^24+2), p−w = 2^24−1, m+u = 2^24, u−m = −(2^24−2).
    T = 2.0 ** 24
    for x, y in (((T, 1, -T, 1), (0, T, 0, -(T - 1))), ((T, 1, 1, 0), (T / 2, (T - 1) / 2, T / 2, -(T - 2) / 2))):
        got = orc.rotate_groups(np.array([x], np.float32), 4)[0]
        assert np.array_equal(got.astype(np.float64), np.array(y)), (x, got)


def test_rotate_groups_runs_span_one_first(orc):
    # G = 16, x0 = 2^24, x1 = x4 = 1 (by hand). Span 1 first: quad 0 → (2^24, 2^24, 2^24−1, −(2^24−1))
    # (the tie drops the 1), quad 1 → (1, 1, 1, −1); then span 4 per column j: j = 2 adds 2^24−1 and
    # 1 exactly → out[2] = 2^24. Span 4 first would give out[2] = 2^24−1. All over √16 = 4.
    T = 2.0 ** 24
    x = np.zeros((1, 16), np.float32)
    x[0, 0], x[0, 1], x[0, 4] = T, 1, 1
    y = np.array([T, T, T, -T, T, T, T, -T, T - 1, T - 1, T - 2, -(T - 2), -(T - 1), -(T - 1), -(T - 2), T - 2]) / 4
    assert np.array_equal(orc.rotate_groups(x, 16)[0].astype(np.float64), y)


def test_rotate_groups_is_its_own_inverse_within_rounding(orc):
    # R = H/√G is symmetric and orthogonal: R·R = I. Two rotations give x back to within the fp32
    # roundings of 2·log4(G) butterfly stages (each a sum of two rounded sums).
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((7, 1024)) * 3).astype(np.float32)
    for g in (4, 16, 64, 256):
        back = orc.rotate_groups(orc.rotate_groups(x, g), g)
        stages = 2 * int(round(math.log(g, 4)))
        assert np.abs(back - x).max() <= 4 * stages * 2.0 ** -24 * np.abs(x).max() * math.sqrt(g) / 4 + 1e-6
        assert np.abs(back - x).max() > 0 or g == 4


# ---- W8A8: Sources/Siliconed/TensorGEMMInt8.swift:4-37, 198-221 ------------------------------------

def test_quantize_rows_rounds_half_to_even(orc):
    # max|y| = 127 → scale exactly 1: the codes are rint of the values themselves, half to even
    # (torch.round, not half away from zero: 2.5 → 2, −0.5 → 0, 63.5 → 64).
    x = np.array([[127.0, 63.5, -0.5, 1.5, 2.5, 0.0, -126.5, 3.49]], np.float32)
    codes, scales = orc.quantize_rows(x)
    assert scales[0] == 1.0
    assert codes[0].tolist() == [127, 64, 0, 2, 2, 0, -126, 3]


def test_quantize_rows_divides_correctly(orc):
    # Found by search and checked with numpy's IEEE division: s = m/127 correctly rounded, and
    # y/s correctly rounded before rint — a reciprocal's product (y·(1/s)) gives 97 here, the
    # division 96; and m·(1/127) is not m/127 for m = 0.6864249110221863.
    m, y = np.float32(2.166764259338379), np.float32(1.646399736404419)
    codes, scales = orc.quantize_rows(np.array([[m, y, -y]], np.float32))
    s = np.float32(m / np.float32(127))
    assert scales[0] == s and codes[0].tolist() == [127, 96, -96]
    assert np.rint(np.float32(y * np.float32(np.float32(1) / s))) == 97
    m2 = np.float32(0.6864249110221863)
    _, s2 = orc.quantize_rows(np.array([[m2]], np.float32))
    assert s2[0] == np.float32(m2 / np.float32(127)) != np.float32(m2 * (np.float32(1) / np.float32(127)))


def test_quantize_rows_floor_and_extremes(orc):
    # A row of zeros takes the floor scale 1e-30 (codes 0); the largest value maps to ±127 exactly
    # and no code leaves [−127, 127] although the clamp allows −128.
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((6, 520)) * 4).astype(np.float32)
    x[2] = 0
    x[4, 17] = -300.0
    codes, scales = orc.quantize_rows(x)
    assert scales[2] == np.float32(1e-30) and not codes[2].any()
    assert codes[4, 17] == -127 and codes.min() >= -127 and codes.max() <= 127
    for r in range(6):
        if r != 2:
            assert np.abs(codes[r]).max() == 127


@pytest.mark.parametrize("g", [0, 16, 64, 256])
def test_quantize_rows_against_numpy(orc, g):
    # The recipe in numpy's own IEEE fp32 operations on the oracle's rotated row (the rotation is
    # pinned above): max, the divide by 127, the 1e-30 floor, the divide, rint, the clamp.
    rng = np.random.default_rng(g + 1)
    x = (rng.standard_normal((9, 768)) * 3).astype(np.float32)
    x[:, 300] *= 300
    y = orc.rotate_groups(x, g) if g else x
    s = np.maximum(np.abs(y).max(axis=1) / np.float32(127), np.float32(1e-30)).astype(np.float32)
    q = np.clip(np.rint(y / s[:, None]), -128, 127).astype(np.int8)
    codes, scales = orc.quantize_rows(x, g)
    assert np.array_equal(scales, s) and np.array_equal(codes, q)


def test_w8a8_product_is_exact_then_scaled(orc):
    # int64 numpy products (exact); the fp32 conversion of a sum past 2^24 rounds half to even;
    # the scale product s_x·s_w is formed first: with acc = −284410, s_x = 0.05983570218086243,
    # s_w = 0.007420313078910112 (found by search), (acc·s_x)·s_w differs from acc·(s_x·s_w).
    rng = np.random.default_rng(9)
    m, k, n = 7, 1100, 13
    codes = rng.integers(-127, 128, (m, k)).astype(np.int8)
    w = rng.integers(-127, 128, (k, n)).astype(np.int8)
    codes[0] = 127
    codes[0, 0] = 126
    w[:, 0] = 127                               # acc = 1100·16129 − 127 = 17 741 773: odd, past 2^24
    sx = rng.uniform(1e-3, 1e-1, m).astype(np.float32)
    sw = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    acc = codes.astype(np.int64) @ w.astype(np.int64)
    expected = acc.astype(np.float32) * (sx[:, None] * sw[None, :]).astype(np.float32)
    got = orc.w8a8_product(codes, sx, w, True, sw)
    assert bitwise_equal(got, expected) == 0
    assert np.array_equal(orc.w8a8_product(codes, sx, np.ascontiguousarray(w.T), False, sw), got)
    assert acc[0, 0] == 17741773 and float(np.float32(acc[0, 0])) == 17741772.0   # the tie goes to the even
    one = orc.w8a8_product(np.array([[1]], np.int8), np.array([0.05983570218086243], np.float32),
                           np.array([[1]], np.int8), True, np.array([0.007420313078910112], np.float32))
    f = np.float32
    a = f(-284410.0) * one[0, 0]
    assert a == f(-284410.0) * f(f(0.05983570218086243) * f(0.007420313078910112))
    assert a != f(f(f(-284410.0) * f(0.05983570218086243)) * f(0.007420313078910112))
    t = orc.w8a8_product(codes[:2], sx[:2], w, True, sw[:1])          # one scale for the tensor
    assert bitwise_equal(t, acc[:2].astype(np.float32) * (sx[:2, None] * sw[0]).astype(np.float32)) == 0
