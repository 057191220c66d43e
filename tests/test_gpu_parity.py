"""Parity of the HIP library (through its C ABI) with the CPU oracle, on an MI355X.

Bars (the reference's own, Sources/Siliconed/Diagnostic.swift:105-107,
CapacityProbes.swift:541-553): per-channel relative error (DiagnosticJudgement.swift:39-71) against
the fp64 truth of the same bf16 activations and 8-bit codes ≤ 1e-5 for fp32 outputs, ≤ max(1e-5,
1.25 × the error of the truth itself rounded to bf16) for bf16 outputs; plus, for bf16 outputs,
max elementwise relative error ≤ 2e-2 with the denominator floored at 1 % of the column's RMS.
Dequantised weights and the bf16 rounding pass are compared bit for bit.
"""
import numpy as np
import pytest
import torch

from refgen import DequantizeGen, bitwise_equal, code_values

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPI = {"none": 0, "gelu": 1, "silu": 2, "situ": 3}


def bf16_dev(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def dev(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def problem(orc, m, k, n, fp8, seed, bias=True):
    """bf16 X ~ N(0,1); int8 codes uniform in [−127, 127] with scales U(1e−3, 2e−2), or fp8 codes of
    N(0, 0.02) weights with amax/448 scales; bias N(0, 0.02). Codes laid out [N, K]."""
    x = orc.normal_bf16(seed, (m, k))
    if fp8:
        q, s = orc.quantize_fp8_per_row(orc.normal_f32(seed + 1, (n, k), 0.0, 0.02))
    else:
        q = orc.uniform_i8(seed + 1, (n, k)).view(np.uint8)
        s = orc.uniform_f32(seed + 2, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(seed + 3, (n,), 0.0, 0.02) if bias else None
    return x, q, s, b


def weight_tensor(q: np.ndarray, fp8: bool, layout: str) -> torch.Tensor:
    w = q if layout == "nk" else np.ascontiguousarray(q.T)
    t = dev(w)
    return t.view(torch.float8_e4m3fn) if fp8 else t.view(torch.int8)


def judge(orc, got, x, q, fp8, s, b, epi, out_dtype, rows=None, values=False):
    """`q`: codes [N, K] (widened here), or with `values` the weight's fp32 values [N, K]."""
    m, k = x.shape
    n = q.shape[0]
    rows = np.arange(m, dtype=np.int32) if rows is None else rows
    wf = q if values else code_values(q, fp8)
    exact = orc.exact_rows(rows, x, wf, False, k, n, scale=s, bias=b, epilogue=EPI[epi])
    g = got[rows]
    assert np.isfinite(g).all(), "non-finite outputs"
    err, ch, _ = orc.channel_error(g, exact)
    if out_dtype == torch.bfloat16:
        floor = orc.channel_error(orc.bf16_to_f32(orc.f32_to_bf16(exact.astype(np.float32))), exact)[0]
        bar = max(1e-5, 1.25 * floor)
        rms = np.sqrt((exact ** 2).mean(axis=0)) + 1e-30
        rel = np.abs(g - exact) / np.maximum(np.abs(exact), 0.01 * rms)
        assert rel.max() <= 2e-2, f"max relative error {rel.max():.3e}"
    else:
        bar = 1e-5
    assert err <= bar, f"channelError {err:.3e} > {bar:.3e} (channel {ch})"
    return err


def run(gemm, x, q, s, b, fp8, layout, epi, out_dtype):
    w = weight_tensor(q, fp8, layout)
    y = gemm.product(bf16_dev(x), w, dev(s), layout=layout, bias=None if b is None else dev(b),
                     epilogue=None if epi == "none" else {"gelu": "gelu_tanh", "silu": "silu_glu", "situ": "situ_glu"}[epi],
                     out_dtype=out_dtype)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


# ---- conversions on the device, bit for bit ------------------------------------------------------

def test_fp8_codes_widen_exactly(gemm, orc):
    codes = np.arange(256, dtype=np.uint8).reshape(1, 256)
    got = gemm.dequantize(dev(codes), None, fp8=True).cpu().numpy()
    assert bitwise_equal(got, orc.e4m3_table().reshape(1, 256)) == 0
    assert bitwise_equal(got, code_values(codes, True)) == 0


def test_int8_codes_widen_exactly(gemm):
    codes = np.arange(256, dtype=np.uint8).reshape(1, 256)
    got = gemm.dequantize(dev(codes).view(torch.int8), None).cpu().numpy()
    assert bitwise_equal(got, codes.view(np.int8).astype(np.float32)) == 0


@pytest.mark.parametrize("fp8", [False, True])
def test_dequantize_reference_vectors(gemm, fp8):
    """DequantizeTests.swift:79-133 on the device: columns, tensor, blocks (mid-block), rows."""
    from siliconed_amd import abi
    g = DequantizeGen()
    view = (lambda t: t) if fp8 else (lambda t: t.view(torch.int8))
    k, n = 300, 500
    q = g.codes(k * n).reshape(k, n)
    for kind, dt in [("bf16", torch.bfloat16), ("f32", torch.float32), ("f16", torch.float16)]:
        raw, s = g.scales(n, kind)
        sd = dev(raw.view(np.int16)).view(dt) if kind != "f32" else dev(raw)
        got = gemm.dequantize(view(dev(q)), sd, layout=abi.SCALE_COLUMNS, fp8=fp8 or None).cpu().numpy()
        assert bitwise_equal(got, code_values(q, fp8) * s[None, :]) == 0
    raw, s = g.scales(4, "f32")
    got = gemm.dequantize(view(dev(q)), dev(raw[:1]), layout=abi.SCALE_TENSOR, fp8=fp8 or None).cpu().numpy()
    assert bitwise_equal(got, code_values(q, fp8) * s[0]) == 0
    kb, nb, b = 100, 2052, 32
    qb = g.codes(kb * nb).reshape(kb, nb)
    raw, s = g.scales((kb + b - 1) // b * nb, "bf16")
    sd = dev(raw.view(np.int16)).view(torch.bfloat16)
    first, rows = 45, 50
    got = gemm.dequantize(view(dev(qb[first:first + rows])), sd, layout=abi.SCALE_BLOCKS, block_rows=b,
                          first_row=first, fp8=fp8 or None).cpu().numpy()
    r = np.arange(rows)[:, None] + first
    want = code_values(qb[first:first + rows], fp8) * s[(r // b) * nb + np.arange(nb)[None, :]]
    assert bitwise_equal(got, want) == 0
    rr, kk = 250, 600
    qr = g.codes(rr * kk).reshape(rr, kk)
    raw, s = g.scales(rr + 7, "bf16")
    sd = dev(raw.view(np.int16)).view(torch.bfloat16)
    got = gemm.dequantize(view(dev(qr)), sd, layout=abi.SCALE_ROWS, first_row=7, fp8=fp8 or None).cpu().numpy()
    assert bitwise_equal(got, code_values(qr, fp8) * s[7:7 + rr, None]) == 0


def test_round_bf16_bits(gemm, orc):
    rng = np.random.default_rng(3)
    u = rng.integers(0, 2 ** 32, size=1 << 16, dtype=np.uint64).astype(np.uint32)
    u[:8] = [0x7F800001, 0xFF800001, 0x7FC00000, 0x7F7FFFFF, 0x3F808000, 0x3F818000, 0x00000001, 0x80000000]
    x = u.view(np.float32)
    got = gemm.round_bf16(dev(x)).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, orc.f32_to_bf16(x))


# ---- the product ---------------------------------------------------------------------------------

SHAPES = [
    (256, 3072, 3072),      # config 0's K and N, rows reduced
    (150, 768, 96),         # the reference's kernel-test shapes (W8A8KernelTests.swift:74-83)
    (70, 10240, 72),
    (65, 448, 130),
    (33, 520, 40),
    (1, 16, 8),
    (300, 200, 1000),
]


@pytest.mark.parametrize("fp8", [False, True], ids=["int8", "fp8"])
@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_product_shapes(gemm, orc, shape, layout, fp8):
    m, k, n = shape
    x, q, s, b = problem(orc, m, k, n, fp8, seed=100 + m + k + n)
    for out in (torch.float32, torch.bfloat16):
        got = run(gemm, x, q, s, b, fp8, layout, "none", out)
        judge(orc, got, x, q, fp8, s, b, "none", out)


@pytest.mark.parametrize("epi", ["gelu", "silu", "situ"])
@pytest.mark.parametrize("fp8", [False, True], ids=["int8", "fp8"])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_product_epilogues(gemm, orc, epi, fp8, layout):
    for m, k, n in [(256, 1024, 768), (65, 448, 130)]:
        x, q, s, b = problem(orc, m, k, n, fp8, seed=7 + n)
        for out in (torch.float32, torch.bfloat16):
            got = run(gemm, x, q, s, b, fp8, layout, epi, out)
            judge(orc, got, x, q, fp8, s, b, epi, out)


def test_zero_row_and_massive_column(gemm, orc):
    # W8A8KernelTests.swift:164-168: a zero row, a ×300 activation column.
    m, k, n = 96, 512, 256
    x, q, s, b = problem(orc, m, k, n, False, seed=5)
    xf = orc.bf16_to_f32(x)
    xf[10, :] = 0.0
    xf[:, 77] *= 300.0
    x = orc.f32_to_bf16(xf)
    got = run(gemm, x, q, s, b, False, "kn", "none", torch.float32)
    assert np.array_equal(got[10], b)  # 0·s + b exactly
    judge(orc, got, x, q, False, s, b, "none", torch.float32)


def test_scale_after_the_sum_and_tensor_scale(gemm, orc):
    m, k, n = 128, 1024, 384
    x, q, s, _ = problem(orc, m, k, n, False, seed=9, bias=False)
    st = np.float32(0.0123)
    w = weight_tensor(q, False, "nk")
    a = gemm.product(bf16_dev(x), w, dev(np.array([st])), layout="nk", out_dtype=torch.float32)
    c = gemm.product(bf16_dev(x), w, dev(np.full(n, st, np.float32)), layout="nk", out_dtype=torch.float32)
    assert torch.equal(a, c)
    # Power-of-two scales commute with the fp32 sum exactly: y(2s) = 2·y(s) bit for bit.
    y1 = gemm.product(bf16_dev(x), w, dev(s), layout="nk", out_dtype=torch.float32)
    y2 = gemm.product(bf16_dev(x), w, dev(2 * s), layout="nk", out_dtype=torch.float32)
    assert torch.equal(2 * y1, y2)


def test_rows_and_columns_are_independent(gemm, orc):
    # Any chunking of rows gives the same rows (WeightProducts.swift:524-528); the first columns of
    # a wider weight are that weight's columns (`submit(…columns:)`, TensorGEMM.swift:296).
    m, k, n = 600, 768, 512
    x, q, s, b = problem(orc, m, k, n, False, seed=11)
    w = weight_tensor(q, False, "kn")
    xt, st, bt = bf16_dev(x), dev(s), dev(b)
    whole = gemm.product(xt, w, st, layout="kn", bias=bt, out_dtype=torch.float32)
    part = gemm.product(xt[123:400], w, st, layout="kn", bias=bt, out_dtype=torch.float32)
    assert torch.equal(part, whole[123:400])
    c = torch.empty((m, n), dtype=torch.float32, device=DEV)
    secs = gemm.linear(xt, int8=w, scales=st, per_column=True, c=c, m=m, k=k, n=n, layout="kn", bias=bt)
    assert secs > 0.0 and torch.equal(c, whole)
    # n = cols with ldw = n of the full weight: the C ABI called directly with the wider stride. A
    # slab-aligned subset runs the same kernel as the whole: the same bits; a ragged one may run
    # another kernel (another order of the fp32 sums): judged against the truth.
    from siliconed_amd import _abi as abi
    for cols in (192, 200):
        c2 = torch.empty((m, cols), dtype=torch.float32, device=DEV)
        st_ = abi.load().sq8_linear(gemm._h, xt.data_ptr(), abi.BF16, k, w.data_ptr(), abi.INT8, abi.KN, n,
                                    st.data_ptr(), abi.SCALE_COLUMNS, bt.data_ptr(), abi.EPI_NONE, c2.data_ptr(),
                                    abi.F32, cols, m, k, cols, None)
        assert st_ == 0
        torch.cuda.synchronize()
        if cols % 64 == 0:
            assert torch.equal(c2, whole[:, :cols])
        judge(orc, c2.cpu().numpy(), x, q[:cols], False, s[:cols], b[:cols], "none", torch.float32)


def test_fp32_activation_is_rounded_first(gemm, orc):
    m, k, n = 200, 640, 320
    x32 = orc.normal_f32(21, (m, k))
    q = orc.uniform_i8(22, (n, k)).view(np.uint8)
    s = orc.uniform_f32(23, (n,), 1e-3, 2e-2)
    w = weight_tensor(q, False, "nk")
    a = gemm.product(dev(x32), w, dev(s), layout="nk", out_dtype=torch.float32)
    r = gemm.product(bf16_dev(orc.f32_to_bf16(x32)), w, dev(s), layout="nk", out_dtype=torch.float32)
    assert torch.equal(a, r)


@pytest.mark.parametrize("head_dim,d", [(0, 512), (128, 512), (48, 240), (0, 200), (40, 200)])
def test_fused_qkv(gemm, orc, head_dim, d):
    # d or head_dim not multiples of 32: a 32-column block straddles two outputs or two heads.
    m, k = 300, 1024
    x, q, s, b = problem(orc, m, k, 3 * d, False, seed=31)
    w = weight_tensor(q, False, "nk")
    whole = gemm.product(bf16_dev(x), w, dev(s), layout="nk", bias=dev(b), out_dtype=torch.bfloat16)
    qq, kk, vv = gemm.product_qkv(bf16_dev(x), w, dev(s), layout="nk", bias=dev(b), head_dim=head_dim)
    for i, t in enumerate((qq, kk, vv)):
        part = whole[:, i * d:(i + 1) * d]
        if head_dim:
            part = part.reshape(m, d // head_dim, head_dim).permute(1, 0, 2)
        assert torch.equal(t, part)


def test_empty_and_refused(gemm):
    from siliconed_amd import abi
    x = torch.zeros((0, 64), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((32, 64), dtype=torch.int8, device=DEV)
    s = torch.ones(32, dtype=torch.float32, device=DEV)
    assert gemm.product(x, w, s).shape == (0, 32)
    with pytest.raises(abi.Unsupported):    # block scales take no rotation (the reference's nil pipeline)
        gemm.linear(x, int8=w, scales=s, per_column=True, c=torch.empty(0, device=DEV), m=0, k=64, n=32, block=32,
                    rotation=4)
    with pytest.raises(ValueError):
        gemm.product(torch.zeros((4, 63), dtype=torch.bfloat16, device=DEV), w, s)


# ---- the baseline's shapes, on sampled rows ----------------------------------------------------

BASELINE_CASES = {
    "c0": (1024, 3072, 3072, False, "none"),             # configs[0] at its full M (64-row tiles)
    "c1_up_gelu": (4096, 3072, 12288, False, "gelu"),
    "c1_down": (4096, 12288, 3072, False, "none"),
    "c2_qkv": (4608, 3072, 9216, False, "none"),
    "c2_text": (512, 3072, 3072, False, "none"),
    "c3_gate_up_fp8": (4096, 3840, 20480, True, "silu"),
    "c3_down_fp8": (4096, 10240, 3840, True, "none"),
    "c3_plain_fp8": (4096, 3840, 12288, True, "none"),   # the plain fp8 W [12288, 3840] of configs[3]
}


@pytest.mark.parametrize("case", ["c0", "c1_up_gelu", "c1_down", "c2_qkv", "c2_text", "c3_gate_up_fp8", "c3_down_fp8",
                                  "c3_plain_fp8"])
def test_baseline_shapes_sampled_rows(gemm, orc, case):
    m, k, n, fp8, epi = BASELINE_CASES[case]
    print(f"baseline shape {case}: {m}x{k}x{n} fp8={fp8} epilogue {epi}", flush=True)
    x, q, s, b = problem(orc, m, k, n, fp8, seed=1000 + k)
    for layout in ("kn", "nk"):
        got = run(gemm, x, q, s, b, fp8, layout, epi, torch.bfloat16)
        judge(orc, got, x, q, fp8, s, b, epi, torch.bfloat16, rows=orc.sample_rows(m, 64))


@pytest.mark.parametrize("head_dim", [0, 128])
def test_fused_qkv_c2_full_shape(gemm, orc, head_dim):
    """configs[2]'s fused QKV at its full shape (X [4608, 3072], W [9216, 3072] int8, packed as staged):
    Q, K and V row-major or head-major ([24 heads, 4608, 128], MossImage.swift:548-560), judged against
    the oracle's fp64 truth on 64 sampled rows across all 9216 columns."""
    m, k, d = 4608, 3072, 3072
    print(f"fused qkv {m}x{k}x{3 * d} head_dim {head_dim}", flush=True)
    x, q, s, b = problem(orc, m, k, 3 * d, False, 2200 + head_dim)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    qq, kk, vv = gemm.product_qkv(bf16_dev(x), w, dev(s), bias=dev(b), head_dim=head_dim)
    torch.cuda.synchronize()
    rows = orc.sample_rows(m, 64)
    ridx = torch.from_numpy(rows.astype(np.int64)).to(DEV)
    parts = []
    for t in (qq, kk, vv):
        t = t.index_select(1, ridx).permute(1, 0, 2).reshape(len(rows), d) if head_dim else t.index_select(0, ridx)
        parts.append(t.float().cpu().numpy())
    judge(orc, np.concatenate(parts, axis=1), x[rows], q, False, s, b, "none", torch.bfloat16,
          rows=np.arange(len(rows)))


def test_c1_down_on_up_gelu_output(gemm, orc):
    """configs[1] as chained: the up projection (X [4096, 3072] ~ N(0, 1), W_up [12288, 3072], bias, GELU)
    and the down projection (W_down [3072, 12288], bias) on the up projection's bf16 output — many
    near-zero activations, not N(0, 1). Each product judged against the oracle on 64 sampled rows, the
    down projection on the very activation the GPU produced."""
    m, k, n = 4096, 3072, 12288
    x, q_up, s_up, b_up = problem(orc, m, k, n, False, 2300)
    _, q_dn, s_dn, b_dn = problem(orc, 8, n, k, False, 2400)
    w_up = gemm.pack(weight_tensor(q_up, False, "nk"), layout="nk")
    w_dn = gemm.pack(weight_tensor(q_dn, False, "nk"), layout="nk")
    h = gemm.product(bf16_dev(x), w_up, dev(s_up), bias=dev(b_up), epilogue="gelu_tanh")
    y = gemm.product(h, w_dn, dev(s_dn), bias=dev(b_dn))
    torch.cuda.synchronize()
    rows = orc.sample_rows(m, 64)
    ridx = torch.from_numpy(rows.astype(np.int64)).to(DEV)
    sub = np.arange(len(rows))
    h_rows = h.index_select(0, ridx)
    h_bits = h_rows.view(torch.int16).cpu().numpy().view(np.uint16)
    judge(orc, h_rows.float().cpu().numpy(), x[rows], q_up, False, s_up, b_up, "gelu", torch.bfloat16, rows=sub)
    near_zero = float((np.abs(orc.bf16_to_f32(h_bits)) < 1e-2).mean())
    assert near_zero > 0.05, near_zero   # the GELU output's distribution, not N(0, 1)
    judge(orc, y.index_select(0, ridx).float().cpu().numpy(), h_bits, q_dn, False, s_dn, b_dn, "none", torch.bfloat16,
          rows=sub)


# ---- the packed layout (sq8_pack_weight) ------------------------------------------------------------

PACKED_SHAPES = [(256, 3072, 3072), (150, 768, 96), (70, 10240, 72), (65, 448, 130), (300, 1024, 1000), (1, 64, 8)]


@pytest.mark.parametrize("fp8", [False, True], ids=["int8", "fp8"])
@pytest.mark.parametrize("shape", PACKED_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_packed_product(gemm, orc, shape, fp8):
    m, k, n = shape
    x, q, s, b = problem(orc, m, k, n, fp8, seed=500 + n)
    xt, st, bt = bf16_dev(x), dev(s), dev(b)
    wnk, wkn = weight_tensor(q, fp8, "nk"), weight_tensor(q, fp8, "kn")
    pk_nk = gemm.pack(wnk, layout="nk", fp8=fp8 or None)
    pk_kn = gemm.pack(wkn, layout="kn", fp8=fp8 or None)
    assert torch.equal(pk_nk.data, pk_kn.data)  # the same codes, the same packed bytes
    for out in (torch.float32, torch.bfloat16):
        y = gemm.product(xt, pk_kn, st, bias=bt, out_dtype=out)
        direct = gemm.product(xt, wnk, st, layout="nk", bias=bt, out_dtype=out)
        torch.cuda.synchronize()
        assert torch.equal(y, direct)  # one kernel, one K order: the same bits
        judge(orc, y.float().cpu().numpy(), x, q, fp8, s, b, "none", out)


@pytest.mark.parametrize("epi", ["gelu", "silu", "situ"])
@pytest.mark.parametrize("fp8", [False, True], ids=["int8", "fp8"])
def test_packed_epilogues(gemm, orc, epi, fp8):
    for m, k, n in [(256, 1024, 768), (65, 448, 130), (512, 3072, 6144)]:
        x, q, s, b = problem(orc, m, k, n, fp8, seed=9 + n)
        glu = epi in ("silu", "situ")
        pk = gemm.pack(weight_tensor(q, fp8, "kn"), layout="kn", glu=glu, fp8=fp8 or None)
        name = {"gelu": "gelu_tanh", "silu": "silu_glu", "situ": "situ_glu"}[epi]
        for out in (torch.float32, torch.bfloat16):
            y = gemm.product(bf16_dev(x), pk, dev(s), bias=dev(b), epilogue=name, out_dtype=out)
            torch.cuda.synchronize()
            judge(orc, y.float().cpu().numpy(), x, q, fp8, s, b, epi, out)


def test_packed_glu_weight_refuses_plain_epilogue(gemm, orc):
    x, q, s, b = problem(orc, 64, 256, 128, False, seed=3)
    pk = gemm.pack(weight_tensor(q, False, "nk"), layout="nk", glu=True)
    with pytest.raises(ValueError):
        gemm.product(bf16_dev(x), pk, dev(s))
    from siliconed_amd import _abi as abi
    assert abi.load().sq8_packed_bytes(100, 130, 0) == 2 * 3 * 4096
    assert abi.load().sq8_packed_bytes(100, 130, 1) == 3 * 2 * 4096
    assert abi.load().sq8_packed_bytes(64, 3, 1) == -1


@pytest.mark.parametrize("case", ["c0", "c1_up_gelu", "c1_down", "c2_qkv", "c2_text", "c3_gate_up_fp8", "c3_down_fp8",
                                  "c3_plain_fp8"])
def test_packed_baseline_shapes(gemm, orc, case):
    # The staged (packed) weight, as bench.py runs every workload.
    m, k, n, fp8, epi = BASELINE_CASES[case]
    print(f"packed baseline shape {case}: {m}x{k}x{n} fp8={fp8} epilogue {epi}", flush=True)
    x, q, s, b = problem(orc, m, k, n, fp8, seed=2000 + k)
    pk = gemm.pack(weight_tensor(q, fp8, "kn"), layout="kn", glu=epi == "silu", fp8=fp8 or None)
    name = {"gelu": "gelu_tanh", "silu": "silu_glu", "none": None}[epi]
    y = gemm.product(bf16_dev(x), pk, dev(s), bias=dev(b), epilogue=name, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    judge(orc, y.float().cpu().numpy(), x, q, fp8, s, b, epi, torch.bfloat16, rows=orc.sample_rows(m, 64))


# ---- every weight-direct kernel on the same problems ----------------------------------------------

TILES = {"main128": "128", "main256": "256", "main224": "224", "main64n": "64n", "main64x192": "64x192",
         "skinny64": "s64", "skinny32": "s32", "k32x32": "k32x32", "k32x64": "k32x64", "k64x64": "k64x64",
         "k64x128": "k64x128", "k64x192": "k64x192"}
# The K-group tiles: groups of waves that split the K steps (their sums added in group order).
K_GROUPS = {"k32x32": 4, "k32x64": 4, "k64x64": 4, "k64x128": 2, "k64x192": 2}
KERNEL_SHAPES = [
    (1, 64, 64),       # one K step: three of the skinny kernel's four waves have none
    (33, 320, 200),    # 5 K steps (not a multiple of the 4 waves), ragged M and N
    (64, 192, 96),     # 3 K steps
    (130, 3072, 520),
    (512, 3072, 3072),  # the C2 skinny shape
]


@pytest.mark.parametrize("fp8", [False, True], ids=["int8", "fp8"])
@pytest.mark.parametrize("shape", KERNEL_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_each_kernel_on_the_same_problem(gemm, orc, tile_gemm, shape, fp8):
    m, k, n = shape
    x, q, s, b = problem(orc, m, k, n, fp8, seed=900 + m + n)
    pk = gemm.pack(weight_tensor(q, fp8, "kn"), layout="kn", fp8=fp8 or None)
    results = {}
    for name, knob in TILES.items():
        for out in (torch.float32, torch.bfloat16):
            y = tile_gemm(knob).product(bf16_dev(x), pk, dev(s), bias=dev(b), epilogue="gelu_tanh", out_dtype=out)
            torch.cuda.synchronize()
            judge(orc, y.float().cpu().numpy(), x, q, fp8, s, b, "gelu", out)
            results[(name, out)] = y
    # Same kernel, same K order: the skinny kernel gives the same bits whatever its tile height.
    for out in (torch.float32, torch.bfloat16):
        assert torch.equal(results[("skinny64", out)], results[("skinny32", out)])
        # The main kernels: one MFMA sequence over K at every height.
        assert torch.equal(results[("main256", out)], results[("main128", out)])
        assert torch.equal(results[("main224", out)], results[("main128", out)])
        assert torch.equal(results[("main64n", out)], results[("main128", out)])
        assert torch.equal(results[("main64x192", out)], results[("main128", out)])
        # The K-group tiles: one family per group count (each group's MFMA sequence, then the groups in
        # order) where K/64 divides among the groups; else they fall back to the tiles without groups.
        for name, groups in K_GROUPS.items():
            if (k // 64) % groups:
                assert torch.equal(results[(name, out)], results[("main128", out)]), name
        if (k // 64) % 4 == 0:
            assert torch.equal(results[("k32x64", out)], results[("k32x32", out)])
            assert torch.equal(results[("k64x64", out)], results[("k32x32", out)])
        if (k // 64) % 2 == 0:
            assert torch.equal(results[("k64x192", out)], results[("k64x128", out)])


@pytest.mark.parametrize("epi", ["silu", "situ"])
def test_skinny_glu_and_qkv(orc, tile_gemm, epi):
    gemm = tile_gemm("s64")
    m, k, n = 77, 640, 264  # GLU: 132 outputs, ragged against 32-column slabs
    x, q, s, b = problem(orc, m, k, n, False, seed=41)
    pk = gemm.pack(weight_tensor(q, False, "kn"), layout="kn", glu=True)
    name = {"silu": "silu_glu", "situ": "situ_glu"}[epi]
    for out in (torch.float32, torch.bfloat16):
        y = gemm.product(bf16_dev(x), pk, dev(s), bias=dev(b), epilogue=name, out_dtype=out)
        torch.cuda.synchronize()
        judge(orc, y.float().cpu().numpy(), x, q, False, s, b, epi, out)
    # Fused QKV through the skinny kernel, heads outermost.
    d, hd = 256, 64
    x, q, s, b = problem(orc, 40, 512, 3 * d, False, seed=43)
    qo, ko, vo = gemm.product_qkv(bf16_dev(x), weight_tensor(q, False, "nk"), dev(s), layout="nk", bias=dev(b),
                                  head_dim=hd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    full = np.concatenate([t.permute(1, 0, 2).reshape(40, d).cpu().numpy() for t in (qo, ko, vo)], axis=1)
    judge(orc, full, x, q, False, s, b, "none", torch.float32)



# ---- the epilogue's rounding, bit for bit -----------------------------------------------------------

@pytest.mark.parametrize("m", [16, 600, 2048], ids=["skinny", "main-small", "main"])
@pytest.mark.parametrize("layout", ["packed", "kn", "nk"])
def test_epilogue_rounds_scale_then_bias(gemm, orc, m, layout):
    # Integer activations and codes make every fp32 sum exact whatever its order (|sum| ≤ 3·5·3072 <
    # 2^24), so the output must be the reference's two roundings bit for bit: the scale after the sum
    # (TensorGEMM.swift:175-179), then the bias (Ops.swift:400-407) — not one fused multiply-add.
    k, n = 3072, 1024
    rng = np.random.default_rng(m)
    a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    q = rng.integers(-5, 6, size=(n, k)).astype(np.int8)
    s = orc.uniform_f32(m + 1, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(m + 2, (n,), 0.0, 0.02)
    sums = (a.astype(np.float64) @ q.astype(np.float64).T).astype(np.float32)
    want = (sums * s) + b  # numpy float32: each operation rounded
    x = torch.from_numpy(a).to(torch.bfloat16).to(DEV)
    w = weight_tensor(q.view(np.uint8), False, "nk" if layout == "nk" else "kn")
    if layout == "packed":
        w = gemm.pack(w, layout="kn")
    y = gemm.product(x, w, dev(s), layout="nk" if layout == "nk" else "kn", bias=dev(b), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), want)


# ---- the gated residual fused into the product (MossImage.swift:15-19, ElementwiseGPUAnima.swift:47-62) ----

@pytest.mark.parametrize("m,layout,gated", [(300, "packed", True), (4096, "packed", False), (40, "nk", True), (1, "packed", True)])
def test_residual_product_is_product_then_residual(gemm, orc, m, layout, gated):
    # x + gate·(s·acc + b) in one pass equals the fp32 product then sq8_gated_residual on it, bit for bit.
    k, n = 1024, 768
    x_, q, s, b = problem(orc, m, k, n, False, m + 7)
    stream = orc.normal_f32(m + 9, (m, n), 0.0, 1.0)
    gate = dev(orc.normal_f32(m + 10, (n,), 0.0, 0.5)) if gated else None
    w = weight_tensor(q, False, "nk")
    if layout == "packed":
        w = gemm.pack(w, layout="nk")
    y = gemm.product(bf16_dev(x_), w, dev(s), layout="nk", bias=dev(b), out_dtype=torch.float32)
    expect = dev(stream)
    gemm.gated_residual(expect, y, gate)
    got = dev(stream)
    gemm.product_residual(got, bf16_dev(x_), w, dev(s), layout="nk", bias=dev(b), gate=gate)
    torch.cuda.synchronize()
    assert bitwise_equal(got.cpu().numpy(), expect.cpu().numpy()) == 0


@pytest.mark.parametrize("k", [96, 3072 + 32])
def test_packed_and_residual_any_k(gemm, orc, k):
    """K not a multiple of 64 on the step kernels (the reference's products take any K,
    TensorGEMM.swift:124-135): a packed weight (zero codes past K) against an activation staged with its
    rows padded by zeros, judged against the oracle; the gated residual on [N, K] codes of the same K
    (repacked per product) bit-equal to that product followed by the residual pass."""
    m, n = 300, 768
    x_, q, s, b = problem(orc, m, k, n, False, k + 5)
    w = weight_tensor(q, False, "nk")
    wp = gemm.pack(w, layout="nk")
    for epi, out in (("gelu", torch.bfloat16), ("none", torch.float32)):
        y = gemm.product(bf16_dev(x_), wp, dev(s), bias=dev(b), epilogue=None if epi == "none" else "gelu_tanh",
                         out_dtype=out)
        torch.cuda.synchronize()
        judge(orc, y.float().cpu().numpy(), x_, q, False, s, b, epi, out)
    y = gemm.product(bf16_dev(x_), wp, dev(s), bias=dev(b), out_dtype=torch.float32)
    stream = orc.normal_f32(k + 9, (m, n), 0.0, 1.0)
    gate = dev(orc.normal_f32(k + 10, (n,), 0.0, 0.5))
    expect = dev(stream)
    gemm.gated_residual(expect, y, gate)
    got = dev(stream)
    gemm.product_residual(got, bf16_dev(x_), w, dev(s), layout="nk", bias=dev(b), gate=gate)
    torch.cuda.synchronize()
    assert bitwise_equal(got.cpu().numpy(), expect.cpu().numpy()) == 0


@pytest.mark.parametrize("m,n,epi,out_dtype", [(1000, 3000, "gelu", torch.bfloat16), (333, 1536, "none", torch.float32),
                                               (512, 2048, "silu", torch.bfloat16)])
def test_tile_heights_same_bits(gemm, orc, tile_gemm, m, n, epi, out_dtype):
    """The weight-direct kernel in 128-, 64- and 32-row tiles and in 64 × 128 tiles of one 32-column block a
    wave (the product's choice by how many tiles fill the CUs): every output the same bits whichever tile
    computes it — each sum runs the same MFMA sequence over K — on ragged shapes, and within the bars of
    the truth on sampled rows."""
    k = 512
    x, q, s, b = problem(orc, m, k, n, False, 31 + m)
    wp = gemm.pack(weight_tensor(q, False, "nk"), layout="nk", glu=epi == "silu")
    outs = {}
    for tile in ("128", "64", "32", "64n", "64x192"):
        y = tile_gemm(tile).product(bf16_dev(x), wp, dev(s), bias=dev(b), out_dtype=out_dtype,
                         epilogue={"gelu": "gelu_tanh", "none": None, "silu": "silu_glu"}[epi])
        torch.cuda.synchronize()
        outs[tile] = y.float().cpu().numpy()
    assert bitwise_equal(outs["64"], outs["128"]) == 0 and bitwise_equal(outs["32"], outs["128"]) == 0
    assert bitwise_equal(outs["64n"], outs["128"]) == 0 and bitwise_equal(outs["64x192"], outs["128"]) == 0
    judge(orc, outs["32"], x, q, False, s, b, epi, out_dtype, rows=orc.sample_rows(m, 64))


@pytest.mark.parametrize("head_dim", [0, 64])
def test_one_block_waves_qkv_and_residual(gemm, orc, tile_gemm, head_dim):
    """The 64 × 128 and 64 × 192 tiles of one 32-column block a wave on the fused QKV split (row-major and head-major:
    a block lies in one output and one head) and on the gated residual epilogue: the same bits as the
    128-row tiles, the QKV outputs judged against the truth."""
    m, k, d = 200, 1024, 192
    x, q, s, b = problem(orc, m, k, 3 * d, False, 45 + head_dim)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    outs = {}
    for tile in ("64n", "64x192", "128"):
        parts = tile_gemm(tile).product_qkv(bf16_dev(x), w, dev(s), bias=dev(b), head_dim=head_dim)
        torch.cuda.synchronize()
        outs[tile] = np.concatenate([(t.permute(1, 0, 2).reshape(m, d) if head_dim else t).float().cpu().numpy()
                                     for t in parts], axis=1)
    assert bitwise_equal(outs["64n"], outs["128"]) == 0 and bitwise_equal(outs["64x192"], outs["128"]) == 0
    judge(orc, outs["64n"], x, q, False, s, b, "none", torch.bfloat16, rows=orc.sample_rows(m, 64))
    stream = orc.normal_f32(46, (m, 3 * d), 0.0, 1.0)
    gate = dev(orc.normal_f32(47, (3 * d,), 0.0, 0.5))
    res = {}
    for tile in ("64n", "64x192", "128"):
        got = dev(stream)
        tile_gemm(tile).product_residual(got, bf16_dev(x), w, dev(s), bias=dev(b), gate=gate)
        torch.cuda.synchronize()
        res[tile] = got.cpu().numpy()
    assert bitwise_equal(res["64n"], res["128"]) == 0 and bitwise_equal(res["64x192"], res["128"]) == 0


@pytest.mark.parametrize("tile", ["k32x32", "k64x128"])
@pytest.mark.parametrize("head_dim", [0, 64])
def test_k_group_tiles_qkv_and_residual(gemm, orc, tile_gemm, tile, head_dim):
    """The K-group tiles (the K steps split over four or two wave groups, the groups' sums added in order)
    on the fused QKV split, row-major and head-major: each output the same bits as the same tile's whole
    product; on the gated residual epilogue: the same bits as the tile's fp32 product followed by the
    residual pass; both judged against the truth."""
    m, k, d = 200, 1024, 192
    x, q, s, b = problem(orc, m, k, 3 * d, False, 48 + head_dim)
    g = tile_gemm(tile)
    w = gemm.pack(weight_tensor(q, False, "nk"), layout="nk")
    whole = g.product(bf16_dev(x), w, dev(s), bias=dev(b))
    parts = g.product_qkv(bf16_dev(x), w, dev(s), bias=dev(b), head_dim=head_dim)
    torch.cuda.synchronize()
    got = np.concatenate([(t.permute(1, 0, 2).reshape(m, d) if head_dim else t).float().cpu().numpy()
                          for t in parts], axis=1)
    assert bitwise_equal(got, whole.float().cpu().numpy()) == 0
    judge(orc, got, x, q, False, s, b, "none", torch.bfloat16, rows=orc.sample_rows(m, 64))
    stream = orc.normal_f32(49, (m, 3 * d), 0.0, 1.0)
    gate = dev(orc.normal_f32(50, (3 * d,), 0.0, 0.5))
    y = g.product(bf16_dev(x), w, dev(s), bias=dev(b), out_dtype=torch.float32)
    expect = dev(stream)
    g.gated_residual(expect, y, gate)
    res = dev(stream)
    g.product_residual(res, bf16_dev(x), w, dev(s), bias=dev(b), gate=gate)
    torch.cuda.synchronize()
    assert bitwise_equal(res.cpu().numpy(), expect.cpu().numpy()) == 0
    judge(orc, y.cpu().numpy(), x, q, False, s, b, "none", torch.float32)


def test_streams_switched_between_products(gemm, orc):
    """Products on fp32 activations (each rounded into the context's scratch) on two streams in turn: the
    switch waits for the work queued on the previous stream, so each product reads its own operand."""
    m, k, n = 512, 1024, 768
    x1, x2 = orc.normal_f32(3, (m, k)), orc.normal_f32(4, (m, k))
    q = orc.uniform_i8(5, (n, k)).view(np.uint8)
    s = orc.uniform_f32(6, (n,), 1e-3, 2e-2)
    w = weight_tensor(q, False, "nk")
    want1 = gemm.product(dev(x1), w, dev(s), layout="nk", out_dtype=torch.float32)
    want2 = gemm.product(dev(x2), w, dev(s), layout="nk", out_dtype=torch.float32)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    a1, a2 = dev(x1), dev(x2)
    try:
        for _ in range(3):
            gemm.set_stream(s1)
            with torch.cuda.stream(s1):
                y1 = gemm.product(a1, w, dev(s), layout="nk", out_dtype=torch.float32)
            gemm.set_stream(s2)
            with torch.cuda.stream(s2):
                y2 = gemm.product(a2, w, dev(s), layout="nk", out_dtype=torch.float32)
            torch.cuda.synchronize()
            assert torch.equal(y1, want1) and torch.equal(y2, want2)
    finally:
        gemm.set_stream(torch.cuda.current_stream())


@pytest.mark.parametrize("route", ["bf16", "fp32", "fp8w"])
def test_non_finite_values_stay_in_their_rows_and_columns(gemm, orc, route):
    """IEEE products as the reference's fp32 route computes them: a NaN in row r of A makes row r NaN,
    +inf times positive codes +inf, times negative codes −inf, times a zero code NaN; an fp8 NaN code
    (0x7F) makes its column NaN. Every other output keeps the bits of the same product without the
    special values (rows and columns are independent)."""
    m, k, n = 100, 256, 192
    x = orc.normal_f32(50, (m, k))
    fp8 = route == "fp8w"
    _, q, s, b = problem(orc, m, k, n, fp8, 51)
    q = q.copy()
    if not fp8:
        # The codes at k = 3 (q is [N, K]): 7 for outputs j < 5, −7 for 5 ≤ j < 10, 0 after.
        q[:, 3] = 0
        q[:5, 3] = np.uint8(7)
        q[5:10, 3] = np.uint8(0xF9)
    else:
        q[17, 40] = 0x7F                         # a NaN code in output column 17
    xs = x.copy()
    xs[5, 7] = np.nan
    xs[9, 3] = np.inf
    w = weight_tensor(q, fp8, "nk")
    kw = dict(layout="nk", bias=dev(b), out_dtype=torch.float32, rounding=route != "fp32")
    if route == "fp32":
        xa, xc = dev(xs), dev(x)
    else:
        xa, xc = bf16_dev(orc.f32_to_bf16(xs)), bf16_dev(orc.f32_to_bf16(x))
    got = gemm.product(xa, w, dev(s), **kw).cpu().numpy()
    clean = gemm.product(xc, w, dev(s), **kw).cpu().numpy()
    torch.cuda.synchronize()
    assert np.isnan(got[5]).all()
    if fp8:
        assert np.isnan(got[:, 17]).all()
        v = code_values(q, True)[:, 3]           # the codes +inf meets, per output column
        live = np.arange(n) != 17
        assert np.isposinf(got[9][live & (v > 0)]).all() and np.isneginf(got[9][live & (v < 0)]).all()
        assert np.isnan(got[9][live & (v == 0)]).all()
        keep = np.ones((m, n), bool)
        keep[5] = keep[9] = False
        keep[:, 17] = False
    else:
        assert np.isposinf(got[9, :5]).all() and np.isneginf(got[9, 5:10]).all() and np.isnan(got[9, 10:]).all()
        keep = np.ones((m, n), bool)
        keep[5] = keep[9] = False
    assert np.array_equal(got[keep].view(np.uint32), clean[keep].view(np.uint32))


@pytest.mark.parametrize("cols", [192, 200])
@pytest.mark.parametrize("rounding,rotation", [(True, None), (False, None), (True, 64)])
def test_submit_first_columns(gemm, orc, rounding, rotation, cols):
    """`submit(…columns:)` (TensorGEMM.swift:292-360): the first `columns` of C computed and written, the
    others untouched; queued, read after a sync. Whole 64-column slabs run the whole product's kernel:
    the same bits as its first columns; a ragged count (200) runs the general kernel where the weight is
    [K, N] and the fp32 route repacks it: within the bars of the truth."""
    m, k, n = 130, 512, 320
    x = orc.normal_f32(61, (m, k))
    q = orc.uniform_i8(62, (k, n))                                    # [K, N], the map's layout
    s = orc.uniform_f32(63, (n,), 1e-3, 2e-2)
    b = orc.normal_f32(64, (n,), 0.0, 0.02)
    a, w, sd, bd = dev(x), dev(q).view(torch.int8), dev(s), dev(b)
    whole = torch.empty((m, n), dtype=torch.float32, device=DEV)
    gemm.linear(a, int8=w, scales=sd, per_column=True, c=whole, m=m, k=k, n=n, rotation=rotation, rounding=rounding,
                bias=bd, epilogue="gelu_tanh")
    part = torch.full((m, n), 7.0, dtype=torch.float32, device=DEV)
    gemm.submit(a, int8=w, scales=sd, per_column=True, c=part, m=m, k=k, n=n, columns=cols, rotation=rotation,
                rounding=rounding, bias=bd, epilogue="gelu_tanh")
    gemm.synchronize()
    assert (part[:, cols:] == 7.0).all()
    if cols % 64 == 0:
        assert torch.equal(part[:, :cols], whole[:, :cols])
    truth_x = orc.rotate_groups(x, rotation) if rotation else x
    if rounding:
        truth_x = orc.f32_to_bf16(truth_x)
    judge(orc, part[:, :cols].cpu().numpy(), truth_x, np.ascontiguousarray(q[:, :cols].T).view(np.uint8), False,
          s[:cols], b[:cols], "gelu", torch.float32)
