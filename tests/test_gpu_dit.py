"""The synthetic DiT block (the C4 workload) against the same block in fp32 with the dequantised
weights and fp32 math attention (tests/dit_reference.py); both round the products' operands to bf16
at the same places (the W8A8 route: both quantize them per row after the same rotation).
Bar: the relative error of the block's update (output − input), in the Frobenius norm, ≤ 2e-2 —
the fused attention's bf16 probabilities dominate it. At the C4 workload itself (4608 tokens, hidden
3072, 24 heads of 128) the check runs on 64 sampled rows, as the reference judges its products on
sampled rows of the real shape (Sources/Siliconed/DiagnosticProbes.swift:75-82)."""
import pytest
import torch

from dit_reference import reference

pytestmark = pytest.mark.gpu


def _update_error(y, x, ref):
    upd, upd_ref = y - x, ref - x
    return float((upd - upd_ref).norm() / upd_ref.norm())


@pytest.mark.parametrize("S,d,heads", [(256, 384, 3), (300, 256, 2)])
def test_block_matches_fp32_reference(S, d, heads):
    from siliconed_amd.dit_block import DiTBlock
    blk = DiTBlock(d=d, heads=heads, mlp=4, seed=S, keep_codes=True)
    g = torch.Generator(device="cuda:0").manual_seed(1)
    x = torch.randn((S, d), device="cuda:0", generator=g)
    temb = torch.randn(d, device="cuda:0", generator=g)
    y = blk.forward(x, temb)
    ref = reference(blk, x, temb)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    rel = _update_error(y, x, ref)
    assert rel <= 2e-2, f"relative error of the update {rel:.3e}"


@pytest.mark.parametrize("S,d,heads,group", [(256, 384, 3, 64), (300, 256, 2, 256), (128, 256, 2, 0)])
def test_w8a8_block_matches_fp32_reference(S, d, heads, group):
    # The W8A8 route (norms writing the int8 operand, int8 × int8 products) against the fp32 block
    # whose operands are quantized the same way (per row after the rotation) — the bar of the bf16
    # route: the fused attention's bf16 probabilities dominate.
    from siliconed_amd.dit_block import DiTBlock
    blk = DiTBlock(d=d, heads=heads, mlp=4, seed=S + group, route="w8a8", group=group, keep_codes=True)
    g = torch.Generator(device="cuda:0").manual_seed(2)
    x = torch.randn((S, d), device="cuda:0", generator=g)
    temb = torch.randn(d, device="cuda:0", generator=g)
    y = blk.forward(x, temb)
    ref = reference(blk, x, temb)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    rel = _update_error(y, x, ref)
    assert rel <= 2e-2, f"relative error of the update {rel:.3e}"


@pytest.mark.parametrize("route,group", [("bf16", 0), ("w8a8", 256)])
def test_c4_block_at_full_size(route, group):
    # C4 as bench.py runs it: 4096 image + 512 text tokens, hidden 3072, 24 heads of 128, MLP 4×;
    # the fp32 block on 64 sampled rows (every key and value still in the attention).
    from siliconed_amd.dit_block import DiTBlock
    S, d, heads = 4608, 3072, 24
    print(f"c4 full size: route {route} group {group} S {S} d {d}", flush=True)
    blk = DiTBlock(d=d, heads=heads, mlp=4, seed=7, route=route, group=group, keep_codes=True)
    g = torch.Generator(device="cuda:0").manual_seed(4)
    x = torch.randn((S, d), device="cuda:0", generator=g)
    temb = torch.randn(d, device="cuda:0", generator=g)
    y = blk.forward(x, temb)
    rows = torch.tensor([(2 * i + 1) * S // 128 for i in range(64)], device="cuda:0")
    ref = reference(blk, x, temb, rows=rows)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    rel = _update_error(y[rows], x[rows], ref)
    assert rel <= 2e-2, f"relative error of the update on the sampled rows {rel:.3e}"
    # Row by row too: no sampled row's update is off by more than the bar.
    per_row = ((y[rows] - ref).norm(dim=1) / (ref - x[rows]).norm(dim=1)).max()
    assert per_row <= 2e-2, f"worst sampled row {float(per_row):.3e}"
    del blk


def test_block_flops():
    from siliconed_amd.dit_block import DiTBlock
    blk = DiTBlock(d=256, heads=2, mlp=4, seed=0, keep_codes=True)
    S, d = 100, 256
    assert blk.flops(S) == 2.0 * (6 * d * d + S * 12 * d * d) + 4.0 * S * S * d


def _bf16_ulps(a: torch.Tensor, b: torch.Tensor) -> int:
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    return int((ia - ib).abs().max())


def test_elementwise_passes_match_fp32():
    # The passes against torch fp32 with the same rounding steps: the sums of squares differ only in
    # order, so at most one bf16 unit in the last place apart.
    from siliconed_amd import context
    ctx = context(0)
    g = torch.Generator(device="cuda:0").manual_seed(3)
    S, d, hd = 300, 3072, 128
    x = torch.randn((S, d), device="cuda:0", generator=g) * 3
    w, sc, sh = (torch.randn(d, device="cuda:0", generator=g) * 0.1 + 1, torch.randn(d, device="cuda:0", generator=g) * 0.2,
                 torch.randn(d, device="cuda:0", generator=g) * 0.2)
    got = ctx.norm_modulate(x, w, sc, sh, 1e-6).double()
    # Against float64: the final bf16 rounding (half a unit of the result: 2^(e-8) for |y| in
    # [2^e, 2^(e+1)), at most 2^-8·|y|) plus a few fp32 units of the terms (the sum of squares in
    # another order; v·(1 + scale) and shift can cancel).
    x64, w64, sc64, sh64 = x.double(), w.double(), sc.double(), sh.double()
    v = x64 / torch.sqrt((x64 * x64).mean(dim=1, keepdim=True) + 1e-6) * w64 * (sc64 + 1.0)
    want = v + sh64
    bound = 2.0 ** -8 * want.abs() + 2.0 ** -21 * (v.abs() + sh64.abs())
    assert bool(((got - want).abs() <= bound).all()), float(((got - want).abs() / bound).max())
    t = (torch.randn((S * 24, hd), device="cuda:0", generator=g) * 2).to(torch.bfloat16)
    wt = torch.randn(hd, device="cuda:0", generator=g) * 0.1 + 1
    t32 = t.float()
    want = ((t32 * (1.0 / torch.sqrt((t32 * t32).mean(dim=1, keepdim=True) + 1e-6))) * wt).to(torch.bfloat16)
    ctx.rms_rows(t, wt, 1e-6)
    assert _bf16_ulps(t, want) <= 1
    y = torch.randn((S, d), device="cuda:0", generator=g).to(torch.bfloat16)
    gate = torch.randn(d, device="cuda:0", generator=g)
    x0 = x.clone()
    ctx.gated_residual(x, y, gate)
    assert torch.equal(x, x0 + gate * y.float())  # one product, one sum: the same rounding
    torch.cuda.synchronize()
