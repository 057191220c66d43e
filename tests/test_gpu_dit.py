"""The synthetic DiT block (the C4 workload) against the same block in fp32 with the dequantised
weights and fp32 math attention; both round the products' operands to bf16 at the same places.
Bar: the relative error of the block's update (output − input), in the Frobenius norm, ≤ 2e-2 —
the fused attention's bf16 probabilities dominate it."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("S,d,heads", [(256, 384, 3), (300, 256, 2)])
def test_block_matches_fp32_reference(S, d, heads):
    from siliconed_amd.dit_block import DiTBlock
    blk = DiTBlock(d=d, heads=heads, mlp=4, seed=S)
    g = torch.Generator(device="cuda:0").manual_seed(1)
    x = torch.randn((S, d), device="cuda:0", generator=g)
    temb = torch.randn(d, device="cuda:0", generator=g)
    y = blk.forward(x, temb)
    ref = blk.reference(x, temb)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    upd, upd_ref = y - x, ref - x
    rel = (upd - upd_ref).norm() / upd_ref.norm()
    assert rel <= 2e-2, f"relative error of the update {rel:.3e}"


def test_block_flops():
    from siliconed_amd.dit_block import DiTBlock
    blk = DiTBlock(d=256, heads=2, mlp=4, seed=0)
    S, d = 100, 256
    assert blk.flops(S) == 2.0 * (6 * d * d + S * 12 * d * d) + 4.0 * S * S * d
