"""The model-facing operator (siliconed_amd.weight_products.WeightProducts.linear, the reference's
`WeightProducts.linear`, Sources/Siliconed/WeightProducts.swift:278-436) on the device: each route of a
map's tensor gives the bits of the product it names, called directly on the same codes — per-column and
convrot int8 on rounded, fp32 and quantized activations, fp8, GGUF-style block scales, a bf16 weight —
and the rounded route is within the reference's bars of the truth."""
import numpy as np
import pytest
import torch

from refgen import bitwise_equal
from siliconed_amd.artifact import Artifact, MapTensor, write_map
from siliconed_amd.weight_products import WeightProducts
from test_gpu_parity import DEV, dev, judge

pytestmark = pytest.mark.gpu


def test_each_route_is_its_product(gemm, orc, tmp_path):
    m, k, n = 150, 512, 320
    q = orc.uniform_i8(1, (k, n))                                     # [K, N] as the map keeps it
    s = orc.uniform_f32(2, (n,), 1e-3, 2e-2)
    f8 = orc.f32_to_e4m3(orc.normal_f32(3, (k, n), 0.0, 20.0))
    blocks = orc.uniform_f32(4, (k // 32, n), 1e-3, 2e-2)
    wb = orc.normal_bf16(5, (k, n))
    b = orc.normal_f32(6, (n,), 0.0, 0.02)
    path = str(tmp_path / "w.silicon")
    write_map(path, {"plain.weight": MapTensor(q, scale=s), "rot.weight": MapTensor(q, scale=s, rotation=64),
                     "fp8.weight": MapTensor(f8, scale=np.array(0.02, np.float32)),
                     "q8.weight": MapTensor(q, scale=blocks, block=32),
                     "bf16.weight": MapTensor(wb, dtype="bfloat16")}, page=4096)
    x = orc.normal_f32(7, (m, k))
    xd = dev(x)
    qd, sd, bd = dev(q).view(torch.int8), dev(s), dev(b)
    c = torch.empty((m, n), dtype=torch.float32, device=DEV)
    f32 = dict(out_dtype=torch.float32)
    with Artifact(path) as a:
        for rounds, quantizes in ((True, False), (False, False), (True, True)):
            wp = WeightProducts(a, gemm, rounds_activations=rounds, quantizes_activations=quantizes)
            for name, group in (("plain.weight", 0), ("rot.weight", 64)):
                assert wp.linear(name, xd, c, m, k, n, bias=bd, epilogue="gelu_tanh") > 0
                if quantizes:
                    want = gemm.product_quantized(xd, qd, sd, group=group, layout="kn", bias=bd, epilogue="gelu_tanh", **f32)
                else:
                    want = gemm.product(xd, qd, sd, layout="kn", bias=bd, epilogue="gelu_tanh", rotation=group,
                                        rounding=rounds, **f32)
                torch.cuda.synchronize()
                assert bitwise_equal(c.cpu().numpy(), want.cpu().numpy()) == 0, (name, rounds, quantizes)
        wp = WeightProducts(a, gemm)
        wp.linear("fp8.weight", xd, c, m, k, n)
        want = gemm.product(xd, dev(f8).view(torch.float8_e4m3fn), dev(np.array([0.02], np.float32)), layout="kn", **f32)
        torch.cuda.synchronize()
        assert bitwise_equal(c.cpu().numpy(), want.cpu().numpy()) == 0
        wp.linear("q8.weight", xd, c, m, k, n)
        want = gemm.product_blocks(xd, qd, dev(blocks), 32, layout="kn", **f32)
        torch.cuda.synchronize()
        assert bitwise_equal(c.cpu().numpy(), want.cpu().numpy()) == 0
        wp.linear("bf16.weight", xd, c, m, k, n)
        want = gemm.product_bf16_weight(gemm.round_bf16(xd), dev(wb.view(np.int16)).view(torch.bfloat16), layout="kn")
        torch.cuda.synchronize()
        assert bitwise_equal(c.cpu().numpy(), want.cpu().numpy()) == 0
        # The rounded per-column route against the truth of its bf16 operand.
        wp.linear("plain.weight", xd, c, m, k, n, bias=bd)
        torch.cuda.synchronize()
        judge(orc, c.cpu().numpy(), orc.f32_to_bf16(x), np.ascontiguousarray(q.T).view(np.uint8), False, s, b, "none",
              torch.float32)
        # Staged once: a second product reads the same staged weight.
        staged = wp.staged("plain.weight")
        wp.linear("plain.weight", xd, c, m, k, n, bias=bd)
        assert wp.staged("plain.weight") is staged
        wp.release()
