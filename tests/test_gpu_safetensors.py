"""Published 8-bit safetensors weights staged for the product (siliconed_amd.safetensors_q8.stage):
the same bits as the product on the same codes passed directly — ComfyUI int8 convrot (scale per
row, group 256), torchao fp8 per row, SDNQ int8 with a bf16 scale, a ComfyUI fp8 with one scale — and
each judged against the oracle's fp64 truth of its codes (convrot: on x·R rounded to bf16)."""
import numpy as np
import pytest
import torch

from refgen import bitwise_equal
from siliconed_amd.safetensors_q8 import Safetensors, recognize, stage
from test_gpu_parity import bf16_dev, dev, judge
from test_safetensors_q8 import _bf16, _f32, _text, _torchao, _write

pytestmark = pytest.mark.gpu


def test_staged_published_weights_give_the_products_of_their_codes(gemm, orc, tmp_path):
    n, k, m = 320, 768, 200
    q = orc.uniform_i8(1, (n, k))                                   # [N, K] as published
    s = orc.uniform_f32(2, (n,), 1e-3, 2e-2)
    f8 = orc.f32_to_e4m3(orc.normal_f32(3, (n, k), 0.0, 20.0))
    sb = orc.f32_to_bf16(orc.uniform_f32(4, (n,), 1e-3, 2e-2))
    tensors = {
        "a.weight": ("I8", [n, k], q.tobytes()), "a.weight_scale": ("F32", [n, 1], _f32(s)),
        "a.comfy_quant": _text({"format": "int8_tensorwise", "convrot": True}),
        "b._weight_qdata": ("F8_E4M3", [n, k], f8.tobytes()), "b._weight_scale": ("F32", [n, 1], _f32(s)),
        "c.weight": ("I8", [n, k], q.tobytes()), "c.scale": ("BF16", [n, 1], sb.tobytes()),
        "d.weight": ("F8_E4M3", [n, k], f8.tobytes()), "d.weight_scale": ("F32", [], _f32(0.0123)),
    }
    meta = {"b.weight": _torchao("Float8Tensor", "F8_E4M3", [1, k], fdt="float8_e4m3fn")}
    st = Safetensors(_write(tmp_path, "w.safetensors", tensors, meta))
    r = recognize(st)
    staged = {name: stage(st, r.groups[name], gemm) for name in ("a.weight", "b.weight", "c.weight", "d.weight")}
    assert staged["a.weight"].group == 256 and staged["b.weight"].dtype == "float8_e4m3"
    x = orc.normal_bf16(5, (m, k))
    xd = bf16_dev(x)
    xr = orc.f32_to_bf16(orc.rotate_groups(orc.bf16_to_f32(x), 256))
    truth = {"a.weight": (xr, q.view(np.uint8), False, s), "b.weight": (x, f8.view(np.uint8), True, s),
             "c.weight": (x, q.view(np.uint8), False, orc.bf16_to_f32(sb)),
             "d.weight": (x, f8.view(np.uint8), True, np.full(n, 0.0123, np.float32))}
    i8, e4 = dev(q).view(torch.int8), dev(f8).view(torch.float8_e4m3fn)
    want = {"a.weight": (i8, dev(s), 256), "b.weight": (e4, dev(s), 0),
            "c.weight": (i8, dev(orc.bf16_to_f32(sb)), 0), "d.weight": (e4, dev(np.array([0.0123], np.float32)), 0)}
    for name, w in staged.items():
        codes, scale, group = want[name]
        got = gemm.product(xd, w.packed, w.scale, rotation=w.group, out_dtype=torch.float32)
        ref = gemm.product(xd, codes, scale, layout="nk", rotation=group, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert bitwise_equal(got.cpu().numpy(), ref.cpu().numpy()) == 0, name
        xt, codes_nk, fp8, sv = truth[name]
        judge(orc, got.cpu().numpy(), xt, codes_nk, fp8, sv, None, "none", torch.float32)
