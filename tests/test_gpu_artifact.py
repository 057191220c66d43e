"""A map's 8-bit weights staged for the product (siliconed_amd.artifact.Artifact.stage): the same
bits as the product on the same codes passed directly — int8 with a convrot rotation, fp8 with a bf16
scale per column, int8 with one scale for the tensor — and each judged against the oracle's fp64 truth of
its codes (the convrot one on x·R rounded to bf16, as the reference rounds the rotated operand)."""
import numpy as np
import pytest
import torch

from refgen import bitwise_equal
from siliconed_amd.artifact import Artifact, MapTensor, write_map
from test_gpu_parity import bf16_dev, dev, judge

pytestmark = pytest.mark.gpu


def test_staged_weights_give_the_products_of_their_codes(gemm, orc, tmp_path):
    k, n, m = 768, 320, 200
    q = orc.uniform_i8(1, (k, n))                                   # [K, N] as the map keeps it
    s = orc.uniform_f32(2, (n,), 1e-3, 2e-2)
    f8 = orc.f32_to_e4m3(orc.normal_f32(3, (k, n), 0.0, 20.0))
    sb = orc.f32_to_bf16(orc.uniform_f32(4, (n,), 1e-3, 2e-2))
    path = str(tmp_path / "w.silicon")
    write_map(path, {"a.weight": MapTensor(q, scale=s, rotation=256),
                     "b.weight": MapTensor(f8, scale=sb, scale_dtype="bfloat16"),
                     "c.weight": MapTensor(q, scale=np.array(0.0123, np.float32))}, page=4096)
    x = orc.normal_bf16(5, (m, k))
    xd = bf16_dev(x)
    with Artifact(path) as a:
        wa, wb, wc = (a.stage(nm, gemm) for nm in ("a.weight", "b.weight", "c.weight"))
    assert wa.group == 256 and wb.group == 0 and wa.dtype == "int8" and wb.dtype == "float8_e4m3"
    got_a = gemm.product(xd, wa.packed, wa.scale, rotation=wa.group, out_dtype=torch.float32)
    want_a = gemm.product(xd, dev(q).view(torch.int8), dev(s), layout="kn", rotation=256, out_dtype=torch.float32)
    got_b = gemm.product(xd, wb.packed, wb.scale, out_dtype=torch.float32)
    want_b = gemm.product(xd, dev(f8).view(torch.float8_e4m3fn), dev(orc.bf16_to_f32(sb)), layout="kn",
                          out_dtype=torch.float32)
    got_c = gemm.product(xd, wc.packed, wc.scale, out_dtype=torch.float32)
    want_c = gemm.product(xd, dev(q).view(torch.int8), dev(np.array([0.0123], np.float32)), layout="kn",
                          out_dtype=torch.float32)
    torch.cuda.synchronize()
    for got, want in ((got_a, want_a), (got_b, want_b), (got_c, want_c)):
        assert bitwise_equal(got.cpu().numpy(), want.cpu().numpy()) == 0
    qt = np.ascontiguousarray(q.T).view(np.uint8)
    ft = np.ascontiguousarray(f8.T).view(np.uint8)
    xr = orc.f32_to_bf16(orc.rotate_groups(orc.bf16_to_f32(x), 256))
    judge(orc, got_a.cpu().numpy(), xr, qt, False, s, None, "none", torch.float32)
    judge(orc, got_b.cpu().numpy(), x, ft, True, orc.bf16_to_f32(sb), None, "none", torch.float32)
    judge(orc, got_c.cpu().numpy(), x, qt, False, np.full(n, 0.0123, np.float32), None, "none", torch.float32)
