"""The model-facing operator's routes (siliconed_amd.weight_products.WeightProducts.route: the reference's
`prepare`, Sources/Siliconed/WeightProducts.swift:874-959, with `readableInt8` :801-807 and `quantizedPlan`
:864-872) over a map written in-test: which product each tensor takes, and where the reference widens,
the refusal this library raises instead. CPU only (the route touches no device)."""
import numpy as np
import pytest

from siliconed_amd import _abi as abi
from siliconed_amd.artifact import Artifact, ArtifactError, MapTensor, write_map
from siliconed_amd.weight_products import Route, WeightProducts


@pytest.fixture
def mapped(tmp_path):
    rng = np.random.default_rng(0)
    k, n = 128, 64
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    f8 = rng.integers(0, 0x7E, (k, n)).astype(np.uint8)
    blocks = rng.uniform(1e-3, 2e-2, (k // 32, n)).astype(np.float32)
    path = str(tmp_path / "w.silicon")
    write_map(path, {
        "plain.weight": MapTensor(q, scale=s),
        "rot.weight": MapTensor(q, scale=s, rotation=64),
        "tensor.weight": MapTensor(q, scale=np.array(0.01, np.float32)),
        "fp8.weight": MapTensor(f8, scale=np.array(0.02, np.float32)),
        "q8.weight": MapTensor(q, scale=blocks, block=32),
        "bf16.weight": MapTensor(rng.integers(0, 1 << 15, (k, n)).astype(np.uint16), dtype="bfloat16"),
        "f32.weight": MapTensor(rng.standard_normal((k, n)).astype(np.float32)),
        "nk.weight": MapTensor(np.ascontiguousarray(q.T), scale=np.array(0.01, np.float32)),
    }, page=4096)
    with Artifact(path) as a:
        yield a, k, n


def products(a, **kw):
    return WeightProducts(a, gemm=object(), **kw)   # the route needs no device


def test_routes_as_prepare_chooses(mapped):
    a, k, n = mapped
    wp = products(a)
    assert wp.route("plain.weight", k, n) == Route("int8", "rounded")
    assert wp.route("rot.weight", k, n) == Route("int8", "rounded", 64)
    assert wp.route("tensor.weight", k, n) == Route("int8", "rounded")
    assert wp.route("fp8.weight", k, n) == Route("float8_e4m3", "rounded")
    assert wp.route("q8.weight", k, n) == Route("q8_0", "rounded", 0, 32)
    assert wp.route("bf16.weight", k, n) == Route("bfloat16", "rounded")
    fp32 = products(a, rounds_activations=False)
    assert fp32.route("plain.weight", k, n) == Route("int8", "fp32")
    assert fp32.route("rot.weight", k, n) == Route("int8", "fp32", 64)
    assert fp32.route("q8.weight", k, n) == Route("q8_0", "fp32", 0, 32)
    assert fp32.route("bf16.weight", k, n) == Route("bfloat16", "fp32")
    # W8A8 (quantizedPlan): int8 per column or tensor, rotation kept; fp8 and block scales keep their route.
    w8 = products(a, quantizes_activations=True)
    assert w8.route("plain.weight", k, n) == Route("int8", "quantized")
    assert w8.route("rot.weight", k, n) == Route("int8", "quantized", 64)
    assert w8.route("fp8.weight", k, n) == Route("float8_e4m3", "rounded")
    assert w8.route("q8.weight", k, n) == Route("q8_0", "rounded", 0, 32)


def test_where_the_reference_widens(mapped):
    a, k, n = mapped
    wp = products(a)
    with pytest.raises(abi.Unsupported):
        wp.route("f32.weight", k, n)                   # an fp32 weight: GEMM.linear's widened route
    with pytest.raises(abi.Unsupported):
        wp.route("nk.weight", k, n)                    # [n, k]: not the map's transposed layout
    with pytest.raises(ArtifactError) as e:
        wp.route("plain.weight", k, n + 1)             # `expect`: the count disagrees
    assert e.value.kind == "bad_header"
    with pytest.raises(ArtifactError) as e:
        wp.route("absent.weight", k, n)
    assert e.value.kind == "missing"
