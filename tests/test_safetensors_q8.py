"""Published 8-bit safetensors (siliconed_amd.safetensors_q8) against the reference's rules:
the header bounds of HostileFilesTests.swift:43-95, the recognizer (Forge/Quantization.swift:430-720)
over the whole published headers of its fixtures (tests/golden/quant_headers.json.gz, laid over
sparse files with the ComfyUI texts written in, as CompactTests.swift:380-406 does), one refusal per
rule on synthetic files, and the operands handed to the product. CPU only."""
import gzip
import json
import os
import struct

import numpy as np
import pytest

from siliconed_amd.artifact import Artifact
from siliconed_amd.safetensors_q8 import (Refused, Safetensors, SafetensorsError, product_operands, recognize,
                                          to_map)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_headers.json.gz")


# ---- the header's bounds -------------------------------------------------------------------------

def _file(tmp_path, name, data: bytes):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def _st(tmp_path, name, header: str, data: int, length=None):
    body = header.encode()
    n = len(body) if length is None else length
    return _file(tmp_path, name, struct.pack("<Q", n) + body + b"\0" * data)


def _refused(path, fragment):
    with pytest.raises(SafetensorsError) as e:
        Safetensors(path)
    assert fragment in str(e.value), e.value


def test_a_valid_file_reads(tmp_path):
    p = _st(tmp_path, "ok.safetensors",
            '{"w": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24]}, "__metadata__": {"format": "pt"}}', 24)
    s = Safetensors(p)
    assert s.entries["w"].shape == [2, 3] and s.entries["w"].bytes == 24 and s.metadata["format"] == "pt"
    assert s.array("w").shape == (2, 3)


def test_hostile_headers_are_refused_by_name(tmp_path):
    for n in (0, 3, 8):
        _refused(_file(tmp_path, f"short{n}.safetensors", b"\1" * n), "cannot hold a safetensors header")
    _refused(_st(tmp_path, "huge.safetensors", "{}", 0, length=2 ** 64 - 1), "length")
    _refused(_st(tmp_path, "past.safetensors", "{}", 0, length=3), "length")
    _refused(_st(tmp_path, "spec.safetensors", "{}", 0, length=100_000_001), "length")
    cases = [
        ('{"w": {"dtype": "F32", "shape": [1], "data_offsets": [-4, 0]}}', "data_offsets"),
        ('{"w": {"dtype": "F32", "shape": [1], "data_offsets": [8, 4]}}', "data_offsets"),
        ('{"w": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}', "data_offsets"),
        ('{"w": {"dtype": "F32", "shape": [-1, -1], "data_offsets": [0, 4]}}', "not a size"),
        ('{"w": {"dtype": "U8", "shape": [4294967296, 4294967296, 4], "data_offsets": [0, 0]}}', "not a size"),
        ('{"w": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}', "8 bytes for [3]"),
        ('{"w": {"dtype": "F32", "shape": [2]}}', "incomplete"),
        ('{"w": {"dtype": "Q4", "shape": [2], "data_offsets": [0, 2]}}', "unknown dtype"),
        ('[1, 2]', "not a JSON object"),
    ]
    for i, (header, fragment) in enumerate(cases):
        _refused(_st(tmp_path, f"bad{i}.safetensors", header, 8), fragment)


# ---- synthetic 8-bit files -------------------------------------------------------------------------

def _write(tmp_path, name, tensors: dict, metadata=None):
    """tensors: name -> (dtype, shape, bytes)."""
    header, blobs, at = {}, [], 0
    for n, (dtype, shape, blob) in tensors.items():
        header[n] = {"dtype": dtype, "shape": list(shape), "data_offsets": [at, at + len(blob)]}
        blobs.append(blob)
        at += len(blob)
    if metadata:
        header["__metadata__"] = metadata
    body = json.dumps(header).encode()
    body += b" " * ((-len(body)) % 8)
    return _file(tmp_path, name, struct.pack("<Q", len(body)) + body + b"".join(blobs))


def _f32(a):
    return np.asarray(a, np.float32).tobytes()


def _bf16(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16).tobytes()


def _i8(a):
    return np.asarray(a, np.int8).tobytes()


def _text(js):
    b = json.dumps(js).encode()
    return ("U8", [len(b)], b)


def _layer(n=8, k=16, rng=0, scale_shape=None, scale_dtype="F32", kind="I8"):
    r = np.random.default_rng(rng)
    q = r.integers(-127, 128, (n, k)).astype(np.int8)
    s = r.uniform(1e-3, 2e-2, n).astype(np.float32)
    sb = _f32(s) if scale_dtype == "F32" else _bf16(s)
    return q, s, {"w.weight": (kind, [n, k], q.tobytes()),
                  "w.weight_scale": (scale_dtype, scale_shape or [n, 1], sb)}


def _torchao(typ, dtype, block, extra_names=(), fdt=None):
    d = {"block_size": block}
    if fdt:
        d["float8_dtype"] = {"_type": "torch.dtype", "_data": fdt}
    return json.dumps({"_type": typ, "_tensor_data_names": ["qdata", "scale", *extra_names], "_data": d})


def _recognized(tmp_path, name, tensors, metadata=None):
    return recognize(Safetensors(_write(tmp_path, name, tensors, metadata)))


def _refuses(tmp_path, name, tensors, fragment, metadata=None):
    with pytest.raises(Refused) as e:
        _recognized(tmp_path, name, tensors, metadata)
    assert fragment in str(e.value), e.value


def test_the_published_layouts_are_recognized(tmp_path):
    q, s, t = _layer(scale_dtype="BF16")
    # ComfyUI int8 convrot, the group under `params`; an input scale; the scaled_fp8 marker.
    cq = {"format": "int8_tensorwise", "params": {"convrot": True, "convrot_groupsize": 16}}
    r = _recognized(tmp_path, "convrot.safetensors",
                    {**t, "w.comfy_quant": _text(cq), "w.input_scale": ("F32", [], _f32(1.0)),
                     "scaled_fp8": ("F8_E4M3", [0], b""), "norm.weight": ("BF16", [16], _bf16(np.ones(16)))})
    g = r.groups["w.weight"]
    assert (g.kind, g.per_row, g.rotation, g.format, g.scale) == ("int8", True, 16, "ComfyUI int8_tensorwise convrot",
                                                                  "w.weight_scale")
    assert {"w.comfy_quant", "w.weight_scale", "w.input_scale", "scaled_fp8"} <= r.consumed
    assert "norm.weight" not in r.groups and any("input_scale" in n for n in r.notes)
    codes, scale = product_operands(Safetensors(_write(tmp_path, "c2.safetensors", t)), g)
    assert np.array_equal(codes, q)
    # the bf16 scale widened exactly
    assert np.array_equal(scale, (np.frombuffer(_bf16(s), np.uint16).astype(np.uint32) << 16).view(np.float32))
    # The convrot default group: 256.
    _, _, t256 = _layer(k=512)
    r = _recognized(tmp_path, "c256.safetensors", {**t256, "w.comfy_quant": _text({"format": "int8_tensorwise",
                                                                                   "convrot": 1})})
    assert r.groups["w.weight"].rotation == 256
    # ComfyUI "scaled" fp8, one scale for the tensor (the older name); a plain fp8 cast.
    f8 = np.arange(128, dtype=np.uint8).reshape(8, 16)
    r = _recognized(tmp_path, "fp8.safetensors", {"a.weight": ("F8_E4M3", [8, 16], f8.tobytes()),
                                                  "a.scale_weight": ("F32", [], _f32(0.5)),
                                                  "b.weight": ("F8_E4M3", [8, 16], f8.tobytes())})
    assert (r.groups["a.weight"].format, r.groups["a.weight"].per_row) == ("ComfyUI scaled", False)
    assert (r.groups["b.weight"].format, r.groups["b.weight"].scale) == ("fp8 cast", None)
    st = Safetensors(_write(tmp_path, "fp8b.safetensors", {"b.weight": ("F8_E4M3", [8, 16], f8.tobytes())}))
    codes, scale = product_operands(st, recognize(st).groups["b.weight"])
    assert codes.dtype == np.uint8 and np.array_equal(codes, f8) and list(scale) == [1.0]
    # SDNQ: `.scale` BF16 [N, 1] beside `.weight` I8; a norm's `.scale` beside no weight stays a tensor.
    r = _recognized(tmp_path, "sdnq.safetensors", {"l.weight": ("I8", [8, 16], q.tobytes()),
                                                   "l.scale": ("BF16", [8, 1], _bf16(s)),
                                                   "prenorm.scale": ("F32", [16], _f32(np.ones(16)))})
    assert r.groups["l.weight"].format == "SDNQ" and "prenorm.scale" not in r.consumed
    # torchao Int8Tensor per row with its zero point (all zeros), Float8Tensor per tensor.
    meta = {"t.weight": _torchao("Int8Tensor", "I8", [1, 16], ["zero_point"]),
            "u.weight": _torchao("Float8Tensor", "F8_E4M3", [8, 16], fdt="float8_e4m3fn")}
    r = _recognized(tmp_path, "ao.safetensors",
                    {"t._weight_qdata": ("I8", [8, 16], q.tobytes()), "t._weight_scale": ("F32", [8, 1], _f32(s)),
                     "t._weight_zero_point": ("I8", [8, 1], bytes(8)),
                     "u._weight_qdata": ("F8_E4M3", [8, 16], f8.tobytes()), "u._weight_scale": ("F32", [], _f32(2.0))},
                    meta)
    assert (r.groups["t.weight"].format, r.groups["t.weight"].per_row) == ("torchao Int8Tensor", True)
    assert (r.groups["u.weight"].kind, r.groups["u.weight"].per_row) == ("float8_e4m3", False)
    assert "t._weight_zero_point" in r.consumed
    # ComfyUI's table in the metadata; its attention preference ignored by its exact content.
    r = _recognized(tmp_path, "table.safetensors",
                    {**t, "b.attn.comfy_attention.config": _text({"attention": "comfy_kitchen_int8"})},
                    {"_quantization_metadata": json.dumps({"layers": {"w": {"format": "int8_tensorwise"}}})})
    assert r.groups["w.weight"].format == "ComfyUI int8_tensorwise" and r.notes[0].startswith("1 ComfyUI attention setting")


def test_siliconed_sq8_is_read_and_its_lower_tiers_refused(tmp_path):
    q = np.random.default_rng(3).integers(-127, 128, (4, 256)).astype(np.int8)
    t = {"l.sq.codes": ("I8", [4, 256], q.tobytes()), "l.sq.scale": ("F32", [4], _f32([0.01, 0.02, 0.03, 0.04])),
         "l.weight": ("BF16", [4, 256], bytes(2048))}
    r = _recognized(tmp_path, "sq8.safetensors", t, {"tiers": json.dumps({"l": "SQ8"})})
    g = r.groups["l.weight"]
    assert (g.values, g.rotation, g.per_row, g.format) == ("l.sq.codes", 256, True, "Siliconed SQ8")
    assert "l.weight" in r.consumed
    _refuses(tmp_path, "sq4.safetensors", {"l.sq.codes": ("U8", [4, 128], bytes(512)),
                                           "l.sq.scale": ("F32", [4], _f32(np.ones(4)))}, "4-bit",
             {"tiers": json.dumps({"l": "SQ4"})})
    _refuses(tmp_path, "sqx.safetensors", t, "names no SQ tier", {"tiers": json.dumps({"l": "SQ3"})})


def test_every_refusal_names_its_rule(tmp_path):
    q, s, t = _layer()
    f8 = ("F8_E4M3", [8, 16], bytes(128))
    cq = lambda js: {**t, "w.comfy_quant": _text(js)}                                   # noqa: E731
    cases = [
        ({**t, "w.weight_scale_2": ("F32", [], _f32(1))}, "4-bit layer"),
        ({**t, "x.weight": ("U8", [4], bytes(4))}, "uint8 codes"),
        ({**t, "x.scales": ("F8_E8M0", [4], bytes(4))}, "mxfp8"),
        ({**t, "x.weight": ("F8_E5M2", [4], bytes(4))}, "E5M2"),
        ({"x.weight": f8, "x.weight_scale_inv": ("F32", [1, 1], _f32([1]))}, "128×128"),
        (cq({"format": "nvfp4"}), "4-bit layer"),
        (cq({"format": "mxfp8"}), "mxfp8"),
        (cq({"format": "int8_blockwise"}), 'format "int8_blockwise"'),
        (cq({"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 8}), "convrot group 8"),
        ({"w.weight": f8, "w.weight_scale": ("F32", [8, 1], _f32(s)),
          "w.comfy_quant": _text({"format": "float8_e4m3fn", "convrot": True})}, "int8_tensorwise weights alone"),
        ({**t, "w.comfy_quant": ("U8", [3], b"{x]")}, "does not parse as JSON"),
        (cq({"format": "float8_e4m3fn"}), 'I8 declared as "float8_e4m3fn"'),
        ({"w.weight": ("I8", [8, 16], q.tobytes())}, "no scale for them"),
        ({"w.weight": f8, "w.comfy_quant": _text({"format": "float8_e4m3fn"})}, "ships no"),
        ({**t, "w.scale_weight": ("F32", [], _f32(1))}, "two scales"),
        ({"w.weight": ("I8", [8, 16], q.tobytes()), "w.weight_scale": ("I32", [8], bytes(32))}, "a scale of type I32"),
        ({"w.weight": ("I8", [8, 16], q.tobytes()), "w.weight_scale": ("F32", [8, 2], bytes(64))}, "shape [8, 2]"),
        ({**t, "w.svd_up": ("BF16", [8, 2], bytes(32))}, "svd_up"),
        ({"w.weight": ("I8", [8, 16], q.tobytes()), "w.weight_scale": ("F32", [], _f32(0.01)),
          "w.comfy_quant": _text({"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 4})}, "one scale"),
        ({"w.weight": ("I8", [8, 18], bytes(144)), "w.weight_scale": ("F32", [8, 1], _f32(s)),
          "w.comfy_quant": _text({"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 4})},
         "multiple of the group"),
        # Subnormal products: an int8 scale under 2^-126; an fp8 one under 2^-117.
        ({"w.weight": ("I8", [8, 16], q.tobytes()), "w.weight_scale": ("F32", [], _f32(2.0 ** -127))}, "subnormal"),
        ({"w.weight": f8, "w.weight_scale": ("F32", [], _f32(2.0 ** -118))}, "subnormal"),
        ({"x._weight_qdata": ("I8", [8, 16], q.tobytes())}, "description is missing"),
        ({"x.weight_thing": ("F32", [1], _f32(1)), "x._weight_extra": ("F32", [1], _f32(1))}, "torchao component"),
    ]
    for i, (tensors, fragment) in enumerate(cases):
        _refuses(tmp_path, f"r{i}.safetensors", tensors, fragment)
    # 2^-125 with an int8 code is a normal product; rotated by 256 (1/16 per code) it is not.
    ok = {"w.weight": ("I8", [8, 256], bytes(2048)), "w.weight_scale": ("F32", [8, 1], _f32([2.0 ** -125] * 8))}
    assert "w.weight" in _recognized(tmp_path, "sub_ok.safetensors", ok).groups
    _refuses(tmp_path, "sub_rot.safetensors", {**ok, "w.comfy_quant": _text({"format": "int8_tensorwise",
                                                                             "convrot": True})}, "subnormal")
    # torchao's rules.
    base = {"t._weight_qdata": ("I8", [8, 16], q.tobytes()), "t._weight_scale": ("F32", [8, 1], _f32(s))}
    ao = [
        ({"t.weight": _torchao("Float8Tensor", "F8_E4M3", [1, 16])}, base, "Float8Tensor of I8"),
        ({"t.weight": json.dumps({"_type": "Int8Tensor", "_tensor_data_names": ["qdata", "act"],
                                  "_data": {"block_size": [1, 16]}})}, base, "torchao parts"),
        ({"t.weight": _torchao("Int8Tensor", "I8", [1, 8])}, base, "torchao block [1, 8]"),
        ({"t.weight": _torchao("Int8Tensor", "I8", [1, 16], ["zero_point"])}, base, "no tensor holds it"),
        ({"t.weight": _torchao("Int8Tensor", "I8", [1, 16], ["zero_point"])},
         {**base, "t._weight_zero_point": ("I8", [8, 1], bytes([0, 0, 3, 0, 0, 0, 0, 0]))},
         "row 2 has zero point 3"),
        ({"t.weight": _torchao("Float8Tensor", "F8_E4M3", [8, 16], fdt="float8_e5m2")},
         {"t._weight_qdata": f8, "t._weight_scale": ("F32", [], _f32(1))}, "float8_e5m2"),
        ({"t.weight": _torchao("Int8Tensor", "I8", [1, 16])},
         {"t._weight_qdata": ("I8", [8, 16], q.tobytes())}, "scale is absent"),
    ]
    for i, (meta, tensors, fragment) in enumerate(ao):
        _refuses(tmp_path, f"ao{i}.safetensors", tensors, fragment, meta)


def test_recognized_weights_write_a_map_the_reader_takes(tmp_path):
    q, s, t = _layer(k=64)
    st = Safetensors(_write(tmp_path, "w.safetensors", {**t, "w.comfy_quant": _text(
        {"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 64})}))
    r = recognize(st)
    path = str(tmp_path / "w.silicon")
    to_map(st, r, path, page=4096)
    with Artifact(path) as a:
        tm = a.tensors["w.weight"]
        assert tm.shape == [64, 8] and tm.rotation.group == 64 and tm.scale.layout == "columns"
        assert np.array_equal(a.values("w.weight"), q.T) and np.array_equal(a.scale("w.weight"), s)


# ---- the reference's fixtures: whole published headers ---------------------------------------------

def _golden():
    with gzip.open(GOLDEN, "rt") as f:
        return json.load(f)


def _sparse(tmp_path, slug, fx):
    """The header over a sparse file of its data's extent, the recorded texts written in."""
    header = fx["header"]
    body = json.dumps(header).encode()
    body += b" " * ((-len(body)) % 8)
    end = max((v["data_offsets"][1] for k, v in header.items() if k != "__metadata__"), default=0)
    path = str(tmp_path / f"{slug}.safetensors")
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(body)) + body)
        f.truncate(8 + len(body) + end)
        for name, text in fx["texts"].items():
            f.seek(8 + len(body) + header[name]["data_offsets"][0])
            f.write(text.encode())
    return path


EXPECTED = {
    # slug: (groups, format, rotation)
    "anima-turbo-convrot": (254, "ComfyUI int8_tensorwise convrot", 256),
    "z-image-sdnq-int8": (269, "SDNQ", 0),
    "qwen21-fp8": (229, "torchao Float8Tensor", 0),
    "qwen21-int8": (224, "torchao Int8Tensor", 0),
}


@pytest.mark.parametrize("slug", ["qwen21-convrot", "qwen21-turbo-convrot", "z-image-convrot", "anima-turbo-convrot",
                                  "krea2-turbo-convrot", "qwen21-encoder-convrot", "krea2-encoder-convrot",
                                  "z-image-sdnq-int8", "z-image-encoder-sdnq-int8", "qwen21-fp8", "qwen21-int8"])
def test_the_published_headers_are_recognized_8bit(tmp_path, slug):
    fx = _golden()[slug]
    st = Safetensors(_sparse(tmp_path, slug, fx))
    r = recognize(st)
    for name in fx["groups"]:
        assert name in r.groups, name
    for name in fx["plain"]:
        assert name not in r.groups and name not in r.consumed, name
    # Every 8-bit tensor of the file is a group's values or consumed; nothing 8-bit stays a tensor.
    values = {g.values for g in r.groups.values()}
    for name, e in st.entries.items():
        if e.dtype in ("I8", "F8_E4M3") and e.count > 0:
            assert name in values or name in r.consumed, name
    if fx.get("group"):
        rotated = [g for g in r.groups.values() if g.rotation]
        assert rotated and all(g.rotation == fx["group"] and g.kind == "int8" and g.per_row for g in rotated)
    if slug in EXPECTED:
        count, fmt, rot = EXPECTED[slug]
        assert len(r.groups) == count and all(g.format == fmt and g.rotation == rot for g in r.groups.values())
    quant = [n for n in st.entries if n.endswith(".comfy_quant")]
    if quant:
        # Each ComfyUI layer is one group, int8 convrot per row (the published `comfy_quant` texts).
        assert len(r.groups) == len(quant) and all(g.rotation == 256 and g.per_row for g in r.groups.values())
    if slug == "z-image-convrot":
        # CompactTests.swift:341-353: 270 8-bit tensors once each fused qkv is split in three.
        qkv = [n for n in r.groups if n.endswith(".qkv.weight")]
        assert qkv and len(r.groups) + 2 * len(qkv) == 270
    if slug == "qwen21-turbo-convrot":
        # CompactTests.swift:325-327: the Turbo's 31 attention preferences, noted and never a tensor.
        assert any(n.startswith("31 ComfyUI attention setting(s)") for n in r.notes), r.notes
        assert all(n in r.consumed for n in st.entries if "comfy_attention" in n)
