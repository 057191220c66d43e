"""The `.silicon` map reader (siliconed_amd.artifact) against the reference's rules
(Sources/Siliconed/Artifact.swift:147-412): the known answers of its robustness tests, a written map
read back, and one refusal per check. CPU only; the staging to the device is in test_gpu_artifact.py."""
import json
import struct

import numpy as np
import pytest

from siliconed_amd.artifact import (Artifact, ArtifactError, MapTensor, element_count, header_length, parse,
                                    write_map)


def test_header_length_and_element_count_known_answers():
    # RobustnessTests.swift:81-83, 103-106.
    assert header_length(2 ** 64 - 1, 1000) is None
    assert header_length(985, 1000) is None
    assert header_length(984, 1000) == 984
    assert element_count([2 ** 63 - 1, 2]) is None
    assert element_count([3, -1]) is None
    assert element_count([]) == 1
    assert element_count([3, 0]) == 0


def _map(tmp_path, **kw):
    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, (512, 96)).astype(np.int8)
    s = rng.uniform(1e-3, 2e-2, 96).astype(np.float32)
    f8 = rng.integers(0, 126, (64, 40)).astype(np.uint8)
    sb = (np.float32(0.5) * np.ones(40, np.float32)).view(np.uint32) >> 16
    tensors = {
        "blocks.0.attn.qkv.weight": MapTensor(q, scale=s, rotation=kw.get("rotation", 256)),
        "blocks.0.mlp.up.weight": MapTensor(f8, scale=sb.astype(np.uint16), scale_dtype="bfloat16"),
        "blocks.0.norm.weight": MapTensor(rng.standard_normal(96).astype(np.float32)),
        "blocks.0.mod.weight": MapTensor(q[:, :8].copy(), scale=np.float32([0.01]).reshape(())),
    }
    path = str(tmp_path / "m.silicon")
    write_map(path, tensors, page=kw.get("page", 4096))
    return path, q, s, f8


def test_a_written_map_reads_back(tmp_path):
    path, q, s, f8 = _map(tmp_path)
    with Artifact(path) as a:
        assert a.page == 4096 and a.order[0] == "blocks.0.attn.qkv.weight"
        t = a.tensors["blocks.0.attn.qkv.weight"]
        assert t.dtype == "int8" and t.shape == [512, 96] and t.offset % a.page == 0
        assert t.scale.layout == "columns" and t.scale.offset == 512 * 96 and t.rotation.group == 256
        assert np.array_equal(a.values(t.name), q) and np.array_equal(a.scale(t.name), s)
        u = a.tensors["blocks.0.mlp.up.weight"]
        assert u.dtype == "float8_e4m3" and u.scale.dtype == "bfloat16"
        assert np.array_equal(a.values(u.name), f8) and np.all(a.scale(u.name) == 0.5)
        assert a.tensors["blocks.0.mod.weight"].scale.layout == "tensor"
        assert a.tensors["blocks.0.norm.weight"].scale is None


def _raw(tmp_path, header, data=b"", version=3, length=None, name="bad.silicon"):
    body = json.dumps(header).encode() if isinstance(header, dict) else header
    n = len(body) if length is None else length
    blob = b"SILICON" + bytes([version]) + struct.pack("<Q", n) + body
    page = header.get("page", 64) if isinstance(header, dict) and isinstance(header.get("page"), int) else 64
    pad = (-len(blob)) % max(page, 1)
    path = tmp_path / name
    path.write_bytes(blob + b"\0" * pad + data)
    return str(path), len(blob) + pad


def _entry(offset, shape, dtype="int8", nbytes=None, **extra):
    n = int(np.prod(shape)) if shape else 1
    e = {"offset": offset, "bytes": n * {"int8": 1, "float32": 4, "bfloat16": 2}.get(dtype, 1) if nbytes is None else nbytes,
         "shape": shape, "dtype": dtype}
    e.update(extra)
    return e


def _refused(path, kind, fragment):
    with pytest.raises(ArtifactError) as e:
        Artifact(path)
    assert e.value.kind == kind and fragment in e.value.why, e.value


def test_refusals(tmp_path):
    # Prologue and header.
    p = tmp_path / "short.silicon"
    p.write_bytes(b"SILICON\x03" + b"\0" * 8)
    _refused(str(p), "truncated", "shorter than a prologue")
    for v in (1, 4):
        path, _ = _raw(tmp_path, {"page": 64, "tensors": {}}, version=v, name=f"v{v}.silicon")
        _refused(path, "bad_magic", "not a Siliconed map's signature")
    path, _ = _raw(tmp_path, {"page": 64, "tensors": {}}, length=10 ** 6, name="len.silicon")
    _refused(path, "truncated", "header length")
    path, _ = _raw(tmp_path, b"[1, 2]", name="notobj.silicon")
    _refused(path, "bad_header", "not a JSON object")
    path, _ = _raw(tmp_path, {"tensors": {}}, name="nopage.silicon")
    _refused(path, "bad_header", "no page size")
    path, _ = _raw(tmp_path, {"page": 0, "tensors": {}}, name="page0.silicon")
    _refused(path, "bad_header", "page size 0")
    path, _ = _raw(tmp_path, {"page": 64}, name="notable.silicon")
    _refused(path, "bad_header", "no tensor table")
    # Tensor entries: written after a header of known size, data at a page boundary.
    cases = [
        ({"w": {"offset": 0, "shape": [2]}}, "bad_header", "incomplete"),
        ({"w": _entry(0, [2], dtype="int4")}, "bad_header", "incomplete"),
        ({"w": _entry(-64, [2])}, "bad_header", "offset -64"),
        ({"w": _entry(64 + 3, [2])}, "unaligned", "not a multiple of 64"),
        ({"w": _entry(1 << 20, [2])}, "truncated", "runs past the end"),
        ({"w": _entry(0, [2, -1], nbytes=0)}, "bad_header", "shape"),
        ({"w": _entry(0, [4, 8], nbytes=31)}, "bad_header", "31 bytes"),
        ({"w": _entry(0, [4, 8], nbytes=64, scale={"offset": 32, "dtype": "float32", "shape": [9]})}, "bad_header",
         "does not fit"),
        ({"w": _entry(0, [4, 8], nbytes=64, scale={"offset": 24, "dtype": "float32", "shape": [8]})}, "bad_header",
         "does not fit"),
        ({"w": _entry(0, [4, 8], nbytes=64, scale={"offset": 32, "dtype": "int8", "shape": [8]})}, "bad_header",
         "scale record is malformed"),
        ({"w": _entry(0, [4, 8], dtype="float32", nbytes=128, scale={"offset": 32, "dtype": "float32", "shape": [8]})},
         "bad_header", "scale record is malformed"),
        ({"w": _entry(0, [4, 8], nbytes=64, scale={"offset": 32, "dtype": "float32", "shape": [8]},
                      rotation={"kind": "hadamard", "group": 4})}, "bad_header", "unknown"),
        ({"w": _entry(0, [4, 8], nbytes=64, scale={"offset": 32, "dtype": "float32", "shape": [8]},
                      rotation={"kind": "convrot", "group": 16})}, "bad_header", "not read"),
        ({"w": _entry(0, [4, 8], dtype="float8_e4m3", nbytes=64, scale={"offset": 32, "dtype": "float32", "shape": [8]},
                      rotation={"kind": "convrot", "group": 4})}, "bad_header", "not read"),
        ({"w": _entry(0, [4, 8], nbytes=40, scale={"offset": 32, "dtype": "float32", "shape": [2, 8], "block": 3})},
         "bad_header", "does not fit"),
    ]
    for i, (table, kind, fragment) in enumerate(cases):
        hdr = {"page": 64, "tensors": table}
        body = json.dumps(hdr).encode()
        start = (16 + len(body) + 63) // 64 * 64
        for e in table.values():
            if isinstance(e.get("offset"), int) and e["offset"] >= 0 and e["offset"] % 64 == 0 and e["offset"] < (1 << 20):
                e["offset"] += start
            elif isinstance(e.get("offset"), int) and e["offset"] == 64 + 3:
                e["offset"] = start + 3
        path, _ = _raw(tmp_path, hdr, data=b"\0" * 256, name=f"case{i}.silicon")
        _refused(path, kind, fragment)
    path, first = _raw(tmp_path, {"page": 64, "tensors": {"w": _entry(128, [2])}, "order": ["w", "v"]}, data=b"\0" * 256,
                       name="order.silicon")
    _refused(path, "bad_header", "disagree")


def test_the_reader_takes_both_versions_and_keeps_the_order(tmp_path):
    rng = np.random.default_rng(1)
    ts = {n: MapTensor(rng.standard_normal(8).astype(np.float32)) for n in ("z", "a", "m")}
    for v in (2, 3):
        path = str(tmp_path / f"v{v}.silicon")
        write_map(path, ts, page=256, version=v, order=["z", "a", "m"])
        with Artifact(path) as a:
            assert a.order == ["z", "a", "m"] and all(a.tensors[n].offset % 256 == 0 for n in a.order)
