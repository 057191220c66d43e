"""GGUF checkpoints (siliconed_amd.gguf_q8) against the reference's reader
(Sources/Siliconed/Forge/GGUF.swift:90-260): the hostile headers of HostileFilesTests.swift:96-135,
the published headers of eleven real GGUF files (the reference's fixtures, tests/golden/gguf_headers.json.gz)
rebuilt byte for byte — their sha256 the manifests' — and parsed over sparse files of the published
size, one refusal per rule, and the Q8_0 blocks taken apart against their definition. CPU only."""
import gzip
import hashlib
import json
import os
import struct

import numpy as np
import pytest

from siliconed_amd.gguf_q8 import (GGUFError, GGUFFile, TYPE_NAMES, Unread, deinterleave_q8_0, parse, write)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "gguf_headers.json.gz")


def le(fmt, *v):
    return struct.pack("<" + fmt, *v)


def gstr(s):
    b = s.encode()
    return le("Q", len(b)) + b


def gguf(tmp_path, name, keys, kv=b"", tensors=0, infos=b"", size=256):
    """HostileFilesTests.swift's builder: header, key/values and infos as bytes, padded to `size`."""
    b = b"GGUF" + le("I", 3) + le("Q", tensors) + le("Q", keys) + kv + infos
    b += b"\0" * max(0, size - len(b))
    p = tmp_path / name
    p.write_bytes(b)
    return str(p)


def refused(path, fragment):
    with pytest.raises(GGUFError) as e:
        GGUFFile(path)
    assert fragment in str(e.value), e.value


def test_hostile_headers(tmp_path):
    # HostileFilesTests.swift:96-135.
    inner = le("I", 5) + le("Q", 1) + le("i", 7)
    nested = gstr("nested") + le("I", 9) + le("I", 9) + le("Q", 1) + inner
    refused(gguf(tmp_path, "nested.gguf", 1, nested), "an array inside an array")
    flat = gstr("flat") + le("I", 9) + inner
    with GGUFFile(gguf(tmp_path, "flat.gguf", 1, flat)) as f:
        assert f.metadata["flat"] == "[1 × i32]"
    refused(gguf(tmp_path, "string.gguf", 1, le("Q", 1 << 40)), "more than the file")
    refused(gguf(tmp_path, "array.gguf", 1, gstr("a") + le("I", 9) + le("I", 10) + le("Q", 30)), "cannot fit")
    refused(gguf(tmp_path, "align.gguf", 1, gstr("general.alignment") + le("I", 10) + le("Q", 1 << 62)),
            "general.alignment")
    # A string-typed alignment is read as the reference's Int(a): an optional sign and ASCII digits.
    for i, text in enumerate(["²", "٣٢", "3 2", ""]):
        refused(gguf(tmp_path, f"salign{i}.gguf", 1, gstr("general.alignment") + le("I", 8) + gstr(text)),
                "general.alignment")
    with GGUFFile(gguf(tmp_path, "plus.gguf", 1, gstr("general.alignment") + le("I", 8) + gstr("+64"))) as f:
        assert f.header.alignment == 64
    info = gstr("w") + le("I", 4) + b"".join(le("Q", 69_000) for _ in range(4)) + le("I", 0) + le("Q", 0)
    refused(gguf(tmp_path, "dims.gguf", 0, b"", 1, info, size=70_000), "overflow a 64-bit count")
    # A header read in part: Unread past the bytes read, never a verdict on zeros; whole, it parses.
    kv = gstr("general.name") + le("I", 8) + gstr("x" * 100)
    data = open(gguf(tmp_path, "part.gguf", 1, kv), "rb").read()
    end = 24 + len(kv)
    with pytest.raises(Unread):
        parse(data, len(data), readable=end - 1)
    assert parse(data, len(data), readable=end).metadata["general.name"] == "x" * 100


def _q8_tensor(rng, n, k):
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    d = rng.uniform(1e-3, 2e-2, (n, k // 32)).astype(np.float16)
    blocks = np.empty((n * k // 32, 34), np.uint8)
    blocks[:, :2] = d.reshape(-1, 1).view(np.uint8)
    blocks[:, 2:] = q.reshape(-1, 32).view(np.uint8)
    return q, d, blocks.tobytes()


def test_every_refusal_names_its_rule(tmp_path):
    rng = np.random.default_rng(0)
    _, _, q8 = _q8_tensor(rng, 4, 64)
    ok = {"w": ("Q8_0", [64, 4], q8)}
    p = str(tmp_path / "ok.gguf")
    write(p, {"general.architecture": ("string", "test")}, ok)
    with GGUFFile(p) as f:
        assert f.entries["w"].shape == [4, 64] and f.entries["w"].dtype == "Q8_0" and f.q8_0_tensors() == ["w"]
    # The type rule: one unread type refuses the file, by name.
    p = str(tmp_path / "q3k.gguf")
    write(p, {}, {"w": ("Q8_0", [64, 4], q8), "v": ("Q3_K", [256], bytes(110))})
    refused(p, "Q3_K (1 tensor(s), first v)")
    # Q8_0 rows of a non-multiple of 32; dimensions 0 and 5; version 1; not GGUF.
    p = str(tmp_path / "rows.gguf")
    write(p, {}, {"w": ("Q8_0", [48, 2], bytes(34 * 3))})
    refused(p, "not a multiple of 32")
    raw = b"GGUF" + le("I", 3) + le("Q", 1) + le("Q", 0) + gstr("w") + le("I", 5)
    refused(gguf(tmp_path, "dims5.gguf", 0, b"", 1, raw[24:]), "declares 5 dimensions")
    refused(gguf(tmp_path, "dims0.gguf", 0, b"", 1, gstr("w") + le("I", 0)), "declares 0 dimensions")
    v1 = tmp_path / "v1.gguf"
    v1.write_bytes(b"GGUF" + le("I", 1) + bytes(64))
    refused(str(v1), "format version 1 is not read")
    notg = tmp_path / "x.gguf"
    notg.write_bytes(b"GGUX" + bytes(64))
    refused(str(notg), "GGUF magic")
    # Offsets: unaligned, past the end, overlapping; a name twice.
    def infos(*items):
        return b"".join(gstr(n) + le("I", 1) + le("Q", ne) + le("I", t) + le("Q", off) for n, ne, t, off in items)
    refused(gguf(tmp_path, "unal.gguf", 0, b"", 1, infos(("w", 4, 0, 8)), size=512), "not a multiple of the alignment 32")
    refused(gguf(tmp_path, "past.gguf", 0, b"", 1, infos(("w", 200, 0, 0)), size=512), "and the file has 512")
    refused(gguf(tmp_path, "over.gguf", 0, b"", 2, infos(("w", 16, 0, 0), ("v", 16, 0, 32)), size=512), "intersect")
    refused(gguf(tmp_path, "twice.gguf", 0, b"", 2, infos(("w", 4, 0, 0), ("w", 4, 0, 32)), size=512), "used by two tensors")
    # A string that is not UTF-8; an unknown value type.
    refused(gguf(tmp_path, "utf.gguf", 1, le("Q", 2) + b"\xff\xfe" + le("I", 4) + le("I", 0)), "no valid UTF-8")
    refused(gguf(tmp_path, "vt.gguf", 1, gstr("k") + le("I", 13)), "metadata value type 13 is not one GGUF defines")


def test_q8_0_blocks_taken_apart(tmp_path):
    """GGUF.deinterleaveQ8_0: the bytes unchanged, w = d·q per block (ggml's dequantize_row_q8_0)."""
    rng = np.random.default_rng(1)
    q, d, blocks = _q8_tensor(rng, 6, 96)
    codes, scales = deinterleave_q8_0(np.frombuffer(blocks, np.uint8), 6, 96)
    assert np.array_equal(codes, q) and np.array_equal(scales.view(np.uint16), d.view(np.uint16))
    p = str(tmp_path / "w.gguf")
    write(p, {}, {"plain": ("F32", [8], np.arange(8, dtype=np.float32).tobytes()), "w": ("Q8_0", [96, 6], blocks)})
    with GGUFFile(p) as f:
        c2, s2 = f.q8_0_operands("w")
        assert np.array_equal(c2, q) and np.array_equal(s2.view(np.uint16), d.view(np.uint16))
        w = c2.astype(np.float32) * np.repeat(s2.astype(np.float32), 32, axis=1)
        assert np.array_equal(w[2, 40], np.float32(q[2, 40]) * np.float32(d[2, 1]))
        with pytest.raises(ValueError):
            f.q8_0_operands("plain")


# ---- the reference's fixtures: published headers, byte for byte ------------------------------------

_CODES = {v: k for k, v in TYPE_NAMES.items()}
_VT = {"u8": (0, "B"), "i8": (1, "b"), "u16": (2, "H"), "i16": (3, "h"), "u32": (4, "I"), "i32": (5, "i"),
       "f32": (6, "f"), "bool": (7, "B"), "string": (8, None), "u64": (10, "Q"), "i64": (11, "q"), "f64": (12, "d")}


def header_bytes(h):
    out = b"GGUF" + le("IQQ", h["version"], len(h["tensors"]), len(h["metadata"]))
    for k, v in h["metadata"].items():
        t, fmt = _VT[v["type"]]
        out += gstr(k) + le("I", t) + (gstr(v["value"]) if t == 8 else le(fmt, v["value"]))
    for name, t in h["tensors"].items():
        out += gstr(name) + le("I", len(t["ne"])) + b"".join(le("Q", x) for x in t["ne"])
        out += le("IQ", _CODES[t["type"]], t["offset"])
    return out + b"\0" * ((-len(out)) % h["alignment"])


def _golden():
    with gzip.open(GOLDEN, "rt") as f:
        return json.load(f)


@pytest.mark.parametrize("slug", sorted(json.load(gzip.open(GOLDEN, "rt"))))
def test_published_headers_rebuild_and_parse(tmp_path, slug):
    fx = _golden()[slug]
    h = fx["header"]
    raw = header_bytes(h)
    assert len(raw) == fx["header_bytes"] == h["data_start"]
    assert hashlib.sha256(raw).hexdigest() == fx["sha256"], "the published header, byte for byte"
    path = tmp_path / f"{slug}.gguf"
    with open(path, "wb") as f:
        f.write(raw)
        f.truncate(fx["file_bytes"])
    with GGUFFile(str(path)) as g:
        assert g.header.version == h["version"] and g.header.alignment == h["alignment"]
        assert g.header.data_start == h["data_start"] and len(g.entries) == len(h["tensors"])
        counts = {}
        for name, t in h["tensors"].items():
            e = g.entries[name]
            assert e.dtype == t["type"] and e.shape == t["shape"] and e.offset == h["data_start"] + t["offset"], name
            counts[e.dtype] = counts.get(e.dtype, 0) + 1
        assert counts == fx["types"]
        assert len(g.q8_0_tensors()) == fx["types"].get("Q8_0", 0)
        for name in g.q8_0_tensors():
            n, k = g.entries[name].shape[0], g.entries[name].shape[-1]
            assert g.entries[name].bytes == n * k // 32 * 34
        for k, v in h["metadata"].items():
            assert k in g.metadata
