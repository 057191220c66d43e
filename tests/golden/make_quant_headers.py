"""Writes quant_headers.json.gz and gguf_headers.json.gz.

quant_headers.json.gz: the published safetensors headers of the reference's 8-bit
fixtures (Tests/SiliconedTests/Fixtures/quant/<slug>/header.json — whole headers of real
checkpoints, pinned there by repository, revision and sha256), ComfyUI's `comfy_quant` texts and
the other U8 texts of each manifest (what CompactTests.swift:380-406 writes into its sparse files),
and which published names each manifest holds quantized and which plain. Data only: the headers as published, the texts as
recorded.

gguf_headers.json.gz: the reference's GGUF fixtures (`*-gguf*/header.json`: version, alignment,
data start, metadata, tensor infos of real published files) with each manifest's header byte count,
sha256 and file size and type counts — what lets a test rebuild the published header bytes, check
them against the sha256, and parse them over a sparse file of the published size.

Run where the reference is mounted: python tests/golden/make_quant_headers.py
"""
import gzip
import json
import os
import sys

SLUGS = ["qwen21-convrot", "qwen21-turbo-convrot", "z-image-convrot", "anima-turbo-convrot", "krea2-turbo-convrot",
         "qwen21-encoder-convrot", "krea2-encoder-convrot", "z-image-sdnq-int8", "z-image-encoder-sdnq-int8",
         "qwen21-fp8", "qwen21-int8"]


def main(root="/root/reference/Tests/SiliconedTests/Fixtures/quant"):
    out = {}
    for slug in SLUGS:
        with open(os.path.join(root, slug, "header.json")) as f:
            header = json.load(f)
        with open(os.path.join(root, slug, "manifest.json")) as f:
            m = json.load(f)
        texts = dict(m.get("comfy_other_u8") or {})
        texts.update(m.get("comfy_quant") or {})
        # The manifest's own split, under the published names: an 8-bit entry of `published` (whose
        # `map` names the model tensors it stands for) is a quantized weight, a 16/32-bit one plain;
        # torchao's and SDNQ's manifests list their quantized weights as {weight, q, s}.
        groups, plain = [], []
        for name, e in (m.get("published") or {}).items():
            if not e.get("map") and "map" in e:
                continue
            (groups if e["dtype"] in ("I8", "F8_E4M3") else plain).append(name)
        for q in m.get("quantized", []):
            if isinstance(q, dict):
                groups.append(q["weight"])
        if not m.get("published"):
            plain += m.get("plain", [])
        parts = (".comfy_quant", ".weight_scale", ".scale_weight", ".scale")
        bases = {g[: -len(".weight")] for g in groups}
        plain = [n for n in plain if not any(n.endswith(x) and n[: -len(x)] in bases for x in parts)]
        out[slug] = {"header": header, "texts": texts, "group": m.get("group"),
                     "groups": sorted(set(groups)), "plain": sorted(set(plain) - set(groups))}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_headers.json.gz")
    with open(path, "wb") as raw, gzip.GzipFile(fileobj=raw, mode="wb", mtime=0) as z:
        z.write(json.dumps(out, sort_keys=True).encode())
    print(path, os.path.getsize(path))
    gguf = {}
    for slug in sorted(os.listdir(root)):
        if "gguf" not in slug:
            continue
        with open(os.path.join(root, slug, "header.json")) as f:
            header = json.load(f)              # key order kept: the file's order
        with open(os.path.join(root, slug, "manifest.json")) as f:
            m = json.load(f)
        gguf[slug] = {"header": header, "sha256": m["header"]["sha256"], "header_bytes": m["header"]["bytes"],
                      "file_bytes": m["file_bytes"], "types": m["types"], "quantized": m.get("quantized", []),
                      "plain": m.get("plain", [])}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gguf_headers.json.gz")
    with open(path, "wb") as raw, gzip.GzipFile(fileobj=raw, mode="wb", mtime=0) as z:
        z.write(json.dumps(gguf).encode())
    print(path, os.path.getsize(path))


if __name__ == "__main__":
    main(*sys.argv[1:])
