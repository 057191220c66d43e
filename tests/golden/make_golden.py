"""Writes the golden fixtures of tests/golden/ from implementations independent of the oracle.

* e4m3fn_table.json — the 256 e4m3fn codes decoded by torch's float8_e4m3fn dtype (fp32 bits).
* bf16_rne.json — fp32 values (ties, carries into the exponent, overflow, subnormals, infinities)
  and torch's bfloat16 conversion of each (bits); the reference rounds "like torch"
  (Sources/Siliconed/Widen.swift:62-76, Forge/Numerics.swift:57-76).
* tiny_products.npz — small products act(s ⊙ (A·q) + b) with bf16 A, int8 q, fp32 s and b,
  computed in float64 by numpy (every sum exact at these sizes) and torch's float64 GELU-tanh /
  SiLU; the references the oracle's fp64 truth is pinned to.

Run: python tests/golden/make_golden.py (deterministic; rerunning rewrites the same bytes).
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def e4m3_table() -> None:
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).to(torch.float32)
    bits = vals.view(torch.int32).numpy().astype(np.uint32)
    out = {"source": f"torch {torch.__version__} float8_e4m3fn -> float32",
           "bits": [f"0x{b:08x}" for b in bits],
           "nan_codes": [int(c) for c in range(256) if np.isnan(vals[c].item())]}
    with open(os.path.join(HERE, "e4m3fn_table.json"), "w") as f:
        json.dump(out, f, indent=1)


def bf16_cases() -> None:
    u = [0x00000000, 0x80000000, 0x3F800000, 0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F817FFF,
         0x3F7FFFFF, 0x7F7FFFFF, 0x7F7F7FFF, 0x7F7F8000, 0xFF7F8000, 0x7F800000, 0xFF800000,
         0x00000001, 0x00008000, 0x00018000, 0x007FFFFF, 0x00800000, 0x40490FDB, 0xC0490FDB,
         0x33800000, 0x3EAAAAAB, 0x477FE000, 0x477FF000, 0x42F6E979]
    rng = np.random.default_rng(20261201)
    u += [int(x) for x in rng.integers(0, 2**32, size=200, dtype=np.uint64)]
    u = [x for x in u if (x & 0x7FFFFFFF) <= 0x7F800000]  # NaNs are checked apart (payload rule)
    f = np.array(u, dtype=np.uint32).view(np.float32)
    b = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)
    out = {"source": f"torch {torch.__version__} float32 -> bfloat16",
           "f32_bits": [f"0x{x:08x}" for x in u], "bf16_bits": [f"0x{int(x):04x}" for x in b]}
    with open(os.path.join(HERE, "bf16_rne.json"), "w") as fh:
        json.dump(out, fh, indent=1)


def tiny_products() -> None:
    rng = np.random.default_rng(7)
    arrays = {}
    for i, (m, k, n) in enumerate([(4, 16, 8), (3, 64, 6), (7, 33, 12), (5, 128, 10)]):
        a32 = rng.standard_normal((m, k)).astype(np.float32)
        a_bf16 = torch.from_numpy(a32).to(torch.bfloat16)
        a = a_bf16.to(torch.float64).numpy()
        q = rng.integers(-128, 128, size=(n, k)).astype(np.int8)
        s = rng.uniform(1e-3, 2e-2, size=n).astype(np.float32)
        b = rng.normal(0, 0.02, size=n).astype(np.float32)
        p = a @ q.astype(np.float64).T  # exact: every term and partial sum fits float64
        y = p * s.astype(np.float64) + b.astype(np.float64)
        t = torch.from_numpy(y)
        h = n // 2
        arrays[f"a_bf16_{i}"] = a_bf16.view(torch.int16).numpy().astype(np.uint16)
        arrays[f"q_{i}"] = q
        arrays[f"s_{i}"] = s
        arrays[f"b_{i}"] = b
        arrays[f"y_none_{i}"] = y
        arrays[f"y_gelu_{i}"] = torch.nn.functional.gelu(t, approximate="tanh").numpy()
        arrays[f"y_silu_glu_{i}"] = (torch.nn.functional.silu(t[:, :h]) * t[:, h:]).numpy()
    np.savez(os.path.join(HERE, "tiny_products.npz"), **arrays)


if __name__ == "__main__":
    e4m3_table()
    bf16_cases()
    tiny_products()
