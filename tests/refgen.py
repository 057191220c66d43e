"""Input generators of the reference's own tests, restated for the parity tests.

`DequantizeGen` is the generator of Tests/SiliconedTests/DequantizeTests.swift:10-42 (SplitMix64
from 0x4D313432; `codes` every one of the 256 codes first; `scales` full-mantissa values
Float(next() % 1 000 000 + 1) · 1.37e−9, the second negative, the third zero). The expected values
of those tests — Float(q) · s, one fp32 multiplication — are computed here with numpy's IEEE
float32 multiply and torch's e4m3fn decoding, independently of the oracle.
"""
from __future__ import annotations

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
M64 = (1 << 64) - 1


class DequantizeGen:
    def __init__(self, seed: int = 0x4D313432):
        self.seed = seed

    def next(self) -> int:
        self.seed = (self.seed + 0x9E3779B97F4A7C15) & M64
        z = self.seed
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)

    def codes(self, count: int) -> np.ndarray:
        return np.array([i if i < 256 else self.next() & 0xFF for i in range(count)], dtype=np.uint8)

    def scales(self, count: int, kind: str):
        """(raw scale array in its published type, fp32 values)."""
        vals = np.empty(count, dtype=np.float32)
        for i in range(count):
            x = np.float32(self.next() % 1_000_000 + 1) * np.float32(1.37e-9)
            if i == 1:
                x = -x
            elif i == 2:
                x = np.float32(0.0)
            vals[i] = x
        if kind == "bf16":
            raw = (vals.view(np.uint32) >> np.uint32(16)).astype(np.uint16)  # truncation, as the test
            return raw, (raw.astype(np.uint32) << np.uint32(16)).view(np.float32)
        if kind == "f16":
            raw = vals.astype(np.float16)
            return raw, raw.astype(np.float32)
        return vals.copy(), vals


def e4m3_torch_table() -> np.ndarray:
    with open(os.path.join(GOLDEN, "e4m3fn_table.json")) as f:
        d = json.load(f)
    return np.array([int(b, 16) for b in d["bits"]], dtype=np.uint32).view(np.float32)


def code_values(codes: np.ndarray, fp8: bool) -> np.ndarray:
    if fp8:
        return e4m3_torch_table()[codes]
    return codes.view(np.int8).astype(np.float32)


def bitwise_equal(got: np.ndarray, expected: np.ndarray) -> int:
    """Count of values whose bits differ (NaN equals NaN)."""
    g = np.asarray(got, dtype=np.float32)
    e = np.asarray(expected, dtype=np.float32)
    same = (g.view(np.uint32) == e.view(np.uint32)) | (np.isnan(g) & np.isnan(e))
    return int((~same).sum())
