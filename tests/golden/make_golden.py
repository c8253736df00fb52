"""Writes tests/golden/fill_det.json: the first values of fill_det for a few
seeds, computed here with Python integers straight from the definition in
tools/test-support/src/lib.rs:9-18 (state = seed * 0x9E3779B97F4A7C15 | 1;
state = state * 6364136223846793005 + 1442695040888963407 mod 2^64;
value = (state >> 40) / 2^24 * 2 - 1, all in f32).  It is an independent
second implementation of the generator, not a copy of the oracle's C code,
so a C-level slip (overflow, shift width, rounding order) shows up as a
fixture mismatch.

    python tests/golden/make_golden.py
"""

import json
from pathlib import Path

import numpy as np

MASK = (1 << 64) - 1


def fill_det(n, seed):
    s = ((seed * 0x9E3779B97F4A7C15) & MASK) | 1
    out = []
    for _ in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & MASK
        bits = np.float32(s >> 40)
        out.append(float(bits / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0)))
    return out


if __name__ == "__main__":
    vals = {str(seed): fill_det(16, seed) for seed in (0, 1, 2, 3, 42, 0xC0FFEE)}
    path = Path(__file__).resolve().parent / "fill_det.json"
    path.write_text(json.dumps({"generator": "tools/test-support/src/lib.rs:9-18", "values": vals}, indent=1))
    print("wrote", path)
