"""Writes the golden fixtures under tests/golden/.

Every value here is computed by plain Python from the format definitions
(E2M1 bit fields, E8M0 = 2**(e-127), IEEE round-to-nearest-even into bf16),
not by the numpy oracle, so the fixtures pin the oracle instead of echoing it.
The reference's own known-answer tests are restated as data
(konradha/cdna3-bench tests/test_smoke.py:6-10, 23-28).

Run: python tests/golden/make_fixtures.py   (seconds; deterministic)
"""

from __future__ import annotations

import json
import math
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def e2m1(code: int) -> float:
    s, e, m = (code >> 3) & 1, (code >> 1) & 3, code & 1
    mag = m * 0.5 if e == 0 else (1.0 + 0.5 * m) * 2.0 ** (e - 1)
    return -mag if s else mag


def f32(x: float) -> float:
    """Round a Python float (binary64) to binary32 (IEEE RNE via struct)."""
    try:
        return struct.unpack("<f", struct.pack("<f", x))[0]
    except OverflowError:
        return math.copysign(math.inf, x)


def bf16_bits(x: float) -> int:
    """binary32 value -> bf16 bits, round to nearest even; NaN -> 0x7FC0|sign."""
    u = struct.unpack("<I", struct.pack("<f", x))[0]
    if (u & 0x7FFFFFFF) > 0x7F800000:
        return ((u >> 16) & 0x8000) | 0x7FC0
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF


def dequant_value(code: int, sbyte: int) -> float:
    # ref.py:69 computes the scale as float64 2**(e-127) cast to float32, then
    # multiplies in float32.
    scale = f32(math.ldexp(1.0, sbyte - 127)) if sbyte < 255 else math.inf
    v = e2m1(code)
    if scale == math.inf:
        return math.nan if v == 0 else math.copysign(math.inf, v)
    return f32(v * scale)


def exhaustive_table() -> np.ndarray:
    """[16 codes, 256 scale bytes] -> bf16 bits of the dequantized value."""
    t = np.zeros((16, 256), dtype=np.uint16)
    for code in range(16):
        for sb in range(256):
            t[code, sb] = bf16_bits(dequant_value(code, sb))
    return t


def tiny_gemm(seed: int = 7, M: int = 4, N: int = 8, K: int = 64):
    """Brute-force float64 GEMM on a [N, K/2] weight; Python loops only."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((M, K)).astype(np.float32)
    a_bits = [[bf16_bits(float(v)) for v in row] for row in a]
    a_val = [[struct.unpack("<f", struct.pack("<I", b << 16))[0] for b in row] for row in a_bits]
    codes = rng.integers(0, 16, (N, K)).tolist()
    exps = rng.integers(118, 134, (N, K // 32)).tolist()
    W = [[codes[n][2 * j] | (codes[n][2 * j + 1] << 4) for j in range(K // 2)] for n in range(N)]
    C = [[0.0] * N for _ in range(M)]
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(K):
                s += a_val[m][k] * dequant_value(codes[n][k], exps[n][k // 32])
            C[m][n] = s
    return {"M": M, "N": N, "K": K, "seed": seed, "A_bits": a_bits, "W_nk": W, "S_nk": exps, "C_f64": C}


def reference_kats():
    """tests/test_smoke.py:23-28 and :6-10 of the reference, as data."""
    return {
        "packing_bit_layout": {"x": [4.0, -4.0] * 16, "scale_byte": 127, "packed": [0xE6] * 16},
        "zeros_roundtrip": {"x": [0.0] * 32, "scale_byte": 0, "packed": [0] * 16},
    }


def main(out_dir: str = HERE) -> None:
    np.save(os.path.join(out_dir, "dequant_table_bf16.npy"), exhaustive_table())
    with open(os.path.join(out_dir, "tiny_gemm.json"), "w") as f:
        json.dump(tiny_gemm(), f)
    with open(os.path.join(out_dir, "reference_kats.json"), "w") as f:
        json.dump(reference_kats(), f, indent=1)
    print("wrote fixtures to", out_dir, file=sys.stderr)


if __name__ == "__main__":
    main()
