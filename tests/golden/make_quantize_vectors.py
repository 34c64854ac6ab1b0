"""Writes tests/golden/quantize_vectors.npz: input/output vectors of the
reference quantizer, quantize_mxfp4 (konradha/cdna3-bench
python/mxfp4_cdna3/ref.py:14-47).

quantize_mxfp4 is the one reference function whose bit-level behaviour the
format definitions do not fix: its argmin tie rule (ref.py:10) and its
float32 ceil(log2(amax / 6)) (ref.py:25-27) at the rounding edges.  This
script therefore imports that single file from the reference checkout, in
the build container only (the reference never travels; only these vectors
do), and records what it returns for inputs built to hit those edges:

* every E2M1 midpoint (ties) and its float32 neighbours, at several scales;
* group maxima 6 * 2**k * (1 + j * 2**-23), j = -3..3, for k from -126 to
  125 (amax / 6 lands on or next to a power of two);
* zeros, -0, subnormals, maxima small enough to clip the exponent at -127,
  maxima near the float32 limit, elements that underflow after scaling;
* seeded N(0, 1) groups at scales 1e-3 .. 1e3;
and a small matrix quantized along axis 0 (the [K, N] weight case).

Run: python tests/golden/make_quantize_vectors.py   (seconds; deterministic;
needs /root/reference).
"""

from __future__ import annotations

import importlib.util
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference/python/mxfp4_cdna3/ref.py"

MIDPOINTS = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
MAGS = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def _load_reference():
    spec = importlib.util.spec_from_file_location("cdna3_bench_ref", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _nudge(x, ulps):
    """x moved by `ulps` float32 steps (x > 0)."""
    b = np.float32(x).view(np.int32) + np.int32(ulps)
    return b.astype(np.int32).view(np.float32)


def edge_groups(rng):
    groups = []
    # ties and their neighbours: amax 6 * 2**k fixes the scale at 2**k
    for k in (-20, -3, 0, 5, 30):
        s = np.float32(2.0) ** np.float32(k)
        vals = []
        for m in MIDPOINTS + MAGS[1:]:
            for u in (-1, 0, 1):
                v = _nudge(np.float32(m), u) if m > 0 else np.float32(0)
                vals += [v * s, -v * s]
        vals = np.array(vals, dtype=np.float32)
        for off in range(0, vals.size, 31):
            chunk = vals[off:off + 31]
            g = np.zeros(32, dtype=np.float32)
            g[0] = np.float32(6.0) * s
            g[1:1 + chunk.size] = chunk
            groups.append(g)
    # amax / 6 on and next to a power of two
    for k in list(range(-126, 126, 7)) + [-127, -5, -4, -1, 0, 1, 3, 4, 5, 8, 16, 64, 100, 120, 124, 125]:
        for j in range(-3, 4):
            base = np.float32(6.0) * (np.float32(2.0) ** np.float32(k)) if k > -127 else np.float32(6.0) * np.float32(2.0 ** -127)
            if not np.isfinite(base) or base == 0:
                continue
            amax = _nudge(base, j)
            if not np.isfinite(amax):
                continue
            g = (rng.standard_normal(32).astype(np.float32) * np.float32(amax / 4)).astype(np.float32)
            g = np.clip(g, -amax, amax).astype(np.float32)
            g[rng.integers(0, 32)] = -amax if j % 2 else amax
            groups.append(g)
    # zeros, signed zeros, subnormals, exponent clip at -127, underflow after scaling
    groups.append(np.zeros(32, dtype=np.float32))
    g = np.zeros(32, dtype=np.float32)
    g[::2] = -0.0
    groups.append(g)
    groups.append((np.arange(32, dtype=np.float32) - 16) * np.float32(1e-45))
    groups.append((rng.standard_normal(32) * 1e-39).astype(np.float32))
    groups.append((rng.standard_normal(32) * 1e-37).astype(np.float32))
    g = (rng.standard_normal(32) * 1e-38).astype(np.float32)
    g[0] = np.float32(1e30)
    groups.append(g)
    g = np.full(32, -1e-38, dtype=np.float32)
    g[5] = np.float32(-3e35)
    groups.append(g)
    g = (rng.standard_normal(32) * 1e37).astype(np.float32)
    g[3] = np.float32(3.4e38)
    groups.append(g)
    # seeded normal groups at many scales
    for scale in (1e-3, 1e-2, 0.1, 1.0, 10.0, 1e3):
        for _ in range(64):
            groups.append((rng.standard_normal(32) * scale).astype(np.float32))
    return np.stack(groups).astype(np.float32)


def main():
    ref = _load_reference()
    rng = np.random.default_rng(2024)
    X = edge_groups(rng)                      # [G, 32]: one scale group per row
    rows = 16
    pad = (-X.shape[0]) % rows
    X = np.concatenate([X, np.zeros((pad, 32), dtype=np.float32)])
    X = X.reshape(-1, rows * 32)              # [R, 16 groups]: quantized along axis -1
    packed, scales = ref.quantize_mxfp4(X, axis=-1)
    W = (rng.standard_normal((128, 48)) * 0.1).astype(np.float32)   # [K, N], axis 0
    packed0, scales0 = ref.quantize_mxfp4(W, axis=0)
    out = os.path.join(HERE, "quantize_vectors.npz")
    np.savez_compressed(out, x=X, packed=packed, scales=scales, w=W, packed0=packed0, scales0=scales0)
    print(f"wrote {out}: x {X.shape}, packed {packed.shape}, scales {scales.shape}; "
          f"w {W.shape}, packed0 {packed0.shape}, scales0 {scales0.shape}")


if __name__ == "__main__":
    main()
