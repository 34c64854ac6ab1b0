"""GPU parity of the quantizer (mxfp4_quantize, device quantize_mxfp4 of
ref.py:14-47): bit-exact codes and scales.

* the reference's recorded vectors (tests/golden/quantize_vectors.npz,
  written from ref.py itself: ties, exponent edges, clipping, subnormals);
* scale exponents on every group maximum within 300 ulps of 6 * 2**k
  against the float32 scale rule (computed here in float64 numpy, so the
  check does not depend on the host's float32 log2);
* seeded matrices, fp32 and bf16 input, both input orientations, every
  output layout, against the oracle;
* quantize -> dequantize recovers the input as the reference's test does
  (tests/test_smoke.py:13-20).
"""

import os

import numpy as np
import pytest

from oracle import mxfp4_oracle as mo
from tests.gpu_util import LAYOUT_TAGS, log
from tests.test_quantize import edge_maxima, model_exponent

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quantize_vectors.npz")


@pytest.fixture(scope="module")
def kk():
    import torch

    assert torch.cuda.is_available()
    from mxfp4_cdna3 import kernels

    return kernels


def _np(t):
    return t.cpu().numpy()


def test_reference_vectors_bit_exact(kk):
    import torch

    d = np.load(GOLDEN)
    log("case quantize reference vectors")
    p, s = kk.quantize(torch.from_numpy(d["x"]).cuda(), -1)
    assert np.array_equal(_np(p), d["packed"]) and np.array_equal(_np(s), d["scales"])
    p0, s0 = kk.quantize(torch.from_numpy(d["w"]).cuda(), 0)
    assert np.array_equal(_np(p0), d["packed0"]) and np.array_equal(_np(s0), d["scales0"])


def test_scale_exponent_edges(kk):
    import torch

    amax = edge_maxima()
    G = amax.size
    X = np.zeros((G, 32), dtype=np.float32)
    X[:, 11] = amax
    X[:, 12] = -amax / np.float32(3.0)
    log(f"case quantize exponent edges groups={G}")
    p, s = kk.quantize(torch.from_numpy(X).cuda(), -1)
    got = _np(s)[:, 0].astype(np.int32) - 127
    assert np.array_equal(got, model_exponent(amax)), int((got != model_exponent(amax)).sum())
    # codes: the oracle's, wherever the host's float32 rule agrees with the model
    op, os_ = mo.quantize_mxfp4(X, axis=-1)
    same = os_[:, 0].astype(np.int32) - 127 == got
    assert same.mean() > 0.999
    assert np.array_equal(_np(p)[same], op[same])


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("axis", [0, -1])
def test_random_matrices_every_layout(kk, dtype, axis):
    import torch

    K, N = 256, 384
    rng = np.random.default_rng(5 + axis)
    W = (rng.standard_normal((K, N)) * 10.0 ** rng.uniform(-3, 3, (K // 32, 1, N)).repeat(32, 0).reshape(K, N))
    W = W.astype(np.float32)
    W[rng.random((K, N)) < 0.01] = 0.0
    if dtype == "bfloat16":
        W = mo.round_to_bf16(W)
    X = W if axis == 0 else np.ascontiguousarray(W.T)
    Xt = torch.from_numpy(X).cuda().to(getattr(torch, dtype))
    Bkn, Skn = mo.quantize_mxfp4(W, axis=0)  # oracle, reference layout
    for layout in ("kn", "nk", "g", "p"):
        log(f"case quantize {dtype} axis={axis} -> {layout}")
        b, s = kk.quantize(Xt, axis, layout)
        wb, ws = mo.to_layout(Bkn, Skn, LAYOUT_TAGS[layout])
        assert np.array_equal(_np(b).ravel(), np.asarray(wb).ravel()), layout
        assert np.array_equal(_np(s).ravel(), np.asarray(ws).ravel()), layout
    # default output layout follows the reference's shapes
    b, s = kk.quantize(Xt, axis)
    assert tuple(b.shape) == ((K // 2, N) if axis == 0 else (N, K // 2))


def test_quantize_dequantize_roundtrip(kk):
    import torch

    rng = np.random.default_rng(0)
    x = rng.standard_normal((8, 64), dtype=np.float32)  # tests/test_smoke.py:13-20
    p, s = kk.quantize(torch.from_numpy(x).cuda(), -1)
    y = _np(kk.dequantize(p, s, "nk", torch.float32)).T
    assert p.shape == (8, 32) and s.shape == (8, 2)
    assert (np.abs(y - x) / (np.abs(x) + 1e-6)).mean() < 0.30
    assert np.array_equal(y, mo.dequantize_mxfp4(_np(p), _np(s), axis=-1))


def test_quantize_rejects_bad_input(kk):
    import torch

    with pytest.raises(RuntimeError, match="not divisible by 32"):
        kk.quantize(torch.zeros(48, 64, device="cuda"), 0)
    with pytest.raises(RuntimeError, match="float32 or bfloat16"):
        kk.quantize(torch.zeros(64, 64, device="cuda", dtype=torch.float16), 0)
    with pytest.raises(RuntimeError, match="layout p needs"):
        kk.quantize(torch.zeros(96, 64, device="cuda"), 0, "p")
