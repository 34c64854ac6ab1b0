"""GPU parity of the reference's package-level functions.

``mxfp4_cdna3.ref`` (re-exported by the package, and ``prepack_b_mxfp4`` by
``kernels``) computes python/mxfp4_cdna3/ref.py's functions on the GPU.
Checked here against:
* the reference's own tests (tests/test_smoke.py:6-38), run unchanged on this
  package;
* the vectors recorded from ref.py itself (tests/golden/quantize_vectors.npz);
* the oracle's restatement of ref.py (numpy), bit for bit for quantize,
  dequantize (every scale byte, 0xFF included) and prepack, and within
  float32 rounding for ref_gemm;
* the reference validate.py flow (seed 42, allclose(1e-2, 2e-2)) written
  with these functions, as validate.py:22-78 does with ref.py's.
"""

import os

import numpy as np
import pytest

from oracle import mxfp4_oracle as mo
from tests.gpu_util import log

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quantize_vectors.npz")


@pytest.fixture(scope="module")
def rr():
    import torch

    assert torch.cuda.is_available()
    from mxfp4_cdna3 import ref

    return ref


@pytest.fixture(scope="module")
def kk():
    from mxfp4_cdna3 import kernels

    return kernels


# ---- the reference's tests/test_smoke.py, on this package ------------------

def test_smoke_quant_dequant_roundtrip_zero(rr):
    x = np.zeros((4, 32), dtype=np.float32)
    p, s = rr.quantize_mxfp4(x, axis=-1)
    y = rr.dequantize_mxfp4(p, s, axis=-1)
    assert np.allclose(y, x)


def test_smoke_quant_dequant_small_values(rr):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((8, 64), dtype=np.float32)
    p, s = rr.quantize_mxfp4(x, axis=-1)
    y = rr.dequantize_mxfp4(p, s, axis=-1)
    assert p.shape == (8, 32)
    assert s.shape == (8, 2)
    assert (np.abs(y - x) / (np.abs(x) + 1e-6)).mean() < 0.30


def test_smoke_quant_packing_bit_layout(rr):
    x = np.array([[4.0, -4.0] * 16], dtype=np.float32)
    p, s = rr.quantize_mxfp4(x, axis=-1)
    assert s[0, 0] == 127
    assert p[0, 0] == 0xE6
    assert (p[0] == 0xE6).all()


def test_smoke_ref_gemm_identity_like(rr):
    rng = np.random.default_rng(1)
    A = rng.standard_normal((16, 32), dtype=np.float32)
    B = rng.standard_normal((32, 16), dtype=np.float32) * 0.1
    p, s = rr.quantize_mxfp4(B, axis=0)
    C = rr.ref_gemm(A, p, s)
    assert C.shape == (16, 16)
    assert np.isfinite(C).all()


def test_package_exports(rr, kk):
    import mxfp4_cdna3

    for name in ("quantize_mxfp4", "dequantize_mxfp4", "ref_gemm", "preshuffle_b"):
        assert getattr(mxfp4_cdna3, name) is getattr(rr, name)
    assert kk.prepack_b_mxfp4 is rr.prepack_b_mxfp4


# ---- bit-exact parity ---------------------------------------------------------

def test_quantize_recorded_vectors(rr):
    d = np.load(GOLDEN)
    log("case ref.quantize_mxfp4 recorded vectors")
    p, s = rr.quantize_mxfp4(d["x"], axis=-1)
    assert isinstance(p, np.ndarray)
    assert np.array_equal(p, d["packed"]) and np.array_equal(s, d["scales"])
    p0, s0 = rr.quantize_mxfp4(d["w"], axis=0)
    assert np.array_equal(p0, d["packed0"]) and np.array_equal(s0, d["scales0"])


@pytest.mark.parametrize("shape,axis", [((3, 64, 5), 1), ((3, 64, 5), -2), ((64,), 0), ((2, 3, 96), -1),
                                        ((96, 7), 0), ((0, 64), -1)])
def test_quantize_any_rank_and_axis(rr, shape, axis):
    import torch

    log(f"case ref.quantize_mxfp4 shape={shape} axis={axis}")
    rng = np.random.default_rng(sum(shape) + axis)
    x = (rng.standard_normal(shape) * np.exp2(rng.integers(-20, 20, shape))).astype(np.float32)
    p, s = rr.quantize_mxfp4(x, axis=axis)
    wp, ws = mo.quantize_mxfp4(x, axis=axis)
    assert p.shape == wp.shape and s.shape == ws.shape
    assert np.array_equal(p, wp) and np.array_equal(s, ws)
    # torch in (CPU or GPU) -> GPU tensors out, same bytes
    pt, st = rr.quantize_mxfp4(torch.from_numpy(x).cuda(), axis=axis)
    assert pt.is_cuda and np.array_equal(pt.cpu().numpy(), wp) and np.array_equal(st.cpu().numpy(), ws)
    pc, _ = rr.quantize_mxfp4(torch.from_numpy(x), axis=axis)
    assert np.array_equal(pc.cpu().numpy(), wp)


def test_quantize_rejects_bad_length(rr):
    with pytest.raises(ValueError, match="not divisible by 32"):
        rr.quantize_mxfp4(np.zeros((4, 48), np.float32), axis=-1)


@pytest.mark.parametrize("axis", [0, -1])
def test_dequantize_every_scale_byte(rr, axis):
    """Every (byte, scale byte) pair, 0xFF included: +-inf and NaN as ref.py."""
    log(f"case ref.dequantize_mxfp4 exhaustive axis={axis}")
    B = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 256, axis=1)   # [K/2=256, N=256]
    S = np.repeat(np.arange(256, dtype=np.uint8)[None, :], 16, axis=0)    # [K/32=16, N=256]
    if axis == -1:
        B, S = np.ascontiguousarray(B.T), np.ascontiguousarray(S.T)
    got = rr.dequantize_mxfp4(B, S, axis=axis)
    want = mo.dequantize_mxfp4(B, S, axis=axis)
    assert got.dtype == np.float32 and got.shape == want.shape
    assert np.array_equal(got, want, equal_nan=True)
    # signs of zeros and infinities too
    num = ~np.isnan(want)
    assert np.array_equal(np.signbit(got[num]), np.signbit(want[num]))
    col = got[:, 255] if axis == 0 else got[255, :]
    assert np.isinf(col).sum() == 512 - 64 and np.isnan(col).sum() == 64


def test_dequantize_rank3(rr):
    rng = np.random.default_rng(3)
    P = rng.integers(0, 256, (2, 32, 3), dtype=np.uint8)
    S = rng.integers(100, 150, (2, 2, 3), dtype=np.uint8)
    assert np.array_equal(rr.dequantize_mxfp4(P, S, axis=1), mo.dequantize_mxfp4(P, S, axis=1))
    with pytest.raises(ValueError):
        rr.dequantize_mxfp4(P, S[:, :1], axis=1)


def test_ref_gemm_float32(rr):
    """float32 A (not bf16 values) times the dequantized weights, fp32 accumulation."""
    rng = np.random.default_rng(5)
    M, N, K = 37, 200, 512
    A = rng.standard_normal((M, K), dtype=np.float32)
    Bp, Bs = mo.quantize_mxfp4(rng.standard_normal((K, N), dtype=np.float32), axis=0)
    got = rr.ref_gemm(A, Bp, Bs)
    W = mo.dequantize_mxfp4(Bp, Bs, axis=0)
    exact = A.astype(np.float64) @ W.astype(np.float64)
    bound = np.abs(A).astype(np.float64) @ np.abs(W).astype(np.float64)
    assert got.dtype == np.float32 and got.shape == (M, N)
    # an fp32 GEMM (any summation order, products rounded or fused) is within
    # (K + 2) units of 2**-24 of sum |a||w| from the exact result
    tol = (K + 2) * 2.0 ** -24 * bound
    assert np.all(np.abs(got - exact) <= tol)
    assert np.all(np.abs(mo.ref_gemm(A, Bp, Bs) - exact) <= tol)


def test_prepack_b_mxfp4(rr, kk):
    import torch

    rng = np.random.default_rng(7)
    K, N = 256, 384
    Bp = rng.integers(0, 256, (K // 2, N), dtype=np.uint8)
    Bs = rng.integers(0, 256, (K // 32, N), dtype=np.uint8)
    gp, gs = kk.prepack_b_mxfp4(Bp, Bs)
    wp, ws = mo.prepack_b_mxfp4(Bp, Bs)
    assert gp.shape == wp.shape and np.array_equal(gp, wp) and np.array_equal(gs, ws)
    tp, ts = rr.prepack_b_mxfp4(torch.from_numpy(Bp).cuda(), torch.from_numpy(Bs).cuda())
    assert np.array_equal(tp.cpu().numpy(), wp) and np.array_equal(ts.cpu().numpy(), ws)
    with pytest.raises(AssertionError, match="multiple of n_tile"):
        rr.prepack_b_mxfp4(Bp[:, :200], Bs[:, :200])
    with pytest.raises(ValueError, match="n_tile=128"):
        rr.prepack_b_mxfp4(Bp, Bs, n_tile=64)
    q0, q1 = rr.preshuffle_b(Bp, Bs)
    assert np.array_equal(q0, Bp) and np.array_equal(q1, Bs)


def test_reference_validate_flow(rr, kk):
    """validate.py:22-78 with this package's functions: strategies J and G."""
    import torch

    for M, N, K in ((256, 256, 128), (512, 512, 256), (1024, 1024, 256)):
        log(f"case validate flow (package functions) M={M} N={N} K={K}")
        rng = np.random.default_rng(42)
        A_f32 = rng.standard_normal((M, K), dtype=np.float32) * 0.1
        A = torch.from_numpy(A_f32).to(torch.bfloat16).cuda()
        B_f32 = rng.standard_normal((K, N), dtype=np.float32) * 0.1
        Bp_np, Bs_np = rr.quantize_mxfp4(B_f32, axis=0)
        assert np.array_equal(Bp_np, mo.quantize_mxfp4(B_f32, axis=0)[0])
        Bp, Bs = torch.from_numpy(Bp_np).cuda(), torch.from_numpy(Bs_np).cuda()
        A_back = A.cpu().to(torch.float32).numpy()
        C_ref = rr.ref_gemm(A_back, Bp_np, Bs_np)
        for fn in (kk.gemm_j, kk.gemm_a):
            assert np.allclose(fn(A, Bp, Bs).cpu().numpy(), C_ref, atol=1e-2, rtol=2e-2)
        Gp, Gs = rr.prepack_b_mxfp4(Bp_np, Bs_np)
        C_g = kk.gemm_g(A, torch.from_numpy(Gp).cuda(), torch.from_numpy(Gs).cuda()).cpu().numpy()
        assert np.allclose(C_g, C_ref, atol=1e-2, rtol=2e-2)
