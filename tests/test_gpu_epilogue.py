"""GPU checks of the fused epilogue C = act(A W + bias) + residual.

Reference: the same plan without epilogue (fp32 C), then bias, activation
(torch's definitions of silu / gelu / gelu(approximate="tanh")) and residual
in float64 on the host.  Tolerances: fp32 C within 1e-5 relative + 1e-6
absolute (a handful of fp32 roundings and the device exp / erf / tanh);
bf16 C within one bf16 rounding (2^-8 relative) of that reference.  Every
kernel family is covered, split-K plans included (the epilogue must run once,
after the reduction), as are K = 0 and a residual that is C itself.
"""

import math

import numpy as np
import pytest

from oracle import mxfp4_oracle as mo
from tests.gpu_util import log, to_dev_bf16, to_dev_u8, weights_for_layout

pytestmark = pytest.mark.gpu

ACTS = [None, "silu", "gelu", "gelu_tanh"]


@pytest.fixture(scope="module")
def kk():
    import torch

    assert torch.cuda.is_available()
    from mxfp4_cdna3 import kernels

    return kernels


def act_f64(name, y):
    if name is None:
        return y
    if name == "silu":
        with np.errstate(over="ignore"):  # exp(-y) = inf -> y / inf = -0, as on the device
            return y / (1.0 + np.exp(-y))
    if name == "gelu":
        erf = np.vectorize(math.erf)
        return 0.5 * y * (1.0 + erf(y / math.sqrt(2.0)))
    return 0.5 * y * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (y + 0.044715 * y ** 3)))


def check(kk, M, N, K, layout, plan, seed=0):
    import torch

    A_bits, W, S = mo.make_inputs(M, N, K, 120, 128, seed=seed)
    B, Sc = weights_for_layout(W, S, layout)
    A, Bd, Sd = to_dev_bf16(A_bits), to_dev_u8(B), to_dev_u8(Sc)
    base = kk.gemm(A, Bd, Sd, None, layout, torch.float32, plan).double().cpu().numpy()
    rng = np.random.default_rng(seed)
    bias32 = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).cuda()
    res32 = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
    cases = [(None, None, None)]
    for act in ACTS:
        cases.append((act, bias32, None))
        cases.append((act, bias32.to(torch.bfloat16), res32.to(torch.bfloat16)))
    cases.append(("silu", None, res32))
    for act, bias, res in cases:
        log(f"case epilogue {layout} plan={plan} M={M} N={N} K={K} act={act} "
            f"bias={None if bias is None else bias.dtype} res={None if res is None else res.dtype}")
        y = base.copy()
        if bias is not None:
            y = y + bias.double().cpu().numpy()[None, :]
        y = act_f64(act, y)
        if res is not None:
            y = y + res.double().cpu().numpy()
        for dt in (torch.float32, torch.bfloat16):
            out = kk.gemm(A, Bd, Sd, None, layout, dt, plan, bias, act, res).double().cpu().numpy()
            tol = (1e-5 * np.abs(y) + 1e-6 * (1 + np.abs(y).max())) if dt == torch.float32 else \
                (2.0 ** -8 * np.abs(y) + 1e-6 * (1 + np.abs(y).max()))
            bad = int((np.abs(out - y) > tol).sum())
            assert bad == 0, f"act={act} dtype={dt}: {bad} outside tolerance, max err {np.abs(out - y).max()}"


@pytest.mark.parametrize("layout,plan", [
    ("kn", (2, 6, 1)), ("kn", (2, 6, 3)), ("nk", (2, 10, 2)), ("g", (2, 6, 1)), ("p", (2, 10, 3)),
    ("kn", (2, 1, 1)), ("nk", (2, 0, 2)), ("kn", (2, 15, 1)), ("kn", (2, 15, 3)),
    ("nk", (2, 15, 1)), ("nk", (2, 15, 3)), ("g", (2, 15, 1)), ("g", (2, 15, 3)),
])
def test_epilogue_tiled(kk, layout, plan):
    check(kk, 300, 512, 640, layout, plan)


@pytest.mark.parametrize("layout,plan", [("kn", (1, 0, 1)), ("kn", (1, 0, 4)), ("nk", (1, 6, 3))])
def test_epilogue_gemv(kk, layout, plan):
    check(kk, 16, 512, 2048, layout, plan, seed=1)


@pytest.mark.parametrize("layout,plan", [("nk", (4, 3, 2)), ("p", (4, 0, 4)), ("nk", (4, 2, 1)),
                                         ("nk", (4, 5, 1)), ("p", (4, 6, 1)), ("nk", (4, 7, 2)), ("nk", (4, 8, 1)),
                                         ("nk", (4, 8, 2)), ("nk", (4, 9, 1)), ("nk", (4, 10, 1)),
                                         ("nk", (4, 11, 1)), ("nk", (4, 11, 4)), ("nk", (4, 12, 4)),
                                         ("nk", (4, 13, 1))])
def test_epilogue_stream(kk, layout, plan):
    M = 32 if plan[1] in (2, 11) else 8 if plan[1] in (8, 10) else 1 if plan[1] in (9, 13) else 16
    K = 16384 if plan[1] == 8 and plan[2] > 1 else 8192 if plan[2] > 1 else 1024
    check(kk, M, 1024, K, layout, plan, seed=2)


def test_epilogue_generic(kk):
    check(kk, 7, 40, 96, "kn", (3, 0, 1), seed=3)


def test_epilogue_k0_and_residual_is_c(kk):
    import torch

    M, N = 5, 64
    A = torch.zeros(M, 0, dtype=torch.bfloat16, device="cuda")
    B = torch.zeros(0, N, dtype=torch.uint8, device="cuda")
    S = torch.zeros(0, N, dtype=torch.uint8, device="cuda")
    bias = torch.linspace(-3, 3, N, device="cuda")
    log("case epilogue K=0")
    out = kk.gemm(A, B, S, None, "kn", torch.float32, None, bias, "silu")
    ref = torch.nn.functional.silu(bias.double().cpu())[None, :].expand(M, N).numpy()
    assert np.allclose(out.double().cpu().numpy(), ref, rtol=1e-6, atol=1e-7)

    # residual = C: C_new = A W + C_old, in place
    A_bits, W, Sc = mo.make_inputs(64, 256, 256, 120, 128, seed=4)
    Bk, Sk = mo.nk_to_kn(W, Sc)
    Ad, Bd, Sd = to_dev_bf16(A_bits), to_dev_u8(Bk), to_dev_u8(Sk)
    for plan in (None, (kk.KERNEL_TILED, 15, 1)):  # auto, and the scheduled kernel's non-temporal stores
        log(f"case epilogue residual aliases C plan={plan}")
        plain = kk.gemm(Ad, Bd, Sd, None, "kn", torch.float32, plan)
        C = torch.randn(64, 256, device="cuda")
        old = C.clone()
        kk.gemm(Ad, Bd, Sd, C, "kn", None, plan, None, None, C)
        assert torch.allclose(C, plain + old, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("plan", [(2, 15, 1), (2, 15, 3), (2, 7, 1)])
def test_epilogue_unaligned_residual(kk, plan):
    """A residual view one element into its buffer (4-byte aligned fp32,
    2-byte aligned bf16): the scheduled kernel reads it per element instead
    of as 4-element vectors; C is bit-identical to the aligned residual's."""
    import torch

    M, N, K = 300, 512, 640
    A_bits, W, S = mo.make_inputs(M, N, K, 120, 128, seed=5)
    B, Sc = weights_for_layout(W, S, "kn")
    A, Bd, Sd = to_dev_bf16(A_bits), to_dev_u8(B), to_dev_u8(Sc)
    bias = torch.randn(N, device="cuda")
    for dt in (torch.float32, torch.bfloat16):
        buf = torch.randn(M * N + 1, device="cuda").to(dt)
        shifted = buf[1:].view(M, N)
        aligned = shifted.clone()
        assert shifted.data_ptr() % 8 != 0
        log(f"case epilogue unaligned residual plan={plan} dtype={dt}")
        want = kk.gemm(A, Bd, Sd, None, "kn", torch.float32, plan, bias, "gelu_tanh", aligned)
        got = kk.gemm(A, Bd, Sd, None, "kn", torch.float32, plan, bias, "gelu_tanh", shifted)
        assert torch.equal(got, want)


def test_epilogue_argument_errors(kk):
    import torch

    A = torch.zeros(16, 64, dtype=torch.bfloat16, device="cuda")
    B = torch.zeros(32, 128, dtype=torch.uint8, device="cuda")
    S = torch.zeros(2, 128, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="activation must be"):
        kk.gemm(A, B, S, activation="relu")
    with pytest.raises(RuntimeError, match=r"bias must be a contiguous \[N\] vector"):
        kk.gemm(A, B, S, bias=torch.zeros(64, device="cuda"))
    with pytest.raises(RuntimeError, match=r"residual must be a contiguous \[M, N\] matrix"):
        kk.gemm(A, B, S, residual=torch.zeros(16, 64, device="cuda"))
    with pytest.raises(RuntimeError, match="bias must be float32 or bfloat16"):
        kk.gemm(A, B, S, bias=torch.zeros(128, device="cuda", dtype=torch.float16))
