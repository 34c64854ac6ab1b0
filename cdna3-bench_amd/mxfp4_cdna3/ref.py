"""The reference's ``mxfp4_cdna3.ref`` functions, computed on the GPU.

Same names, arguments, shapes and errors as python/mxfp4_cdna3/ref.py:1-101,
so reference callers (validate.py, bench.py, tests/test_smoke.py) run
unchanged; the work runs in this build's gfx950 kernels:

  quantize_mxfp4(x, axis=-1)           ref.py:14-47  -> mxfp4_quantize
  dequantize_mxfp4(packed, scales, axis=-1)
                                       ref.py:50-72  -> mxfp4_dequant (fp32)
  ref_gemm(A_bf16, B_packed, B_scales) ref.py:75-78  -> mxfp4_dequant + an
                                       fp32 GEMM on the device (torch.matmul)
  preshuffle_b(B_packed, B_scales, N_tile=128, K_tile=128)
                                       ref.py:81-82  (identity: contiguous copies)
  prepack_b_mxfp4(B_packed, B_scales, n_tile=128)
                                       ref.py:85-101 -> mxfp4_convert_layout
                                       into the strategy-G layout

Arrays may be numpy (the reference's type: numpy in, numpy out) or torch
tensors (CPU or GPU; the result is a tensor on the GPU).  There is no CPU
path: without a GPU every function except preshuffle_b raises RuntimeError.

``ref_gemm`` keeps the reference's meaning: float32 A times the float32
dequantized weights, with float32 accumulation.  It does not call the MXFP4
GEMM kernel, so comparing a kernel against it (validate.py) still compares
two different computations.

Differences: quantize_mxfp4 on NaN / inf inputs gives unspecified codes (the
reference's depend on numpy's NaN-to-int cast); prepack_b_mxfp4 supports
n_tile=128 only (the block width of strategy G and of this build's G layout).
"""

import numpy as np

# E2M1 magnitudes of codes 0..7 (the format's table; bit 3 is the sign)
E2M1_MAGNITUDES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)

_GROUP = 32


def _torch():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("mxfp4_cdna3: no GPU available; this build has no CPU path")
    return torch


def _kernels():
    from . import kernels

    return kernels


def _is_tensor(x):
    try:
        import torch
    except ImportError:  # pragma: no cover
        return False
    return isinstance(x, torch.Tensor)


def _device(x, dtype):
    """x (numpy or torch) as a contiguous GPU tensor of ``dtype``."""
    torch = _torch()
    if _is_tensor(x):
        t = x.detach()
        if not t.is_cuda:
            t = t.cuda()
        return t.to(dtype).contiguous()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda().to(dtype).contiguous()


def _out(t, like_tensor):
    return t if like_tensor else t.cpu().numpy()


def _axis(ndim, axis):
    if not -ndim <= axis < ndim:
        raise np.exceptions.AxisError(axis, ndim)
    return axis % ndim


def quantize_mxfp4(x, axis=-1):
    """E2M1 codes (two per byte, low nibble = even index along ``axis``) and
    one E8M0 scale byte per 32 elements along ``axis``; any rank."""
    torch = _torch()
    is_t = _is_tensor(x)
    if is_t:
        xt = x.detach()
        if xt.dtype not in (torch.float32, torch.bfloat16):
            xt = xt.float()
        shape = tuple(xt.shape)
    else:
        x = np.asarray(x, dtype=np.float32)
        shape = x.shape
    ax = _axis(len(shape), axis)
    L = shape[ax]
    if L % _GROUP != 0:
        raise ValueError(f"axis {axis} length {L} not divisible by {_GROUP}")
    lead = shape[:ax] + shape[ax + 1:]
    R = int(np.prod(lead, dtype=np.int64))
    if is_t:
        X = xt.movedim(ax, -1).reshape(R, L)
        X = (X if X.is_cuda else X.cuda()).contiguous()
    else:
        X = torch.from_numpy(np.ascontiguousarray(np.moveaxis(x, ax, -1).reshape(R, L))).cuda()
    P, S = _kernels().quantize(X, -1, "nk")  # [R, L/2], [R, L/32]
    P = P.reshape(*lead, L // 2).movedim(-1, ax).contiguous()
    S = S.reshape(*lead, L // _GROUP).movedim(-1, ax).contiguous()
    return _out(P, is_t), _out(S, is_t)


def dequantize_mxfp4(packed, scales, axis=-1):
    """float32 values sign * |e2m1| * 2**(e - 127), the inverse layout of
    quantize_mxfp4 along ``axis`` (scale byte 255 gives +-inf, and NaN for
    codes 0 and 8, as numpy's float32 arithmetic does)."""
    torch = _torch()
    is_t = _is_tensor(packed)
    pshape = tuple(packed.shape)
    sshape = tuple(scales.shape)
    ax = _axis(len(pshape), axis)
    Lh = pshape[ax]
    L = 2 * Lh
    rest = pshape[:ax] + pshape[ax + 1:]
    if L % _GROUP != 0 or len(sshape) != len(pshape) or sshape[ax] != L // _GROUP or \
            sshape[:ax] + sshape[ax + 1:] != rest:
        raise ValueError(f"packed {pshape} and scales {sshape} are not MXFP4 arrays along axis {axis}")
    R = int(np.prod(rest, dtype=np.int64))
    if is_t:
        B = packed.detach().movedim(ax, 0).reshape(Lh, R)
        S = scales.detach().movedim(ax, 0).reshape(L // _GROUP, R)
        B = _device(B, torch.uint8)
        S = _device(S, torch.uint8)
    else:
        B = _device(np.moveaxis(np.asarray(packed, dtype=np.uint8), ax, 0).reshape(Lh, R), torch.uint8)
        S = _device(np.moveaxis(np.asarray(scales, dtype=np.uint8), ax, 0).reshape(L // _GROUP, R), torch.uint8)
    W = _kernels().dequantize(B, S, "kn", torch.float32)  # [L, R]
    W = W.reshape(L, *rest).movedim(0, ax)
    return _out(W, is_t)


def ref_gemm(A_bf16, B_packed, B_scales):
    """float32 A [M, K] @ dequantize_mxfp4(B_packed [K/2, N], B_scales [K/32, N], axis=0)."""
    torch = _torch()
    is_t = _is_tensor(A_bf16)
    A = _device(A_bf16, torch.float32)
    if A.dim() != 2:
        raise ValueError("A must be 2-D [M, K]")
    Bp = _device(B_packed, torch.uint8)
    Bs = _device(B_scales, torch.uint8)
    if Bp.dim() != 2 or Bs.dim() != 2 or Bp.shape[0] * 2 != A.shape[1]:
        raise ValueError(f"A {tuple(A.shape)}, B_packed {tuple(Bp.shape)}: expected [M, K] and [K/2, N]")
    W = _kernels().dequantize(Bp, Bs, "kn", torch.float32)  # [K, N] float32, exact
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False  # full fp32 products, as numpy's matmul
    try:
        C = A @ W
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32
    return _out(C, is_t)


def preshuffle_b(B_packed, B_scales, N_tile=128, K_tile=128):
    """The reference's placeholder (ref.py:81-82): the same bytes, contiguous."""
    if _is_tensor(B_packed):
        return B_packed.contiguous(), B_scales.contiguous()
    return np.ascontiguousarray(B_packed), np.ascontiguousarray(B_scales)


def prepack_b_mxfp4(B_packed, B_scales, n_tile=128):
    """Strategy G's prepacked arrays of [K/2, N] / [K/32, N] weights, flat:
    B_prep[nb, K-byte / 4, ni, K-byte % 4] and Bs_prep[nb, K / 32, ni] for
    column n = 128 nb + ni (ref.py:85-101), rewritten on the device."""
    torch = _torch()
    is_t = _is_tensor(B_packed)
    K_half, N = tuple(B_packed.shape)
    assert N % n_tile == 0, "N must be a multiple of n_tile"
    if n_tile != 128:
        raise ValueError("prepack_b_mxfp4: this build's G layout has 128-column blocks (n_tile=128)")
    if (2 * K_half) % _GROUP != 0 or tuple(B_scales.shape) != (2 * K_half // _GROUP, N):
        raise ValueError(f"B_packed {(K_half, N)} / B_scales {tuple(B_scales.shape)}: expected [K/2, N], "
                         f"[K/32, N] with K % 32 == 0")
    Bp, Sp = _kernels().prepack(_device(B_packed, torch.uint8), _device(B_scales, torch.uint8), "g")
    return _out(Bp.reshape(-1), is_t), _out(Sp.reshape(-1), is_t)
