"""Operator API: the reference's python/mxfp4_cdna3/kernels.py surface on gfx950.

Every function calls the native extension ``_C`` (which calls the C ABI in
include/mxfp4_mi355x.h); there is no CPU or torch fallback.  Importing this
module raises if the extension is missing, as the reference does
(python/mxfp4_cdna3/kernels.py:3-6).

Reference functions and their counterparts:
  gemm_a .. gemm_m  (kernels.py:35-94)  same names/arguments/accepted shapes;
                                        all run the library's chosen plan
  gemm_g            (kernels.py:59-60)  prepacked (strategy G) layout, read directly
  gemm_auto         (kernels.py:63-74)  every shape with K % 32 == 0
  device_info, shape_supported_{c,d,e,f,g} (kernels.py:11-32)
  prepack_b_mxfp4   (kernels.py:8, re-exported from ref.py:85-101) the
                    device prepack into the strategy-G arrays
Additions: ``gemm`` (any weight layout, bf16/fp32 out, explicit plan),
``dequantize`` (device dequant tile), ``quantize`` (device quantize_mxfp4,
ref.py:14-47), ``prepack`` / ``convert_layout``
(device counterpart of ref.py:85-101 ``prepack_b_mxfp4``, between any two
layouts), ``select_plan``.
"""

import torch  # noqa: F401  (loads the HIP runtime symbols _C links against)

try:
    from . import _C as _ext
except ImportError as e:  # pragma: no cover - exercised only without a build
    raise RuntimeError(
        "mxfp4_cdna3._C not built; run `python cdna3-bench_amd/build.py`"
    ) from e

from .ref import prepack_b_mxfp4  # noqa: F401,E402  (kernels.py:8 of the reference)

LAYOUT_KN = "kn"  # B [K/2, N], S [K/32, N]  (reference API layout)
LAYOUT_NK = "nk"  # B [N, K/2], S [N, K/32]  (K-contiguous weights)
LAYOUT_G = "g"    # B [N/128, K/8, 128, 4], S [N/128, K/32, 128]  (strategy G prepack, N % 128 == 0)
LAYOUT_P = "p"    # B [N/32, K/64, 2, 32, 16], S [N/32, K/64, 2, 32]  (panels, N % 32 == 0, K % 64 == 0)

KERNEL_AUTO, KERNEL_GEMV, KERNEL_TILED, KERNEL_GENERIC, KERNEL_STREAM = 0, 1, 2, 3, 4
PLAN_STREAM_NO_POLL = 1  # plan flag (tests): streaming split-K groups reduced by their last arrival


def device_info(dev_id=0):
    return _ext.device_info(dev_id)


def shape_supported_c(M, N, K):
    return _ext.shape_supported_c(M, N, K)


def shape_supported_d(M, N, K):
    return _ext.shape_supported_d(M, N, K)


def shape_supported_e(M, N, K):
    return _ext.shape_supported_e(M, N, K)


def shape_supported_f(M, N, K):
    return _ext.shape_supported_f(M, N, K)


def shape_supported_g(M, N, K):
    return _ext.shape_supported_g(M, N, K)


def gemm_a(A, B_packed, B_scales, C=None):
    return _ext.gemm_a(A, B_packed, B_scales, C)


def gemm_b(A, B_packed, B_scales, C=None):
    return _ext.gemm_b(A, B_packed, B_scales, C)


def gemm_c(A, B_packed, B_scales, C=None):
    return _ext.gemm_c(A, B_packed, B_scales, C)


def gemm_d(A, B_packed, B_scales, C=None):
    return _ext.gemm_d(A, B_packed, B_scales, C)


def gemm_e(A, B_packed, B_scales, C=None):
    return _ext.gemm_e(A, B_packed, B_scales, C)


def gemm_f(A, B_packed, B_scales, C=None):
    return _ext.gemm_f(A, B_packed, B_scales, C)


def gemm_g(A, B_prep, Bs_prep, C=None):
    return _ext.gemm_g(A, B_prep, Bs_prep, C)


def gemm_h(A, B_packed, B_scales, C=None):
    return _ext.gemm_h(A, B_packed, B_scales, C)


def gemm_i(A, B_packed, B_scales, C=None):
    return _ext.gemm_i(A, B_packed, B_scales, C)


def gemm_k(A, B_packed, B_scales, C=None):
    return _ext.gemm_k(A, B_packed, B_scales, C)


def gemm_j(A, B_packed, B_scales, C=None):
    return _ext.gemm_j(A, B_packed, B_scales, C)


def gemm_m(A, B_packed, B_scales, C=None):
    return _ext.gemm_m(A, B_packed, B_scales, C)


def gemm_auto(A, B_packed, B_scales, C=None):
    """Any M, N; K % 32 == 0.  C=None -> fp32 (the reference's default)."""
    return _ext.gemm_auto(A, B_packed, B_scales, C)


def gemm(A, B, S, C=None, layout=LAYOUT_KN, out_dtype=None, plan=None, bias=None, activation=None,
         residual=None):
    """C = act(A @ dequant(B, S) + bias) + residual in any weight layout (g / p:
    any shape of the layout's size, N = B.numel() / (K/2)).

    out_dtype: torch.float32 (default) or torch.bfloat16 when C is None.
    plan: optional (kernel, variant, split_k[, flags]) overriding the cost
    model (flags: include/mxfp4_mi355x.h MXFP4_PLAN_*).
    Split-K plans use a workspace the extension keeps per (device, stream);
    under HIP graph capture, run the call once on the capturing stream first.
    bias [N], residual [M, N] (fp32 or bf16; residual may be C itself) and
    activation (None, "silu", "gelu", "gelu_tanh") are fused into the
    kernel's store, in fp32 before the rounding to C's dtype.
    """
    return _ext.gemm(A, B, S, C, layout, out_dtype, None if plan is None else list(plan), bias, activation,
                     residual)


def dequantize(B, S, layout=LAYOUT_KN, out_dtype=torch.bfloat16, K=None):
    """Dequantized weights [K, N] on the device (bf16 or fp32).  K is needed
    only for flat g / p weights."""
    return _ext.dequant(B, S, layout, out_dtype, K)


def quantize(X, axis=-1, layout=None):
    """Device quantize_mxfp4 (ref.py:14-47) of a 2-D fp32 / bf16 tensor,
    bit-exact with the reference for finite inputs.  axis=0: X is [K, N]
    (returns [K/2, N], [K/32, N] by default); axis=-1: X is [N, K] (returns
    [N, K/2], [N, K/32]).  ``layout`` asks for "kn", "nk", "g" or "p" instead.
    """
    return _ext.quantize(X, axis, layout)


def convert_layout(B, S, src, dst, K=None):
    """(codes, scales) of the same weights in layout ``dst``, rewritten on the
    device.  K is needed only for flat g / p sources."""
    return _ext.convert_layout(B, S, src, dst, K)


def prepack(B_packed, B_scales, layout=LAYOUT_P):
    """Device prepack of reference-layout weights ([K/2, N], [K/32, N]).

    layout "g" gives the strategy-G arrays of ref.py:85-101 (flattened, as
    ``prepack_b_mxfp4`` returns them, ready for ``gemm_g``): the fastest
    layout for M > 32 (the hand-scheduled tiled kernel reads it directly).
    "p" (default) gives the panel layout: the fastest for decode shapes
    (M <= 32, the streaming kernels).
    """
    Bp, Sp = _ext.convert_layout(B_packed, B_scales, LAYOUT_KN, layout, None)
    return (Bp.reshape(-1), Sp.reshape(-1)) if layout == LAYOUT_G else (Bp, Sp)


def select_plan(M, N, K, layout=LAYOUT_KN):
    """(kernel, variant, split_k, description) the cost model picks."""
    return _ext.select_plan(M, N, K, layout)


def describe_plan(plan):
    """Description of a (kernel, variant, split_k[, flags]) plan."""
    return _ext.describe_plan(list(plan))


def version():
    return _ext.version()
