"""mxfp4_cdna3 -- MXFP4-weight x BF16-activation GEMM for MI355X (gfx950).

Drop-in for konradha/cdna3-bench's ``mxfp4_cdna3`` operator package
(python/mxfp4_cdna3/__init__.py:1-22): the same lazily loaded kernel API
(``gemm_a`` .. ``gemm_m``, ``gemm_g``, ``gemm_auto``, ``device_info``,
``shape_supported_*``), backed by hand-written gfx950 HIP kernels through the
C ABI in include/mxfp4_mi355x.h.  The kernels load on first attribute access
so ``import mxfp4_cdna3`` works on a host without a GPU.

The reference's package-level functions (``quantize_mxfp4``,
``dequantize_mxfp4``, ``ref_gemm``, ``preshuffle_b``; __init__.py:1) come
from ``mxfp4_cdna3.ref``, which computes them on the GPU with the same
arguments and shapes as python/mxfp4_cdna3/ref.py.
"""

from .ref import dequantize_mxfp4, preshuffle_b, quantize_mxfp4, ref_gemm

__version__ = "0.1.0"

_KERNEL_NAMES = (
    "gemm_a", "gemm_b", "gemm_c", "gemm_d", "gemm_e", "gemm_f", "gemm_g", "gemm_h",
    "gemm_i", "gemm_j", "gemm_k", "gemm_m", "gemm_auto", "gemm", "dequantize", "quantize", "convert_layout", "prepack",
    "select_plan", "describe_plan", "device_info", "shape_supported_c", "shape_supported_d",
    "shape_supported_e", "shape_supported_f", "shape_supported_g", "version",
    "LAYOUT_KN", "LAYOUT_NK", "LAYOUT_G", "LAYOUT_P", "KERNEL_AUTO", "KERNEL_GEMV", "KERNEL_TILED", "KERNEL_GENERIC", "KERNEL_STREAM", "PLAN_STREAM_NO_POLL",
)

__all__ = ["dequantize_mxfp4", "preshuffle_b", "quantize_mxfp4", "ref_gemm"] + list(_KERNEL_NAMES)


def __getattr__(name):
    if name in _KERNEL_NAMES:
        from . import kernels

        return getattr(kernels, name)
    raise AttributeError(name)
