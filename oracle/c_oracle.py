"""ctypes loader for the C restatement (mxfp4_oracle.c).

TEST INFRASTRUCTURE ONLY (see mxfp4_oracle.py's header).  The shared library
is built by ``oracle/Makefile`` (called from ``__graft_entry__.build()``).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_mxfp4.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.mxo_dequant_bf16.argtypes = [p, p, i64, i64, ctypes.c_int, p]
        L.mxo_dequant_bf16.restype = None
        L.mxo_gemm_f64.argtypes = [p, p, p, i64, i64, i64, ctypes.c_int, p, p]
        L.mxo_gemm_f64.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def dequant_bf16(B, S, K, N, layout):
    B = np.ascontiguousarray(B, dtype=np.uint8)
    S = np.ascontiguousarray(S, dtype=np.uint8)
    out = np.empty((K, N), dtype=np.uint16)
    lib().mxo_dequant_bf16(_ptr(B), _ptr(S), K, N, layout, _ptr(out))
    return out


def gemm_f64(A_bits, B, S, M, N, K, layout, with_abs=True):
    A_bits = np.ascontiguousarray(A_bits, dtype=np.uint16)
    B = np.ascontiguousarray(B, dtype=np.uint8)
    S = np.ascontiguousarray(S, dtype=np.uint8)
    C = np.empty((M, N), dtype=np.float64)
    Ca = np.empty((M, N), dtype=np.float64) if with_abs else None
    rc = lib().mxo_gemm_f64(_ptr(A_bits), _ptr(B), _ptr(S), M, N, K, layout, _ptr(C),
                            _ptr(Ca) if Ca is not None else None)
    if rc != 0:
        raise MemoryError("mxo_gemm_f64 failed to allocate")
    return C, Ca
