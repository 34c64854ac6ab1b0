"""CPU checks of the weight layouts: the oracle's packers and the device code's
index functions.

* ``panel_pack`` (the panel layout P) is pinned by its definition evaluated
  with plain-Python index loops, by being a bijection and by its inverse.
* The C++ index functions every kernel uses (cdna3-bench_amd/csrc/
  mxfp4_layout.h) are compiled for the host with g++ and must put every code
  and scale byte exactly where the oracle's packers put it, for all four
  layouts (KN, NK, G = ref.py:85-101, P).
* The C-ABI enforces each layout's shape rule and plans a native kernel.
"""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from oracle import mxfp4_oracle as mo

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "cdna3-bench_amd", "csrc")
HEADER = os.path.join(REPO, "include", "mxfp4_mi355x.h")
LIB = os.path.join(REPO, "cdna3-bench_amd", "mxfp4_cdna3", "libmxfp4_mi355x.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

hipSuccess, hipErrorInvalidValue = 0, 1


def test_panel_pack_matches_its_definition():
    rng = np.random.default_rng(3)
    K, N = 192, 96
    B = rng.integers(0, 256, (K // 2, N), dtype=np.uint8)
    S = rng.integers(0, 256, (K // 32, N), dtype=np.uint8)
    P, Ps = mo.panel_pack(B, S)
    # definition: block (p, t) = 32 columns x 64 K, 1 KB; lane 32h + c holds
    # the 16 bytes of column 32p + c for K 64t + 32h .. +31 (byte j = K pair
    # 32t + 16h + j); the block's 64 scale bytes follow the same lane order.
    for p in range(N // 32):
        for t in range(K // 64):
            blk = p * (K // 64) + t
            for h in range(2):
                for c in range(32):
                    lane = 32 * h + c
                    for j in range(16):
                        assert P[blk * 1024 + lane * 16 + j] == B[32 * t + 16 * h + j, 32 * p + c]
                    assert Ps[blk * 64 + lane] == S[2 * t + h, 32 * p + c]


def test_panel_pack_is_a_bijection_with_inverse():
    K, N = 256, 64
    ids_b = np.arange(K // 2 * N, dtype=np.int64).reshape(K // 2, N)
    ids_s = np.arange(K // 32 * N, dtype=np.int64).reshape(K // 32, N)
    P, Ps = mo.panel_pack(ids_b, ids_s)
    assert np.array_equal(np.sort(P), ids_b.ravel()) and np.array_equal(np.sort(Ps), ids_s.ravel())
    B2, S2 = mo.panel_unpack(P, Ps, K, N)
    assert np.array_equal(B2, ids_b) and np.array_equal(S2, ids_s)
    with pytest.raises(ValueError):
        mo.panel_pack(ids_b[:, :48], ids_s[:, :48])


@pytest.mark.parametrize("layout", [mo.LAYOUT_KN, mo.LAYOUT_NK, mo.LAYOUT_G, mo.LAYOUT_P])
def test_from_layout_inverts_to_layout(layout):
    rng = np.random.default_rng(layout)
    K, N = 128, 256
    B = rng.integers(0, 256, (K // 2, N), dtype=np.uint8)
    S = rng.integers(0, 256, (K // 32, N), dtype=np.uint8)
    X, Xs = mo.to_layout(B, S, layout)
    B2, S2 = mo.from_layout(X, Xs, layout, K, N)
    assert np.array_equal(B2, B) and np.array_equal(S2, S)


def test_header_layout_tags_match_oracle():
    text = open(HEADER).read()
    m = re.search(r"enum \{ MXFP4_LAYOUT_KN = (\d), MXFP4_LAYOUT_NK = (\d), MXFP4_LAYOUT_G = (\d), "
                  r"MXFP4_LAYOUT_P = (\d) \};", text)
    assert m, "layout enum not found"
    assert tuple(int(x) for x in m.groups()) == (mo.LAYOUT_KN, mo.LAYOUT_NK, mo.LAYOUT_G, mo.LAYOUT_P)


@pytest.fixture(scope="module")
def index_dump(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("layout") / "layout_index_dump")
    src = os.path.join(REPO, "tests", "native", "layout_index_dump.cpp")
    subprocess.run(["g++", "-O1", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include",
                    f"-I{CSRC}", src, "-o", exe], check=True)

    def run(layout, K, N):
        out = subprocess.run([exe, str(layout), str(K), str(N)], check=True, capture_output=True).stdout
        a = np.frombuffer(out, dtype=np.uint64)
        nb, ns = K // 2 * N, K // 32 * N
        assert a.size == nb + ns + 1
        return a[:nb].reshape(K // 2, N), a[nb:nb + ns].reshape(K // 32, N), int(a[-1])

    return run


@pytest.mark.parametrize("layout,K,N", [
    (mo.LAYOUT_KN, 64, 40), (mo.LAYOUT_KN, 96, 48), (mo.LAYOUT_NK, 64, 40), (mo.LAYOUT_NK, 96, 48),
    (mo.LAYOUT_G, 64, 256), (mo.LAYOUT_G, 96, 128), (mo.LAYOUT_P, 128, 64), (mo.LAYOUT_P, 192, 96),
])
def test_device_index_functions_match_oracle(index_dump, layout, K, N):
    code_off, scale_off, bad_inverse = index_dump(layout, K, N)
    assert bad_inverse == 0  # code_position / scale_position invert the offsets
    ids_b = np.arange(K // 2 * N, dtype=np.int64).reshape(K // 2, N)
    ids_s = np.arange(K // 32 * N, dtype=np.int64).reshape(K // 32, N)
    X, Xs = mo.to_layout(ids_b, ids_s, layout)
    X, Xs = np.asarray(X).ravel(), np.asarray(Xs).ravel()
    # byte (kp, n) sits at code_offset(kp, n) in the oracle's packed array
    assert np.array_equal(X[code_off.astype(np.int64)], ids_b)
    assert np.array_equal(Xs[scale_off.astype(np.int64)], ids_s)


# ---- C-ABI: layout rules and plans (no kernel runs) ----------------------------

class Plan(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int32), ("variant", ctypes.c_int32),
                ("split_k", ctypes.c_int32), ("flags", ctypes.c_int32)]


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libmxfp4_mi355x.so not built (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB)
    i64, p = ctypes.c_int64, ctypes.c_void_p
    L.mxfp4_select_plan.argtypes = [i64, i64, i64, ctypes.c_int, p]
    L.mxfp4_gemm_workspace_bytes.argtypes = [i64, i64, i64, ctypes.c_int, p]
    L.mxfp4_gemm_workspace_bytes.restype = ctypes.c_size_t
    L.mxfp4_gemm.argtypes = [p, p, p, p, ctypes.c_int, i64, i64, i64, ctypes.c_int, p, ctypes.c_size_t, p]
    L.mxfp4_dequant.argtypes = [p, p, p, ctypes.c_int, i64, i64, ctypes.c_int, p]
    L.mxfp4_convert_layout.argtypes = [p, p, ctypes.c_int, p, p, ctypes.c_int, i64, i64, p]
    L.mxfp4_plan_describe.argtypes = [p, ctypes.c_char_p, ctypes.c_size_t]
    return L


def _plan(lib, M, N, K, layout):
    p = Plan()
    rc = lib.mxfp4_select_plan(M, N, K, layout, ctypes.byref(p))
    if rc != hipSuccess:
        return rc, None, None
    buf = ctypes.create_string_buffer(128)
    assert lib.mxfp4_plan_describe(ctypes.byref(p), buf, 128) == hipSuccess
    return rc, p, buf.value.decode()


def test_layout_shape_rules(lib):
    assert _plan(lib, 16, 8192 + 64, 8192, mo.LAYOUT_G)[0] == hipErrorInvalidValue  # N % 128
    assert _plan(lib, 16, 8192 + 16, 8192, mo.LAYOUT_P)[0] == hipErrorInvalidValue  # N % 32
    assert _plan(lib, 16, 8192, 8192 + 32, mo.LAYOUT_P)[0] == hipErrorInvalidValue  # K % 64
    assert _plan(lib, 16, 8192, 8192 + 32, mo.LAYOUT_G)[0] == hipSuccess
    assert _plan(lib, 16, 8192, 8192, 4)[0] == hipErrorInvalidValue
    dummy = ctypes.c_void_p(0x1000)
    assert lib.mxfp4_gemm(dummy, dummy, dummy, dummy, 0, 16, 8192 + 64, 8192, mo.LAYOUT_G, None, 0,
                          None) == hipErrorInvalidValue
    assert lib.mxfp4_dequant(dummy, dummy, dummy, 1, 8192 + 32, 64, mo.LAYOUT_P, None) == hipErrorInvalidValue


@pytest.mark.parametrize("M,N,K,layout,kernel,prefix", [
    (16, 8192, 8192, mo.LAYOUT_P, 4, "stream"),
    (32, 8192, 8192, mo.LAYOUT_P, 4, "stream"),
    (16, 8192, 8192, mo.LAYOUT_G, 2, "tiled-"),  # the scheduled or the pipelined kernel, split-K
    (4096, 12288, 3072, mo.LAYOUT_G, 2, "tiled-sched"),
    (4096, 12288, 3072, mo.LAYOUT_P, 2, "tiled-pipe"),
    (64, 96, 64, mo.LAYOUT_P, 2, "tiled-pipe"),
])
def test_prepacked_layouts_plan_native_kernels(lib, M, N, K, layout, kernel, prefix):
    rc, p, desc = _plan(lib, M, N, K, layout)
    assert rc == hipSuccess
    assert p.kernel == kernel and desc.startswith(prefix), desc
    # the first tiled kernel has no G / P loader: rejected
    assert lib.mxfp4_gemm_workspace_bytes(M, N, K, layout, ctypes.byref(Plan(2, 1, 2, 0))) == 0
    # the GEMV family has none either
    assert lib.mxfp4_gemm_workspace_bytes(M, N, K, layout, ctypes.byref(Plan(1, 0, 2, 0))) == 0


def test_convert_layout_argument_errors(lib):
    a, b = ctypes.c_void_p(0x100000), ctypes.c_void_p(0x200000)
    s, t = ctypes.c_void_p(0x300000), ctypes.c_void_p(0x400000)
    cv = lib.mxfp4_convert_layout
    assert cv(a, s, 0, b, t, 3, 64, 48, None) == hipErrorInvalidValue   # P needs N % 32
    assert cv(a, s, 0, b, t, 2, 64, 64, None) == hipErrorInvalidValue   # G needs N % 128
    assert cv(a, s, 0, b, t, 3, 96, 64, None) == hipErrorInvalidValue   # P needs K % 64
    assert cv(a, s, 0, b, t, 5, 64, 64, None) == hipErrorInvalidValue   # unknown layout
    assert cv(a, s, 0, b, t, 1, 48, 64, None) == hipErrorInvalidValue   # K % 32
    assert cv(a, s, 0, a, t, 1, 64, 64, None) == hipErrorInvalidValue   # codes overlap
    assert cv(a, s, 0, b, s, 1, 64, 64, None) == hipErrorInvalidValue   # scales overlap
    assert cv(a, s, 0, ctypes.c_void_p(0x200008), t, 1, 64, 64, None) == hipErrorInvalidValue  # unaligned
    assert cv(None, None, 0, None, None, 1, 0, 64, None) == hipSuccess  # empty
