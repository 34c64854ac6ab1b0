"""GPU parity of the gfx950 path against the CPU oracle.

Bar: the dequantized bf16 tile is bit-exact; GEMM outputs are within the
BASELINE tolerance |out - ref| <= 1e-2*sqrt(K/4096) + 2e-2*|ref| of a float64
oracle on the same seeded inputs (the wide-exponent 70B sweep uses the
cancellation-aware bound with c = 4, see oracle.mxfp4_oracle).  Everything
goes through the native extension (no fallback exists).
"""

import math
import os

import numpy as np
import pytest

from oracle import mxfp4_oracle as mo
from tests.gpu_util import full_check_fp32, log, oracle_f64, run_gemm, sample_indices, to_dev_bf16, to_dev_u8

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def kk():
    import torch

    assert torch.cuda.is_available()
    from mxfp4_cdna3 import kernels

    return kernels


def test_device_is_gfx950(kk):
    info = kk.device_info(0)
    log(f"device: {info}")
    assert info["gcn_arch_name"].startswith("gfx950")
    assert info["warp_size"] == 64
    assert info["multi_processor_count"] >= 32


# --------------------------------------------------------------------------- dequant tile

def _table_inputs():
    B = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 256, axis=1)   # [K/2=256, N=256]
    S = np.repeat(np.arange(256, dtype=np.uint8)[None, :], 16, axis=0)    # [K/32=16, N=256]
    return B, S


@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_dequant_exhaustive_bit_exact(kk, layout):
    import torch

    log(f"case dequant exhaustive layout={layout}")
    B, S = _table_inputs()
    if layout == "nk":
        B, S = mo.kn_to_nk(B, S)
    out = kk.dequantize(to_dev_u8(B), to_dev_u8(S), layout, torch.bfloat16)
    torch.cuda.synchronize()
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)  # [512, 256]
    table = np.load(os.path.join(GOLDEN, "dequant_table_bf16.npy"))  # [16 codes, 256 scales]
    Bkn, Skn = _table_inputs()
    want = mo.dequantize_to_bf16_bits(Bkn, Skn, axis=0)
    # Scale bytes 0..254: bit-exact with ref.py (byte 0 = 2**-127, bf16 subnormals kept).
    finite = slice(0, 255)
    assert np.array_equal(got[:, finite], want[:, finite]), "bf16 tile differs for scale bytes 0..254"
    # the fixture (plain-Python brute force) agrees on the same entries
    for code in range(16):
        assert np.array_equal(got[2 * code, finite], table[code, finite])
    # Scale byte 255: ref.py gives +-inf, and NaN for codes 0 and 8 (0 * inf);
    # the tile matches bit for bit except for the NaN payloads (any NaN).
    got255, want255 = mo.bf16_bits_to_f32(got[:, 255]), mo.bf16_bits_to_f32(want[:, 255])
    log(f"scale byte 255 -> {sorted(set(got[:, 255].tolist()))}")
    nan = np.isnan(want255)
    assert nan.sum() == 64 and np.array_equal(np.isnan(got255), nan)
    assert np.array_equal(got[~nan, 255], want[~nan, 255])
    assert np.all(np.isinf(got255[~nan]))


def test_dequant_float32_output(kk):
    import torch

    A_bits, W, S = mo.make_inputs(1, 96, 320, 100, 150, seed=4)
    Bkn, Skn = mo.nk_to_kn(W, S)
    out = kk.dequantize(to_dev_u8(Bkn), to_dev_u8(Skn), "kn", torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), mo.weights_f32(Bkn, Skn, mo.LAYOUT_KN))


# --------------------------------------------------------------------------- GEMM parity

SMALL_SHAPES = [
    # (M, N, K): tails in every dimension, both kernel families
    (1, 256, 256), (3, 128, 64), (16, 2048, 2048), (17, 512, 96), (32, 1024, 512),
    (33, 256, 128), (64, 128, 64), (100, 384, 416), (128, 512, 1024), (257, 768, 320),
    (512, 1024, 256), (300, 272, 160),
]


@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("M,N,K", SMALL_SHAPES)
def test_gemm_small_shapes(kk, M, N, K, layout):
    import torch

    log(f"case gemm M={M} N={N} K={K} layout={layout}")
    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M * 7 + N + K)
    ref = oracle_f64(A_bits, W, S)
    for dt in (torch.float32, torch.bfloat16):
        out = run_gemm(kk, A_bits, W, S, layout, dt)
        assert out.shape == (M, N)
        bad = mo.strict_violations(out, ref, K)
        assert bad == 0, f"{bad} elements outside tolerance (dtype {dt})"


def test_generic_kernel_odd_n(kk):
    import torch

    M, N, K = 40, 100, 96
    log(f"case generic M={M} N={N} K={K}")
    A_bits, W, S = mo.make_inputs(M, N, K, 120, 132, seed=1)
    ref = oracle_f64(A_bits, W, S)
    for layout in ("kn", "nk"):
        out = run_gemm(kk, A_bits, W, S, layout, torch.float32)
        assert mo.strict_violations(out, ref, K) == 0


TILED_VARIANTS = range(16)
PIPE_VARIANTS = range(6, 15)  # pipelined kernel; [N,K/2] needs K % 128 == 0
SCHED_VARIANT = 15            # hand-scheduled kernel: [K/2,N] and G with K % 64 == 0, [N,K/2] with K % 128 == 0
GEMV_VARIANTS = range(15)


@pytest.mark.parametrize("layout,K", [("kn", 672), ("nk", 672), ("nk", 640)])
def test_every_tiled_variant_and_split(kk, layout, K):
    import torch

    M, N = 300, 512  # M tail, 2 N tiles at BN=256; K = 672: K % 64 == 32
    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=21)
    ref = oracle_f64(A_bits, W, S)
    for v in TILED_VARIANTS:
        for split in (1, 2, 3, (K + 63) // 64):  # the last: one 64-K step per split
            log(f"case tiled variant={v} split={split} layout={layout} K={K}")
            plan = (kk.KERNEL_TILED, v, split)
            if (layout == "nk" and K % 128 and v in PIPE_VARIANTS) or (
                    v == SCHED_VARIANT and K % (64 if layout == "kn" else 128)):
                with pytest.raises(RuntimeError, match="invalid argument"):
                    run_gemm(kk, A_bits, W, S, layout, torch.float32, plan=plan)
                continue
            out = run_gemm(kk, A_bits, W, S, layout, torch.float32, plan=plan)
            bad = mo.strict_violations(out, ref, K)
            assert bad == 0, f"variant {v} split {split}: {bad} bad"


@pytest.mark.parametrize("layout", ["kn", "nk", "g"])
@pytest.mark.parametrize("M,N,K", [(300, 528, 640), (64, 256, 128), (513, 1040, 1536)])
def test_sched_kernel_tails_and_splits(kk, layout, M, N, K):
    """Hand-scheduled kernel: M / N tails (N % 256 != 0), splits down to one
    64-K step (odd first steps: the [N,K/2] scale dword half), fp32 and bf16
    out, against the float64 oracle; every split count sums the same 64-K
    partial products (fp32), so splits agree to within fp32 reassociation,
    and bf16 out is the fp32 result rounded."""
    import torch

    if layout == "g":
        N = -(-N // 128) * 128  # G blocks are 128 columns; 640 / 1152 leave a half-empty last tile
    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=33)
    ref = oracle_f64(A_bits, W, S)
    plan = lambda split: (kk.KERNEL_TILED, SCHED_VARIANT, split)
    base = None
    for split in sorted({s for s in (1, 2, 3, K // 64) if s <= K // 64}):
        log(f"case sched {layout} M={M} N={N} K={K} split={split}")
        out = run_gemm(kk, A_bits, W, S, layout, torch.float32, plan=plan(split))
        assert mo.strict_violations(out, ref, K) == 0, f"split {split}"
        again = run_gemm(kk, A_bits, W, S, layout, torch.float32, plan=plan(split))
        assert np.array_equal(out, again), f"split {split}: not deterministic"
        out16 = run_gemm(kk, A_bits, W, S, layout, torch.bfloat16, plan=plan(split))
        assert np.array_equal(out16, mo.bf16_bits_to_f32(mo.f32_to_bf16_bits(out))), f"split {split}: bf16 rounding"
        if base is None:
            base = out
        else:
            np.testing.assert_allclose(out, base, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("N", [514, 260, 42])
def test_tiled_nk_column_tails(kk, N):
    """[N,K/2] weights with N % 16 != 0 on the tiled kernels.  The scheduled
    kernel stores 4 adjacent columns per lane and row, so it takes N % 4 == 0
    only (N = 514 and 42 are rejected before launch, and the auto plan picks
    a kernel with per-column stores); the others store per column.  Every
    variant that takes the shape, and the auto plan, against the oracle."""
    import torch

    M, K = 300, 640
    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=N)
    ref = oracle_f64(A_bits, W, S)
    for plan in [None] + [(kk.KERNEL_TILED, v, s) for v in TILED_VARIANTS for s in (1, 3)]:
        log(f"case tiled nk column tail N={N} plan={plan}")
        if plan is not None and plan[1] == SCHED_VARIANT and N % 4:
            with pytest.raises(RuntimeError, match="invalid argument"):
                run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
            continue
        out = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
        assert mo.strict_violations(out, ref, K) == 0, f"plan {plan}"


def test_kn_weights_of_one_gib(kk):
    """[K/2,N] codes of exactly 1 GiB (K = 32768, N = 65536): past the
    scheduled kernel's descriptor range, so an explicit scheduled plan is
    rejected and the auto plan takes a kernel that rebases per K step; C
    against the float64 oracle on sampled rows and columns (edges included)."""
    import torch

    M, N, K = 300, 65536, 32768
    rng = np.random.default_rng(7)
    A_bits = mo.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    W = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)  # uniform E2M1 codes
    S = rng.integers(122, 131, size=(N, K // 32), dtype=np.uint8)
    Bkn, Skn = mo.nk_to_kn(W, S)
    A, B, Sd = to_dev_bf16(A_bits), to_dev_u8(Bkn), to_dev_u8(Skn)
    del Bkn
    kind, variant, split, desc = kk.select_plan(M, N, K, "kn")
    log(f"case kn 1 GiB auto plan {desc}")
    assert not desc.startswith("tiled-sched")
    with pytest.raises(RuntimeError, match="invalid argument"):
        kk.gemm(A, B, Sd, None, "kn", torch.float32, (kk.KERNEL_TILED, SCHED_VARIANT, 1))
    out = kk.gemm(A, B, Sd, None, "kn", torch.float32)
    torch.cuda.synchronize()
    rows, cols = sample_indices(M, 6, rng), sample_indices(N, 40, rng)
    got = out[torch.from_numpy(rows).cuda()][:, torch.from_numpy(cols).cuda()].cpu().numpy()
    ref = oracle_f64(A_bits, W, S, rows=rows, cols=cols)
    assert mo.strict_violations(got, ref, K) == 0


@pytest.mark.parametrize("K", [192, 448, 1600])
def test_sched_g_odd_step_counts(kk, K):
    """G weights with an odd number of 64-K steps (K % 128 == 64): the G
    loader moves whole 64-K steps, so the scheduled kernel takes these K
    (only [N,K/2] pairs steps for its scale dwords).  Auto plan and explicit
    splits, against the float64 oracle and the [K/2,N] result."""
    import torch

    M, N = 200, 768
    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=K)
    ref = oracle_f64(A_bits, W, S)
    for plan in [None] + [(kk.KERNEL_TILED, SCHED_VARIANT, s) for s in (1, 2, 3) if s <= K // 64]:
        log(f"case sched g K={K} plan={plan}")
        out = run_gemm(kk, A_bits, W, S, "g", torch.float32, plan=plan)
        assert mo.strict_violations(out, ref, K) == 0, f"plan {plan}"
        if plan is not None:
            assert np.array_equal(out, run_gemm(kk, A_bits, W, S, "kn", torch.float32, plan=plan)), f"plan {plan}"


@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("M", [1, 16, 29])
def test_every_gemv_variant_and_split(kk, layout, M):
    import torch

    N, K = 512, 1536
    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M)
    ref = oracle_f64(A_bits, W, S)
    ran = 0
    for v in GEMV_VARIANTS:
        for split in (1, 2, 5):
            try:
                out = run_gemm(kk, A_bits, W, S, layout, torch.float32, plan=(kk.KERNEL_GEMV, v, split))
            except RuntimeError as e:  # shape not valid for this M / layout
                assert "invalid argument" in str(e)
                continue
            log(f"case gemv variant={v} split={split} layout={layout} M={M}")
            ran += 1
            bad = mo.strict_violations(out, ref, K)
            assert bad == 0, f"variant {v} split {split}: {bad} bad"
    assert ran >= 6


# (variant, rows it covers, K per split, K per wave)
STREAM_VARIANTS = [(0, 16, 2048, 256), (1, 16, 1024, 256), (2, 32, 1024, 256),
                   (3, 16, 4096, 512), (4, 32, 2048, 512)]


@pytest.mark.parametrize("variant,mmax,kr,kw", STREAM_VARIANTS)
def test_stream_variants(kk, variant, mmax, kr, kw):
    """Streaming split-K kernel ([N,K/2], M <= 32): ragged M / N, one split,
    a partial last split (K = kr + kw) and the largest split count (K = 8192)."""
    import torch

    for M in (1, 7, mmax):
        for N, K in ((512, min(kr, 2048)), (1000, kr + kw), (4096, 8192), (96, kw)):
            splits = -(-K // kr)
            log(f"case stream variant={variant} M={M} N={N} K={K} splits={splits}")
            A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M + N + K)
            ref = oracle_f64(A_bits, W, S)
            for dt in (torch.float32, torch.bfloat16):
                out = run_gemm(kk, A_bits, W, S, "nk", dt, plan=(kk.KERNEL_STREAM, variant, splits))
                bad = mo.strict_violations(out, ref, K)
                assert bad == 0, f"M={M} N={N} K={K} {dt}: {bad} bad"


# (variant, K per wave, largest K = 16 waves)
WHOLE_VARIANTS = [(5, 512, 8192), (6, 256, 4096)]


@pytest.mark.parametrize("variant,kw,kmax", WHOLE_VARIANTS)
def test_stream_whole_variants(kk, variant, kw, kmax):
    """Whole-K streaming kernel ([N,K/2], M <= 16): one wave (K = kw) up to
    16 waves (K = kmax), ragged M, N % 32 != 0 and odd N (element stores),
    fp32 and bf16 out; repeat calls are bitwise identical and bf16 out is the
    fp32 result rounded."""
    import torch

    for M in (1, 7, 16):
        for N, K in ((512, kw), (1000, 3 * kw), (1001, 2 * kw), (4096, kmax), (96, kmax)):
            log(f"case stream-whole variant={variant} M={M} N={N} K={K}")
            A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M + N + K + 7)
            ref = oracle_f64(A_bits, W, S)
            plan = (kk.KERNEL_STREAM, variant, 1)
            out = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
            bad = mo.strict_violations(out, ref, K)
            assert bad == 0, f"M={M} N={N} K={K}: {bad} bad"
            again = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
            assert np.array_equal(out, again), f"M={M} N={N} K={K}: not deterministic"
            out16 = run_gemm(kk, A_bits, W, S, "nk", torch.bfloat16, plan=plan)
            assert np.array_equal(out16, mo.bf16_bits_to_f32(mo.f32_to_bf16_bits(out))), f"M={M} N={N} K={K}"


@pytest.mark.parametrize("variant,kw,kmax", WHOLE_VARIANTS)
def test_stream_whole_rejects(kk, variant, kw, kmax):
    import torch

    for M, K, split in ((17, kw, 1), (16, kmax + kw, 1), (16, kmax + kw, 2), (16, kw + 32, 1)):
        A_bits, W, S = mo.make_inputs(M, 64, K, 120, 132, seed=4)
        with pytest.raises(RuntimeError, match="invalid argument"):  # M > 16, K > 16 waves, K % kw
            run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=(kk.KERNEL_STREAM, variant, split))


# decode kernel variants: (variant, rows, K per split, K granularity)
DECODE_VARIANTS = [(7, 16, 4096, 512), (8, 8, 8192, 1024)]


@pytest.mark.parametrize("variant,rows,kr,kg", DECODE_VARIANTS)
def test_decode_variants(kk, variant, rows, kr, kg):
    """Decode kernel ([N,K/2], M <= rows): one split, a partial last split,
    up to 8 splits, ragged M, N % 64 != 0 and odd N (element stores), fp32
    and bf16 out; repeat calls are bitwise identical and bf16 out is the
    fp32 result rounded."""
    import torch

    for M in sorted({1, 7, rows}):
        for N, K in ((512, kg), (1000, kr + kg), (1001, 2 * kg), (4096, 8192), (96, 8192), (200, 3 * kr),
                     (256, 8 * kr)):
            splits = -(-K // kr)
            log(f"case decode variant={variant} M={M} N={N} K={K} splits={splits}")
            A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M + N + K + 11)
            ref = oracle_f64(A_bits, W, S)
            plan = (kk.KERNEL_STREAM, variant, splits)
            out = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
            bad = mo.strict_violations(out, ref, K)
            assert bad == 0, f"M={M} N={N} K={K}: {bad} bad"
            again = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
            assert np.array_equal(out, again), f"M={M} N={N} K={K}: not deterministic"
            out16 = run_gemm(kk, A_bits, W, S, "nk", torch.bfloat16, plan=plan)
            assert np.array_equal(out16, mo.bf16_bits_to_f32(mo.f32_to_bf16_bits(out))), f"M={M} N={N} K={K}"


@pytest.mark.parametrize("variant,rows,kr,kg", DECODE_VARIANTS)
def test_decode_rejects(kk, variant, rows, kr, kg):
    import torch

    for M, K, layout, split in ((rows + 1, kg, "nk", 1), (rows, 8 * kr + kg, "nk", 9), (rows, kg + 256, "nk", 1),
                                (rows, kg, "p", 1), (rows, kg, "kn", 1), (rows, 2 * kr, "nk", 1)):
        A_bits, W, S = mo.make_inputs(M, 64, K, 120, 132, seed=4)
        with pytest.raises(RuntimeError, match="invalid argument"):  # M, splits, K granularity, layout, split count
            run_gemm(kk, A_bits, W, S, layout, torch.float32, plan=(kk.KERNEL_STREAM, variant, split))


# resident kernel variants: (variant, rows)
RESIDENT_VARIANTS = [(9, 1), (10, 8), (13, 1)]  # 13: the M = 1 form with dot products


@pytest.mark.parametrize("variant,rows", RESIDENT_VARIANTS)
def test_resident_variants(kk, variant, rows):
    """Resident kernel ([N,K/2], M <= rows, K % 512 == 0, K <= 8192): one wave
    (K = 512) up to 16 waves (K = 8192), ragged M, N % 32 != 0 and odd N,
    fp32 and bf16 out; repeat calls are bitwise identical and bf16 out is
    the fp32 result rounded."""
    import torch

    for M in sorted({1, min(5, rows), rows}):
        for N, K in ((512, 512), (1000, 1536), (1001, 4096), (4096, 8192), (96, 8192), (33, 2560)):
            log(f"case resident variant={variant} M={M} N={N} K={K}")
            A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M + N + K + 13)
            ref = oracle_f64(A_bits, W, S)
            plan = (kk.KERNEL_STREAM, variant, 1)
            out = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
            bad = mo.strict_violations(out, ref, K)
            assert bad == 0, f"M={M} N={N} K={K}: {bad} bad"
            again = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
            assert np.array_equal(out, again), f"M={M} N={N} K={K}: not deterministic"
            out16 = run_gemm(kk, A_bits, W, S, "nk", torch.bfloat16, plan=plan)
            assert np.array_equal(out16, mo.bf16_bits_to_f32(mo.f32_to_bf16_bits(out))), f"M={M} N={N} K={K}"


@pytest.mark.parametrize("variant,rows", RESIDENT_VARIANTS)
def test_resident_rejects(kk, variant, rows):
    import torch

    for M, K, layout, split in ((rows + 1, 512, "nk", 1), (rows, 8704, "nk", 1), (rows, 8704, "nk", 2),
                                (rows, 768, "nk", 1), (rows, 512, "p", 1), (rows, 512, "kn", 1), (rows, 512, "nk", 2)):
        A_bits, W, S = mo.make_inputs(M, 64, K, 120, 132, seed=4)
        with pytest.raises(RuntimeError, match="invalid argument"):  # M, K > 8192, K % 512, layout, split count
            run_gemm(kk, A_bits, W, S, layout, torch.float32, plan=(kk.KERNEL_STREAM, variant, split))


@pytest.mark.parametrize("variant,rows", [(11, 32), (12, 16)])
def test_resident_split_variant(kk, variant, rows):
    """Resident split kernel (variant 11: [N,K/2], M <= 32, 128 columns x 2048
    K per CTA, S = ceil(K / 2048) <= 8 splits): one wave's K (K = 256), a
    partial last split, 4 and 8 splits, ragged M and N, fp32 and bf16 out;
    repeat calls are bitwise identical and bf16 out is the fp32 result
    rounded (the counter-arbitration path: test_gpu_c_abi.py)."""
    import torch

    for M in sorted({1, rows // 2 + 1, rows}):
        for N, K in ((512, 256), (1000, 2048 + 256), (1001, 4096), (4096, 8192), (96, 16384), (200, 6144 + 512)):
            splits = -(-K // 2048)
            log(f"case resident-split variant={variant} M={M} N={N} K={K} splits={splits}")
            A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M + N + K + 17)
            ref = oracle_f64(A_bits, W, S)
            plan = (kk.KERNEL_STREAM, variant, splits)
            out = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
            bad = mo.strict_violations(out, ref, K)
            assert bad == 0, f"M={M} N={N} K={K}: {bad} bad"
            again = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
            assert np.array_equal(out, again), f"M={M} N={N} K={K}: not deterministic"
            out16 = run_gemm(kk, A_bits, W, S, "nk", torch.bfloat16, plan=plan)
            assert np.array_equal(out16, mo.bf16_bits_to_f32(mo.f32_to_bf16_bits(out))), f"M={M} N={N} K={K}"


@pytest.mark.parametrize("variant,rows", [(11, 32), (12, 16)])
def test_resident_split_rejects(kk, variant, rows):
    import torch

    for M, K, layout, split in ((rows + 1, 2048, "nk", 1), (rows, 16384 + 256, "nk", 9), (rows, 2048 + 128, "nk", 2),
                                (rows, 2048, "p", 1), (rows, 2048, "kn", 1), (rows, 4096, "nk", 1)):
        A_bits, W, S = mo.make_inputs(M, 64, K, 120, 132, seed=4)
        with pytest.raises(RuntimeError, match="invalid argument"):  # M, splits, K % 256, layout, split count
            run_gemm(kk, A_bits, W, S, layout, torch.float32, plan=(kk.KERNEL_STREAM, variant, split))


@pytest.mark.parametrize("M", [24, 32])
def test_wide_nk_decode_takes_gemv(kk, M):
    """[N,K/2], 16 < M <= 32, N >= 16384 with K too short to give the
    resident split kernel 192 CTAs: the auto plan is the GEMV family
    (128-column CTAs); checked against the oracle on sampled columns."""
    import torch

    N, K = 16384, 1024
    kind, _, _, desc = kk.select_plan(M, N, K, "nk")
    assert kind == kk.KERNEL_GEMV, desc
    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M + 70)
    cols = np.sort(np.random.default_rng(M).choice(N, 512, replace=False))
    ref = oracle_f64(A_bits, W, S, cols=cols)
    log(f"case wide nk decode M={M} plan={desc}")
    out = run_gemm(kk, A_bits, W, S, "nk", torch.float32)
    assert mo.strict_violations(out[:, cols], ref, K) == 0


def test_stream_rejects_unsupported(kk):
    import torch

    A_bits, W, S = mo.make_inputs(17, 512, 2048, 120, 132, seed=3)
    with pytest.raises(RuntimeError, match="invalid argument"):  # M > 16 for a 16-row variant
        run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=(kk.KERNEL_STREAM, 0, 1))
    with pytest.raises(RuntimeError, match="invalid argument"):  # [K/2,N] weights
        run_gemm(kk, A_bits[:16], W, S, "kn", torch.float32, plan=(kk.KERNEL_STREAM, 0, 1))


def test_stream_repeat_and_shared_workspace(kk):
    """Counters and packets return to zero after every call: repeated calls are
    bitwise identical, also when other split-K kernels use the same
    workspace in between."""
    import torch

    A16, W16, S16 = mo.make_inputs(16, 8192, 8192, 122, 130, seed=9)
    ref = oracle_f64(A16, W16, S16)
    first = run_gemm(kk, A16, W16, S16, "nk", torch.float32)
    assert mo.strict_violations(first, ref, 8192) == 0
    assert kk.select_plan(16, 8192, 8192, "nk")[0] == kk.KERNEL_STREAM
    Am, Wm, Sm = mo.make_inputs(300, 512, 672, 118, 134, seed=2)
    for i in range(3):
        again = run_gemm(kk, A16, W16, S16, "nk", torch.float32)
        assert np.array_equal(first, again), f"repeat {i}"
        run_gemm(kk, Am, Wm, Sm, "kn", torch.float32, plan=(kk.KERNEL_TILED, 6, 3))
        run_gemm(kk, A16, W16, S16, "kn", torch.float32, plan=(kk.KERNEL_GEMV, 0, 4))


def test_split_k_is_deterministic(kk):
    import torch

    M, N, K = 200, 512, 2048
    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=5)
    for plan in ((kk.KERNEL_TILED, 2, 4), (kk.KERNEL_TILED, 0, 3)):
        a = run_gemm(kk, A_bits, W, S, "kn", torch.float32, plan)
        b = run_gemm(kk, A_bits, W, S, "kn", torch.float32, plan)
        assert np.array_equal(a, b)
    A16, W16, S16 = mo.make_inputs(16, 4096, 4096, 122, 130, seed=6)
    a = run_gemm(kk, A16, W16, S16, "kn", torch.float32)
    b = run_gemm(kk, A16, W16, S16, "kn", torch.float32)
    assert np.array_equal(a, b)


def test_empty_and_k0(kk):
    import torch

    A = torch.zeros(0, 64, dtype=torch.bfloat16, device="cuda")
    B = torch.zeros(32, 128, dtype=torch.uint8, device="cuda")
    S = torch.zeros(2, 128, dtype=torch.uint8, device="cuda")
    assert kk.gemm_auto(A, B, S).shape == (0, 128)
    A = torch.ones(4, 0, dtype=torch.bfloat16, device="cuda")
    C = torch.full((4, 128), 7.0, device="cuda")
    out = kk.gemm_auto(A, torch.zeros(0, 128, dtype=torch.uint8, device="cuda"),
                       torch.zeros(0, 128, dtype=torch.uint8, device="cuda"), C)
    torch.cuda.synchronize()
    assert torch.all(out == 0)
    # C a view at an odd bf16 offset (not 16-byte aligned): all of C cleared,
    # the elements on either side kept
    buf = torch.full((4 * 130 + 2,), 5.0, dtype=torch.bfloat16, device="cuda")
    Cv = buf[1:1 + 4 * 130].view(4, 130)
    kk.gemm(A, torch.zeros(0, 130, dtype=torch.uint8, device="cuda"),
            torch.zeros(0, 130, dtype=torch.uint8, device="cuda"), Cv, "kn")
    torch.cuda.synchronize()
    assert torch.all(buf[1:-1] == 0) and buf[0].item() == 5.0 and buf[-1].item() == 5.0


# --------------------------------------------------------------------------- reference API

def test_letter_api_matches_auto_and_rejects_like_reference(kk):
    import torch

    M, N, K = 256, 256, 128
    A_bits, W, S = mo.make_inputs(M, N, K, 120, 132, seed=3)
    Bkn, Skn = mo.nk_to_kn(W, S)
    A, B, Sd = to_dev_bf16(A_bits), to_dev_u8(Bkn), to_dev_u8(Skn)
    ref = kk.gemm_auto(A, B, Sd)
    assert ref.dtype == torch.float32
    for name in "abcdefhijkm":
        out = getattr(kk, f"gemm_{name}")(A, B, Sd)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), name
    C = torch.empty(M, N, dtype=torch.float32, device="cuda")
    assert kk.gemm_j(A, B, Sd, C).data_ptr() == C.data_ptr()
    # M % 64 != 0: A/B return invalid argument, J raises the strategy message
    A48 = A[:48].contiguous()
    with pytest.raises(RuntimeError, match="launch_strategy_b: invalid argument"):
        kk.gemm_b(A48, B, Sd)
    with pytest.raises(RuntimeError, match="Strategy J requires"):
        kk.gemm_j(A48, B, Sd)
    with pytest.raises(RuntimeError, match="B_scales shape"):
        kk.gemm_auto(A, B, Sd[:1].contiguous())
    with pytest.raises(RuntimeError, match="A must be bfloat16"):
        kk.gemm_auto(A.float(), B, Sd)


def test_reference_validate_flow(kk):
    """validate.py:22-62 of the reference: A, B = 0.1*N(0,1) (seed 42), B quantized
    along K, np.allclose(atol=1e-2, rtol=2e-2) against ref_gemm."""
    for M, N, K in ((256, 256, 128), (512, 512, 256), (1024, 1024, 256)):
        log(f"case validate-flow M={M} N={N} K={K}")
        rng = np.random.default_rng(42)
        A_f32 = rng.standard_normal((M, K), dtype=np.float32) * 0.1
        A_bits = mo.f32_to_bf16_bits(A_f32)
        B_f32 = rng.standard_normal((K, N), dtype=np.float32) * 0.1
        Bp, Bs = mo.quantize_mxfp4(B_f32, axis=0)
        C_ref = mo.ref_gemm(mo.bf16_bits_to_f32(A_bits), Bp, Bs)
        out = kk.gemm_j(to_dev_bf16(A_bits), to_dev_u8(Bp), to_dev_u8(Bs)).cpu().numpy()
        assert np.allclose(out, C_ref, atol=1e-2, rtol=2e-2)


# --------------------------------------------------------------------------- BASELINE configs

def _check_config(kk, cfg, layout, rows_k=24, cols_k=1536, strict=True):
    import torch

    rng = np.random.default_rng(1234)
    A_bits, W, S = mo.make_config_inputs(cfg)
    out = run_gemm(kk, A_bits, W, S, layout, torch.bfloat16)
    rows = sample_indices(cfg.M, rows_k, rng)
    cols = sample_indices(cfg.N, cols_k, rng)
    ref, absref = oracle_f64(A_bits, W, S, rows, cols, with_abs=True)
    got = out[np.ix_(rows, cols)]
    strict_bad = mo.strict_violations(got, ref, cfg.K)
    canc_bad = mo.cancellation_violations(got, ref, absref, cfg.K, c=4.0)
    log(f"config {cfg.name} layout={layout}: checked {got.size} elements, strict violations "
        f"{strict_bad}, cancellation-aware (c=4) violations {canc_bad}")
    assert canc_bad == 0
    if strict:
        assert strict_bad == 0
    # size-independent property at full size: every output finite, and a row
    # permutation of A permutes C exactly (rows are independent, fixed K order)
    assert np.isfinite(out).all()
    # every element against a float32 torch reference on the GPU (c = 8: the
    # 4 of the float64 checks above for our sums plus 4 for the reference's)
    full_strict, full_canc = full_check_fp32(A_bits, W, S, out, c=8.0)
    log(f"config {cfg.name} layout={layout}: all {out.size} elements against the float32 reference: strict "
        f"violations {full_strict}, cancellation-aware (c=8) violations {full_canc}")
    assert full_canc == 0
    return A_bits, W, S, out


@pytest.mark.parametrize("name", ["plumbing", "decode_m1", "decode_m8", "decode_m16", "decode_m32"])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_baseline_memory_bound_configs(kk, name, layout):
    cfg = {c.name: c for c in mo.baseline_configs()}[name]
    log(f"case config {name} layout={layout}")
    _check_config(kk, cfg, layout, rows_k=32, cols_k=4096)


@pytest.mark.parametrize("layout", ["kn", "nk", "g"])
@pytest.mark.parametrize("name", ["dit_up", "dit_down"])
def test_baseline_mfma_bound_configs(kk, name, layout):
    """Full size in every layout the scheduled kernel reads."""
    import torch

    cfg = {c.name: c for c in mo.baseline_configs()}[name]
    log(f"case config {name} layout={layout}")
    A_bits, W, S, out = _check_config(kk, cfg, layout)
    perm = np.random.default_rng(0).permutation(cfg.M)
    outp = run_gemm(kk, A_bits[perm], W, S, layout, torch.bfloat16)
    assert np.array_equal(outp, out[perm])
    # linearity in A: 2A -> 2C exactly (power-of-two scaling)
    A2 = mo.f32_to_bf16_bits(2.0 * mo.bf16_bits_to_f32(A_bits))
    out2 = run_gemm(kk, A2, W, S, layout, torch.float32)
    out1 = run_gemm(kk, A_bits, W, S, layout, torch.float32)
    assert np.array_equal(out2, 2.0 * out1)


@pytest.mark.parametrize("m", [1, 16, 128, 512, 2048, 8192])
def test_baseline_70b_sweep(kk, m):
    cfg = {c.name: c for c in mo.baseline_configs()}[f"ffn70b_m{m}"]
    log(f"case config {cfg.name}")
    _check_config(kk, cfg, "kn" if m % 2 else "nk", rows_k=16, cols_k=1024, strict=False)
