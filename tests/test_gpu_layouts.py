"""GPU parity of the prepacked weight layouts: the device layout conversion
(prepack) and the G / P loaders of the GEMM kernels.

Bars:
* layout conversion is a byte permutation: bit-exact against the oracle's
  packers (ref.py:85-101 for G; the panel layout's definition for P), for
  every pair of layouts;
* the dequantized tile from G / P weights is bit-identical to the one from
  the reference layout;
* a GEMM over G (P) weights gives bit-identical results to the same plan
  over [K/2,N] ([N,K/2]) weights -- the loaders feed the MFMAs the same
  operands in the same order -- and meets the BASELINE tolerance against the
  float64 oracle;
* gemm_g follows the reference's validate flow (validate.py:66-79) and
  rejects what the reference rejects, with the same messages.
"""

import numpy as np
import pytest

from oracle import mxfp4_oracle as mo
from tests.gpu_util import LAYOUT_TAGS, log, oracle_f64, run_gemm, to_dev_bf16, to_dev_u8

pytestmark = pytest.mark.gpu

LAYOUTS = ["kn", "nk", "g", "p"]


@pytest.fixture(scope="module")
def kk():
    import torch

    assert torch.cuda.is_available()
    from mxfp4_cdna3 import kernels

    return kernels


def _rand_weights(K, N, seed):
    rng = np.random.default_rng(seed)
    B = rng.integers(0, 256, (K // 2, N), dtype=np.uint8)
    S = rng.integers(0, 256, (K // 32, N), dtype=np.uint8)
    return B, S


def _host(B, S, layout):
    X, Xs = mo.to_layout(B, S, LAYOUT_TAGS[layout])
    return np.ascontiguousarray(X), np.ascontiguousarray(Xs)


# [N,K/2] -> G conversion tiles hold 64 code dwords (512 K): K = 64 and 192
# fill one partly, 1024 two exactly, 4160 eight and a partial ninth
@pytest.mark.parametrize("K,N", [(64, 128), (192, 384), (1024, 256), (4160, 256)])
def test_convert_layout_every_pair(kk, K, N):
    import torch

    B, S = _rand_weights(K, N, K + N)
    for src in LAYOUTS:
        Xb, Xs = _host(B, S, src)
        db, ds = to_dev_u8(Xb), to_dev_u8(Xs)
        for dst in LAYOUTS:
            log(f"case convert {src}->{dst} K={K} N={N}")
            ob, os_ = kk.convert_layout(db, ds, src, dst, K)
            torch.cuda.synchronize()
            Yb, Ys = _host(B, S, dst)
            assert np.array_equal(ob.cpu().numpy().ravel(), Yb.ravel()), f"codes {src}->{dst}"
            assert np.array_equal(os_.cpu().numpy().ravel(), Ys.ravel()), f"scales {src}->{dst}"


def test_convert_kn_nk_ragged_n(kk):
    import torch

    K, N = 96, 40  # N % 16 != 0: [K/2,N] rows end inside a 16-byte vector
    B, S = _rand_weights(K, N, 7)
    log("case convert kn<->nk N=40")
    nb, ns = kk.convert_layout(to_dev_u8(B), to_dev_u8(S), "kn", "nk")
    kb, ks = kk.convert_layout(nb, ns, "nk", "kn")
    torch.cuda.synchronize()
    assert np.array_equal(nb.cpu().numpy(), B.T) and np.array_equal(ns.cpu().numpy(), S.T)
    assert np.array_equal(kb.cpu().numpy(), B) and np.array_equal(ks.cpu().numpy(), S)


def test_prepack_is_reference_prepack(kk):
    import torch

    K, N = 512, 384
    B, S = _rand_weights(K, N, 11)
    log("case prepack g / p")
    gb, gs = kk.prepack(to_dev_u8(B), to_dev_u8(S), "g")
    pb, ps = kk.prepack(to_dev_u8(B), to_dev_u8(S), "p")
    torch.cuda.synchronize()
    rb, rs = mo.prepack_b_mxfp4(B, S)
    assert gb.dim() == 1 and np.array_equal(gb.cpu().numpy(), rb) and np.array_equal(gs.cpu().numpy(), rs)
    qb, qs = mo.panel_pack(B, S)
    assert np.array_equal(pb.cpu().numpy().ravel(), qb) and np.array_equal(ps.cpu().numpy().ravel(), qs)


@pytest.mark.parametrize("layout", ["g", "p"])
def test_dequant_prepacked_bit_exact(kk, layout):
    import torch

    # every code byte x every scale byte (K/2 = 256 rows of codes 0..255)
    B = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 256, axis=1)
    S = np.repeat(np.arange(256, dtype=np.uint8)[None, :], 16, axis=0)
    log(f"case dequant exhaustive layout={layout}")
    base = kk.dequantize(to_dev_u8(B), to_dev_u8(S), "kn", torch.bfloat16)
    Xb, Xs = _host(B, S, layout)
    got = kk.dequantize(to_dev_u8(Xb), to_dev_u8(Xs), layout, torch.bfloat16, 512)
    f32 = kk.dequantize(to_dev_u8(Xb), to_dev_u8(Xs), layout, torch.float32, 512)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), base.view(torch.int16))
    assert torch.equal(f32.view(torch.int32), (base.view(torch.int16).to(torch.int32) << 16))


PIPE_VARIANTS = range(6, 15)


@pytest.mark.parametrize("pre,base,K", [("g", "kn", 640), ("g", "kn", 672), ("p", "nk", 640)])
def test_tiled_prepacked_equals_base_layout(kk, pre, base, K):
    import torch

    M, N = 300, 512  # M tail; two 256-column tiles; K = 672 leaves a half 64-K step (G only)
    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=31)
    ref = oracle_f64(A_bits, W, S)
    for v in PIPE_VARIANTS:
        for split in (1, 3):
            log(f"case tiled-pipe {pre} vs {base} variant={v} split={split} K={K}")
            plan = (kk.KERNEL_TILED, v, split)
            a = run_gemm(kk, A_bits, W, S, pre, torch.float32, plan=plan)
            b = run_gemm(kk, A_bits, W, S, base, torch.float32, plan=plan)
            assert np.array_equal(a, b), f"variant {v} split {split}"
            assert mo.strict_violations(a, ref, K) == 0


VIA_G = 2  # MXFP4_PLAN_TILED_VIA_G


@pytest.mark.parametrize("M,N,K,split", [(300, 512, 640, 1), (300, 512, 640, 2), (130, 1280, 4224, 3)])
def test_tiled_via_g_equals_direct_nk(kk, M, N, K, split):
    """A via-G plan ([N,K/2] weights rewritten to G in the workspace, after
    the split-K region, then the scheduled kernel on G) is bit-identical to
    the same scheduled plan on the [N,K/2] weights -- both feed the MFMAs
    the same operands in the same K order -- and meets the tolerance.  The
    cases run in order on one stream's workspace: a split-K call after a
    split-1 via-G call finds its counters zero (the G copy once overwrote
    them)."""
    import torch

    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M + K)
    ref = oracle_f64(A_bits, W, S)
    log(f"case via-g M={M} N={N} K={K} split={split}")
    plan = (kk.KERNEL_TILED, 15, split)
    a = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan + (VIA_G,))
    b = run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=plan)
    assert np.array_equal(a, b)
    assert mo.strict_violations(a, ref, K) == 0
    c = run_gemm(kk, A_bits, W, S, "nk", torch.bfloat16, plan=plan + (VIA_G,))
    d = run_gemm(kk, A_bits, W, S, "nk", torch.bfloat16, plan=plan)
    assert np.array_equal(c, d)


def test_tiled_via_g_rejected_where_g_cannot_hold_the_weights(kk):
    import torch

    A_bits, W, S = mo.make_inputs(64, 320, 640, 118, 134, seed=5)  # N % 128 != 0
    log("case via-g rejected N=320")
    with pytest.raises(RuntimeError):
        run_gemm(kk, A_bits, W, S, "nk", torch.float32, plan=(kk.KERNEL_TILED, 15, 1, VIA_G))
    A_bits, W, S = mo.make_inputs(64, 256, 640, 118, 134, seed=6)
    with pytest.raises(RuntimeError):  # [K/2,N] weights: the flag is for [N,K/2] only
        run_gemm(kk, A_bits, W, S, "kn", torch.float32, plan=(kk.KERNEL_TILED, 15, 1, VIA_G))
    torch.cuda.synchronize()


@pytest.mark.parametrize("M", [16, 300])
def test_tiled_p_odd_step_count(kk, M):
    """P weights with K % 128 == 64 (an odd number of 64-K panels): the
    pipelined kernel reads P scales per panel, so it takes these K; the
    streaming kernels need K % 256 and leave them to it.  Auto plan and every
    pipelined variant, against the float64 oracle."""
    import torch

    N, K = 512, 576
    A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=41)
    ref = oracle_f64(A_bits, W, S)
    for plan in [None] + [(kk.KERNEL_TILED, v, s) for v in PIPE_VARIANTS for s in (1, 3)]:
        log(f"case tiled p M={M} K={K} plan={plan}")
        out = run_gemm(kk, A_bits, W, S, "p", torch.float32, plan=plan)
        assert mo.strict_violations(out, ref, K) == 0, f"plan {plan}"


def test_tiled_rejects_prepacked_without_loader(kk):
    import torch

    A_bits, W, S = mo.make_inputs(128, 256, 256, 120, 132, seed=1)
    for layout in ("g", "p"):
        with pytest.raises(RuntimeError, match="invalid argument"):  # non-pipelined tiled variant
            run_gemm(kk, A_bits, W, S, layout, torch.float32, plan=(kk.KERNEL_TILED, 1, 1))
        with pytest.raises(RuntimeError, match="invalid argument"):  # GEMV family
            run_gemm(kk, A_bits[:16], W, S, layout, torch.float32, plan=(kk.KERNEL_GEMV, 0, 1))


STREAM_VARIANTS = [(0, 16, 2048, 256), (1, 16, 1024, 256), (2, 32, 1024, 256),
                   (3, 16, 4096, 512), (4, 32, 2048, 512)]


@pytest.mark.parametrize("variant,mmax,kr,kw", STREAM_VARIANTS)
def test_stream_panels_equal_nk(kk, variant, mmax, kr, kw):
    import torch

    for M in (1, mmax):
        for N, K in ((512, min(kr, 2048)), (992, kr + kw), (4096, 8192), (96, kw)):
            splits = -(-K // kr)
            log(f"case stream p vs nk variant={variant} M={M} N={N} K={K} splits={splits}")
            A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M + N + K + 1)
            ref = oracle_f64(A_bits, W, S)
            plan = (kk.KERNEL_STREAM, variant, splits)
            for dt in (torch.float32, torch.bfloat16):
                a = run_gemm(kk, A_bits, W, S, "p", dt, plan=plan)
                b = run_gemm(kk, A_bits, W, S, "nk", dt, plan=plan)
                assert np.array_equal(a, b), f"M={M} N={N} K={K} {dt}"
                assert mo.strict_violations(a, ref, K) == 0


@pytest.mark.parametrize("variant,kw,kmax", [(5, 512, 8192), (6, 256, 4096)])
def test_stream_whole_panels_equal_nk(kk, variant, kw, kmax):
    import torch

    for M in (1, 16):
        for N, K in ((512, kw), (992, 3 * kw), (4096, kmax)):
            log(f"case stream-whole p vs nk variant={variant} M={M} N={N} K={K}")
            A_bits, W, S = mo.make_inputs(M, N, K, 118, 134, seed=M + N + K + 3)
            ref = oracle_f64(A_bits, W, S)
            plan = (kk.KERNEL_STREAM, variant, 1)
            for dt in (torch.float32, torch.bfloat16):
                a = run_gemm(kk, A_bits, W, S, "p", dt, plan=plan)
                b = run_gemm(kk, A_bits, W, S, "nk", dt, plan=plan)
                assert np.array_equal(a, b), f"M={M} N={N} K={K} {dt}"
                assert mo.strict_violations(a, ref, K) == 0


@pytest.mark.parametrize("M", [1, 16, 32])
def test_auto_plans_on_prepacked_decode_shapes(kk, M):
    """Decode shapes through the auto plan: P streams, G runs the tiled kernel
    with split-K."""
    import torch

    N, K = 8192, 8192
    A_bits, W, S = mo.make_inputs(M, N, K, 122, 130, seed=40 + M)
    cols = np.sort(np.random.default_rng(M).choice(N, 1024, replace=False))
    ref = oracle_f64(A_bits, W, S, cols=cols)
    assert kk.select_plan(M, N, K, "p")[0] == kk.KERNEL_STREAM
    assert kk.select_plan(M, N, K, "g")[0] == kk.KERNEL_TILED
    for layout in ("g", "p"):
        log(f"case auto decode layout={layout} M={M} plan={kk.select_plan(M, N, K, layout)}")
        out = run_gemm(kk, A_bits, W, S, layout, torch.bfloat16)
        assert mo.strict_violations(out[:, cols], ref, K) == 0


def test_gemm_g_reference_validate_flow(kk):
    """validate.py:66-79: prepack_b_mxfp4 on the host, gemm_g, allclose(1e-2, 2e-2)."""
    for M, N, K in ((256, 256, 128), (512, 512, 256), (1024, 1024, 256)):
        log(f"case gemm_g validate-flow M={M} N={N} K={K}")
        rng = np.random.default_rng(42)
        A_f32 = rng.standard_normal((M, K), dtype=np.float32) * 0.1
        A_bits = mo.f32_to_bf16_bits(A_f32)
        B_f32 = rng.standard_normal((K, N), dtype=np.float32) * 0.1
        Bp, Bs = mo.quantize_mxfp4(B_f32, axis=0)
        C_ref = mo.ref_gemm(mo.bf16_bits_to_f32(A_bits), Bp, Bs)
        Gp, Gs = mo.prepack_b_mxfp4(Bp, Bs)
        out = kk.gemm_g(to_dev_bf16(A_bits), to_dev_u8(Gp), to_dev_u8(Gs)).cpu().numpy()
        assert out.dtype == np.float32 and out.shape == (M, N)
        assert np.allclose(out, C_ref, atol=1e-2, rtol=2e-2)
        # the letter API over the reference layout agrees within float32 rounding
        ref_letter = kk.gemm_d(to_dev_bf16(A_bits), to_dev_u8(Bp), to_dev_u8(Bs)).cpu().numpy()
        assert np.allclose(out, ref_letter, atol=1e-5, rtol=1e-5)


def test_gemm_g_dit_up_full_size(kk):
    """dit_up (M=4096, N=12288, K=3072) through gemm_g vs the same plan over
    [K/2,N] weights: bit-identical; sampled rows x columns vs float64."""
    import torch

    cfg = next(c for c in mo.baseline_configs() if c.name == "dit_up")
    A_bits, W, S = mo.make_config_inputs(cfg)
    M, N, K = cfg.M, cfg.N, cfg.K
    B, Sk = mo.nk_to_kn(W, S)
    Gp, Gs = mo.prepack_b_mxfp4(B, Sk)
    A = to_dev_bf16(A_bits)
    log("case gemm_g dit_up")
    out_g = kk.gemm_g(A, to_dev_u8(Gp), to_dev_u8(Gs))
    plan = kk.select_plan(M, N, K, "g")
    out_kn = kk.gemm(A, to_dev_u8(B), to_dev_u8(Sk), None, "kn", torch.float32, list(plan[:3]))
    torch.cuda.synchronize()
    assert torch.equal(out_g, out_kn), plan
    rng = np.random.default_rng(0)
    rows = np.sort(rng.choice(M, 16, replace=False))
    cols = np.sort(rng.choice(N, 1024, replace=False))
    ref = oracle_f64(A_bits, W, S, rows=rows, cols=cols)
    got = out_g.cpu().numpy()[np.ix_(rows, cols)]
    assert mo.strict_violations(got, ref, K) == 0


def test_gemm_g_rejects_like_reference(kk):
    import torch

    A = torch.zeros(64, 256, dtype=torch.bfloat16, device="cuda")
    Bp = torch.zeros(128 * 128, dtype=torch.uint8, device="cuda")
    Bs = torch.zeros(256 * 128 // 32, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match=r"Strategy G requires M%128==0, N%128==0, K%64==0"):
        kk.gemm_g(A, Bp, Bs)
    A = torch.zeros(128, 256, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="B_prep size not consistent with K/2 byte stride"):
        kk.gemm_g(A, Bp[:-1], Bs)
    with pytest.raises(RuntimeError, match=r"Bs_prep size != K\*N/32"):
        kk.gemm_g(A, Bp, Bs[:-1])
    with pytest.raises(RuntimeError, match="A bf16"):
        kk.gemm_g(A.float(), Bp, Bs)
