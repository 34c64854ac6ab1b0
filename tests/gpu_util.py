"""Helpers for the GPU parity tests: device tensors from oracle inputs and the
sampled float64 oracle."""

import sys

import numpy as np

from oracle import mxfp4_oracle as mo


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def to_dev_bf16(A_bits):
    import torch

    return torch.from_numpy(np.ascontiguousarray(A_bits).view(np.int16)).view(torch.bfloat16).cuda()


def to_dev_u8(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


LAYOUT_TAGS = {"kn": mo.LAYOUT_KN, "nk": mo.LAYOUT_NK, "g": mo.LAYOUT_G, "p": mo.LAYOUT_P}


def weights_for_layout(W_nk, S_nk, layout):
    """[N, K/2] weights in ``layout`` (g and p flat, as the oracle packers give them)."""
    if layout == "nk":
        return W_nk, S_nk
    B, S = mo.nk_to_kn(W_nk, S_nk)
    return mo.to_layout(B, S, LAYOUT_TAGS[layout])


def run_gemm(kk, A_bits, W_nk, S_nk, layout="kn", out_dtype=None, plan=None):
    import torch

    B, S = weights_for_layout(W_nk, S_nk, layout)
    out = kk.gemm(to_dev_bf16(A_bits), to_dev_u8(B), to_dev_u8(S), None, layout,
                  out_dtype if out_dtype is not None else torch.float32, plan)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def oracle_f64(A_bits, W_nk, S_nk, rows=None, cols=None, with_abs=False):
    """float64 C (and sum |a||w|) on the given row/column subsets ([N, K/2] weights)."""
    A = mo.bf16_bits_to_f32(A_bits if rows is None else A_bits[rows])
    W = W_nk if cols is None else W_nk[cols]
    S = S_nk if cols is None else S_nk[cols]
    Wf = mo.weights_f32(W, S, mo.LAYOUT_NK)
    ref = mo.gemm_f64(A, Wf)
    return (ref, mo.gemm_abs_f64(A, Wf)) if with_abs else ref


def sample_indices(n, k, rng, edge=True):
    """Sorted unique sample of range(n): k random plus both ends."""
    if n <= k:
        return np.arange(n)
    idx = set(rng.choice(n, size=k, replace=False).tolist())
    if edge:
        idx |= {0, n - 1}
    return np.array(sorted(idx))


# E2M1 values of the 16 codes (sign bit 3; ref.py:3 magnitudes), for the
# torch-side dequantization below
_E2M1_CODES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def full_check_fp32(A_bits, W_nk, S_nk, out, c=8.0):
    """Every element of ``out`` (numpy [M, N]) against a float32 reference built
    on the GPU with plain torch ops, independent of the HIP library: codes from
    the nibbles (low nibble = even K), the E2M1 table, 2**(e - 127) per 32-K
    group (ref.py:50-72), then torch.matmul in float32 (TF32 off), and
    sum |a||w| the same way.  Returns (strict, cancellation-aware) violation
    counts; the cancellation-aware limit adds c * 2**-24 * sum |a||w|, with c
    covering both float32 summations (ours and the reference's)."""
    import torch

    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        Wt = to_dev_u8(W_nk)
        St = to_dev_u8(S_nk)
        N, Kh = Wt.shape
        K = 2 * Kh
        lut = torch.tensor(_E2M1_CODES, dtype=torch.float32, device="cuda")
        codes = torch.stack([Wt & 0x0F, Wt >> 4], dim=-1).reshape(N, K).long()
        del Wt
        scale = torch.ldexp(torch.ones((), device="cuda"), St.to(torch.int32) - 127).to(torch.float32)
        Wf = (lut[codes].view(N, K // 32, 32) * scale[..., None]).view(N, K)
        del codes, scale
        WfT = Wf.t().contiguous()  # [K, N]
        del Wf
        A = to_dev_bf16(A_bits).float()
        ref = A @ WfT
        absref = A.abs() @ WfT.abs_()
        del WfT, A
        got = torch.from_numpy(np.ascontiguousarray(out, dtype=np.float32)).cuda()
        err = (got.double() - ref.double()).abs()
        base = mo.atol_for(K) + mo.RTOL * ref.double().abs()
        strict = int((~(err <= base)).sum().item())
        canc = int((~(err <= base + c * 2.0 ** -24 * absref.double())).sum().item())
        torch.cuda.synchronize()
        return strict, canc
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
