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
