"""The fused epilogue's float64 reference (tests/test_gpu_epilogue.py act_f64)
against torch.nn.functional's own silu / gelu / gelu(approximate="tanh") on
the CPU: a transcription slip in the formulas (a constant, a sign) fails here
rather than passing on both sides of the GPU test."""

import numpy as np
import pytest

from tests.test_gpu_epilogue import act_f64


@pytest.mark.parametrize("name", ["silu", "gelu", "gelu_tanh"])
def test_act_f64_matches_torch(name):
    import torch
    import torch.nn.functional as F

    rng = np.random.default_rng(0)
    y = np.concatenate([rng.standard_normal(4000) * 3.0, np.linspace(-30.0, 30.0, 1201),
                        [0.0, -0.0, 1e-30, -1e-30, 50.0, -50.0, 88.0, -88.0]])
    t = torch.from_numpy(y)  # float64
    if name == "silu":
        want = F.silu(t)
    elif name == "gelu":
        want = F.gelu(t)
    else:
        want = F.gelu(t, approximate="tanh")
    got = act_f64(name, y)
    # float64 rounding of the two formulations (the tails cancel: compare
    # against the input's scale, not the tiny outputs there)
    err = np.abs(got - want.numpy())
    assert np.all(err <= 1e-14 * np.maximum(1.0, np.abs(y))), float(err.max())
    # a slip in a constant is far outside that: 0.044715 -> 0.04471 moves gelu_tanh by > 1e-6
    if name == "gelu_tanh":
        c = np.sqrt(2.0 / np.pi)
        slip = 0.5 * y * (1.0 + np.tanh(c * (y + 0.04471 * y ** 3)))
        assert np.max(np.abs(slip - want.numpy())) > 1e-6
    assert act_f64(None, y) is y
