"""Python cost model (mxfp4_cdna3/cost_model.py) against closed forms.

Counterpart of python/mxfp4_cdna3/cost_model.py:10-167 in the reference; the
MFMA peak there counts one MFMA pipe per CU (4x low, per CDNA's four SIMDs).
"""

import csv
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "cdna3-bench_amd"))

from mxfp4_cdna3 import cost_model as cm  # noqa: E402


def test_mfma_peaks_are_published_dense_figures():
    # MI355X: 256 CUs x 4 SIMDs x 1024 bf16 flops/clk x 2.4 GHz
    assert cm.MI355X.mfma_peak_tflops == pytest.approx(2516.58, abs=0.01)
    # MI300X: AMD's published 1307.4 TFLOP/s dense bf16
    assert cm.MI300X.mfma_peak_tflops == pytest.approx(1307.4, abs=0.1)
    # the reference's formula (2*16^3 flops / 16 cycles per CU) gives a quarter
    ref = 2 * 16 * 16 * 16 / 16 * 304 * 2.1e9 / 1e12
    assert cm.MI300X.mfma_peak_tflops / ref == pytest.approx(4.0)


def test_hbm_bytes_closed_forms():
    # BASELINE plumbing config and the decode config of bench.py
    assert cm.ProblemShape(16, 2048, 2048).hbm_bytes() == 2 * 16 * 2048 + 1024 * 2048 + 64 * 2048 + 2 * 16 * 2048
    assert cm.ProblemShape(16, 8192, 8192).hbm_bytes() == 36175872
    # the reference's fp32 C and the two-pass scratch
    s = cm.ProblemShape(64, 256, 128)
    assert s.hbm_bytes(c_bytes=4) - s.hbm_bytes() == 2 * 64 * 256
    assert s.hbm_bytes(extra_b_passes=2) - s.hbm_bytes() == 2 * 128 * 256 * 2


def test_counts():
    s = cm.ProblemShape(4096, 12288, 3072)
    assert s.flops == 2.0 * 4096 * 12288 * 3072
    assert s.n_mfma_16x16x32 * 16 * 16 * 32 * 2 == s.flops
    assert s.dequant_calls * 8 == 3072 * 12288
    # ceil for ragged shapes
    assert cm.ProblemShape(17, 16, 32).n_mfma_16x16x32 == 2


def test_predict_binding_and_max_rule():
    up = cm.predict(cm.STRATEGY_BY_NAME["tiled-sched"], cm.ProblemShape(4096, 12288, 3072))
    assert up.binding == "compute"
    dec = cm.predict(cm.STRATEGY_BY_NAME["stream"], cm.ProblemShape(16, 8192, 8192))
    assert dec.binding == "hbm"
    for p in (up, dec):
        assert p.predicted_ns == max(p.compute_ns + p.dequant_ns_unhidden, p.hbm_ns, p.lds_ns)
        assert p.predicted_tflops == pytest.approx(p.shape.flops / (p.predicted_ns * 1e3))
    # compute time at efficiency e is the peak time / e
    st = cm.STRATEGY_BY_NAME["tiled-sched"]
    peak_ns = up.shape.flops / (cm.MI355X.mfma_peak_tflops * 1e12) * 1e9
    assert up.compute_ns == pytest.approx(peak_ns / st.achievable_eff)
    # the decode HBM time at full bandwidth is the 4.52 us floor
    assert dec.hbm_ns * cm.STRATEGY_BY_NAME["stream"].hbm_eff == pytest.approx(36175872 / 8e12 * 1e9)
    # a fully hidden dequant adds nothing; the two-pass strategy hides none
    assert up.dequant_ns_unhidden == 0.0
    two = cm.predict(cm.STRATEGY_BY_NAME["two-pass"], up.shape)
    assert two.dequant_ns_unhidden == pytest.approx(two.dequant_ns_total) and two.dequant_ns_total > 0


def test_fit_efficiency_inverts_predict(tmp_path):
    shapes = [cm.ProblemShape(4096, 12288, 3072), cm.ProblemShape(2048, 28672, 8192),
              cm.ProblemShape(512, 28672, 8192)]
    effs = {"x": [0.5, 0.6, 0.55], "y": [0.3, 0.3, 0.3]}
    path = tmp_path / "bench.csv"
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["strategy", "M", "N", "K", "ns"])
        for name, es in effs.items():
            for sh, e in zip(shapes, es):
                peak_ns = sh.flops / (cm.MI355X.mfma_peak_tflops * 1e12) * 1e9
                for jitter in (1.0, 1.01, 0.99):  # per-iteration rows; the median is used
                    w.writerow([name, sh.M, sh.N, sh.K, peak_ns / e * jitter])
    fit = cm.fit_efficiency(str(path))
    assert fit["x"] == pytest.approx(0.55, rel=1e-9)  # median over shapes
    assert fit["y"] == pytest.approx(0.3, rel=1e-9)


def test_predictions_csv(tmp_path):
    rows = cm.predict_all(cm.BASELINE_SHAPES)
    assert len(rows) == len(cm.BASELINE_SHAPES) * len(cm.STRATEGIES)
    out = tmp_path / "pred.csv"
    cm.write_predictions_csv(rows, str(out))
    with open(out) as f:
        got = list(csv.DictReader(f))
    assert len(got) == len(rows) and {"M", "N", "K", "binding", "predicted_ns"} <= set(got[0])


def test_selector_efficiencies_are_the_committed_sweep_fit():
    """The C++ selector's efficiencies of the re-measured tiled variants (6, 7,
    15) are the fit of the committed BASELINE sweep (profiles/
    sweep_baseline_configs.md, made by bench.py --sweep and
    cost_model --fit --summary)."""
    import re

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    fit = {}
    with open(os.path.join(repo, "profiles", "sweep_baseline_configs.md")) as f:
        for line in f:
            m = re.match(r"\| (tiled-v\d+-(kn|nk|g)) \| ([0-9.]+) \|", line)
            if m:
                fit[m.group(1)] = float(m.group(3))
    src = open(os.path.join(repo, "cdna3-bench_amd", "csrc", "mxfp4_api.hip")).read()
    table = {}
    for m in re.finditer(r"\{\{[0-9, ]+\}, ([0-9.]+), ([0-9.]+), \d, kFamily\w+\},?\s*// (\d+):", src):
        table[int(m.group(3))] = (float(m.group(1)), float(m.group(2)))
    for v in (6, 7, 15):
        assert abs(table[v][0] - fit[f"tiled-v{v}-kn"]) < 0.0015, (v, table[v], fit)
        assert abs(table[v][1] - fit[f"tiled-v{v}-nk"]) < 0.0015, (v, table[v], fit)
