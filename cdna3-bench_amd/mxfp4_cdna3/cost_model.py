"""Roofline cost model of the MXFP4 GEMM for reports, re-derived for MI355X.

Counterpart of the reference's python/mxfp4_cdna3/cost_model.py:10-167 (same
names: HwProfile, ProblemShape, StrategyDesc, STRATEGIES, Prediction,
predict, predict_all, fit_efficiency, write_predictions_csv).  What changes:

* MFMA peak.  The reference divides one MFMA's flops by its cycle count per
  CU (cost_model.py:22-25), i.e. it counts one MFMA pipe per CU; every CDNA
  CU has four (one per SIMD), so its peaks are 4x low.  Here a SIMD retires
  ``mfma_flops_per_simd_clk`` dense flops per clock: 1024 bf16 on gfx950
  (v_mfma_f32_16x16x32_bf16: 16384 flops in 16 clocks), 512 on gfx942.
  MI355X: 256 CUs x 4 x 1024 x 2.4 GHz = 2.52 PF/s (AMD's 2.5 PF/s dense).
* Dequant cost.  One v_cvt_scalef32_pk_bf16_fp4 per byte (two E2M1 codes,
  scale applied): 4 VALU instructions per 8 elements, against the reference's
  22 (LUT perm + cvt + scale + RNE, cost_model.py:124-125).
* C is bf16 (2 bytes) unless stated; the reference's fp32 C is c_bytes=4.
* Strategies are this build's kernel families with the efficiencies measured
  on MI355X (the C++ selector in csrc/mxfp4_api.hip uses the same figures and
  also models waves of CTAs and split-K; ``plan`` asks it directly).

No GPU is needed: everything here is arithmetic on shapes.
"""

from __future__ import annotations

import argparse
import csv
import logging
from dataclasses import asdict, dataclass

log = logging.getLogger("mxfp4_cdna3.cost_model")


@dataclass(frozen=True)
class HwProfile:
    name: str
    num_cus: int
    num_xcds: int
    clock_ghz: float
    hbm_bw_tbps: float
    lds_bytes_per_clk_per_cu: int = 128
    simds_per_cu: int = 4
    mfma_flops_per_simd_clk: int = 1024  # dense bf16
    valu_lanes_per_simd: int = 16        # a wave64 VALU instruction takes 4 clocks

    @property
    def mfma_peak_tflops(self) -> float:
        return self.mfma_flops_per_simd_clk * self.simds_per_cu * self.num_cus * self.clock_ghz / 1e3

    @property
    def valu_peak_gops(self) -> float:
        """Lane-operations per second / 1e9 (a convert counts 64 lane-ops per wave)."""
        return self.valu_lanes_per_simd * self.simds_per_cu * self.num_cus * self.clock_ghz

    @property
    def lds_bw_aggregate_tbps(self) -> float:
        return self.lds_bytes_per_clk_per_cu * self.num_cus * self.clock_ghz / 1e3


MI355X = HwProfile("MI355X", 256, 8, 2.4, 8.0)
# The reference's two CDNA3 profiles with the per-SIMD MFMA rate (1307 TF/s
# dense bf16 for MI300X at 2.1 GHz).
MI300A = HwProfile("MI300A", 228, 6, 2.1, 5.3, mfma_flops_per_simd_clk=512)
MI300X = HwProfile("MI300X", 304, 8, 2.1, 5.3, mfma_flops_per_simd_clk=512)


@dataclass(frozen=True)
class ProblemShape:
    M: int
    N: int
    K: int

    @property
    def flops(self) -> float:
        return 2.0 * self.M * self.N * self.K

    def hbm_bytes(self, extra_b_passes: int = 0, c_bytes: int = 2) -> int:
        """Compulsory bytes: A bf16, packed B (half a byte per element), one
        E8M0 byte per 32 K, C (bf16 by default), plus extra_b_passes passes of
        a bf16 K x N scratch (the two-pass strategy)."""
        a = self.M * self.K * 2
        bp = (self.K // 2) * self.N
        s = (self.K // 32) * self.N
        c = self.M * self.N * c_bytes
        return a + bp + s + c + extra_b_passes * self.K * self.N * 2

    @property
    def n_mfma_16x16x32(self) -> int:
        return -(-self.M // 16) * -(-self.N // 16) * -(-self.K // 32)

    @property
    def dequant_calls(self) -> int:
        """Groups of 8 FP4 elements (the reference's unit, cost_model.py:64-66)."""
        return (self.K * self.N) // 8


@dataclass(frozen=True)
class StrategyDesc:
    name: str
    block_m: int
    block_n: int
    block_k: int
    lds_kib_per_cta: int
    extra_b_hbm_passes: int
    dequant_overlap: float  # 0..1 fraction of the converts hidden behind MFMA
    achievable_eff: float   # 0..1 of mfma_peak_tflops sustained (compute-bound shapes)
    hbm_eff: float = 1.0    # 0..1 of hbm_bw_tbps sustained (memory-bound shapes)
    converts_per_b: float = 1.0  # times each B element is converted (M-blocks per column)
    # LDS bytes read per v_mfma_f32_16x16x32_bf16 (or its flop equivalent):
    # the reference's model reads both operands afresh for every MFMA (1 KB
    # each); a wave tile reuses each A operand across its column blocks and
    # each B word across its row blocks.
    lds_bytes_per_mfma: int = 2048


# Measured on MI355X with seeded random data (A ~ N(0,1), uniform codes):
#  * tiled-sched: dit_up 0.55 ([K/2,N]), 0.57 (G), 0.49 ([N,K/2]), 70B FFN
#    M=2048..8192 0.58 (plan variant 15);
#  * tiled-pipe: dit_up 0.52 ([K/2,N]), 0.40 ([N,K/2]) (plan variant 6);
#  * stream: decode M=16 N=K=8192 [N,K/2] 2.69 TB/s, P layout 3.03 TB/s;
#  * stream-whole: M=1 N=K=8192 [N,K/2] 3.37 TB/s (P 3.59), N=28672 3.87 TB/s;
#  * gemv: [K/2,N] decode 2.15 TB/s at N=8192, 3.56 TB/s at N=28672.
STRATEGIES = (
    # 64 x 128 per wave: 4 A reads (1 KB) + 8 raw B words (256 B) per 32 MFMAs
    StrategyDesc("tiled-sched", 128, 256, 64, 75, 0, dequant_overlap=1.0, achievable_eff=0.55,
                 converts_per_b=2.0, lds_bytes_per_mfma=192),
    # 64 x 128 per wave, 32x32x16: 2 A reads + 4 raw B words per 8 MFMAs (16 equivalents)
    StrategyDesc("tiled-pipe", 256, 256, 64, 122, 0, dequant_overlap=1.0, achievable_eff=0.52,
                 converts_per_b=4.0, lds_bytes_per_mfma=192),
    StrategyDesc("stream", 16, 32, 512, 140, 0, dequant_overlap=1.0, achievable_eff=0.10, hbm_eff=0.34),
    # one CTA per 32 columns x the whole K (M <= 8 in the C++ selector)
    StrategyDesc("stream-whole", 16, 32, 8192, 136, 0, dequant_overlap=1.0, achievable_eff=0.10, hbm_eff=0.42),
    StrategyDesc("gemv", 16, 128, 32, 8, 0, dequant_overlap=1.0, achievable_eff=0.10, hbm_eff=0.30),
    # dequantize to a bf16 scratch, then a bf16 GEMM (the reference's strategy A)
    StrategyDesc("two-pass", 128, 256, 64, 0, 2, dequant_overlap=0.0, achievable_eff=0.60,
                 lds_bytes_per_mfma=256),
)
STRATEGY_BY_NAME = {s.name: s for s in STRATEGIES}


@dataclass
class Prediction:
    strategy: str
    hw: str
    shape: ProblemShape
    compute_ns: float
    hbm_ns: float
    lds_ns: float
    dequant_ns_total: float
    dequant_ns_unhidden: float
    binding: str
    predicted_ns: float
    predicted_tflops: float

    def to_row(self) -> dict:
        d = {k: v for k, v in asdict(self).items() if k != "shape"}
        d.update({"M": self.shape.M, "N": self.shape.N, "K": self.shape.K})
        return d


def predict(strategy: StrategyDesc, shape: ProblemShape, hw: HwProfile = MI355X, c_bytes: int = 2) -> Prediction:
    """max(compute + unhidden dequant, HBM, LDS), as cost_model.py:117-146."""
    compute_ns = shape.flops / (hw.mfma_peak_tflops * strategy.achievable_eff * 1e12) * 1e9
    hbm_ns = shape.hbm_bytes(strategy.extra_b_hbm_passes, c_bytes) / (hw.hbm_bw_tbps * strategy.hbm_eff * 1e12) * 1e9
    lds_ns = shape.n_mfma_16x16x32 * strategy.lds_bytes_per_mfma / (hw.lds_bw_aggregate_tbps * 1e12) * 1e9
    # Dequant: one convert (a lane-op) per byte = 4 per 8 elements, times the
    # number of M-blocks that convert each B element.
    dequant_ops = shape.dequant_calls * 4 * strategy.converts_per_b
    dequant_ns_total = dequant_ops / (hw.valu_peak_gops * 1e9) * 1e9
    dequant_ns_unhidden = dequant_ns_total * (1.0 - strategy.dequant_overlap)
    candidates = {"compute": compute_ns + dequant_ns_unhidden, "hbm": hbm_ns, "lds": lds_ns}
    binding = max(candidates, key=candidates.get)
    predicted_ns = candidates[binding]
    return Prediction(strategy.name, hw.name, shape, compute_ns, hbm_ns, lds_ns, dequant_ns_total,
                      dequant_ns_unhidden, binding, predicted_ns, shape.flops / (predicted_ns * 1e3))


def predict_all(shapes, hw: HwProfile = MI355X, strategies=STRATEGIES):
    return [predict(s, sh, hw) for sh in shapes for s in strategies]


def fit_efficiency(bench_csv: str, hw: HwProfile = MI355X, peak_tflops: float | None = None) -> dict[str, float]:
    """Invert measured times -> achievable_eff per strategy (median across
    shapes of peak time / measured time), as cost_model.py:153-167.  The CSV
    has columns strategy, M, N, K, ns (one row per iteration or per shape).
    ``peak_tflops`` overrides the hardware peak (the C++ selector's
    efficiencies are fractions of 2500 TFLOP/s)."""
    peak = peak_tflops if peak_tflops else hw.mfma_peak_tflops
    per_strategy: dict[str, list[float]] = {}
    for (strat, M, N, K), p50 in _p50_rows(bench_csv).items():
        peak_ns = ProblemShape(M, N, K).flops / (peak * 1e12) * 1e9
        per_strategy.setdefault(strat, []).append(peak_ns / p50)
    return {s: float(sorted(v)[len(v) // 2]) for s, v in per_strategy.items()}


def _p50_rows(bench_csv: str) -> dict[tuple, float]:
    """{(strategy, M, N, K): median ns} of a bench CSV."""
    rows: dict[tuple, list[float]] = {}
    with open(bench_csv, newline="") as f:
        for r in csv.DictReader(f):
            key = (r["strategy"], int(r["M"]), int(r["N"]), int(r["K"]))
            rows.setdefault(key, []).append(float(r["ns"]))
    return {k: sorted(v)[len(v) // 2] for k, v in rows.items()}


def write_sweep_summary(bench_csv: str, path: str, command: str = "", peak_tflops: float = 2500.0):
    """Markdown summary of a ``bench.py --sweep`` CSV: every (config, strategy)
    with its plan, median time and roofline fraction, then the efficiencies
    fitted for the selector's tiled variants (fractions of ``peak_tflops``)."""
    plans, fracs = {}, {}
    with open(bench_csv, newline="") as f:
        for r in csv.DictReader(f):
            key = (r["strategy"], int(r["M"]), int(r["N"]), int(r["K"]))
            plans[key] = r.get("plan", "")
            fracs[key] = (r.get("bound", ""), r.get("frac", ""))
    p50 = _p50_rows(bench_csv)
    lines = ["# Sweep of the BASELINE configs (bench.py --sweep)", ""]
    if command:
        lines += [f"command: `{command}`", ""]
    lines += ["| M | N | K | strategy | plan | median us | bound | roofline frac |", "|---|---|---|---|---|---|---|---|"]
    for (strat, M, N, K), ns in sorted(p50.items(), key=lambda kv: (kv[0][1], kv[0][2], kv[0][3], kv[0][0])):
        bound, frac = fracs[(strat, M, N, K)]
        us = f"{ns / 1e3:.3f}" if strat != "cpu-torch-fp32" else f"{ns / 1e3:.1f}"
        lines.append(f"| {M} | {N} | {K} | {strat} | {plans[(strat, M, N, K)]} | {us} | {bound} | {frac} |")
    fit = fit_efficiency(bench_csv, peak_tflops=peak_tflops)
    lines += ["", f"## fitted efficiencies (median over the MFMA-bound configs of peak time / measured time, "
                  f"peak {peak_tflops:.0f} TFLOP/s)", "", "| strategy | efficiency |", "|---|---|"]
    for st in sorted(k for k in fit if k.startswith("tiled-v")):
        lines.append(f"| {st} | {fit[st]:.3f} |")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def write_predictions_csv(rows: list[Prediction], path: str):
    fields = list(rows[0].to_row().keys())
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for r in rows:
            w.writerow(r.to_row())


def plan(M: int, N: int, K: int, layout: str = "kn") -> str:
    """The plan the library's C++ selector picks (loads the extension; no GPU needed)."""
    from . import kernels

    return kernels.select_plan(M, N, K, layout)[3]


BASELINE_SHAPES = (
    ProblemShape(16, 2048, 2048),
    ProblemShape(16, 8192, 8192),
    ProblemShape(4096, 12288, 3072),
    ProblemShape(4608, 3072, 12288),
    ProblemShape(128, 28672, 8192),
    ProblemShape(2048, 28672, 8192),
)


def main(argv=None):
    ap = argparse.ArgumentParser(description="MI355X roofline predictions for the MXFP4 GEMM")
    ap.add_argument("--out", default=None, help="write predictions as CSV")
    ap.add_argument("--fit", default=None, help="bench CSV (strategy,M,N,K,ns) to fit efficiencies")
    ap.add_argument("--peak", type=float, default=None, help="--fit: peak TFLOP/s (default: the hardware's)")
    ap.add_argument("--summary", default=None, help="--fit: write a markdown summary of the CSV here")
    ap.add_argument("--command", default="", help="--summary: the command that produced the CSV")
    a = ap.parse_args(argv)
    if a.fit:
        for s, e in sorted(fit_efficiency(a.fit, peak_tflops=a.peak).items()):
            print(f"{s}: achievable_eff = {e:.3f}")
        if a.summary:
            write_sweep_summary(a.fit, a.summary, a.command, a.peak or 2500.0)
        return
    rows = predict_all(BASELINE_SHAPES)
    for r in rows:
        print(f"{r.strategy:12s} {r.shape.M:5d}x{r.shape.N:5d}x{r.shape.K:5d}  {r.binding:8s} "
              f"{r.predicted_ns / 1e3:9.2f} us  {r.predicted_tflops:8.1f} TF/s")
    if a.out:
        write_predictions_csv(rows, a.out)


if __name__ == "__main__":
    main()
