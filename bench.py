#!/usr/bin/env python3
"""Benchmark of the MXFP4-weight x BF16-activation GEMM on one MI355X.

Headline (BASELINE.json metric): TFLOP/s and % of the 2.5 PF/s dense bf16
MFMA peak at M=4096, N=12288, K=3072 (DiT MLP up-projection), plus HBM GB/s
at M=16, N=K=8192 (decode) against 8 TB/s.

A "step" is one GEMM call on inputs already resident in HBM.  Weights are
rotated over >= 640 MB of distinct copies so the 256 MB MALL cannot serve
them.  Per leg:
  1. W eager warm-up launches, then K eager launches between two events
     (eager_ms_per_step);
  2. the K steps are captured once in a HIP graph; the graph is replayed for
     a fixed GPU time (--warm-s, default 1 s, whatever --warmup says) so the
     clocks settle on this kernel;
  3. REPLAYS (5) replays of the K-step graph are timed one by one, each
     between two events on the launch stream with a synchronize on both
     sides; ms_per_step = median replay / K, and the spread (min, max) is
     reported beside it.
The reference times 50 warm-up + 100 events-bracketed launches and reports
p50 (python/mxfp4_cdna3/bench.py:31-49,105-108).

The CPU baseline is the reference CPU path (torch dequant + torch.matmul in
fp32, python/mxfp4_cdna3/ref.py:75-78) on the dit_up workload, repeated for
~10 s with every host core (median reported).  roofline.traffic is read from
the committed rocprofv3 summary of the same kernel and workload
(profiles/<kernel>_<workload>.md: FETCH_SIZE + WRITE_SIZE, copy-calibrated).

--sweep times every BASELINE config (plumbing, decode M in {1,8,16,32},
dit_up, dit_down, 70B FFN M in {1,16,128,512,2048,8192}) with the auto plan
and the re-measured tiled variants, writes the reference's CSV schema
(strategy,M,N,K,iter,ns; python/mxfp4_cdna3/bench.py:69-119) plus bytes,
flops and roofline columns, and times the CPU path per config.  The CSV
feeds ``python -m mxfp4_cdna3.cost_model --fit <csv>`` (the reference's
scripts/run_bench.sh:12-14 -> cost_model.py:153-167).

--leg CONFIG:LAYOUT[:KIND,VARIANT,SPLIT] times one config in one layout (auto
or explicit plan) and prints its record: the unit of the committed rocprofv3
summaries (profiles/), one kernel per run.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--layout kn|nk|g]
                       [--no-cpu] [--no-decode] [--no-extra] [--calibrate-copy]
                       [--sweep [--csv PATH]] [--leg CONFIG:LAYOUT[:PLAN]]
"""

import argparse
import csv
import json
import math
import os
import platform
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "cdna3-bench_amd"))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E
ROTATE_BYTES = 640 << 20   # > 2x the 256 MB MALL
REPLAYS = 5                # timed graph replays per leg (median reported)

# BASELINE.json configs.  "N(0,2)" of the 70B sweep is read as variance 2.
CONFIGS = {"plumbing": dict(M=16, N=2048, K=2048, exp_lo=122, exp_hi=130, a_std=1.0)}
CONFIGS.update({f"decode_m{m}": dict(M=m, N=8192, K=8192, exp_lo=122, exp_hi=130, a_std=1.0)
                for m in (1, 8, 16, 32)})
CONFIGS["dit_up"] = dict(M=4096, N=12288, K=3072, exp_lo=120, exp_hi=132, a_std=1.0)
CONFIGS["dit_down"] = dict(M=4608, N=3072, K=12288, exp_lo=120, exp_hi=132, a_std=1.0)
CONFIGS.update({f"ffn70b_m{m}": dict(M=m, N=28672, K=8192, exp_lo=110, exp_hi=140, a_std=math.sqrt(2.0))
                for m in (1, 16, 128, 512, 2048, 8192)})
for _name, _cfg in CONFIGS.items():
    _cfg["name"] = _name
UP = CONFIGS["dit_up"]
DECODE = CONFIGS["decode_m16"]

# tiled variants whose efficiency the selector uses (mxfp4_api.hip kTiled):
# timed explicitly at split 1 on the MFMA-bound configs in --sweep
FIT_VARIANTS = (6, 7, 15)
MFMA_BOUND = ("dit_up", "dit_down", "ffn70b_m512", "ffn70b_m2048", "ffn70b_m8192")


def make_inputs(cfg, layout, seed=0):
    """Seeded synthetic inputs with the BASELINE distributions.

    numpy PCG64, draw order A, codes, exponents: A ~ N(0, a_std^2) rounded to
    bf16, E2M1 codes uniform over 0..15 (two per byte, low nibble = even K),
    E8M0 exponents uniform over [exp_lo, exp_hi], one per 32 K.
    """
    import torch

    M, N, K = cfg["M"], cfg["N"], cfg["K"]
    rng = np.random.default_rng(seed)
    A = torch.from_numpy(rng.standard_normal((M, K), dtype=np.float32) * np.float32(cfg["a_std"]))
    A = A.to(torch.bfloat16).cuda()
    codes = rng.integers(0, 16, (N, K), dtype=np.uint8)
    W = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    del codes
    S = rng.integers(cfg["exp_lo"], cfg["exp_hi"] + 1, (N, K // 32), dtype=np.uint8)
    if layout == "kn":
        W, S = np.ascontiguousarray(W.T), np.ascontiguousarray(S.T)
    W, S = torch.from_numpy(W).cuda(), torch.from_numpy(S).cuda()
    if layout in ("g", "p"):  # the device prepack of the [N,K/2] weights
        from mxfp4_cdna3 import kernels as kk

        W, S = kk.convert_layout(W, S, "nk", layout)
    return A, W, S


def gemm_bytes(M, N, K, c_bytes=2):
    return 2 * M * K + N * K // 2 + N * K // 32 + c_bytes * M * N


_CAPTURE_STREAM = []


def capture_stream():
    """One graph-capture stream for the run (the library keeps a split-K workspace per stream)."""
    import torch

    if not _CAPTURE_STREAM:
        _CAPTURE_STREAM.append(torch.cuda.Stream())
    return _CAPTURE_STREAM[0]


def time_steps(step, steps, warmup, warm_s):
    """Eager and graph-replayed time per step of ``step(i)`` (see the module doc)."""
    import torch

    main = torch.cuda.current_stream()
    cap = capture_stream()
    cap.wait_stream(main)
    with torch.cuda.stream(cap):
        step(0)  # allocates the capture stream's split-K workspace outside the capture
    main.wait_stream(cap)
    for i in range(max(warmup, 1)):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / steps

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        for i in range(steps):
            step(i)
    torch.cuda.synchronize()
    t0, n = time.perf_counter(), 0
    while True:  # fixed-time warm-up on this kernel
        g.replay()
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
            if time.perf_counter() - t0 >= warm_s:
                break
    torch.cuda.synchronize()
    per_step = []
    for _ in range(REPLAYS):
        torch.cuda.synchronize()
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        per_step.append(e0.elapsed_time(e1) / steps)
    del g
    s = sorted(per_step)
    return {"ms": s[len(s) // 2], "min_ms": s[0], "max_ms": s[-1], "replays_ms": per_step,
            "eager_ms": eager_ms, "warm_replays": n}


def measure(kk, cfg, layout, steps, warmup, warm_s, plan=None, inputs=None):
    """Time of one GEMM on cfg's shape in ``layout`` under ``plan`` (None: auto)."""
    import torch

    M, N, K = cfg["M"], cfg["N"], cfg["K"]
    A, B, S = inputs if inputs is not None else make_inputs(cfg, layout)
    per_set = B.numel() + S.numel()
    rot = max(1, math.ceil(ROTATE_BYTES / per_set))
    Bs = [B] + [B.clone() for _ in range(rot - 1)]
    Ss = [S] + [S.clone() for _ in range(rot - 1)]
    C = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")

    def step(i):
        kk.gemm(A, Bs[i % rot], Ss[i % rot], C, layout, None, plan)

    r = time_steps(step, steps, warmup, warm_s)
    del Bs, Ss
    r["plan"] = kk.select_plan(M, N, K, layout)[3] if plan is None else kk.describe_plan(plan)
    r["rotation_sets"] = rot
    return r


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(cfg, budget_s=10.0, min_runs=3):
    """Reference CPU path on the full workload, repeated for ~budget_s (median)."""
    import torch

    sys.path.insert(0, REPO)
    from oracle import mxfp4_oracle as mo  # CPU baseline leg only

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    M, N, K = cfg["M"], cfg["N"], cfg["K"]
    A_bits, W, S = mo.make_inputs(M, N, K, cfg["exp_lo"], cfg["exp_hi"], cfg["a_std"], seed=0)
    Bkn, Skn = mo.nk_to_kn(W, S)
    del W, S
    A_t = torch.from_numpy(A_bits.view(np.int16)).view(torch.bfloat16)

    def run():
        t0 = time.perf_counter()
        mo.ref_gemm_torch(A_t, Bkn, Skn, mo.LAYOUT_KN)
        return time.perf_counter() - t0

    run()  # warmup
    times, t_start = [], time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s and len(times) < 200):
        times.append(run())
    t = sorted(times)[len(times) // 2]
    return {
        "value": round(2.0 * M * N * K / t / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": cpu_model(),
        "ms": round(t * 1e3, 3),
        "sample": f"full {cfg['name']} workload {M}x{N}x{K} (torch fp32 dequant + matmul per call, as "
                  f"ref.py:75-78), {len(times)} runs in {sum(times):.1f} s, median {t:.3f} s, "
                  f"{threads} threads of {cpu_model()}",
    }


def profile_traffic(name):
    """traffic_bytes_per_launch from a committed rocprofv3 summary (profiles/<name>.md)."""
    path = os.path.join(REPO, "profiles", name + ".md")
    try:
        with open(path) as f:
            for line in f:
                if "traffic_bytes_per_launch" in line:
                    return int(float(line.split("=")[1]))
    except (OSError, ValueError, IndexError):
        pass
    return None


def copy_calibration(nbytes=1 << 30):
    """A plain device copy of known size on a cold source (for PMC byte-counter scales)."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(3)
    flush = torch.empty(2 * nbytes, dtype=torch.uint8, device="cuda").fill_(5)  # evict src from L2
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del flush


def leg_record(cfg, r, c_bytes=2):
    """Roofline figures of one timed leg: MFMA-bound (TFLOP/s) or HBM-bound (GB/s)."""
    M, N, K = cfg["M"], cfg["N"], cfg["K"]
    flops = 2.0 * M * N * K
    nbytes = gemm_bytes(M, N, K, c_bytes)
    t = r["ms"] * 1e-3
    mfma_bound = flops / nbytes > PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBPS * 1e9)
    tf, gb = flops / t / 1e12, nbytes / t / 1e9
    rec = {"us_per_step": round(r["ms"] * 1e3, 3),
           "spread_us": [round(r["min_ms"] * 1e3, 3), round(r["max_ms"] * 1e3, 3)],
           "plan": r["plan"], "tflops": round(tf, 2), "gbps": round(gb, 1)}
    if mfma_bound:
        rec["roofline"] = {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS,
                           "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4)}
    else:
        rec["roofline"] = {"bound": "hbm", "achieved": round(gb, 1), "peak": PEAK_HBM_GBPS,
                           "unit": "GB/s", "frac": round(gb / PEAK_HBM_GBPS, 4)}
    return rec


def headline(args, kk):
    up = measure(kk, UP, args.layout, args.steps, args.warmup, args.warm_s)
    M, N, K = UP["M"], UP["N"], UP["K"]
    flops = 2.0 * M * N * K
    tflops = flops / (up["ms"] * 1e-3) / 1e12
    layout_names = {"kn": "[K/2,N] (reference layout)", "nk": "[N,K/2]", "g": "G (reference prepack)"}
    result = {
        "metric": "TFLOP/s & % BF16 MFMA peak (M=4096,N=12288,K=3072); HBM GB/s at M=16",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(up["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded; E2M1 codes uniform, E8M0 120..132, A ~ N(0,1))",
        "config": {
            "workload": f"dit_up M={M} N={N} K={K}, weights {layout_names[args.layout]}, bf16 out",
            "M": M, "N": N, "K": K, "layout": args.layout, "plan": up["plan"],
            "rotation_sets": up["rotation_sets"],
            "timing": f"hip graph of K launches; {args.warm_s:g} s replay warm-up; median of "
                      f"{REPLAYS} timed replays (events)",
        },
        "pct_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "ms_per_step_spread": [round(up["min_ms"], 5), round(up["max_ms"], 5)],
        "eager_ms_per_step": round(up["eager_ms"], 5),
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": None,
        },
    }

    # the same workload with the other weight layouts: [N,K/2] (the BASELINE
    # configs store W so; the reference extension takes [K/2,N]) and G (the
    # reference's prepack_b_mxfp4 format, prepacked outside the timed region
    # as the reference's bench does for strategy G)
    result["other_layouts"] = {}
    for other in [lay for lay in ("kn", "nk", "g") if lay != args.layout]:
        up2 = measure(kk, UP, other, args.steps, args.warmup, args.warm_s)
        tf2 = flops / (up2["ms"] * 1e-3) / 1e12
        result["other_layouts"][other] = {"value": round(tf2, 2), "unit": "TFLOP/s",
                                          "pct_bf16_peak": round(100.0 * tf2 / PEAK_BF16_TFLOPS, 2),
                                          "ms_per_step": round(up2["ms"], 5),
                                          "ms_per_step_spread": [round(up2["min_ms"], 5), round(up2["max_ms"], 5)],
                                          "plan": up2["plan"]}

    dsteps = max(args.steps, 200)
    if not args.no_decode:
        dbytes = gemm_bytes(DECODE["M"], DECODE["N"], DECODE["K"])
        legs = {}
        for lay in ("nk", "kn", "p"):
            d = measure(kk, DECODE, lay, dsteps, args.warmup, args.warm_s)
            legs[lay] = (d, dbytes / (d["ms"] * 1e-3) / 1e9)
        d, gbps = legs["nk"]
        result["hbm_decode"] = {
            "metric": "HBM GB/s at M=16, N=K=8192 (weights [N,K/2] as in the BASELINE configs)",
            "value": round(gbps, 1),
            "unit": "GB/s",
            "pct_hbm_peak": round(100.0 * gbps / PEAK_HBM_GBPS, 2),
            "us_per_step": round(d["ms"] * 1e3, 3),
            "us_per_step_spread": [round(d["min_ms"] * 1e3, 3), round(d["max_ms"] * 1e3, 3)],
            "eager_us_per_step": round(d["eager_ms"] * 1e3, 3),
            "plan": d["plan"],
            "rotation_sets": d["rotation_sets"],
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS,
                         "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4),
                         "bytes_per_launch": dbytes, "traffic": profile_traffic("stream_decode_m16_nk")},
        }
        for lay, prof in (("kn", "gemv_decode_m16_kn"), ("p", "stream_decode_m16_p")):
            dl, gl = legs[lay]
            result["hbm_decode"][f"{lay}_layout"] = {
                "value": round(gl, 1), "pct_hbm_peak": round(100.0 * gl / PEAK_HBM_GBPS, 2),
                "us_per_step": round(dl["ms"] * 1e3, 3), "plan": dl["plan"], "traffic": profile_traffic(prof)}
        # the other M of the BASELINE decode config ([N,K/2], N = K = 8192)
        sweep = {}
        for m in (1, 8, 32):
            cfg = CONFIGS[f"decode_m{m}"]
            dm = measure(kk, cfg, "nk", dsteps, args.warmup, args.warm_s)
            gb = gemm_bytes(m, cfg["N"], cfg["K"]) / (dm["ms"] * 1e-3) / 1e9
            sweep[f"M{m}"] = {"value": round(gb, 1), "unit": "GB/s", "pct_hbm_peak": round(100.0 * gb / PEAK_HBM_GBPS, 2),
                              "us_per_step": round(dm["ms"] * 1e3, 3), "plan": dm["plan"]}
        result["hbm_decode"]["m_sweep"] = sweep

    if not args.no_extra:
        # dit_down and the 70B FFN sweep: roofline fraction per config (weights
        # [N,K/2], the BASELINE layout)
        extra = {}
        for name in ("dit_down",) + tuple(f"ffn70b_m{m}" for m in (1, 16, 128, 512, 2048, 8192)):
            cfg = CONFIGS[name]
            st = dsteps if cfg["M"] <= 32 else args.steps
            extra[name] = leg_record(cfg, measure(kk, cfg, "nk", st, args.warmup, min(args.warm_s, 0.5)))
        result["other_configs"] = extra

    # the committed rocprof summary of the kernel the plan runs
    family = "tiled_sched" if up["plan"].startswith("tiled-sched") else "tiled"
    result["roofline"]["traffic"] = profile_traffic(f"{family}_dit_up_{args.layout}")
    if args.calibrate_copy:
        copy_calibration()
    result["cpu_baseline"] = None if args.no_cpu else cpu_baseline(UP)
    return result


def sweep(args, kk):
    """Every BASELINE config: auto plan in every layout it takes, plus the
    selector's tiled variants at split 1 on the MFMA-bound configs."""
    rows, summary = [], {}
    for name, cfg in CONFIGS.items():
        M, N, K = cfg["M"], cfg["N"], cfg["K"]
        steps = max(args.steps, 200) if M <= 32 else args.steps
        layouts = ["kn", "nk"] + (["g"] if N % 128 == 0 else []) + (["p"] if N % 32 == 0 and K % 64 == 0 else [])
        for lay in layouts:
            inputs = make_inputs(cfg, lay)
            legs = [("auto", None)]
            if name in MFMA_BOUND and lay in ("kn", "nk", "g"):
                legs += [(f"tiled-v{v}", (2, v, 1)) for v in FIT_VARIANTS]
            for label, plan in legs:
                try:
                    r = measure(kk, cfg, lay, steps, args.warmup, args.warm_s, plan, inputs)
                except RuntimeError as ex:  # a variant that does not take this layout / shape
                    print(f"sweep: {name} {lay} {label}: skipped ({ex})", file=sys.stderr, flush=True)
                    continue
                rec = leg_record(cfg, r)
                strategy = f"{label}-{lay}"
                summary.setdefault(name, {})[strategy] = rec
                for i, ms in enumerate(r["replays_ms"]):
                    rows.append({"strategy": strategy, "M": M, "N": N, "K": K, "iter": i,
                                 "ns": round(ms * 1e6, 1), "plan": r["plan"],
                                 "bytes": gemm_bytes(M, N, K), "flops": 2 * M * N * K,
                                 "bound": rec["roofline"]["bound"], "frac": rec["roofline"]["frac"]})
                print(f"sweep: {name} {strategy}: {rec['us_per_step']} us ({r['plan']}), "
                      f"{rec['roofline']['bound']} frac {rec['roofline']['frac']}", flush=True)
            del inputs
        if not args.no_cpu:
            cb = cpu_baseline(cfg, budget_s=args.cpu_s, min_runs=1)
            summary.setdefault(name, {})["cpu"] = cb
            rows.append({"strategy": "cpu-torch-fp32", "M": M, "N": N, "K": K, "iter": 0,
                         "ns": round(cb["ms"] * 1e6, 1), "plan": f"{cb['cores']} threads",
                         "bytes": gemm_bytes(M, N, K), "flops": 2 * M * N * K, "bound": "cpu", "frac": ""})
            print(f"sweep: {name} cpu: {cb['ms']} ms ({cb['value']} TFLOP/s, {cb['cores']} threads)", flush=True)
    if args.csv:
        os.makedirs(os.path.dirname(os.path.abspath(args.csv)), exist_ok=True)
        with open(args.csv, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=["strategy", "M", "N", "K", "iter", "ns", "plan", "bytes",
                                              "flops", "bound", "frac"])
            w.writeheader()
            w.writerows(rows)
    return {"sweep": summary, "cpu_model": cpu_model(), "csv": args.csv}


def single_leg(args, kk):
    """One config in one layout: the record of a profiled run."""
    parts = args.leg.split(":")
    cfg = CONFIGS[parts[0]]
    lay = parts[1] if len(parts) > 1 else "kn"
    plan = tuple(int(x) for x in parts[2].split(",")) if len(parts) > 2 else None
    steps = max(args.steps, 200) if cfg["M"] <= 32 else args.steps
    rec = leg_record(cfg, measure(kk, cfg, lay, steps, args.warmup, args.warm_s, plan))
    if args.calibrate_copy:
        copy_calibration()
    return {"leg": args.leg, "M": cfg["M"], "N": cfg["N"], "K": cfg["K"], "layout": lay, "steps": steps, **rec}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--warm-s", type=float, default=1.0,
                    help="seconds of graph replays before each leg is timed (independent of --warmup)")
    ap.add_argument("--layout", choices=["kn", "nk", "g"], default="kn")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode HBM leg")
    ap.add_argument("--no-extra", action="store_true", help="skip dit_down and the 70B FFN sweep")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a cold 1 GiB device copy (scale for PMC byte counters)")
    ap.add_argument("--sweep", action="store_true", help="time every BASELINE config (CSV)")
    ap.add_argument("--csv", default=None, help="--sweep: CSV output path")
    ap.add_argument("--cpu-s", type=float, default=3.0, help="--sweep: CPU seconds per config")
    ap.add_argument("--leg", default=None, help="one config: CONFIG:LAYOUT[:KIND,VARIANT,SPLIT]")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print("bench.py: this build runs on one GPU only; sharding over several GPUs is "
              "designed but not built or measured. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    from mxfp4_cdna3 import kernels as kk

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.synchronize()
    result = single_leg(args, kk) if args.leg else sweep(args, kk) if args.sweep else headline(args, kk)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
