"""Summaries of rocprofv3 runs: kernel durations, PMC counters, roofline figures.

Counterpart of the reference's python/mxfp4_cdna3/profile_summary.py:41-165,
re-derived for MI355X (256 CUs, 8 TB/s HBM, 2.5 PF/s dense bf16 MFMA):

* kernel durations come from the rocprofv3 rocpd database (``*_results.db``)
  or a ``*kernel_trace.csv``;
* counters are averaged per dispatch of the selected kernel;
* HBM bytes per dispatch = FETCH_SIZE and WRITE_SIZE (KiB) scaled by what the
  same counters read for a plain copy of known size (``--copy-bytes``): the
  copy kernel reads and writes exactly that many bytes, so its counters give
  the per-counter scale;
* MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (SQ_BUSY_CU_CYCLES x 4 SIMDs) when both
  are present -- per-SIMD cycles over per-SIMD cycles (the reference divides
  MFMAs summed over CUs by one global counter, cost_model/profile_summary F9).

Usage:
  python -m mxfp4_cdna3.profile_summary --trace DIR_OR_DB --kernel REGEX
      [--pmc DB ...] [--copy-bytes N] [--flops F] [--alg-bytes B]
      [--title T] [--command C] [--out FILE.md]
"""

from __future__ import annotations

import argparse
import csv
import glob
import os
import re
import sqlite3
import statistics
import sys

PEAK_TFLOPS = 2500.0
PEAK_GBPS = 8000.0
COPY_KERNEL_RE = r"copyBuffer|CatArrayBatchedCopy|elementwise_kernel.*copy|direct_copy"


def _find_db(path: str) -> str | None:
    if os.path.isfile(path):
        return path
    hits = sorted(glob.glob(os.path.join(path, "**", "*_results.db"), recursive=True))
    return hits[0] if hits else None


def kernel_durations(path: str) -> dict[str, list[float]]:
    """{kernel name: [duration ns, ...] in dispatch order} from a rocpd db or kernel_trace.csv."""
    out: dict[str, list[float]] = {}
    db = _find_db(path)
    if db:
        con = sqlite3.connect(db)
        for name, dur in con.execute("select name, duration from kernels order by start"):
            out.setdefault(name, []).append(float(dur))
        return out
    csvs = sorted(glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True))
    for f in csvs:
        with open(f) as fh:
            for row in csv.DictReader(fh):
                name = row.get("Kernel_Name") or row.get("KernelName") or ""
                start = float(row.get("Start_Timestamp") or row.get("BeginNs") or 0)
                end = float(row.get("End_Timestamp") or row.get("EndNs") or 0)
                out.setdefault(name, []).append(end - start)
    return out


def counters(path: str, reduce: str = "avg") -> dict[str, dict[str, float]]:
    """{kernel name: {counter: value per dispatch}} from a rocpd db; reduce = avg | max."""
    db = _find_db(path)
    if not db:
        return {}
    con = sqlite3.connect(db)
    fn = {"avg": "avg", "max": "max"}[reduce]
    rows = con.execute(
        f"select kernel_name, counter_name, {fn}(value) from counters_collection "
        "group by kernel_name, counter_name").fetchall()
    out: dict[str, dict[str, float]] = {}
    for kname, cname, val in rows:
        out.setdefault(kname, {})[cname] = float(val)
    return out


def _select(names, regex):
    rx = re.compile(regex)
    return [n for n in names if rx.search(n)]


def summarize(trace: str, kernel_re: str, pmc: list[str], copy_bytes: float | None,
              flops: float | None, alg_bytes: float | None, title: str, command: str,
              last: int | None = None) -> tuple[str, dict]:
    durs = kernel_durations(trace)
    if last:
        durs = {k: v[-last:] for k, v in durs.items()}
    sel = _select(durs, kernel_re)
    lines = [f"# {title}", "", f"command: `{command}`" if command else "", ""]
    if last:
        lines += [f"durations: the last {last} dispatches of each kernel (the timed graph replay)", ""]
    lines += ["| kernel | dispatches | avg us | median us | min us | max us |", "|---|---|---|---|---|---|"]
    result: dict = {}
    all_d = []
    for n in sel:
        d = durs[n]
        all_d += d
        lines.append(f"| `{n[:110]}` | {len(d)} | {statistics.mean(d)/1e3:.3f} | "
                     f"{statistics.median(d)/1e3:.3f} | {min(d)/1e3:.3f} | {max(d)/1e3:.3f} |")
    if all_d:
        avg_ns = statistics.mean(all_d)
        result["avg_us"] = avg_ns / 1e3
        if flops:
            result["tflops"] = flops / avg_ns / 1e3
            lines += ["", f"achieved (algorithmic) = {flops:.4g} flop / {avg_ns/1e3:.3f} us = "
                          f"{result['tflops']:.1f} TFLOP/s = {100*result['tflops']/PEAK_TFLOPS:.1f}% of {PEAK_TFLOPS:.0f}"]
        if alg_bytes:
            result["gbps"] = alg_bytes / avg_ns
            lines += ["", f"achieved (algorithmic) = {alg_bytes:.4g} B / {avg_ns/1e3:.3f} us = "
                          f"{result['gbps']:.0f} GB/s = {100*result['gbps']/PEAK_GBPS:.1f}% of {PEAK_GBPS:.0f}"]
    # counters
    merged: dict[str, float] = {}
    copy_c: dict[str, float] = {}
    for db in pmc:
        c = counters(db)
        for n in _select(c, kernel_re):
            merged.update(c[n])
        # calibration copy = the largest copy dispatch (the run also copies smaller buffers)
        cmax = counters(db, "max")
        for n in _select(cmax, COPY_KERNEL_RE):
            copy_c.update(cmax[n])
    if merged:
        lines += ["", "## counters (mean per dispatch)", "", "| counter | value |", "|---|---|"]
        for k in sorted(merged):
            lines.append(f"| {k} | {merged[k]:.6g} |")
        if "SQ_VALU_MFMA_BUSY_CYCLES" in merged and "SQ_BUSY_CU_CYCLES" in merged:
            busy = merged["SQ_VALU_MFMA_BUSY_CYCLES"] / (4.0 * merged["SQ_BUSY_CU_CYCLES"])
            result["mfma_busy"] = busy
            lines += ["", f"MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (4 x SQ_BUSY_CU_CYCLES) = {100*busy:.1f}%"]
        # latency, occupancy and cache figures from the raw counters
        derived = []
        if "VmemLatency" in merged:
            result["vmem_latency_cycles"] = merged["VmemLatency"]
            derived.append(f"- vector memory latency (VmemLatency: accumulated SQ_INST_LEVEL_VMEM / SQ_INSTS_VMEM) = "
                           f"{merged['VmemLatency']:.0f} cycles")
        if "MeanOccupancyPerActiveCU" in merged:
            result["waves_per_busy_cu"] = merged["MeanOccupancyPerActiveCU"]
            derived.append(f"- resident waves per SIMD of a busy CU (MeanOccupancyPerActiveCU) = "
                           f"{merged['MeanOccupancyPerActiveCU']:.2f}")
        if "VmemLatency" not in merged and merged.get("SQ_INSTS_VMEM") and "SQ_INST_LEVEL_VMEM" in merged:
            v = merged["SQ_INST_LEVEL_VMEM"] / merged["SQ_INSTS_VMEM"]
            result["vmem_latency_cycles"] = v
            derived.append(f"- vector memory latency = SQ_INST_LEVEL_VMEM / SQ_INSTS_VMEM = {v:.0f} cycles")
        if "MeanOccupancyPerActiveCU" not in merged and merged.get("SQ_BUSY_CU_CYCLES") and "SQ_LEVEL_WAVES" in merged:
            v = merged["SQ_LEVEL_WAVES"] / merged["SQ_BUSY_CU_CYCLES"]
            result["waves_per_busy_cu"] = v
            derived.append(f"- resident waves per busy CU = SQ_LEVEL_WAVES / SQ_BUSY_CU_CYCLES = {v:.2f}")
        hit, miss = merged.get("TCC_HIT_sum", merged.get("TCC_HIT")), merged.get("TCC_MISS_sum", merged.get("TCC_MISS"))
        if hit is not None and miss is not None and hit + miss > 0:
            result["l2_hit"] = hit / (hit + miss)
            derived.append(f"- L2 hit rate = TCC_HIT / (TCC_HIT + TCC_MISS) = {100 * hit / (hit + miss):.1f}%")
        lvl = merged.get("TCC_EA0_RDREQ_LEVEL_sum", merged.get("TCC_EA0_RDREQ_LEVEL"))
        req = merged.get("TCC_EA0_RDREQ_sum", merged.get("TCC_EA0_RDREQ"))
        if lvl is not None and req:
            result["ea_read_latency_cycles"] = lvl / req
            derived.append(f"- L2-miss (EA) read latency = TCC_EA0_RDREQ_LEVEL / TCC_EA0_RDREQ = {lvl / req:.0f} cycles")
        if merged.get("SQ_WAIT_INST_ANY") is not None and merged.get("SQ_WAVES"):
            derived.append(f"- cycles a wave waited on any instruction dependency, per wave = "
                           f"{merged['SQ_WAIT_INST_ANY'] / merged['SQ_WAVES']:.0f}")
        # LDS: SQ_LDS_IDX_ACTIVE and SQ_LDS_BANK_CONFLICT are cycles summed over
        # CUs, like SQ_BUSY_CU_CYCLES
        lds_active = merged.get("SQ_LDS_IDX_ACTIVE")
        if lds_active and merged.get("SQ_BUSY_CU_CYCLES"):
            result["lds_active_frac"] = lds_active / merged["SQ_BUSY_CU_CYCLES"]
            derived.append(f"- LDS active per busy CU cycle = SQ_LDS_IDX_ACTIVE / SQ_BUSY_CU_CYCLES = "
                           f"{100 * lds_active / merged['SQ_BUSY_CU_CYCLES']:.1f}%")
        if lds_active and merged.get("SQ_LDS_BANK_CONFLICT") is not None:
            result["lds_conflict_frac"] = merged["SQ_LDS_BANK_CONFLICT"] / lds_active
            derived.append(f"- LDS bank-conflict cycles / LDS active cycles = "
                           f"{100 * merged['SQ_LDS_BANK_CONFLICT'] / lds_active:.1f}%")
        if derived:
            lines += ["", "## latency, occupancy, cache", ""] + derived
    if copy_bytes and copy_c and ("FETCH_SIZE" in merged or "WRITE_SIZE" in merged):
        lines += ["", f"## HBM traffic (copy calibration: {copy_bytes/2**20:.0f} MiB copy)", ""]
        traffic = 0.0
        for cn in ("FETCH_SIZE", "WRITE_SIZE"):
            if cn in merged and cn in copy_c and copy_c[cn] > 0:
                scale = copy_bytes / (copy_c[cn] * 1024.0)
                b = merged[cn] * 1024.0 * scale
                traffic += b
                result[cn.lower() + "_bytes"] = b
                lines.append(f"- {cn}: kernel {merged[cn]:.6g} KiB, copy {copy_c[cn]:.6g} KiB "
                             f"-> scale {scale:.4f} -> {b/1e6:.2f} MB per dispatch")
        result["traffic_bytes"] = traffic
        lines.append(f"- traffic_bytes_per_launch = {traffic:.0f}")
        if alg_bytes:
            lines.append(f"- traffic / algorithmic bytes = {traffic/alg_bytes:.3f}")
    return "\n".join(l for l in lines if l is not None) + "\n", result


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--trace", required=True, help="rocprofv3 --kernel-trace output dir or db")
    ap.add_argument("--kernel", required=True, help="regex selecting the kernel")
    ap.add_argument("--pmc", nargs="*", default=[], help="rocprofv3 --pmc output dirs or dbs")
    ap.add_argument("--copy-bytes", type=float, default=None)
    ap.add_argument("--flops", type=float, default=None)
    ap.add_argument("--alg-bytes", type=float, default=None)
    ap.add_argument("--title", default="rocprofv3 summary")
    ap.add_argument("--command", default="")
    ap.add_argument("--out", default=None)
    ap.add_argument("--last", type=int, default=None, help="only the last N dispatches of each kernel")
    a = ap.parse_args(argv)
    text, _ = summarize(a.trace, a.kernel, a.pmc, a.copy_bytes, a.flops, a.alg_bytes, a.title, a.command,
                        a.last)
    if a.out:
        with open(a.out, "w") as f:
            f.write(text)
    sys.stdout.write(text)


if __name__ == "__main__":
    main()
