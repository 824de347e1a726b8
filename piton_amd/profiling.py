"""Summaries of rocprofv3 output for the benchmark kernels.

    python -m piton_amd.profiling KT_DIR FETCH_DIR WRITE_DIR [--json OUT]
    python -m piton_amd.profiling PMC_DIR --mfma

KT_DIR holds a `--kernel-trace --stats` run of `python3 bench.py` (*_kernel_trace.csv);
FETCH_DIR / WRITE_DIR hold `--pmc FETCH_SIZE` / `--pmc WRITE_SIZE` runs of
`python3 bench.py --pmc-probe` (*_counter_collection.csv). Prints a markdown summary: each
kernel's average duration, and its HBM traffic per launch, each counter scaled by the factor
that maps the calibration add of known size (bench.py CAL_ELEMS: reads 2 x 256 MiB, writes
256 MiB) onto its true bytes. --json writes {kernel: {fetch_bytes, write_bytes, ...}}.
With --mfma, PMC_DIR holds a `--pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES` run of
`python3 bench.py --pmc-probe`: the MFMA pipe occupancy of the benchmark's MFMA kernels.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import sys

CAL_READ = 2 * 64 * 2 ** 20 * 4
CAL_WRITE = 64 * 2 ** 20 * 4

# benchmark launches, identified by kernel name prefix and Grid_Size_X (work-items):
# (workload, algorithmic HBM bytes per launch, algorithmic FLOPs per launch)
BENCH = {
    ("gemm_direct_kernel<false, true, false>", 262144): ("matmul 4096^3", 3 * 4096 * 4096 * 4, 2 * 4096 ** 3),
    ("softmax_rows_kernel<4, true>", 262144): ("softmax 4096 x 1024", 2 * 4 * 4096 * 1024, None),
    ("softmax_wg_kernel<2, 512, true>", 2097152): ("softmax 4096 x 4096", 2 * 4 * 4096 * 4096, None),
    ("softmax_rows_kernel<8, false>", 196608): ("softmax 4096 x 1823", 2 * 4 * 4096 * 1823, None),
    ("attn_fwd_fast<64, true>", 131072): ("attention 32 x 1024 x 64 causal", 4 * 32 * 1024 * 64 * 4,
                                          4 * 1024 * 1024 * 64 * 32 // 2),
}


def short(name: str) -> str:
    name = name.split("(")[0]
    name = re.sub(r"^void ", "", name)
    return name.replace("piton::", "")


def _one(pattern):
    files = glob.glob(pattern)
    if not files:
        raise FileNotFoundError(pattern)
    return files[0]


def kernel_stats(kt_dir, timed_steps=0):
    """Per (kernel, grid) launch statistics from the per-dispatch trace. With timed_steps, the
    4096^3 matmul group also reports the average of its last `timed_steps` dispatches in
    dispatch order: bench.py's timed region (its earlier dispatches are the untimed clock ramp
    and warm-up)."""
    groups = {}
    for r in csv.DictReader(open(_one(os.path.join(kt_dir, "*_kernel_trace.csv")))):
        if "piton::" in r["Kernel_Name"]:
            key = (short(r["Kernel_Name"]), int(r["Grid_Size_X"]))
            groups.setdefault(key, []).append((int(r["Start_Timestamp"]),
                                               int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    rows = []
    for (k, grid), td in sorted(groups.items(), key=lambda kv: -sum(d for _, d in kv[1])):
        in_order = [d for _, d in sorted(td)]
        d = sorted(in_order)
        row = dict(kernel=k, grid=grid, calls=len(d), avg_ns=sum(d) / len(d), min_ns=d[0],
                   median_ns=d[len(d) // 2], max_ns=d[-1], workload=BENCH.get((k, grid), ("",))[0])
        if timed_steps and row["workload"] == "matmul 4096^3" and len(in_order) >= timed_steps:
            last = in_order[-timed_steps:]
            row["timed_avg_ns"] = sum(last) / len(last)
        rows.append(row)
    return rows


def counters(pmc_dir, counter):
    agg = {}
    for r in csv.DictReader(open(_one(os.path.join(pmc_dir, "*_counter_collection.csv")))):
        if r["Counter_Name"] != counter or "piton::" not in r["Kernel_Name"]:
            continue
        key = (short(r["Kernel_Name"]), int(r["Grid_Size"]))
        agg.setdefault(key, []).append(float(r["Counter_Value"]) * 1024.0)  # KiB -> bytes
    return {k: sum(v) / len(v) for k, v in agg.items()}


def summarize(kt_dir, fetch_dir, write_dir, timed_steps=0):
    fetch, write = counters(fetch_dir, "FETCH_SIZE"), counters(write_dir, "WRITE_SIZE")
    cal = [k for k in fetch if k[0].startswith("add_vec4_kernel")]
    if not cal:
        raise RuntimeError("no calibration add in the counter runs")
    f_fetch = CAL_READ / fetch[cal[0]]
    f_write = CAL_WRITE / write[cal[0]]
    traffic = {}
    for k in fetch:
        if k in write and k in BENCH:
            label, algo, _ = BENCH[k]
            traffic[label] = dict(kernel=k[0], grid=k[1], fetch_bytes=fetch[k] * f_fetch,
                                  write_bytes=write[k] * f_write,
                                  traffic_bytes=fetch[k] * f_fetch + write[k] * f_write, algorithmic_bytes=algo)
    return kernel_stats(kt_dir, timed_steps), traffic, f_fetch, f_write


def mfma_busy(pmc_dir, xcds=8, simds=1024):
    """MFMA pipe occupancy per benchmark MFMA kernel from a
    `--pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES` run: SQ_VALU_MFMA_BUSY_CYCLES is summed
    over the SIMDs and GRBM_GUI_ACTIVE over the XCDs (both as rocprofv3 reports them), so
    busy = MFMA cycles / (GUI cycles / xcds * simds), a ratio of cycles that does not depend
    on the clock the kernel ran at."""
    per = {}
    for r in csv.DictReader(open(_one(os.path.join(pmc_dir, "*_counter_collection.csv")))):
        key = (short(r["Kernel_Name"]), int(r["Grid_Size"]))
        if key not in BENCH or not BENCH[key][2]:
            continue
        per.setdefault((key, r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
    out = {}
    for (key, _), d in per.items():
        if "GRBM_GUI_ACTIVE" in d and "SQ_VALU_MFMA_BUSY_CYCLES" in d:
            out.setdefault(key, []).append(d["SQ_VALU_MFMA_BUSY_CYCLES"] / (d["GRBM_GUI_ACTIVE"] / xcds * simds))
    return {BENCH[k][0]: dict(kernel=k[0], dispatches=len(v), mfma_busy=sum(v) / len(v)) for k, v in out.items()}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("kt_dir")
    ap.add_argument("fetch_dir", nargs="?")
    ap.add_argument("write_dir", nargs="?")
    ap.add_argument("--json")
    ap.add_argument("--timed-steps", type=int, default=20,
                    help="bench.py --steps of the traced run: the matmul's timed dispatches are its last ones")
    ap.add_argument("--commit", default=None, help="the commit the traced runs were made at (recorded)")
    ap.add_argument("--mfma", action="store_true",
                    help="kt_dir is a --pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES run: print MFMA occupancy")
    a = ap.parse_args(argv)
    if a.mfma:
        sys.stdout.write("| workload | kernel | dispatches | MFMA pipe busy |\n|---|---|---|---|\n")
        for label, m in mfma_busy(a.kt_dir).items():
            sys.stdout.write(f"| {label} | `{m['kernel']}` | {m['dispatches']} | {100 * m['mfma_busy']:.1f} % |\n")
        return
    stats, traffic, ff, fw = summarize(a.kt_dir, a.fetch_dir, a.write_dir, a.timed_steps)
    out = sys.stdout
    if a.commit:
        out.write(f"Traced at commit {a.commit}.\n\n")
    for r in stats:
        if "timed_avg_ns" in r:
            flops = BENCH[(r["kernel"], r["grid"])][2]
            out.write(f"bench.py's timed region: the last {a.timed_steps} `{r['kernel']}` dispatches (after the "
                      f"untimed clock ramp and warm-up) average {r['timed_avg_ns'] / 1e3:.2f} us = "
                      f"{flops / r['timed_avg_ns'] / 1e3:.1f} TFLOP/s.\n\n")
    out.write("## Kernel durations (rocprofv3 --kernel-trace, per dispatch, grouped by grid)\n\n")
    out.write("| kernel | grid (work-items) | benchmark workload | calls | avg us | median us | min us | max us | "
              "achieved |\n|---|---|---|---|---|---|---|---|---|\n")
    for r in stats:
        bench = BENCH.get((r["kernel"], r["grid"]))
        ach = ""
        if bench:
            _, nbytes, flops = bench
            ach = (f"{flops / r['avg_ns'] / 1e3:.1f} TFLOP/s" if flops else f"{nbytes / r['avg_ns']:.0f} GB/s")
        out.write(f"| `{r['kernel']}` | {r['grid']} | {r['workload']} | {r['calls']} | {r['avg_ns'] / 1e3:.2f} | "
                  f"{r['median_ns'] / 1e3:.2f} | {r['min_ns'] / 1e3:.2f} | {r['max_ns'] / 1e3:.2f} | {ach} |\n")
    out.write(f"\n## HBM traffic per launch (FETCH_SIZE x {ff:.3f}, WRITE_SIZE x {fw:.3f})\n\n")
    out.write("Scale factors: the calibration add reads 512 MiB and writes 256 MiB; the counters read "
              f"{CAL_READ / ff / 2 ** 20:.1f} MiB and {CAL_WRITE / fw / 2 ** 20:.1f} MiB for it.\n\n")
    out.write("| workload | kernel | fetch MB | write MB | traffic MB | algorithmic MB | traffic / algorithmic |\n")
    out.write("|---|---|---|---|---|---|---|\n")
    for label, t in traffic.items():
        algo = t["algorithmic_bytes"]
        out.write(f"| {label} | `{t['kernel']}` | {t['fetch_bytes'] / 1e6:.1f} | {t['write_bytes'] / 1e6:.1f} | "
                  f"{t['traffic_bytes'] / 1e6:.1f} | {algo / 1e6:.1f} | {t['traffic_bytes'] / algo:.2f} |\n")
    if a.json:
        with open(a.json, "w") as f:
            json.dump(dict(commit=a.commit, fetch_factor=ff, write_factor=fw, kernels=traffic), f, indent=1)


if __name__ == "__main__":
    main()
