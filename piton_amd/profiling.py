"""Summaries of rocprofv3 output for the benchmark kernels.

    python -m piton_amd.profiling KT_DIR FETCH_DIR WRITE_DIR [--json OUT]
    python -m piton_amd.profiling PMC_DIR --mfma

KT_DIR holds a `--kernel-trace --stats` run of `python3 bench.py` (*_kernel_trace.csv);
FETCH_DIR / WRITE_DIR hold `--pmc FETCH_SIZE` / `--pmc WRITE_SIZE` runs of
`python3 bench.py --pmc-probe` (*_counter_collection.csv). Prints a markdown summary: each
kernel's average duration, each benchmark workload's kernel time per step (the sum over its
launches), and its HBM traffic per step, each counter scaled by the factor that maps the
calibration add of known size (bench.py CAL_ELEMS: reads 2 x 256 MiB, writes 256 MiB) onto its
true bytes. --json writes {workload: {fetch_bytes, write_bytes, ...}}.
With --mfma, PMC_DIR holds a `--pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES` run of
`python3 bench.py --pmc-probe`: the MFMA pipe occupancy of the benchmark's MFMA workloads.
With --lds, PMC_DIR holds a `--pmc GRBM_GUI_ACTIVE SQ_WAVE_CYCLES SQ_LDS_IDX_ACTIVE
SQ_LDS_BANK_CONFLICT` run of the same: each workload's mean resident waves per SIMD and its LDS
bank-conflict cycles per conflict-free LDS cycle.
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

# benchmark workloads: (algorithmic HBM bytes per step, algorithmic FLOPs per step)
WORKLOADS = {
    "matmul 4096^3": (3 * 4096 * 4096 * 4, 2 * 4096 ** 3),
    "softmax 4096 x 1024": (2 * 4 * 4096 * 1024, None),
    "softmax 4096 x 4096": (2 * 4 * 4096 * 4096, None),
    "softmax 4096 x 1823": (2 * 4 * 4096 * 1823, None),
    "attention 32 x 1024 x 64 causal": (4 * 32 * 1024 * 64 * 4, 4 * 1024 * 1024 * 64 * 32 // 2),
}
# their launches, identified by kernel name and Grid_Size_X (work-items), with the number of
# times a step runs each (the 4096^3 matmul: two launches of 256 tiles of 128 x 256, one per CU)
LAUNCHES = {
    ("gemm_direct_kernel<true, true, false, 4>", 65536): ("matmul 4096^3", 2),
    ("softmax_rows_kernel<4, true>", 262144): ("softmax 4096 x 1024", 1),
    ("softmax_wg_kernel<2, 512, true>", 2097152): ("softmax 4096 x 4096", 1),
    ("softmax_rows_kernel<8, false>", 196608): ("softmax 4096 x 1823", 1),
    ("attn_fwd_fast<64, true>", 131072): ("attention 32 x 1024 x 64 causal", 1),
}
TIMED = "matmul 4096^3"  # the workload of bench.py's timed region


def short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "").split("(")[0]
    name = re.sub(r"^void ", "", name)
    return name.replace("piton::", "")


def _one(pattern):
    files = glob.glob(pattern)
    if not files:
        raise FileNotFoundError(pattern)
    return files[0]


def kernel_stats(kt_dir, timed_steps=0):
    """Per (kernel, grid) launch statistics from the per-dispatch trace. With timed_steps, the
    launches of the 4096^3 matmul also report the average of their last `timed_steps` dispatches
    in dispatch order: bench.py's timed region (their earlier dispatches are the untimed clock
    ramp and warm-up)."""
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
                   median_ns=d[len(d) // 2], max_ns=d[-1], workload=LAUNCHES.get((k, grid), ("", 0))[0],
                   per_step=LAUNCHES.get((k, grid), ("", 0))[1])
        if timed_steps and row["workload"] == TIMED and len(in_order) >= timed_steps * row["per_step"]:
            last = in_order[-timed_steps * row["per_step"]:]
            row["timed_avg_ns"] = sum(last) / len(last)
        rows.append(row)
    return rows


def workload_steps(stats):
    """Per benchmark workload: its launches' average durations, each times the launches of it a
    step makes, summed (the kernel time of one step, gaps between the launches excluded), the
    timed region's too where known."""
    out = {}
    for label, (nbytes, flops) in WORKLOADS.items():
        rows = [r for r in stats if r["workload"] == label]
        if not rows:
            continue
        step_ns = sum(r["avg_ns"] * r["per_step"] for r in rows)
        d = dict(launches=[f"{r['kernel']}" + (f" x {r['per_step']}" if r["per_step"] > 1 else "") for r in rows],
                 step_ns=step_ns, algorithmic_bytes=nbytes, flops=flops)
        if all("timed_avg_ns" in r for r in rows):
            d["timed_step_ns"] = sum(r["timed_avg_ns"] * r["per_step"] for r in rows)
        out[label] = d
    return out


def counters(pmc_dir, counter):
    agg = {}
    for r in csv.DictReader(open(_one(os.path.join(pmc_dir, "*_counter_collection.csv")))):
        if r["Counter_Name"] != counter or "piton::" not in r["Kernel_Name"]:
            continue
        key = (short(r["Kernel_Name"]), int(r["Grid_Size"]))
        agg.setdefault(key, []).append(float(r["Counter_Value"]) * 1024.0)  # KiB -> bytes
    return {k: sum(v) / len(v) for k, v in agg.items()}


def summarize(kt_dir, fetch_dir, write_dir, timed_steps=0):
    """Launch statistics, and per workload its HBM traffic per step: each launch's average
    counter values summed over the step's launches, each counter scaled by the calibration
    add's factor."""
    fetch, write = counters(fetch_dir, "FETCH_SIZE"), counters(write_dir, "WRITE_SIZE")
    cal = [k for k in fetch if k[0].startswith("add_vec4_kernel")]
    if not cal:
        raise RuntimeError("no calibration add in the counter runs")
    f_fetch = CAL_READ / fetch[cal[0]]
    f_write = CAL_WRITE / write[cal[0]]
    traffic = {}
    for label, (algo, _) in WORKLOADS.items():
        keys = [k for k, (w, _) in LAUNCHES.items() if w == label and k in fetch and k in write]
        if not keys:
            continue
        fb = sum(fetch[k] * LAUNCHES[k][1] for k in keys) * f_fetch
        wb = sum(write[k] * LAUNCHES[k][1] for k in keys) * f_write
        traffic[label] = dict(kernel=" + ".join(k[0] for k in keys), grid=[k[1] for k in keys], fetch_bytes=fb,
                              write_bytes=wb, traffic_bytes=fb + wb, algorithmic_bytes=algo)
    return kernel_stats(kt_dir, timed_steps), traffic, f_fetch, f_write


def mfma_busy(pmc_dir, xcds=8, simds=1024):
    """MFMA pipe occupancy per benchmark MFMA workload from a
    `--pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES` run: SQ_VALU_MFMA_BUSY_CYCLES is summed
    over the SIMDs and GRBM_GUI_ACTIVE over the XCDs (both as rocprofv3 reports them), so
    busy = MFMA cycles / (GUI cycles / xcds * simds), a ratio of cycles that does not depend
    on the clock the kernel ran at; over all dispatches of a workload's launches (weighted by
    their cycles)."""
    per = {}
    for r in csv.DictReader(open(_one(os.path.join(pmc_dir, "*_counter_collection.csv")))):
        key = (short(r["Kernel_Name"]), int(r["Grid_Size"]))
        if key not in LAUNCHES or not WORKLOADS[LAUNCHES[key][0]][1]:
            continue
        per.setdefault((key, r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
    out = {}
    for (key, _), d in per.items():
        if "GRBM_GUI_ACTIVE" in d and "SQ_VALU_MFMA_BUSY_CYCLES" in d:
            w = out.setdefault(LAUNCHES[key][0], dict(kernels=[], dispatches=0, busy=0.0, cycles=0.0))
            if key[0] not in w["kernels"]:
                w["kernels"].append(key[0])
            w["dispatches"] += 1
            w["busy"] += d["SQ_VALU_MFMA_BUSY_CYCLES"]
            w["cycles"] += d["GRBM_GUI_ACTIVE"] / xcds * simds
    return {label: dict(kernel=" + ".join(w["kernels"]), dispatches=w["dispatches"], mfma_busy=w["busy"] / w["cycles"])
            for label, w in out.items()}


def _per_dispatch(pmc_dir):
    """{((kernel, grid), dispatch): {counter: value}} for the benchmark launches."""
    per = {}
    for r in csv.DictReader(open(_one(os.path.join(pmc_dir, "*_counter_collection.csv")))):
        key = (short(r["Kernel_Name"]), int(r["Grid_Size"]))
        if key in LAUNCHES:
            per.setdefault((key, r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
    return per


def lds_occupancy(pmc_dir, xcds=8, cus=256, simds_per_cu=4):
    """Per benchmark workload, from a `--pmc GRBM_GUI_ACTIVE SQ_WAVE_CYCLES SQ_LDS_IDX_ACTIVE
    SQ_LDS_BANK_CONFLICT` run (each counter summed over the chip, as rocprofv3 reports them):
    waves per SIMD = 4 SQ_WAVE_CYCLES (counted in units of 4 cycles) / (GUI cycles per XCD x
    SIMDs), the time-averaged resident waves, against the kernel's launch limit; LDS conflicts =
    SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE - SQ_LDS_BANK_CONFLICT), the cycles lost to bank
    conflicts per conflict-free cycle of LDS access (the LdsBankConflict definition of
    rocprofiler-sdk's counter_defs.yaml for gfx950). Sums over all dispatches of a workload."""
    out = {}
    for (key, _), d in _per_dispatch(pmc_dir).items():
        need = ("GRBM_GUI_ACTIVE", "SQ_WAVE_CYCLES", "SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT")
        if not all(c in d for c in need):
            continue
        w = out.setdefault(LAUNCHES[key][0], dict(kernels=[], dispatches=0, wave=0.0, cycles=0.0, lds=0.0, conf=0.0))
        if key[0] not in w["kernels"]:
            w["kernels"].append(key[0])
        w["dispatches"] += 1
        w["wave"] += 4 * d["SQ_WAVE_CYCLES"]
        w["cycles"] += d["GRBM_GUI_ACTIVE"] / xcds * cus * simds_per_cu
        w["lds"] += d["SQ_LDS_IDX_ACTIVE"]
        w["conf"] += d["SQ_LDS_BANK_CONFLICT"]
    return {label: dict(kernel=" + ".join(w["kernels"]), dispatches=w["dispatches"],
                        waves_per_simd=w["wave"] / w["cycles"],
                        lds_active=w["lds"], lds_conflict_cycles=w["conf"],
                        lds_conflict_ratio=w["conf"] / (w["lds"] - w["conf"]) if w["lds"] > w["conf"] else None)
            for label, w in out.items()}


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
    ap.add_argument("--lds", action="store_true",
                    help="kt_dir is a --pmc GRBM_GUI_ACTIVE SQ_WAVE_CYCLES SQ_LDS_IDX_ACTIVE SQ_LDS_BANK_CONFLICT run: "
                         "print resident waves and LDS bank conflicts")
    a = ap.parse_args(argv)
    if a.lds:
        sys.stdout.write("| workload | kernel | dispatches | resident waves per SIMD | LDS active cycles "
                         "| bank-conflict cycles | conflict cycles per conflict-free LDS cycle |\n"
                         "|---|---|---|---|---|---|---|\n")
        for label, m in lds_occupancy(a.kt_dir).items():
            ratio = "—" if m["lds_conflict_ratio"] is None else f"{m['lds_conflict_ratio']:.3f}"
            sys.stdout.write(f"| {label} | `{m['kernel']}` | {m['dispatches']} | {m['waves_per_simd']:.2f} | "
                             f"{m['lds_active']:.3g} | {m['lds_conflict_cycles']:.3g} | {ratio} |\n")
        return
    if a.mfma:
        sys.stdout.write("| workload | kernel | dispatches | MFMA pipe busy |\n|---|---|---|---|\n")
        for label, m in mfma_busy(a.kt_dir).items():
            sys.stdout.write(f"| {label} | `{m['kernel']}` | {m['dispatches']} | {100 * m['mfma_busy']:.1f} % |\n")
        return
    stats, traffic, ff, fw = summarize(a.kt_dir, a.fetch_dir, a.write_dir, a.timed_steps)
    steps = workload_steps(stats)
    out = sys.stdout
    if a.commit:
        out.write(f"Traced at commit {a.commit}.\n\n")
    t = steps.get(TIMED)
    if t and "timed_step_ns" in t:
        out.write(f"bench.py's timed region: the last {a.timed_steps} steps' dispatches of "
                  f"{', '.join(f'`{k}`' for k in t['launches'])} (after the untimed clock ramp and warm-up) "
                  f"take {t['timed_step_ns'] / 1e3:.2f} us per step together = "
                  f"{t['flops'] / t['timed_step_ns'] / 1e3:.1f} TFLOP/s.\n\n")
    out.write("## Benchmark workloads (kernel time per step: the averages of the step's launches, summed)\n\n")
    out.write("| workload | launches per step | us per step | achieved |\n|---|---|---|---|\n")
    for label, w in steps.items():
        ach = (f"{w['flops'] / w['step_ns'] / 1e3:.1f} TFLOP/s" if w["flops"]
               else f"{w['algorithmic_bytes'] / w['step_ns']:.0f} GB/s")
        out.write(f"| {label} | {' + '.join(f'`{k}`' for k in w['launches'])} | {w['step_ns'] / 1e3:.2f} | {ach} |\n")
    out.write("\n## Kernel durations (rocprofv3 --kernel-trace, per dispatch, grouped by grid)\n\n")
    out.write("| kernel | grid (work-items) | benchmark workload | calls | avg us | median us | min us | max us |\n"
              "|---|---|---|---|---|---|---|---|\n")
    for r in stats:
        out.write(f"| `{r['kernel']}` | {r['grid']} | {r['workload']} | {r['calls']} | {r['avg_ns'] / 1e3:.2f} | "
                  f"{r['median_ns'] / 1e3:.2f} | {r['min_ns'] / 1e3:.2f} | {r['max_ns'] / 1e3:.2f} |\n")
    out.write(f"\n## HBM traffic per step (FETCH_SIZE x {ff:.3f}, WRITE_SIZE x {fw:.3f})\n\n")
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
