"""Summaries of rocprofv3 output for the benchmark kernels.

    python -m piton_amd.profiling KT_DIR FETCH_DIR WRITE_DIR [--json OUT]
    python -m piton_amd.profiling PMC_DIR --mfma [--trace KT_DIR --clock GHZ]

KT_DIR holds a `--kernel-trace --stats` run of `python3 bench.py` (*_kernel_trace.csv);
FETCH_DIR / WRITE_DIR hold `--pmc FETCH_SIZE` / `--pmc WRITE_SIZE` runs of
`python3 bench.py --pmc-probe` (*_counter_collection.csv). Prints a markdown summary: each
kernel's average duration, each benchmark workload's kernel time per step (the sum over its
launches), and its HBM traffic per step, each counter scaled by the factor that maps the
calibration add of known size (bench.py CAL_ELEMS: reads 2 x 256 MiB, writes 256 MiB) onto its
true bytes. --json writes {workload: {fetch_bytes, write_bytes, ...}}.
With --mfma, PMC_DIR holds a `--pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES` run of
`python3 bench.py --pmc-probe`: the MFMA pipe occupancy of the benchmark's MFMA workloads, per
cycle of each dispatch's own span and per cycle of the counter window.
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

def _mm(M, N, K):
    return (4 * (M * K + K * N + M * N), 2 * M * N * K)


# the digits MLP over 1797 images: x, the three layers' weights and biases, logits and predictions
_MLP_BYTES = 4 * (1797 * 64 + 64 * 128 + 128 + 128 * 64 + 64 + 64 * 10 + 10 + 1797 * 10 + 1797)
_MLP_FLOPS = 2 * 1797 * (64 * 128 + 128 * 64 + 64 * 10)

# benchmark workloads: (algorithmic HBM bytes per step, algorithmic FLOPs per step)
WORKLOADS = {
    "matmul 4096^3": _mm(4096, 4096, 4096),
    "matmul 512^3": _mm(512, 512, 512),
    "matmul 1024^3": _mm(1024, 1024, 1024),
    "matmul 1000 x 1800 x 700 (row strides 703 / 1805 / 1807)": _mm(1000, 1800, 700),
    "matmul 1024^3, B column-major": _mm(1024, 1024, 1024),
    "softmax 4096 x 1024": (2 * 4 * 4096 * 1024, None),
    "softmax 4096 x 4096": (2 * 4 * 4096 * 4096, None),
    "softmax 4096 x 1823": (2 * 4 * 4096 * 1823, None),
    "attention 32 x 1024 x 64 causal": (4 * 32 * 1024 * 64 * 4, 4 * 1024 * 1024 * 64 * 32 // 2),
    "digits MLP, 1797 images": (_MLP_BYTES, _MLP_FLOPS),
}
# their launches, identified by kernel name and Grid_Size_X (work-items), with the number of
# times a step runs each (the 4096^3 matmul: two launches of 256 tiles of 128 x 256, one per CU;
# the split GEMM's template arguments are <row blocks, column blocks, waves splitting K, A's
# layout (0: rows 16-byte aligned, 1: unaligned rows), B column-major, K % 32 != 0>; the ragged
# shape runs 240 wide tiles of 64 x 128)
LAUNCHES = {
    ("gemm_direct_kernel<true, true, false, 4>", 65536): ("matmul 4096^3", 2),
    ("gemm_split_kernel<1, 1, 4, 0, false, false>", 65536): ("matmul 512^3", 1),
    ("gemm_split_kernel<2, 2, 4, 0, false, false>", 65536): ("matmul 1024^3", 1),
    ("gemm_split_kernel<2, 4, 4, 1, false, true>", 61440): ("matmul 1000 x 1800 x 700 (row strides 703 / 1805 / 1807)", 1),
    ("gemm_split_kernel<2, 2, 4, 0, true, false>", 65536): ("matmul 1024^3, B column-major", 1),
    ("softmax_rows_kernel<4, true>", 262144): ("softmax 4096 x 1024", 1),
    ("softmax_wg_kernel<2, 512, true>", 2097152): ("softmax 4096 x 4096", 1),
    ("softmax_rows_kernel<8, false>", 196608): ("softmax 4096 x 1823", 1),
    ("attn_fwd_fast<64, true>", 131072): ("attention 32 x 1024 x 64 causal", 1),
    ("mlp3_rows16_kernel<64, 128, 64, 10>", 28928): ("digits MLP, 1797 images", 1),
}
MAX_CLOCK_GHZ = 2.4  # the engine clock's maximum: a lower bound on busy cycles per busy time
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
    `--pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES` run, in two normalisations (summed over all
    dispatches of a workload's launches):
      * per GUI cycle: SQ_VALU_MFMA_BUSY_CYCLES (summed over the SIMDs) / (GRBM_GUI_ACTIVE / xcds *
        simds). GRBM_GUI_ACTIVE counts every cycle of the counter window, which under the
        profiler is longer than the kernel (the dispatch and its drain), so this understates the
        kernel's own occupancy, most for short launches;
      * per kernel cycle: the same busy cycles / (simds * the dispatch's own duration, End_Timestamp -
        Start_Timestamp, * MAX_CLOCK_GHZ): the occupancy over the kernel's span at the maximum
        clock (a lower bound: the clock is at most that).
    `window_over_kernel` is the ratio of the two denominators."""
    per = {}
    for r in csv.DictReader(open(_one(os.path.join(pmc_dir, "*_counter_collection.csv")))):
        key = (short(r["Kernel_Name"]), int(r["Grid_Size"]))
        if key not in LAUNCHES or not WORKLOADS[LAUNCHES[key][0]][1]:
            continue
        d = per.setdefault((key, r["Dispatch_Id"]), {})
        d[r["Counter_Name"]] = float(r["Counter_Value"])
        d["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    out = {}
    for (key, _), d in per.items():
        if "GRBM_GUI_ACTIVE" in d and "SQ_VALU_MFMA_BUSY_CYCLES" in d:
            w = out.setdefault(LAUNCHES[key][0], dict(kernels=[], dispatches=0, busy=0.0, cycles=0.0, kcycles=0.0,
                                                      ns=0))
            if key[0] not in w["kernels"]:
                w["kernels"].append(key[0])
            w["dispatches"] += 1
            w["busy"] += d["SQ_VALU_MFMA_BUSY_CYCLES"]
            w["cycles"] += d["GRBM_GUI_ACTIVE"] / xcds * simds
            w["kcycles"] += d["ns"] * MAX_CLOCK_GHZ * simds
            w["ns"] += d["ns"]
    return {label: dict(kernel=" + ".join(w["kernels"]), dispatches=w["dispatches"], mfma_busy=w["busy"] / w["cycles"],
                        mfma_busy_kernel=w["busy"] / w["kcycles"], kernel_us=w["ns"] / w["dispatches"] / 1e3,
                        window_over_kernel=w["cycles"] / w["kcycles"],
                        busy_cycles_per_launch=w["busy"] / w["dispatches"])
            for label, w in out.items()}


def mfma_busy_traced(pmc_dir, kt_dir, clock_ghz, simds=1024):
    """The busy cycles of each MFMA workload's launch (a count of the work: MFMAs x their cycles,
    the same with or without the profiler) over the cycles of its median span in a kernel trace
    (where the kernels run as in the benchmark; under --pmc they run slower) at `clock_ghz`, the
    clock the device sustains (bench.py's mfma_sustained)."""
    spans = {}
    for r in kernel_stats(kt_dir):
        key = (r["kernel"], r["grid"])
        if key in LAUNCHES:
            spans[LAUNCHES[key][0]] = (r["median_ns"], LAUNCHES[key][1])
    out = {}
    for label, m in mfma_busy(pmc_dir, simds=simds).items():
        if label in spans:
            ns, per_step = spans[label]
            out[label] = dict(m, traced_median_us=ns / 1e3,
                              mfma_busy_traced=m["busy_cycles_per_launch"] / (simds * ns * clock_ghz))
    return out


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
    ap.add_argument("--trace", default=None,
                    help="with --mfma: a --kernel-trace run of bench.py, whose median spans normalise the busy cycles")
    ap.add_argument("--clock", type=float, default=MAX_CLOCK_GHZ,
                    help="with --trace: the engine clock in GHz (bench.py's mfma_sustained clock_ghz)")
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
        traced = mfma_busy_traced(a.kt_dir, a.trace, a.clock) if a.trace else {}
        sys.stdout.write("| workload | kernel | dispatches | busy cycles per launch | kernel us under --pmc | "
                         f"busy per cycle of that span (at {MAX_CLOCK_GHZ} GHz) | busy per GUI cycle | "
                         "counter window / span |" + (f" traced median us | busy per cycle of the traced span "
                                                      f"(at {a.clock} GHz) |" if traced else "") + "\n" +
                         "|---" * (8 + (2 if traced else 0)) + "|\n")
        for label, m in mfma_busy(a.kt_dir).items():
            t = traced.get(label)
            sys.stdout.write(f"| {label} | `{m['kernel']}` | {m['dispatches']} | {m['busy_cycles_per_launch']:.4g} | "
                             f"{m['kernel_us']:.2f} | {100 * m['mfma_busy_kernel']:.1f} % | "
                             f"{100 * m['mfma_busy']:.1f} % | {m['window_over_kernel']:.2f} |" +
                             (f" {t['traced_median_us']:.2f} | {100 * t['mfma_busy_traced']:.1f} % |" if t else
                              (" — | — |" if traced else "")) + "\n")
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
    out.write("The 4096^3 row leads with bench.py's timed steps (the dispatches of its timed region); every row "
              "also gives the average over all of the workload's dispatches (warm-up, clock ramp and the "
              "HIP-graph replays included).\n\n")
    out.write("| workload | launches per step | us per step (timed steps) | achieved (timed steps) | "
              "us per step (all dispatches) | achieved (all dispatches) |\n|---|---|---|---|---|---|\n")

    def achieved(w, ns):
        return (f"{w['flops'] / ns / 1e3:.1f} TFLOP/s" if w["flops"] else f"{w['algorithmic_bytes'] / ns:.0f} GB/s")

    for label, w in steps.items():
        timed = (f"{w['timed_step_ns'] / 1e3:.2f} | {achieved(w, w['timed_step_ns'])}" if "timed_step_ns" in w
                 else "— | —")
        out.write(f"| {label} | {' + '.join(f'`{k}`' for k in w['launches'])} | {timed} | "
                  f"{w['step_ns'] / 1e3:.2f} | {achieved(w, w['step_ns'])} |\n")
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
