"""A/B gate for a change to the library (perf/ab.py:1-15, 50-62): the performance suite runs
alternately against two builds of libpiton_mi355x.so, A (the baseline) and B (the change).

    python -m piton_amd.ab --a base/libpiton_mi355x.so --b piton_amd/lib/libpiton_mi355x.so \\
        [cases ...] [--target softmax matmul] [--rounds 2]

Each round runs every case under A and under B, in separate processes (A B, then B A, ...),
and keeps each build's best time per case. Outputs: B's checked sample must equal A's bit for
bit ("identical") or, failing that, pass the case's own tolerance against float64 ("within
tolerance"); a wrong or failed case rejects the change. The verdict follows the reference's
rule: accept when every case is correct, some target case (default: any) is more than 2 %
faster, and no case is more than 2 % slower.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

THRESHOLD = 0.02


def run_suite(lib: str, cases, small: bool, workdir: str, tag: str, timeout: int = 900):
    """(rows by name, samples) of one suite run against the library at `lib`."""
    js, npz = os.path.join(workdir, tag + ".json"), os.path.join(workdir, tag + ".npz")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PITON_MI355X_LIB=os.path.abspath(lib),
               PYTHONPATH=os.pathsep.join([root, os.environ.get("PYTHONPATH", "")]))
    cmd = [sys.executable, "-m", "piton_amd.perf_suite", *cases, "--json", js, "--outputs", npz]
    if small:
        cmd.append("--small")
    r = subprocess.run(cmd, env=env, timeout=timeout, capture_output=True, text=True)
    if not os.path.exists(js):
        raise RuntimeError(f"suite against {lib} failed ({r.returncode}):\n{r.stderr[-3000:]}")
    rows = {row["name"]: row for row in json.load(open(js))}
    with np.load(npz) as z:
        samples = {k: z[k] for k in z.files}
    return rows, samples


def compare(rows_a, rows_b, samples_a, samples_b, best_a, best_b):
    """One result row per case: speedup of B over A, and how B's outputs relate to A's."""
    out = []
    for name in rows_a:
        ra, rb = rows_a[name], rows_b[name]
        if not rb.get("ok"):
            status = "wrong"
        elif name in samples_a and np.array_equal(samples_a[name], samples_b[name]):
            status = "identical"
        else:
            status = "within tolerance"
        out.append(dict(name=name, a_us=best_a[name], b_us=best_b[name], speedup=best_a[name] / best_b[name],
                        outputs=status, errors=rb.get("error")))
    return out


def verdict(results, targets=()) -> tuple:
    """(accepted, reason) by the reference's rule (perf/ab.py:50-62)."""
    bad = [r["name"] for r in results if r["outputs"] == "wrong"]
    if bad:
        return False, "wrong: " + ", ".join(bad)
    slower = [f"{r['name']} {r['speedup']:.3f}x" for r in results if r["speedup"] < 1 - THRESHOLD]
    if slower:
        return False, "slower: " + ", ".join(slower)
    faster = [r for r in results if (not targets or r["name"] in targets) and r["speedup"] > 1 + THRESHOLD]
    if not faster:
        return False, "no target case more than 2% faster"
    return True, "faster: " + ", ".join(f"{r['name']} {r['speedup']:.3f}x" for r in faster)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--a", required=True, help="baseline libpiton_mi355x.so")
    ap.add_argument("--b", required=True, help="changed libpiton_mi355x.so")
    ap.add_argument("cases", nargs="*")
    ap.add_argument("--target", nargs="*", default=[])
    ap.add_argument("--rounds", type=int, default=2)
    ap.add_argument("--small", action="store_true")
    ap.add_argument("--json")
    a = ap.parse_args(argv)
    from .perf_suite import CASES
    cases = a.cases or list(CASES)
    work = tempfile.mkdtemp(prefix="piton_ab_")
    best = {"a": {}, "b": {}}
    rows, samples = {}, {}
    for rnd in range(a.rounds):
        order = ("a", "b") if rnd % 2 == 0 else ("b", "a")
        for side in order:
            r, s = run_suite(getattr(a, side), cases, a.small, work, f"{side}{rnd}")
            rows.setdefault(side, r)
            samples.setdefault(side, s)
            for name, row in r.items():
                if not row.get("ok"):
                    rows[side][name] = row
                best[side][name] = min(best[side].get(name, float("inf")), row["us"])
    results = compare(rows["a"], rows["b"], samples["a"], samples["b"], best["a"], best["b"])
    ok, why = verdict(results, a.target)
    for r in results:
        print(f"{r['name']:12s} A {r['a_us']:10.2f} us  B {r['b_us']:10.2f} us  {r['speedup']:6.3f}x  {r['outputs']}")
    print(("ACCEPT: " if ok else "REJECT: ") + why)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(dict(results=results, accepted=ok, reason=why), f, indent=1)


if __name__ == "__main__":
    main()
