"""The performance suite on one MI355X (perf/suite.py, perf/profile_pi.py, perf/analyze.py):
every kernel of the library at a size that fills the chip, timed from HIP-graph replays, its
output checked on a sample against float64 with the suite's tolerance.

    python -m piton_amd.perf_suite                      # every case, a table
    python -m piton_amd.perf_suite copy exp matmul --json out.json --outputs out.npz
    python -m piton_amd.perf_suite copy --pmc FETCH_SIZE   # one rocprofv3 counter pass
    python -m piton_amd.perf_suite --small              # reduced sizes (tests)

Each case reports its algorithmic bytes (every input read once, every output written once)
or FLOPs, the time per launch, and the fraction of the MI355X roof that bounds it (8 TB/s
HBM, or 157.3 TFLOP/s fp32 MFMA). --outputs saves each case's checked sample for the A/B
gate (piton_amd.ab). --pmc runs the named cases once under `rocprofv3 --pmc` (one pass: at
most 8 SQ, 4 TCC, 4 TCP, 2 TA, 2 TD, 2 GRBM counters; FETCH_SIZE takes 3 TCC) and prints the
counters of this library's kernels.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import subprocess
import sys
import tempfile
from dataclasses import dataclass
from typing import Callable

import numpy as np

PEAK_HBM = 8.0e12
PEAK_FP32_MFMA = 157.3e12


@dataclass
class Built:
    run: Callable[[int], None]             # launch i (a graph records iters of them)
    sample: Callable[[], np.ndarray]       # the checked outputs, on the host
    want: Callable[[], np.ndarray]         # their float64 (or exact) expectation
    rtol: float
    atol: float
    nbytes: float
    flops: float = 0.0
    exact: bool = False


def _gen(seed):
    import torch
    return torch.Generator(device="cuda").manual_seed(seed)


def _uniform(n, lo, hi, seed):
    import torch
    return torch.rand(n, device="cuda", generator=_gen(seed)) * (hi - lo) + lo


def _sample_idx(n, k=4099):
    return np.arange(0, n, k)


def _elementwise(op_name, n_in, lo, hi, ref, rtol, atol, alpha=None, sfu_op=None):
    def build(size):
        import torch

        from .runtime import mi355x as rt
        n = size
        xs = [_uniform(n, lo, hi, 11 + i) for i in range(n_in)]
        out = torch.empty(n, device="cuda")
        fn = getattr(rt, op_name)
        extra = [alpha] if alpha is not None else ([sfu_op] if sfu_op is not None else [])
        idx = _sample_idx(n)
        ti = torch.from_numpy(idx).cuda()
        return Built(run=lambda i: fn(*xs, out, n, *extra),
                     sample=lambda: out[ti].cpu().numpy(),
                     want=lambda: ref(*[x[ti].cpu().numpy().astype(np.float64) for x in xs]),
                     rtol=rtol, atol=atol, nbytes=4.0 * n * (n_in + 1))
    return build


def _idiv(size):
    import torch

    from .runtime import mi355x as rt
    n = size
    g = _gen(5)
    x = torch.randint(-2 ** 31, 2 ** 31 - 1, (n,), device="cuda", generator=g, dtype=torch.int32)
    y = (torch.randint(-2 ** 31, 2 ** 31 - 1, (n,), device="cuda", generator=g, dtype=torch.int32) >> 8) | 1
    q, r = torch.empty_like(x), torch.empty_like(x)
    ti = torch.from_numpy(_sample_idx(n)).cuda()

    def want():
        a, b = x[ti].cpu().numpy().astype(np.int64), y[ti].cpu().numpy().astype(np.int64)
        qq = np.sign(a) * np.sign(b) * (np.abs(a) // np.abs(b))
        return np.concatenate([qq, a - qq * b])

    return Built(run=lambda i: rt.idiv(x, y, q, r, n),
                 sample=lambda: np.concatenate([q[ti].cpu().numpy(), r[ti].cpu().numpy()]).astype(np.int64),
                 want=want, rtol=0, atol=0, nbytes=16.0 * n, exact=True)


def _row(op_name, ref, rtol):
    def build(size):
        import torch

        from .runtime import mi355x as rt
        m = size
        x = _uniform(m * m, -1, 1, 21)
        out = torch.empty(m, device="cuda")
        rows = torch.arange(0, m, 61, device="cuda")
        fn = getattr(rt, op_name)
        return Built(run=lambda i: fn(x, out, m, m, m), sample=lambda: out[rows].cpu().numpy(),
                     want=lambda: ref(x.view(m, m)[rows].cpu().numpy().astype(np.float64), axis=1),
                     rtol=rtol, atol=1e-5, nbytes=4.0 * m * (m + 1))
    return build


def _transpose(size):
    import torch

    from .runtime import mi355x as rt
    m = size
    x = _uniform(m * m, -1, 1, 31)
    out = torch.empty(m * m, device="cuda")
    rows = torch.arange(0, m, 67, device="cuda")
    return Built(run=lambda i: rt.transpose(x, out, m, m, m, m), sample=lambda: out.view(m, m)[rows].cpu().numpy(),
                 want=lambda: x.view(m, m)[:, rows].t().cpu().numpy().astype(np.float64), rtol=0, atol=0,
                 nbytes=8.0 * m * m, exact=True)


def _softmax(size):
    import torch

    from . import next_power_of_2
    from .runtime import mi355x as rt
    rows, n = 4096, size
    x = torch.randn((rows, n), device="cuda", generator=_gen(41)) * 4
    out = torch.empty_like(x)
    sel = torch.arange(0, rows, 97, device="cuda")

    def want():
        a = x[sel].cpu().numpy().astype(np.float64)
        e = np.exp(a - a.max(axis=1, keepdims=True))
        return e / e.sum(axis=1, keepdims=True)

    return Built(run=lambda i: rt.softmax(out, x, n, n, n, rows, next_power_of_2(n)),
                 sample=lambda: out[sel].cpu().numpy(), want=want, rtol=2e-5, atol=1e-8, nbytes=8.0 * rows * n)


def _matmul(size):
    import torch

    from .runtime import mi355x as rt
    n = size
    a = torch.rand((n, n), device="cuda", generator=_gen(51)) * 2 - 1
    b = torch.rand((n, n), device="cuda", generator=_gen(52)) * 2 - 1
    c = torch.empty((n, n), device="cuda")
    sel = torch.arange(0, n, 257, device="cuda")
    return Built(run=lambda i: rt.matmul(a, b, c, n, n, n, n, 1, n, 1, n, 1, 8), sample=lambda: c[sel].cpu().numpy(),
                 want=lambda: a[sel].cpu().numpy().astype(np.float64) @ b.cpu().numpy().astype(np.float64),
                 rtol=1e-3, atol=2e-4 * n, nbytes=12.0 * n * n, flops=2.0 * n ** 3)


def _attention(size):
    import torch

    from .kernels.attention import attention_flops
    from .runtime import mi355x as rt
    from .timing import timed_graph  # noqa: F401  (same timing as every case)
    H, N, D = 32, size, 64
    g = _gen(61)
    q, k, v = (torch.randn((H, N, D), device="cuda", generator=g) for _ in range(3))
    o = torch.empty_like(q)
    hs = [0, H // 2, H - 1]

    def want():
        outs = []
        for h in hs:
            qq, kk, vv = (t[h].cpu().numpy().astype(np.float64) for t in (q, k, v))
            s = qq @ kk.T / 8.0
            s = np.where(np.tril(np.ones((N, N), bool)), s, -np.inf)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            outs.append((p / p.sum(axis=1, keepdims=True)) @ vv)
        return np.stack(outs)

    return Built(run=lambda i: rt.attn_fwd(q, k, v, o, 0.125, N * D, D, N * D, D, 1, N * D, D, N * D, D, N, H, D, True),
                 sample=lambda: o[hs].cpu().numpy(), want=want, rtol=0, atol=2e-5, nbytes=16.0 * H * N * D,
                 flops=attention_flops(N, D, causal=True, heads=H))


def _dense(size):
    import torch

    from .runtime import mi355x as rt
    m, k, n = size, 64, 128
    x = _uniform(m * k, 0, 1, 71).view(m, k)
    w = _uniform(k * n, -0.3, 0.3, 72).view(k, n)
    b = _uniform(n, -0.1, 0.1, 73)
    y = torch.empty((m, n), device="cuda")
    return Built(run=lambda i: rt.dense(x, w, b, y, m, n, k, True, True),
                 sample=lambda: y.cpu().numpy(),
                 want=lambda: np.maximum(x.cpu().numpy().astype(np.float64) @ w.cpu().numpy().astype(np.float64)
                                         + b.cpu().numpy(), 0),
                 rtol=1e-4, atol=1e-4, nbytes=4.0 * (m * k + k * n + n + m * n), flops=2.0 * m * n * k)


# name -> (builder, full size, small size)
CASES = {
    "copy": (_elementwise("copy", 1, -1, 1, lambda x: x, 1e-6, 1e-6), 1 << 26, 1 << 16),
    "mul": (_elementwise("mul", 2, -1, 1, lambda x, y: x * y, 1e-6, 1e-6), 1 << 26, 1 << 16),
    "fma": (_elementwise("fma", 2, -1, 1, lambda x, y: x * 1.5 + y, 1e-6, 1e-6, alpha=1.5), 1 << 26, 1 << 16),
    "scaled_relu": (_elementwise("scaled_relu", 1, -1, 1, lambda x: np.where(x > 0, x * 0.5, 0.0), 1e-6, 1e-6,
                                 alpha=0.5), 1 << 26, 1 << 16),
    "exp": (_elementwise("sfu", 1, -8, 8, np.exp, 4e-6, 1e-30, sfu_op=4), 1 << 26, 1 << 16),
    "exp2": (_elementwise("sfu", 1, -8, 8, np.exp2, 4e-6, 1e-30, sfu_op=0), 1 << 26, 1 << 16),
    "log": (_elementwise("log", 1, 0.01, 100, np.log, 4e-6, 4e-7), 1 << 26, 1 << 16),
    "log2": (_elementwise("sfu", 1, 0.01, 100, np.log2, 4e-6, 4e-7, sfu_op=1), 1 << 26, 1 << 16),
    "recip": (_elementwise("sfu", 1, 0.01, 100, lambda x: 1 / x, 4e-6, 1e-30, sfu_op=2), 1 << 26, 1 << 16),
    "rsqrt": (_elementwise("sfu", 1, 0.01, 100, lambda x: 1 / np.sqrt(x), 4e-6, 1e-30, sfu_op=3), 1 << 26, 1 << 16),
    "sqrt": (_elementwise("sfu", 1, 0.01, 100, np.sqrt, 4e-6, 1e-30, sfu_op=5), 1 << 26, 1 << 16),
    "idiv": (_idiv, 1 << 26, 1 << 16),
    "row_sum": (_row("row_sum", np.sum, 1e-5), 8192, 256),
    "row_max": (_row("row_max", np.max, 0.0), 8192, 256),
    "transpose": (_transpose, 8192, 256),
    "softmax": (_softmax, 4096, 256),
    "matmul": (_matmul, 4096, 256),
    "attention": (_attention, 1024, 128),
    "dense_relu": (_dense, 1797, 64),
}


def check(b: Built) -> tuple:
    got, want = b.sample(), b.want()
    if b.exact:
        bad = np.flatnonzero(got != want)
        return got, None if bad.size == 0 else f"{bad.size} wrong, first at {bad[0]}"
    g = np.asarray(got, np.float64)
    if not np.isfinite(g).all():
        return got, f"{int((~np.isfinite(g)).sum())} non-finite outputs"
    err = np.abs(g - want)
    bad = np.flatnonzero(err > b.atol + b.rtol * np.abs(want))
    return got, None if bad.size == 0 else f"{bad.size} outside tolerance, worst {err.max():.3g}"


def run_cases(names, small=False, iters=16, time_it=True):
    """[{name, us, gbs, frac, ok, error, ...}] and {name: sampled output}."""
    import torch

    from .timing import timed_graph
    rows, samples = [], {}
    for name in names:
        build, full, reduced = CASES[name]
        b = build(reduced if small else full)
        b.run(0)
        torch.cuda.synchronize()
        got, err = check(b)
        samples[name] = got
        row = dict(name=name, size=reduced if small else full, ok=err is None, error=err)
        if time_it:
            t = timed_graph(b.run, iters)
            row.update(us=round(t * 1e6, 3), gbs=round(b.nbytes / t / 1e9, 1))
            if b.flops:
                row.update(tflops=round(b.flops / t / 1e12, 2), frac=round(b.flops / t / PEAK_FP32_MFMA, 4),
                           bound="mfma")
            else:
                row.update(frac=round(b.nbytes / t / PEAK_HBM, 4), bound="hbm")
        rows.append(row)
        del b
        torch.cuda.empty_cache()
    return rows, samples


def pmc(names, counters, small=False, timeout=60):
    """One rocprofv3 --pmc pass over the cases (each launched once): {kernel: {counter: value}}."""
    out = tempfile.mkdtemp(prefix="piton_pmc_")
    cmd = ["rocprofv3", "--pmc", *counters, "-d", out, "-o", "p", "--output-format", "csv", "--",
           sys.executable, "-m", "piton_amd.perf_suite", "--once", *(["--small"] if small else []), *names]
    env = dict(os.environ, TMPDIR="/tmp", PYTHONPATH=os.pathsep.join(
        [os.path.dirname(os.path.dirname(os.path.abspath(__file__))), os.environ.get("PYTHONPATH", "")]))
    subprocess.run(cmd, cwd="/tmp", env=env, check=True, timeout=timeout, stdout=subprocess.DEVNULL)
    res = {}
    for f in glob.glob(os.path.join(out, "**", "*_counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if "piton::" in r["Kernel_Name"]:
                k = r["Kernel_Name"].split("(")[0].replace("void ", "").replace("piton::", "")
                res.setdefault(k, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in res.items()}


def main(argv=None):
    ap = argparse.ArgumentParser(description="the performance suite on one MI355X")
    ap.add_argument("cases", nargs="*", help=f"cases (default: all of {', '.join(CASES)})")
    ap.add_argument("--small", action="store_true", help="reduced sizes")
    ap.add_argument("--json", help="write the rows here")
    ap.add_argument("--outputs", help="save each case's checked sample here (.npz)")
    ap.add_argument("--once", action="store_true", help="launch each case once, no timing (counter passes)")
    ap.add_argument("--pmc", help="comma-separated counters: one rocprofv3 pass over the cases")
    a = ap.parse_args(argv)
    names = a.cases or list(CASES)
    unknown = [n for n in names if n not in CASES]
    if unknown:
        ap.error(f"unknown cases {unknown}")
    if a.pmc:
        res = pmc(names, a.pmc.split(","), a.small)
        print(json.dumps(res, indent=1))
        return
    rows, samples = run_cases(names, a.small, time_it=not a.once)
    if a.once:
        return
    for r in rows:
        extra = f"{r.get('tflops', '')} TFLOP/s" if "tflops" in r else f"{r['gbs']} GB/s"
        print(f"{r['name']:12s} {r['us']:10.2f} us  {extra:>16s}  {100 * r['frac']:5.1f}% of {r['bound']}  "
              f"{'ok' if r['ok'] else 'WRONG: ' + r['error']}")
    if a.json:
        with open(a.json, "w") as f:
            json.dump(rows, f, indent=1)
    if a.outputs:
        np.savez(a.outputs, **samples)
    if not all(r["ok"] for r in rows):
        sys.exit(1)


if __name__ == "__main__":
    main()
