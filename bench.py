"""Benchmark: fp32 grouped matmul at 4096^3 on one MI355X (TFLOP/s and % of the fp32 MFMA peak),
plus the row softmax (HBM GB/s, cold cache) and causal attention at their benchmark shapes.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]

Prints ONE JSON line. A "step" is one matmul_kernel launch over A, B (4096 x 4096, U[-1, 1],
already resident in HBM). `value` is 2*M*N*K*steps / the timed region's wall time. The
`roofline` object is the matmul kernel's: algorithmic FLOPs per launch / its average launch
time (HIP events on the launch stream at the two ends of the timed region, / steps) against
the 157.3 TFLOP/s dense fp32 MFMA peak. The
`cpu_baseline` object is the oracle (the C restatement of the reference's round-toward-zero
emulator arithmetic) timed on a bounded sample of rows of the same product on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA = 157.3e12  # MI355X dense fp32 matrix, FLOP/s
PEAK_HBM = 8.0e12          # MI355X HBM3E, B/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--no-extras", action="store_true", help="matmul only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run each benchmark kernel twice plus the calibration add of known size (for "
                         "rocprofv3 --pmc passes), print nothing")
    return ap.parse_args()


CAL_ELEMS = 64 * 2 ** 20  # calibration add: reads 2 x 256 MiB, writes 256 MiB
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_bench_kernels.json")


def measured_traffic(workload):
    """HBM bytes per launch of a benchmark workload from the committed counter summary (two
    rocprofv3 --pmc passes, FETCH_SIZE then WRITE_SIZE, over `bench.py --pmc-probe`, scaled
    by the calibration add), or None when the summary does not cover it."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)["kernels"][workload]
    except (OSError, KeyError, ValueError):
        return None
    return int(round(t["traffic_bytes"]))


def pmc_probe(n):
    """Launches for the counter passes: the calibration add (known bytes), then two of each
    benchmark kernel at its benchmark shape (softmax on cold buffers)."""
    import torch

    from piton_amd import next_power_of_2
    from piton_amd.runtime import mi355x as rt
    x = torch.ones(CAL_ELEMS, device="cuda")
    y = torch.ones(CAL_ELEMS, device="cuda")
    z = torch.empty(CAL_ELEMS, device="cuda")
    rt.add(x, y, z, CAL_ELEMS)
    torch.cuda.synchronize()
    del x, y, z
    a = torch.rand((n, n), device="cuda")
    b = torch.rand((n, n), device="cuda")
    c = torch.empty((n, n), device="cuda")
    for _ in range(2):
        rt.matmul(a, b, c, n, n, n, n, 1, n, 1, n, 1, 8)
    torch.cuda.synchronize()
    del a, b, c
    for nc in (1024, 4096, 1823):
        xs = [torch.randn((4096, nc), device="cuda") for _ in range(6)]
        ys = [torch.empty_like(t) for t in xs]
        for i in range(2):
            rt.softmax(ys[i * 3], xs[i * 3], nc, nc, nc, 4096, next_power_of_2(nc))
        torch.cuda.synchronize()
        del xs, ys
    q, k, v = (torch.randn((32, 1024, 64), device="cuda") for _ in range(3))
    o = torch.empty_like(q)
    for _ in range(2):
        rt.attn_fwd(q, k, v, o, 0.125, 65536, 64, 65536, 64, 1, 65536, 64, 65536, 64, 1024, 32, 64, True)
    torch.cuda.synchronize()


def timed_graph(fn, iters, reps=5):
    from piton_amd.timing import timed_graph as tg
    return tg(fn, iters, reps)


def bench_matmul(n, steps, warmup):
    import torch

    from piton_amd import cdiv
    from piton_amd.kernels import matmul_kernel
    g = torch.Generator(device="cuda").manual_seed(0)
    a = torch.rand((n, n), device="cuda", generator=g) * 2 - 1
    b = torch.rand((n, n), device="cuda", generator=g) * 2 - 1
    c = torch.empty((n, n), device="cuda")
    grid = (cdiv(n, 128) * cdiv(n, 128),)
    launch = matmul_kernel[grid]

    def step(_i=0):
        launch(a, b, c, n, n, n, n, 1, n, 1, n, 1, BLOCK_SIZE_M=128, BLOCK_SIZE_N=128, BLOCK_SIZE_K=32,
               GROUP_SIZE_M=8, device="mi355x")

    stream = torch.cuda.current_stream()
    # clock ramp before the warm-up steps: the engine clock climbs over the first few tens of
    # milliseconds of sustained work after the idle set-up (otherwise the first timed launches
    # run up to 10 % slow); untimed, like the warm-up
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.2:
        for _ in range(8):
            step()
        torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # timed region: K steps bracketed by synchronize on both sides; HIP events on the launch
    # stream at its two ends give the average launch duration (no events between launches,
    # which would put a marker packet between every two kernels)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    flops = 2.0 * n * n * n
    return dict(wall=wall, kernel_s=e0.elapsed_time(e1) * 1e-3 / steps, flops=flops, a=a, b=b, c=c)


def bench_softmax(n, rows=4096, launches=48):
    """Cold-cache GB/s: buffer pairs rotated so the inputs span >= 1 GiB, four times the
    256 MB last-level cache, and each launch reads from HBM; the launches replay from a HIP
    graph, back to back."""
    import torch

    from piton_amd import next_power_of_2
    from piton_amd.runtime import mi355x as rt
    pair_bytes = 2 * 4 * rows * n
    pairs = max(2, -(-2 ** 30 // (pair_bytes // 2)))
    g = torch.Generator(device="cuda").manual_seed(n)
    xs = [torch.randn((rows, n), device="cuda", generator=g) * 4 for _ in range(pairs)]
    ys = [torch.empty_like(x) for x in xs]
    block = next_power_of_2(n)

    def step(i):
        rt.softmax(ys[i % pairs], xs[i % pairs], n, n, n, rows, block)

    avg = timed_graph(step, max(launches, pairs))
    # the copy ceiling of the same traffic: this library's copy (16-byte nontemporal loads and
    # stores, one vector per thread) over the same rotated buffers
    copy = timed_graph(lambda i: rt.copy(xs[i % pairs], ys[i % pairs], rows * n), max(launches, pairs))
    del xs, ys
    torch.cuda.empty_cache()
    return dict(n=n, rows=rows, bytes=pair_bytes, us=round(avg * 1e6, 3), gbs=round(pair_bytes / avg / 1e9, 1),
                frac=round(pair_bytes / avg / PEAK_HBM, 4), copy_gbs=round(pair_bytes / copy / 1e9, 1),
                traffic=measured_traffic(f"softmax {rows} x {n}"))


def bench_attention(launches=32):
    import torch

    from piton_amd.kernels.attention import attention_flops
    from piton_amd.runtime import mi355x as rt
    H, N, D = 32, 1024, 64
    g = torch.Generator(device="cuda").manual_seed(4)
    q, k, v = (torch.randn((H, N, D), device="cuda", generator=g) for _ in range(3))
    out = torch.empty_like(q)
    scale = 1.0 / D ** 0.5

    def step(_i):
        rt.attn_fwd(q, k, v, out, scale, N * D, D, N * D, D, 1, N * D, D, N * D, D, N, H, D, True)

    avg = timed_graph(step, launches)
    flops = attention_flops(N, D, causal=True, heads=H)
    nbytes = 4 * 4 * H * N * D
    return dict(shape=[H, N, D], causal=True, us=round(avg * 1e6, 3), tflops=round(flops / avg / 1e12, 3),
                frac_mfma=round(flops / avg / PEAK_FP32_MFMA, 4), gbs=round(nbytes / avg / 1e9, 1),
                traffic=measured_traffic(f"attention {H} x {N} x {D} causal"))


def bench_mlp(reps=3):
    """Digits MLP 64 -> 128 -> 64 -> 10 over a batch of 1797: three dense launches and the
    fused argmax, replayed from a HIP graph."""
    import numpy as np
    import torch

    from piton_amd import digits
    layers = digits.he_normal_mlp(seed=1729)
    mlp = digits.MLP(layers, max_batch=1797)
    x = torch.from_numpy(np.random.default_rng(0).integers(0, 17, (1797, 64)).astype(np.float32)).cuda()
    avg = timed_graph(lambda i: mlp.run(x), 16, reps)
    return dict(batch=1797, us=round(avg * 1e6, 3), images_per_s=round(1797 / avg, 1))


def bench_tinygpt():
    """TinyGPT greedy decoding: 64 prompts x 32 tokens, 128 new tokens each, K/V cache; the
    whole timed generate() call: prompt copy-in, the decode (prefill and 127 steps) replayed
    from the HIP graph the warm-up call captured, token copy-out."""
    import torch

    from piton_amd import tinygpt
    w = tinygpt.init_weights(seed=0)
    prompts = tinygpt.seeded_prompts()
    model = tinygpt.TinyGPT(w, batch=64)
    model.generate(prompts, 128)  # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    model.generate(prompts, 128)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return dict(sequences=64, prompt=32, new_tokens=128, s=round(dt, 4), tokens_per_s=round(64 * 128 / dt, 1),
                graph=True)


def _oracle_rate(an, bn, threads, budget_s):
    """Rows per second of the oracle's matmul on row blocks of A (cycling), about budget_s."""
    import oracle
    M = an.shape[0]
    rows, spent, total_rows, r0 = threads, 0.0, 0, 0
    while spent < budget_s:
        rows = min(rows, M - r0)
        t0 = time.perf_counter()
        oracle.matmul_fast(an[r0:r0 + rows], bn, threads=threads)
        dt = time.perf_counter() - t0
        spent += dt
        total_rows += rows
        r0 = (r0 + rows) % M
        if dt < budget_s / 8:
            rows *= 2
    return total_rows, spent


def cpu_baseline(a, b, budget_s=10.0, c_gpu=None):
    """The oracle's matmul (round-toward-zero restatement, vectorised) over row blocks of the
    same product, cycling through A's rows, with all host threads up to 16 for about budget_s
    (the reported value), then with one thread and numpy's float64 matmul for a tenth of that
    each. With c_gpu (the first rows of the GPU's C), the relative Frobenius error of the GPU
    and of the oracle against float64 on those rows."""
    import numpy as np

    import oracle
    from oracle import fp64
    an, bn = a.cpu().numpy(), b.cpu().numpy()
    threads = max(1, min(16, os.cpu_count() or 1))
    M, n, K = an.shape[0], bn.shape[1], bn.shape[0]
    total_rows, spent = _oracle_rate(an, bn, threads, budget_s)
    flops_row = 2.0 * n * K
    out = dict(value=total_rows * flops_row / spent / 1e12, unit="TFLOP/s", cores=threads, kind="port",
               sample=f"{total_rows} rows of C = A B at {M}x{n}x{K}, cycling over A's rows ({spent:.1f} s)")
    rows1, spent1 = _oracle_rate(an, bn, 1, budget_s / 10)
    out["value_1_thread"] = rows1 * flops_row / spent1 / 1e12
    rows64, spent64, r0 = 0, 0.0, 0
    while spent64 < budget_s / 10:
        t0 = time.perf_counter()
        np.matmul(an[r0:r0 + 64].astype(np.float64), bn.astype(np.float64))
        spent64 += time.perf_counter() - t0
        rows64 += 64
        r0 = (r0 + 64) % max(1, M - 63)
    out["numpy_fp64"] = dict(value=rows64 * flops_row / spent64 / 1e12, unit="TFLOP/s",
                             threads=os.environ.get("OMP_NUM_THREADS", "numpy default"))
    if c_gpu is not None:
        rows = c_gpu.shape[0]
        ref = fp64.matmul(an[:rows], bn)
        out["err_vs_fp64"] = dict(rows=rows, gpu=fp64.rel_fro(np.asarray(c_gpu), ref),
                                  oracle=fp64.rel_fro(np.asarray(oracle.matmul_fast(an[:rows], bn, threads=threads)), ref))
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    from piton_amd.runtime import mi355x as rt
    info = rt.device_info()
    n = args.size
    if args.pmc_probe:
        pmc_probe(n)
        return
    mm = bench_matmul(n, args.steps, args.warmup)
    avg = mm["kernel_s"]
    achieved = mm["flops"] / avg
    value = mm["flops"] * args.steps / mm["wall"] / 1e12
    line = {
        "metric": "fp32 matmul TFLOPS (% MFMA peak) at 4096^3; softmax/attn HBM GB/s",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mm["wall"] / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: A, B ~ U[-1, 1] fp32 from a fixed seed, resident in HBM",
        "config": {"workload": f"grouped matmul C = A B, fp32, M = N = K = {n}, GROUP_SIZE_M = 8",
                   "M": n, "N": n, "K": n, "group_size_m": 8, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 3),
                     "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA, 4), "traffic": measured_traffic(f"matmul {n}^3"),
                     "kernel_us": round(avg * 1e6, 2)},
        "device": {k: info[k] for k in ("arch", "cu_count", "max_clock_khz", "hbm_bytes")},
    }
    a_host, b_host = (mm["a"].cpu(), mm["b"].cpu()) if not args.no_cpu else (None, None)
    c_rows = mm["c"][:64].cpu().numpy() if not args.no_cpu else None
    del mm
    torch.cuda.empty_cache()
    if not args.no_extras:
        line["softmax"] = [bench_softmax(nc) for nc in (1024, 4096, 1823)]
        line["attention"] = bench_attention()
        line["mlp"] = bench_mlp()
        line["tinygpt"] = bench_tinygpt()
    if not args.no_cpu:  # last: the GPU idles while the host cores work
        line["cpu_baseline"] = cpu_baseline(a_host, b_host, c_gpu=c_rows)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
