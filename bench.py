"""Benchmark: fp32 grouped matmul at 4096^3 on one MI355X (TFLOP/s and % of the fp32 MFMA peak),
plus every other benchmark workload of the kernel set at its benchmark shape: the matmul at
512^3, 1024^3 and ragged 1000 x 1800 x 700 with padded strides, the row softmax (HBM GB/s, cold
cache), causal attention, the digits MLP and TinyGPT greedy decoding; and, timed in the same run
on this host's cores, the reference's CPU path for each of them.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]

Prints ONE JSON line. A "step" is one matmul_kernel launch over A, B (4096 x 4096, U[-1, 1],
already resident in HBM). `value` is 2*M*N*K*steps / the timed region's wall time. The
`roofline` object is the matmul kernel's: algorithmic FLOPs per launch / its average launch
time (HIP events on the launch stream at the two ends of the timed region, / steps) against
the 157.3 TFLOP/s dense fp32 MFMA peak; its `traffic` is HBM bytes per launch from the
committed counter passes (`traffic_source` names them).

The CPU path of the reference is its emulator's arithmetic and its numpy float64 host
references. Here they are the oracle (the C restatement of the emulator's round-toward-zero
arithmetic, `kind: "port"`), timed at one thread and at `threads` threads on a bounded sample of
each workload, and numpy float64; every entry carries its thread count and its error against
float64 beside the GPU's on the same sample. `cpu_baseline` is the matmul's; `cpu` holds the
other workloads'; `host` names the host.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import functools
import json
import os
import subprocess
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
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU legs")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run each benchmark kernel twice plus the calibration add of known size (for "
                         "rocprofv3 --pmc passes), print nothing")
    return ap.parse_args()


CAL_ELEMS = 64 * 2 ** 20  # calibration add: reads 2 x 256 MiB, writes 256 MiB
# the matmul config's other shapes: (M, N, K, lda, ldb, ldc, B column-major); the ragged one with
# rows of A, B and C not 16-byte aligned
MATMUL_SHAPES = [(512, 512, 512, 512, 512, 512, False), (1024, 1024, 1024, 1024, 1024, 1024, False),
                 (1000, 1800, 700, 703, 1805, 1807, False), (1024, 1024, 1024, 1024, 1024, 1024, True),
                 (4096, 4096, 4096, 4096, 4096, 4096, True)]
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_bench_kernels.json")


def _traffic_doc():
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def measured_traffic(workload):
    """HBM bytes per launch of a benchmark workload from the committed counter summary (two
    rocprofv3 --pmc passes, FETCH_SIZE then WRITE_SIZE, over `bench.py --pmc-probe`, scaled
    by the calibration add), or None when the summary does not cover it."""
    t = _traffic_doc().get("kernels", {}).get(workload)
    return None if t is None else int(round(t["traffic_bytes"]))


def traffic_source():
    doc = _traffic_doc()
    commit = doc.get("commit", "unrecorded")
    return (f"profiles/{os.path.basename(TRAFFIC_FILE)}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes over "
            f"bench.py --pmc-probe at commit {commit}, not measured in this run")


def cpu_threads() -> int:
    """Host threads for the CPU legs: the cores this process may run on, at most 16."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    return max(1, min(16, n))


@functools.lru_cache(maxsize=1)
def host_info():
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name")), None)
    except (OSError, subprocess.SubprocessError):
        pass
    if not model:
        try:
            with open("/proc/cpuinfo") as f:
                model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), None)
        except OSError:
            pass
    blas = None
    try:
        from threadpoolctl import threadpool_info
        blas = max((p.get("num_threads", 0) for p in threadpool_info() if p.get("user_api") == "blas"), default=None)
    except Exception:  # noqa: BLE001  (optional information)
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        affinity = None
    return dict(cpu_count=os.cpu_count(), affinity=affinity, model=model, threads_used=cpu_threads(),
                numpy_blas_threads=blas)


def _blas_threads():
    return host_info()["numpy_blas_threads"]


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
    del q, k, v, o
    # the matmul config's other shapes (the split GEMM), as bench_matmul_shape lays them out
    for (M, N, K, lda, ldb, ldc, bt) in MATMUL_SHAPES[:4]:
        A = torch.rand((M, lda), device="cuda") * 2 - 1
        B = torch.rand((N, ldb) if bt else (K, ldb), device="cuda") * 2 - 1
        C = torch.empty((M, ldc), device="cuda")
        s_bk, s_bn = (1, ldb) if bt else (ldb, 1)
        for _ in range(2):
            rt.matmul(A, B, C, M, N, K, lda, 1, s_bk, s_bn, ldc, 1, 8)
        torch.cuda.synchronize()
    # the digits MLP over 1797 images
    from piton_amd import digits
    mlp = digits.MLP(digits.he_normal_mlp(seed=1729), max_batch=1797)
    x = torch.randint(0, 17, (1797, 64), device="cuda").float()
    for _ in range(2):
        mlp.run(x)
    torch.cuda.synchronize()


def timed_graph(fn, iters, reps=5):
    from piton_amd.timing import timed_graph as tg
    return tg(fn, iters, reps)


# -- GPU legs ------------------------------------------------------------------------------------

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
        return launch(a, b, c, n, n, n, n, 1, n, 1, n, 1, BLOCK_SIZE_M=128, BLOCK_SIZE_N=128, BLOCK_SIZE_K=32,
                      GROUP_SIZE_M=8, device="mi355x")

    stream = torch.cuda.current_stream()
    # clock ramp before the warm-up steps: the engine clock climbs over the first few tens of
    # milliseconds of sustained work after the idle set-up (otherwise the first timed launches
    # run up to 10 % slow); untimed, like the warm-up
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.2:
        for _ in range(8):
            rec = step()
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
    return dict(wall=wall, kernel_s=e0.elapsed_time(e1) * 1e-3 / steps, flops=flops, a=a, b=b, c=c,
                kernel=" + ".join(f"{l['kernel']} x {l['grid'][0]}" for l in rec.last_stats["launches"]))


def bench_matmul_shape(M, N, K, lda, ldb, ldc, launches=32, b_transposed=False):
    """Config 2's other shapes (HIP-graph replays, back to back): TFLOP/s and MFMA fraction.
    b_transposed: B stored column-major (stride_bk = 1, stride_bn = ldb)."""
    import torch

    from piton_amd.runtime import mi355x as rt
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    A = torch.rand((M, lda), device="cuda", generator=g) * 2 - 1
    B = torch.rand((N, ldb) if b_transposed else (K, ldb), device="cuda", generator=g) * 2 - 1
    C = torch.empty((M, ldc), device="cuda")
    s_bk, s_bn = (1, ldb) if b_transposed else (ldb, 1)

    def step(_i):
        rt.matmul(A, B, C, M, N, K, lda, 1, s_bk, s_bn, ldc, 1, 8)

    step(0)
    kernel = " + ".join(f"{l['kernel']} x {l['grid'][0]}" for l in rt.last_launches())
    avg = timed_graph(step, launches)
    flops = 2.0 * M * N * K
    line = dict(M=M, N=N, K=K, lda=lda, ldb=ldb, ldc=ldc, b_transposed=b_transposed, kernel=kernel,
                us=round(avg * 1e6, 3), tflops=round(flops / avg / 1e12, 3),
                frac_mfma=round(flops / avg / PEAK_FP32_MFMA, 4))
    # HBM bytes per launch from the committed counter passes, where they cover the shape
    label = {(512, 512, 512, 512, False): "matmul 512^3", (1024, 1024, 1024, 1024, False): "matmul 1024^3",
             (1000, 1800, 700, 703, False): "matmul 1000 x 1800 x 700 (row strides 703 / 1805 / 1807)",
             (1024, 1024, 1024, 1024, True): "matmul 1024^3, B column-major"}.get((M, N, K, lda, b_transposed))
    if label:
        line["traffic"] = measured_traffic(label)
    return line


def bench_softmax(n, rows=4096, launches=48, sample_rows=256):
    """Cold-cache GB/s: buffer pairs rotated so the inputs span >= 1 GiB, four times the
    256 MB last-level cache, and each launch reads from HBM; the launches replay from a HIP
    graph, back to back. Returns the line and (input, GPU output) of a strided sample of rows."""
    import torch

    from piton_amd import next_power_of_2
    from piton_amd.runtime import mi355x as rt
    pair_bytes = 2 * 4 * rows * n
    pairs = max(2, -(-2 ** 30 // (pair_bytes // 2)))
    g = torch.Generator(device="cuda").manual_seed(n)
    xs = [torch.randn((rows, n), device="cuda", generator=g) * 4 for _ in range(pairs)]
    ys = [torch.empty_like(x) for x in xs]
    block = next_power_of_2(n)
    # the special rows of the config: a +inf entry, a -inf entry, one all -inf row
    xs[0][1, 5] = float("inf")
    xs[0][2, 7] = float("-inf")
    xs[0][3] = float("-inf")

    def step(i):
        rt.softmax(ys[i % pairs], xs[i % pairs], n, n, n, rows, block)

    step(0)
    kernel = rt.last_launches()[0]["kernel"]
    avg = timed_graph(step, max(launches, pairs))
    # the copy ceiling of the same traffic: this library's copy (16-byte nontemporal loads and
    # stores, one vector per thread) over the same rotated buffers
    copy = timed_graph(lambda i: rt.copy(xs[i % pairs], ys[i % pairs], rows * n), max(launches, pairs))
    # the two halves of the traffic apart: a read-only pass over the inputs (this library's row
    # sum over the same bytes seen as n rows of 4096 aligned floats: reads every float, writes
    # one per row) and a write-only pass over the outputs (torch's fill), plus an empty graph
    # node (a one-float copy) for the per-launch cost
    sums = torch.empty(max(rows, n), device="cuda")
    read = timed_graph(lambda i: rt.row_sum(xs[i % pairs].view(n, rows), sums, n, rows, rows), max(launches, pairs))
    write = timed_graph(lambda i: ys[i % pairs].fill_(0.5), max(launches, pairs))
    one = torch.zeros(1, device="cuda")
    node = timed_graph(lambda i: rt.copy(one, sums, 1), launches)
    step(0)
    torch.cuda.synchronize()
    # the special rows and a strided sample of the others
    idx = torch.cat([torch.arange(1, 4), torch.arange(0, rows, rows // sample_rows)]).cuda()
    sample = (xs[0][idx].cpu().numpy(), ys[0][idx].cpu().numpy())
    del xs, ys, sums, one
    torch.cuda.empty_cache()
    half = pair_bytes // 2
    line = dict(n=n, rows=rows, kernel=kernel, bytes=pair_bytes, us=round(avg * 1e6, 3),
                gbs=round(pair_bytes / avg / 1e9, 1), frac=round(pair_bytes / avg / PEAK_HBM, 4),
                copy_gbs=round(pair_bytes / copy / 1e9, 1), traffic=measured_traffic(f"softmax {rows} x {n}"),
                bound=dict(read_us=round(read * 1e6, 3), read_gbs=round(half / read / 1e9, 1),
                           write_us=round(write * 1e6, 3), write_gbs=round(half / write / 1e9, 1),
                           two_pass_us=round((read + write) * 1e6, 3), node_us=round(node * 1e6, 3),
                           frac_of_two_pass=round((read + write) / avg, 4)))
    return line, sample


def bench_mfma_sustained(cus, iters=2000):
    """The device's sustained fp32 MFMA rate in this run (piton_mi355x_mfma_probe: two waves
    per SIMD, two independent 32x32x2 chains each), and the engine clock it implies (one
    4096-flop MFMA per 64 clocks per SIMD). The published peak assumes 2.4 GHz; each MFMA
    fraction is also given against the rate measured here, so a fraction below 1 is the
    kernel's and not the clock's."""
    import torch

    from piton_amd.runtime import mi355x as rt
    wgs = 2 * cus
    out = torch.empty(wgs * 256, device="cuda")
    avg = timed_graph(lambda i: rt.mfma_probe(out, wgs, iters), 4)
    flops = wgs * 4 * iters * 32 * 4096
    rate = flops / avg
    return dict(tflops=round(rate / 1e12, 2), clock_ghz=round(rate / (cus * 4 * 64) / 1e9, 3),
                frac_of_published=round(rate / PEAK_FP32_MFMA, 4), launch_ms=round(avg * 1e3, 3),
                probe="piton_mi355x_mfma_probe, %d workgroups x 4 waves x %d x 32 MFMAs" % (wgs, iters))


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

    step(0)
    kernel = rt.last_launches()[0]["kernel"]
    avg = timed_graph(step, launches)
    flops = attention_flops(N, D, causal=True, heads=H)
    nbytes = 4 * 4 * H * N * D
    line = dict(shape=[H, N, D], causal=True, kernel=kernel, us=round(avg * 1e6, 3),
                tflops=round(flops / avg / 1e12, 3), frac_mfma=round(flops / avg / PEAK_FP32_MFMA, 4),
                gbs=round(nbytes / avg / 1e9, 1), traffic=measured_traffic(f"attention {H} x {N} x {D} causal"))
    torch.cuda.synchronize()
    return line, tuple(t.cpu().numpy() for t in (q, k, v, out))


MLP_BATCHES = (1, 16, 64, 256, 1797)


def bench_mlp(reps=3):
    """Digits MLP 64 -> 128 -> 64 -> 10 over batches of 1, 16, 64, 256 and 1797 unnormalised
    [0, 16] images (the batches of the reference's latency table), one fused launch (three dense
    layers and the argmax): `us` per batch from launches replayed back to back from a HIP graph,
    and `us_call`, the median wall time of one host call (launch and synchronisation)."""
    import numpy as np
    import torch

    from piton_amd import digits
    layers = digits.he_normal_mlp(seed=1729)
    mlp = digits.MLP(layers, max_batch=1797)
    xh = np.random.default_rng(0).integers(0, 17, (1797, 64)).astype(np.float32)
    x = torch.from_numpy(xh).cuda()
    batches = []
    for m in MLP_BATCHES:
        xm = x[:m]
        avg = timed_graph(lambda i: mlp.run(xm), 16, reps)
        calls = []
        for _ in range(50):
            t0 = time.perf_counter()
            mlp.run(xm)
            torch.cuda.synchronize()
            calls.append(time.perf_counter() - t0)
        batches.append(dict(batch=m, us=round(avg * 1e6, 3), images_per_s=round(m / avg, 1),
                            us_call=round(sorted(calls)[len(calls) // 2] * 1e6, 1)))
    logits, pred = mlp.run(x)
    torch.cuda.synchronize()
    full = batches[-1]
    line = dict(batch=1797, us=full["us"], images_per_s=full["images_per_s"], kernel=mlp_kernel_name(),
                batches=batches)
    return line, (layers, xh, logits.cpu().numpy(), pred.cpu().numpy())


def mlp_kernel_name():
    from piton_amd.runtime import mi355x as rt
    return rt.last_launches()[0]["kernel"]


def bench_tinygpt():
    """TinyGPT greedy decoding: 64 prompts x 32 tokens, 128 new tokens each, K/V cache; the
    whole timed generate() call: prompt copy-in, the decode (prefill and 127 steps) replayed
    from the HIP graph the warm-up call captured, token copy-out."""
    import torch

    from piton_amd import tinygpt
    w = tinygpt.init_weights(seed=0)
    prompts = tinygpt.seeded_prompts()
    model = tinygpt.TinyGPT(w, batch=64)
    model.generate(prompts, 128)  # warm-up (captures the graph)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tokens = model.generate(prompts, 128)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    line = dict(sequences=64, prompt=32, new_tokens=128, s=round(dt, 4), tokens_per_s=round(64 * 128 / dt, 1),
                graph=True)
    return line, (w, prompts, tokens)


# -- CPU legs: the reference's path (the oracle and numpy float64) on this host ---------------------

def _timed_units(run, units, budget_s, threads):
    """Runs run(u) for u in units cyclically until about budget_s has passed, `threads` at a time
    (ctypes releases the GIL, so oracle calls run in parallel); returns (units done, seconds)."""
    done, spent, i = 0, 0.0, 0
    with cf.ThreadPoolExecutor(threads) as ex:
        while spent < budget_s:
            batch = [units[(i + j) % len(units)] for j in range(threads)]
            t0 = time.perf_counter()
            list(ex.map(run, batch))
            spent += time.perf_counter() - t0
            done += len(batch)
            i += threads
    return done, spent


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
    same product, cycling through A's rows, with `cpu_threads()` threads for about budget_s
    (the reported value), then with one thread and numpy's float64 matmul for a tenth of that
    each. With c_gpu (the first rows of the GPU's C), the relative Frobenius error of the GPU
    and of the oracle against float64 on those rows."""
    import numpy as np

    import oracle
    from oracle import fp64
    an, bn = a.cpu().numpy(), b.cpu().numpy()
    threads = cpu_threads()
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
                             threads=_blas_threads())
    if c_gpu is not None:
        rows = c_gpu.shape[0]
        ref = fp64.matmul(an[:rows], bn)
        out["err_vs_fp64"] = dict(rows=rows, gpu=fp64.rel_fro(np.asarray(c_gpu), ref),
                                  oracle=fp64.rel_fro(np.asarray(oracle.matmul_fast(an[:rows], bn, threads=threads)), ref))
    return out


def _finite_rows(x):
    import numpy as np
    return np.isfinite(x).all(axis=1)


def cpu_softmax(n, sample, budget_s=1.0):
    """The oracle's softmax (the emulator's exp, reductions and division order) and numpy float64
    on a strided sample of the benchmark's rows: GB/s at the kernel's 8 bytes per element."""
    import numpy as np

    import oracle
    from oracle import fp64
    x, y_gpu = sample
    block = 1 << (n - 1).bit_length()
    ok = _finite_rows(x)
    ref = fp64.softmax(x[ok])
    chunks = [x[i:i + 8] for i in range(0, x.shape[0] - 7, 8)]
    out = dict(n=n, sample_rows=int(x.shape[0]), unit="GB/s", kind="port")
    for label, th in (("oracle_1_thread", 1), ("oracle", cpu_threads())):
        done, spent = _timed_units(lambda c: oracle.softmax(c, n, block), chunks, budget_s, th)
        out[label] = dict(value=round(8.0 * 8 * n * done / spent / 1e9, 4), threads=th)
    t0 = time.perf_counter()
    fp64.softmax(x)
    out["numpy_fp64"] = dict(value=round(8.0 * x.size / (time.perf_counter() - t0) / 1e9, 4),
                             threads=_blas_threads())
    orc = oracle.softmax(x, n, block)
    out["err_vs_fp64"] = dict(rows=int(ok.sum()), gpu=fp64.rel_fro(y_gpu[ok], ref), oracle=fp64.rel_fro(orc[ok], ref))
    # the special rows keep the emulator's NaN pattern: a +inf entry or an all -inf row gives a
    # NaN row, a -inf entry an exact zero
    out["special_rows_match_oracle"] = bool(np.array_equal(np.isnan(y_gpu[~ok]), np.isnan(orc[~ok])))
    return out


def cpu_attention(sample, budget_s=1.5):
    """The oracle's attention (the emulator's block order and math) and numpy float64 per head:
    TFLOP/s at the tutorial's count (4 N^2 d / 2 per causal head). One thread works through
    query rows of head 0 from the last (the longest rows) for about budget_s; `threads` threads
    each take a whole head."""
    import numpy as np

    import oracle
    from oracle import fp64
    q, k, v, o_gpu = sample
    H, N, D = q.shape
    scale = 1.0 / np.sqrt(D)
    out = dict(shape=[H, N, D], causal=True, unit="TFLOP/s", kind="port")
    rows, spent, r1 = [], 0.0, N
    got = np.full((N, D), np.nan, np.float32)
    while spent < budget_s and r1 > 0:
        r0 = max(0, r1 - 32)
        t0 = time.perf_counter()
        got[r0:r1] = oracle.attention(q[0], k[0], v[0], True, scale, block_n=32, rows=(r0, r1))[r0:r1]
        spent += time.perf_counter() - t0
        rows.append((r0, r1))
        r1 = r0
    flops1 = sum(4.0 * D * (i + 1) for a, b in rows for i in range(a, b))
    out["oracle_1_thread"] = dict(value=flops1 / spent / 1e12, threads=1, sample=f"query rows {r1}-{N} of head 0")
    th = min(cpu_threads(), H)
    heads = [(1 + i) % H for i in range(th)]
    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(th) as ex:
        list(ex.map(lambda h: oracle.attention(q[h], k[h], v[h], True, scale, block_n=32), heads))
    dt = time.perf_counter() - t0
    out["oracle"] = dict(value=th * 2.0 * N * N * D / dt / 1e12, threads=th, sample=f"{th} whole heads")
    t0 = time.perf_counter()
    ref = fp64.attention_reference(q[0], k[0], v[0], True, scale)
    out["numpy_fp64"] = dict(value=2.0 * N * N * D / (time.perf_counter() - t0) / 1e12,
                             threads=_blas_threads())
    sel = slice(r1, N)
    out["err_vs_fp64"] = dict(rows=N - r1, gpu=fp64.rel_fro(o_gpu[0][sel], ref[sel]),
                              oracle=fp64.rel_fro(got[sel], ref[sel]))
    return out


def cpu_mlp(sample, budget_s=1.0):
    """The oracle's three dense layers (RTZ, the emulator's order) and argmax over the 1797
    images, numpy float64 for the same chain; the GPU's predictions against the oracle's. Per
    batch of the reference's latency table: the oracle's time for one batch on one thread and
    numpy float64's (median of a few runs)."""
    import numpy as np

    import oracle
    from oracle import fp64
    layers, x, logits_gpu, pred_gpu = sample
    chain = [(w, b, i < 2) for i, (w, b) in enumerate(layers)]
    chunks = [x[i:i + 64] for i in range(0, x.shape[0], 64)]
    out = dict(batch=int(x.shape[0]), unit="images/s", kind="port")
    for label, th in (("oracle_1_thread", 1), ("oracle", cpu_threads())):
        done, spent = _timed_units(lambda c: oracle.mlp_forward(c, chain), chunks, budget_s, th)
        imgs = sum(chunks[i % len(chunks)].shape[0] for i in range(done))
        out[label] = dict(value=round(imgs / spent, 1), threads=th)
    t0 = time.perf_counter()
    h = x.astype(np.float64)
    for w, b, relu in chain:
        h = fp64.dense(h, w, b, relu)
    out["numpy_fp64"] = dict(value=round(x.shape[0] / (time.perf_counter() - t0), 1),
                             threads=_blas_threads())
    orc = oracle.mlp_forward(x, chain)
    pred_orc = oracle.argmax_rows(orc, 10)
    out["err_vs_fp64"] = dict(gpu=fp64.rel_fro(logits_gpu, h), oracle=fp64.rel_fro(orc, h))
    out["predictions_equal_oracle"] = int((pred_gpu == pred_orc).sum())

    def median_us(fn, reps):
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return round(sorted(ts)[len(ts) // 2] * 1e6, 1)

    def f64_chain(xb):
        hb = xb.astype(np.float64)
        for w, b, relu in chain:
            hb = fp64.dense(hb, w, b, relu)
        return np.argmax(hb[:, :10], axis=1)

    out["batches"] = [dict(batch=m, oracle_1_thread_us=median_us(lambda: oracle.mlp_forward(x[:m], chain),
                                                                  3 if m < 1797 else 1),
                           numpy_fp64_us=median_us(lambda: f64_chain(x[:m]), 5))
                      for m in MLP_BATCHES]
    return out


def cpu_tinygpt(sample):
    """The float64 decoder (the composition's host reference) over the whole config: tokens/s,
    and the GPU's token ids against it (first divergences with their float64 top-2 margins)."""
    from oracle import tinygpt64
    w, prompts, tokens_gpu = sample
    t0 = time.perf_counter()
    want, margins = tinygpt64.generate(w, prompts, 128)
    dt = time.perf_counter() - t0
    div = tinygpt64.first_divergence(tokens_gpu, want, margins, prompts.shape[1])
    return dict(unit="tokens/s", kind="port", numpy_fp64=dict(value=round(64 * 128 / dt, 1),
                                                             threads=_blas_threads()),
                sequences_equal=64 - len(div), divergences=div)


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
                     "kernel_us": round(avg * 1e6, 2), "kernel": mm["kernel"], "traffic_source": traffic_source()},
        "device": {k: info[k] for k in ("arch", "cu_count", "max_clock_khz", "hbm_bytes")},
    }
    sustained = bench_mfma_sustained(info["cu_count"])
    line["mfma_sustained"] = sustained
    line["roofline"]["frac_of_sustained"] = round(achieved / (sustained["tflops"] * 1e12), 4)
    a_host, b_host = (mm["a"].cpu(), mm["b"].cpu()) if not args.no_cpu else (None, None)
    c_rows = mm["c"][:64].cpu().numpy() if not args.no_cpu else None
    del mm
    torch.cuda.empty_cache()
    samples = {}
    if not args.no_extras:
        line["matmul_shapes"] = [bench_matmul_shape(*sh[:6], launches=8 if sh[0] == 4096 else 32, b_transposed=sh[6])
                                 for sh in MATMUL_SHAPES]
        line["softmax"] = []
        for nc in (1024, 4096, 1823):
            sm, samples[f"softmax {nc}"] = bench_softmax(nc)
            line["softmax"].append(sm)
        line["attention"], samples["attention"] = bench_attention()
        line["attention"]["frac_of_sustained"] = round(line["attention"]["tflops"] / sustained["tflops"], 4)
        line["mlp"], samples["mlp"] = bench_mlp()
        line["tinygpt"], samples["tinygpt"] = bench_tinygpt()
    if not args.no_cpu:  # last: the GPU idles while the host cores work
        line["host"] = host_info()
        line["cpu_baseline"] = cpu_baseline(a_host, b_host, c_gpu=c_rows)
        if samples:
            line["cpu"] = {
                "softmax": [cpu_softmax(nc, samples[f"softmax {nc}"]) for nc in (1024, 4096, 1823)],
                "attention": cpu_attention(samples["attention"]),
                "mlp": cpu_mlp(samples["mlp"]),
                "tinygpt": cpu_tinygpt(samples["tinygpt"]),
            }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
