"""Launch phases of the HBM-bound softmax, the one-generation attention kernel, the decode
attention of the KV-cached decoder, its fused decode step, the split GEMM of the small and
ragged matmul shapes and the digits MLP (diagnostics).

`python -m piton_amd.phase_trace` builds a traced copy of the library beside the product one
(-DPITON_PHASE_TRACE: every traced wave keeps s_memrealtime stamps -- a 100 MHz clock shared by
the whole chip -- and stores one record into its own slot at its end; the product build
compiles none of it), replays launches back to back from a HIP graph as bench.py does (each
launch writes its own record area, handed to it by the host) and prints, per workload, the
median over the launches of: when the last wave started, when the first wave had its first row
(softmax) or its Q tile (attention), each wave's own wait for it, when the last wave finished,
and the gap to the next launch's first wave. For softmax the bytes over the window from first
data to last wave end give the streaming rate while the kernel runs, apart from its start and
its drain.
"""
from __future__ import annotations

import argparse
import ctypes
import os
import statistics

from . import build as _build

TRACE_LIB = os.path.join(_build.LIB_DIR, "libpiton_mi355x_trace.so")
TRACE_OBJ = os.path.join(_build.HERE, "_build_trace")
TICK_US = 0.01  # s_memrealtime: 100 MHz
K_PHASE_WAVES = 1 << 16  # records per launch area (kPhaseWaves in csrc/common.h)


class Record(ctypes.Structure):
    _fields_ = [("t", ctypes.c_uint64 * 4), ("kernel", ctypes.c_uint32), ("block", ctypes.c_uint32)]


def build_traced(verbose: bool = False) -> str:
    return _build.build(verbose=verbose, extra_flags=["-DPITON_PHASE_TRACE"], obj_dir=TRACE_OBJ, lib=TRACE_LIB)


def _trace(tu: str, fn, launches: int):
    """Stamps of `launches` back-to-back launches replayed from a HIP graph, one list per launch
    (the i-th launch after the attach writes area i)."""
    import numpy as np
    import torch

    from .runtime import mi355x as rt
    L = rt.lib()
    attach = getattr(L, f"piton_phase_attach_{tu}")
    attach.argtypes, attach.restype = [ctypes.c_void_p, ctypes.c_uint], ctypes.c_int
    rec = ctypes.sizeof(Record)
    log = torch.zeros(launches * K_PHASE_WAVES * rec, dtype=torch.uint8, device="cuda")
    assert attach(None, 0) == 0
    fn(0)
    torch.cuda.synchronize()
    graph_off = torch.cuda.CUDAGraph()  # records off: brings the clocks up
    with torch.cuda.graph(graph_off):
        for i in range(launches):
            fn(i)
    assert attach(ctypes.c_void_p(log.data_ptr()), launches) == 0
    graph = torch.cuda.CUDAGraph()  # the same launches, each with its own record area
    with torch.cuda.graph(graph):
        for i in range(launches):
            fn(i)
    assert attach(None, 0) == 0
    for _ in range(20):
        graph_off.replay()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    t = np.frombuffer(log.cpu().numpy().tobytes(), dtype=np.uint64).reshape(launches, K_PHASE_WAVES, rec // 8)
    # (t0, t1, t2, t3, kernel | wave << 32) per traced wave
    return [[tuple(int(x) for x in r[:5]) for r in t[k][t[k][:, 0] > 0]] for k in range(launches)]


def _summary(launches, stamps: int, nbytes: int | None = None):
    """Medians over the launches (the first and the last left out) of the phases, in us from the
    launch's first wave start."""
    rows = []
    last = stamps - 1
    for k in range(1, len(launches) - 1):
        ls, nxt = launches[k], launches[k + 1]
        t0 = min(r[0] for r in ls)
        d = dict(waves=len(ls), last_wave_start=max(r[0] for r in ls) - t0,
                 first_data=min(r[1] for r in ls) - t0,
                 wave_wait=statistics.median(r[1] - r[0] for r in ls),
                 end=max(r[last] for r in ls) - t0,
                 gap_to_next=min(r[0] for r in nxt) - max(r[last] for r in ls))
        if stamps == 4:
            d["loop"] = statistics.median(r[2] - r[1] for r in ls)
            d["merge"] = statistics.median(r[3] - r[2] for r in ls)
        rows.append(d)
    med = {k: statistics.median(r[k] for r in rows) * (1 if k == "waves" else TICK_US) for k in rows[0]}
    if nbytes:
        med["stream_tbs"] = nbytes / ((med["end"] - med["first_data"]) * 1e-6) / 1e12
    return med


def softmax_phases(n: int, rows: int = 4096, launches: int = 12):
    import torch

    from . import next_power_of_2
    from .runtime import mi355x as rt
    pair_bytes = 2 * 4 * rows * n
    pairs = max(2, -(-2 ** 30 // (pair_bytes // 2)))  # inputs over >= 1 GiB: every launch reads HBM
    g = torch.Generator(device="cuda").manual_seed(n)
    xs = [torch.randn((rows, n), device="cuda", generator=g) * 4 for _ in range(pairs)]
    ys = [torch.empty_like(x) for x in xs]
    block = next_power_of_2(n)
    per = _trace("softmax", lambda i: rt.softmax(ys[i % pairs], xs[i % pairs], n, n, n, rows, block), launches)
    return _summary([[r[:3] for r in ls] for ls in per], 3, pair_bytes)


def attention_phases(heads: int = 32, n: int = 1024, d: int = 64, launches: int = 12):
    import torch

    from .runtime import mi355x as rt
    g = torch.Generator(device="cuda").manual_seed(4)
    q, k, v = (torch.randn((heads, n, d), device="cuda", generator=g) for _ in range(3))
    o = torch.empty_like(q)
    per = _trace("attention", lambda i: rt.attn_fwd(q, k, v, o, d ** -0.5, n * d, d, n * d, d, 1, n * d, d, n * d, d,
                                                    n, heads, d, True), launches)
    return _summary(per, 4)


def decode_phases(n_keys: int, batch: int = 64, heads: int = 4, d_head: int = 64, launches: int = 12):
    """TinyGPT's decode attention: one query per (sequence, head) against n_keys cached keys,
    in the decoder's cache layout (row t*batch + b of [context * batch, 3 * d_model])."""
    import torch

    from .runtime import mi355x as rt
    D = heads * d_head
    g = torch.Generator(device="cuda").manual_seed(n_keys)
    cache = torch.randn((n_keys * batch, 3 * D), device="cuda", generator=g)
    att = torch.empty((batch, D), device="cuda")
    q = cache[(n_keys - 1) * batch:]
    per = _trace("attention", lambda i: rt.attn_decode(q, cache[:, D:], cache[:, 2 * D:], att, d_head ** -0.5,
                                                       3 * D, d_head, 3 * D, d_head, batch * 3 * D, 3 * D, d_head,
                                                       batch * 3 * D, D, d_head, n_keys, batch, heads, d_head),
                 launches)
    return _summary(per, 4)


def decode_layer_phases(n_keys: int, batch: int = 64, heads: int = 4, d_head: int = 64, launches: int = 12):
    """TinyGPT's fused decode step of a layer (piton_mi355x_decode_layer): per launch, medians
    over waves of the layernorm phase (to the barrier after it), of the projection on waves 0-5
    and of the cache copies on waves 6 and 7 (both from that barrier), and of the attention after
    the two meet."""
    import torch

    from .runtime import mi355x as rt
    D = heads * d_head
    g = torch.Generator(device="cuda").manual_seed(n_keys)
    cache = torch.randn((n_keys * batch, 3 * D), device="cuda", generator=g)
    x = torch.randn((batch, D), device="cuda", generator=g)
    w = torch.randn((D, 3 * D), device="cuda", generator=g) * 0.05
    att = torch.empty((batch, D), device="cuda")
    per = _trace("decode_layer", lambda i: rt.decode_layer(x, D, 1e-5, w, None, cache, 3 * D, att, D, d_head ** -0.5,
                                                          n_keys, batch, heads, d_head, D), launches)
    rows = []
    for k in range(1, len(per) - 1):
        ls = per[k]
        t0 = min(r[0] for r in ls)
        # the record's wave index is blockIdx.x * 8 + wave: waves 0-5 project, 6 and 7 copy the cache
        proj = [r for r in ls if (r[4] >> 32) % 8 < 6]
        copy = [r for r in ls if (r[4] >> 32) % 8 >= 6]
        rows.append(dict(layernorm=statistics.median(r[1] - r[0] for r in ls),
                         projection=statistics.median(r[2] - r[1] for r in proj),
                         cache_copies=statistics.median(r[2] - r[1] for r in copy),
                         attention=statistics.median(r[3] - r[2] for r in ls),
                         end=max(r[3] for r in ls) - t0,
                         gap_to_next=min(r[0] for r in per[k + 1]) - max(r[3] for r in ls)))
    return {key: statistics.median(r[key] for r in rows) * TICK_US for key in rows[0]}


def mlp_phases(batch: int, launches: int = 12):
    """The digits MLP in one launch (piton_mi355x_mlp3, 16 rows per workgroup): per launch,
    medians over waves of the wait for every operand (x, the three layers' weights and biases),
    of layers 1 and 2 to the barrier after layer 2, and of wave 0's layer 3, logits and argmax."""
    import numpy as np
    import torch

    from . import digits
    from .runtime import mi355x as rt
    layers = digits.he_normal_mlp(seed=1729)
    mlp = digits.MLP(layers, max_batch=batch)
    x = torch.from_numpy(np.random.default_rng(0).integers(0, 17, (batch, 64)).astype(np.float32)).cuda()
    per = _trace("mlp", lambda i: mlp.run(x), launches)
    rows = []
    for k in range(1, len(per) - 1):
        ls = per[k]
        t0 = min(r[0] for r in ls)
        w0 = [r for r in ls if (r[4] >> 32) % 4 == 0]
        rows.append(dict(waves=len(ls), last_wave_start=max(r[0] for r in ls) - t0,
                         operands=statistics.median(r[1] - r[0] for r in ls),
                         layers12=statistics.median(r[2] - r[1] for r in ls),
                         layer3=statistics.median(r[3] - r[2] for r in w0),
                         end=max(r[3] for r in ls) - t0,
                         gap_to_next=min(r[0] for r in per[k + 1]) - max(r[3] for r in ls)))
    return {key: statistics.median(r[key] for r in rows) * (1 if key == "waves" else TICK_US) for key in rows[0]}


def gemm_split_phases(M: int, N: int, K: int, lda: int, ldb: int, ldc: int, launches: int = 12):
    """The split GEMM (the small and ragged matmul shapes) on U[-1, 1] inputs: per launch, the
    last wave's start, medians over waves of the wait for the first K tile's operands, of the K
    loop and of the partial-tile sum and stores, and when the last wave ends."""
    import torch

    from .runtime import mi355x as rt
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    a = torch.rand((M, lda), device="cuda", generator=g) * 2 - 1
    b = torch.rand((K, ldb), device="cuda", generator=g) * 2 - 1
    c = torch.empty((M, ldc), device="cuda")
    per = _trace("matmul", lambda i: rt.matmul(a, b, c, M, N, K, lda, 1, ldb, 1, ldc, 1, 8), launches)
    rows = []
    for k in range(1, len(per) - 1):
        ls = per[k]
        t0 = min(r[0] for r in ls)
        rows.append(dict(waves=len(ls), last_wave_start=max(r[0] for r in ls) - t0,
                         first_tile=statistics.median(r[1] - r[0] for r in ls),
                         loop=statistics.median(r[2] - r[1] for r in ls),
                         loop_max=max(r[2] - r[1] for r in ls),
                         epilogue=statistics.median(r[3] - r[2] for r in ls),
                         end=max(r[3] for r in ls) - t0,
                         gap_to_next=min(r[0] for r in per[k + 1]) - max(r[3] for r in ls)))
    return {key: statistics.median(r[key] for r in rows) * (1 if key == "waves" else TICK_US) for key in rows[0]}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--no-build", action="store_true", help="use the traced library already built")
    a = ap.parse_args()
    if not a.no_build:
        build_traced()
    os.environ["PITON_MI355X_LIB"] = TRACE_LIB  # before the runtime loads a library

    def us(v):
        return f"{v:.2f} us"

    print("| workload | waves | last wave starts | first data | a wave's own wait | last wave ends | "
          "gap to next launch | streaming between first data and end |")
    print("|---|---|---|---|---|---|---|---|")
    for n in (1024, 4096, 1823):
        m = softmax_phases(n)
        print(f"| softmax 4096 x {n} | {int(m['waves'])} | {us(m['last_wave_start'])} | {us(m['first_data'])} | "
              f"{us(m['wave_wait'])} | {us(m['end'])} | {us(m['gap_to_next'])} | {m['stream_tbs']:.2f} TB/s |")
    m = attention_phases()
    print(f"| attention 32 x 1024 x 64 causal | {int(m['waves'])} | {us(m['last_wave_start'])} | "
          f"{us(m['first_data'])} (Q staged) | {us(m['wave_wait'])} | {us(m['end'])} | {us(m['gap_to_next'])} | "
          f"per wave: loop {us(m['loop'])}, merge {us(m['merge'])} |")
    for nk in (96, 160):
        m = decode_phases(nk)
        print(f"| decode attention 64 x 4 heads x 64, {nk} keys | {int(m['waves'])} | {us(m['last_wave_start'])} | "
              f"{us(m['first_data'])} (K, V in) | {us(m['wave_wait'])} | {us(m['end'])} | {us(m['gap_to_next'])} | "
              f"per wave: scores and max {us(m['loop'])}, exp, sum, P V {us(m['merge'])} |")
    print()
    print("| fused decode step, 64 x 4 heads x 64 | layernorm | projection (waves 0-5) | cache copies (waves 6, 7) | "
          "attention | last wave ends | gap to next launch |")
    print("|---|---|---|---|---|---|---|")
    for nk in (96, 160):
        m = decode_layer_phases(nk)
        print(f"| {nk} keys | {us(m['layernorm'])} | {us(m['projection'])} | {us(m['cache_copies'])} | "
              f"{us(m['attention'])} | {us(m['end'])} | {us(m['gap_to_next'])} |")
    print()
    print("| split GEMM | waves | last wave starts | first K tile in | K loop (median / max) | partial-tile sum "
          "and stores | last wave ends | gap to next launch |")
    print("|---|---|---|---|---|---|---|---|")
    for shape in ((512, 512, 512, 512, 512, 512), (1024, 1024, 1024, 1024, 1024, 1024),
                  (1000, 1800, 700, 703, 1805, 1807)):
        m = gemm_split_phases(*shape)
        print(f"| {shape[0]} x {shape[1]} x {shape[2]} | {int(m['waves'])} | {us(m['last_wave_start'])} | "
              f"{us(m['first_tile'])} | {us(m['loop'])} / {us(m['loop_max'])} | {us(m['epilogue'])} | "
              f"{us(m['end'])} | {us(m['gap_to_next'])} |")
    print()
    print("| digits MLP, one launch | waves | last wave starts | every operand in | layers 1 and 2 | "
          "layer 3 and argmax (wave 0) | last wave ends | gap to next launch |")
    print("|---|---|---|---|---|---|---|---|")
    for b in (1, 256, 1797):
        m = mlp_phases(b)
        print(f"| batch {b} | {int(m['waves'])} | {us(m['last_wave_start'])} | {us(m['operands'])} | "
              f"{us(m['layers12'])} | {us(m['layer3'])} | {us(m['end'])} | {us(m['gap_to_next'])} |")


if __name__ == "__main__":
    main()
