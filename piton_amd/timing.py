"""Timing of launch sequences on one GPU."""
from __future__ import annotations

import time


def timed_graph(fn, iters, reps=5):
    """Average duration (s) of fn(i), i = 0..iters-1, launched back to back from a captured HIP
    graph (no host work between launches), timed with HIP events around each replay; the
    median over `reps` replays."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(0)  # warm: library loaded, kernels resident
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(iters):
            fn(i)
    # warm: replay for at least 50 ms so clocks have ramped after any idle host phase
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.05:
        graph.replay()
        torch.cuda.synchronize()
    out = []
    stream = torch.cuda.current_stream()
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        out.append(a.elapsed_time(b) * 1e-3 / iters)
    return sorted(out)[len(out) // 2]
