"""TEST INFRASTRUCTURE ONLY (part of the oracle): the float64 host references that the
reference validates its kernels against, restated with numpy, plus its deterministic input
recipes. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this.
"""
from __future__ import annotations

import numpy as np

LCG_A, LCG_C = 1664525, 1013904223


def lcg_u32(n: int, seed: int) -> np.ndarray:
    """First n outputs of the board LCG s <- s*1664525 + 1013904223 mod 2^32
    (pi/runtime/piton_rt.h:60-63; perf/suite.py:39-49), by the closed form
    s_k = a^k s_0 + c (a^0 + ... + a^(k-1)); uint64 arithmetic wraps mod 2^64, which keeps
    the low 32 bits exact."""
    with np.errstate(over="ignore"):
        powers = np.cumprod(np.full(n, LCG_A, dtype=np.uint64))
        sums = np.cumsum(np.concatenate(([np.uint64(1)], powers[:-1])).astype(np.uint64))
        s = powers * np.uint64(seed & 0xFFFFFFFF) + sums * np.uint64(LCG_C)
    return (s & np.uint64(0xFFFFFFFF)).astype(np.uint32)


def lcg_floats(n: int, seed: int) -> np.ndarray:
    """piton_lcg_float (pi/runtime/piton_rt.h:64-67; perf/suite.py:52-54): the top 24 bits of
    each LCG output scaled into [-1, 1)."""
    top = (lcg_u32(n, seed) >> np.uint32(8)).astype(np.float32)
    return top * np.float32(1.0 / 8388608.0) - np.float32(1.0)


def rel_fro(x, ref) -> float:
    """Relative Frobenius error ||x - ref||_F / ||ref||_F in float64."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm((x - ref).ravel()) / max(np.linalg.norm(ref.ravel()), 1e-300))


def matmul(a, b) -> np.ndarray:
    return np.asarray(a, np.float64) @ np.asarray(b, np.float64)


def softmax(x, n_cols=None, block=None) -> np.ndarray:
    """Row softmax over the first min(n_cols, block) columns (examples/kernels.py:60-76;
    perf/suite.py:222-231). Other columns are NaN."""
    x = np.atleast_2d(np.asarray(x, np.float64))
    n = x.shape[1] if n_cols is None else int(n_cols)
    if block is not None:
        n = min(n, int(block))
    out = np.full(x.shape, np.nan)
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp(x[:, :n] - x[:, :n].max(axis=1, keepdims=True))
        out[:, :n] = e / e.sum(axis=1, keepdims=True)
    return out


def attention_reference(q, k, v, causal=False, sm_scale=None) -> np.ndarray:
    """softmax(q k^T * sm_scale) v in float64 for [N, D] or [H, N, D] inputs, with the causal
    lower-triangle mask (examples/attention.py:180-191)."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    scale = 1.0 / np.sqrt(q.shape[-1]) if sm_scale is None else float(sm_scale)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    if causal:
        keep = np.tril(np.ones((s.shape[-2], s.shape[-1]), bool))
        s = np.where(keep, s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.matmul(p, v)


def attention_flops(n_ctx, head_dim, causal=False, heads=1) -> float:
    """The two products' FLOPs as Triton tutorial 06 counts them (examples/attention.py:194-197)."""
    return 4.0 * n_ctx * n_ctx * head_dim * heads * (0.5 if causal else 1.0)


def dense(x, w, b=None, relu=False) -> np.ndarray:
    y = np.asarray(x, np.float64) @ np.asarray(w, np.float64)
    if b is not None:
        y = y + np.asarray(b, np.float64)
    return np.maximum(y, 0.0) if relu else y


def layernorm(x, n=None, eps=1e-5) -> np.ndarray:
    """(x - mean) / sqrt(var + eps) over the first n columns, biased variance, no affine
    (tests/test_reroll_reduce.py:199-231)."""
    x = np.atleast_2d(np.asarray(x, np.float64))
    n = x.shape[1] if n is None else int(n)
    xs = x[:, :n]
    d = xs - xs.mean(axis=1, keepdims=True)
    return d / np.sqrt((d * d).mean(axis=1, keepdims=True) + eps)


def mlp_with_bounds(x, layers, unit: float = 2.0 ** -23):
    """Float64 logits and a per-logit absolute error bound for a chain of fp32 dense layers
    whose every operation has relative error <= unit (2^-23: round-toward-zero; 2^-24: round-
    to-nearest), generalising examples/digits_reference.py:14-55 to any input range: each
    length-K output takes K products, K sums and a bias add, so
    err' = (err |W|)(1 + g) + g(|a| |W| + |b|) with g = (2K+1)u / (1 - (2K+1)u); ReLU is
    1-Lipschitz and keeps the bound. layers = [(w, b, relu), ...]."""
    a = np.asarray(x, np.float32).astype(np.float64)
    err = np.zeros_like(a)
    for w, b, relu in layers:
        w64 = np.asarray(w, np.float32).astype(np.float64)
        b64 = np.asarray(b, np.float32).astype(np.float64)
        k = w64.shape[0]
        num = (2 * k + 1) * unit
        g = num / (1.0 - num)
        aw = np.abs(w64)
        err = (err @ aw) * (1.0 + g) + g * (np.abs(a) @ aw + np.abs(b64))
        a = a @ w64 + b64
        if relu:
            a = np.maximum(a, 0.0)
    return a, err


def certified_argmax(logits, bounds, n=None):
    """(argmax, certified) per row: certified when the top logit beats every other by more
    than the sum of their error bounds, so any arithmetic within the bounds picks it too."""
    lg = np.asarray(logits, np.float64)
    bd = np.asarray(bounds, np.float64)
    if n is not None:
        lg, bd = lg[:, :n], bd[:, :n]
    top = np.argmax(lg, axis=1)
    rows = np.arange(lg.shape[0])
    gap = lg[rows, top][:, None] - lg
    need = bd[rows, top][:, None] + bd
    gap[rows, top] = np.inf
    return top, (gap > need).all(axis=1)


def top2_margin(logits, n=None) -> np.ndarray:
    lg = np.asarray(logits, np.float64)
    if n is not None:
        lg = lg[:, :n]
    s = np.sort(lg, axis=1)
    return s[:, -1] - s[:, -2]
