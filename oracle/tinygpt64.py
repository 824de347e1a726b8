"""TEST INFRASTRUCTURE ONLY (part of the oracle): the decoder of piton_amd/tinygpt.py restated
in float64 numpy, with greedy decoding, as the checker of the GPU token ids.

The reference has no decoder (its parity is unpinned); this model fixes the composition from
the reference's pieces: the no-affine layernorm with biased variance of
tests/test_reroll_reduce.py:199-208, dense layers Y = X W + b (examples/nn_kernels.py:23-74),
causal softmax(Q K^T / sqrt(d)) V (examples/attention.py:180-191), ReLU, and numpy's first-index
argmax (examples/digits_model.py:137-139).
"""
from __future__ import annotations

import numpy as np


def layernorm(x, eps):
    d = x - x.mean(axis=-1, keepdims=True)
    return d / np.sqrt((d * d).mean(axis=-1, keepdims=True) + eps)


def generate(weights: dict, prompts, steps: int, n_layers=4, n_heads=4, eps=1e-5, score_scale=None,
             activation=None):
    """Greedy decoding in float64 with a K/V cache. Returns (tokens [B, T0 + steps], margins
    [B, steps]: the top-1 minus top-2 logit of every step). score_scale (default 1/sqrt(d_head))
    and activation (default ReLU) exist so that tests can plant a wrong one."""
    w = {k: np.asarray(v, np.float64) for k, v in weights.items()}
    prompts = np.asarray(prompts)
    B, T0 = prompts.shape
    D = w["tok"].shape[1]
    Dh = D // n_heads
    scale = 1.0 / np.sqrt(Dh) if score_scale is None else score_scale
    act = (lambda z: np.maximum(z, 0.0)) if activation is None else activation
    total = T0 + steps
    tokens = np.zeros((B, total), np.int64)
    tokens[:, :T0] = prompts
    margins = np.zeros((B, steps))
    kcache = np.zeros((n_layers, B, n_heads, total, Dh))
    vcache = np.zeros_like(kcache)

    def forward(p0, p1):
        """Positions [p0, p1) of every sequence; returns the last position's logits."""
        x = w["tok"][tokens[:, p0:p1]] + w["pos"][p0:p1][None]          # [B, T, D]
        T = p1 - p0
        for i in range(n_layers):
            h = layernorm(x, eps)
            qkv = h @ w[f"wqkv{i}"] + w[f"bqkv{i}"]                      # [B, T, 3D]
            q, k, v = (qkv[..., j * D:(j + 1) * D].reshape(B, T, n_heads, Dh).transpose(0, 2, 1, 3)
                       for j in range(3))
            kcache[i, :, :, p0:p1] = k
            vcache[i, :, :, p0:p1] = v
            keys, vals = kcache[i, :, :, :p1], vcache[i, :, :, :p1]
            s = (q @ keys.transpose(0, 1, 3, 2)) * scale                  # [B, H, T, p1]
            qpos = np.arange(p0, p1)[:, None]
            s = np.where(np.arange(p1)[None, :] <= qpos, s, -np.inf)
            s = s - s.max(axis=-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=-1, keepdims=True)
            a = (p @ vals).transpose(0, 2, 1, 3).reshape(B, T, D)
            x = x + a @ w[f"wo{i}"] + w[f"bo{i}"]
            h = layernorm(x, eps)
            x = x + act(h @ w[f"w1{i}"] + w[f"b1{i}"]) @ w[f"w2{i}"] + w[f"b2{i}"]
        return layernorm(x[:, -1], eps) @ w["lm"]

    logits = forward(0, T0)
    for step in range(steps):
        t = T0 + step
        srt = np.sort(logits, axis=1)
        margins[:, step] = srt[:, -1] - srt[:, -2]
        tokens[:, t] = np.argmax(logits, axis=1)
        if step + 1 < steps:
            logits = forward(t, t + 1)
    return tokens, margins


def first_divergence(got, want, margins, t0):
    """[(sequence, position, fp64 top-2 margin at that step)] where two greedy decodes first
    differ; later positions of a diverged sequence are not compared."""
    out = []
    for b in range(got.shape[0]):
        diff = np.flatnonzero(got[b] != want[b])
        if diff.size:
            pos = int(diff[0])
            out.append((b, pos, float(margins[b, pos - t0]) if pos >= t0 else float("nan")))
    return out
