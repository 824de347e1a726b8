"""Pins the float64 decoder oracle (oracle/tinygpt64.py): its K/V-cache decode equals a full
recompute of the prefix, and with the blocks' weights zero the logits have the closed form
LN(tok[id] + pos[t]) Wlm."""
import numpy as np

from oracle import tinygpt64
from piton_amd import tinygpt


def small_weights(seed=0, zero_blocks=False):
    cfg = tinygpt.Config(d_model=32, n_heads=2, d_mlp=64, vocab=17, context=24, n_layers=2)
    w = tinygpt.init_weights(cfg, seed)
    if zero_blocks:
        for k in w:
            if k[:2] in ("wq", "wo", "w1", "w2"):
                w[k][:] = 0
    return cfg, w


def test_kv_cache_equals_recompute():
    cfg, w = small_weights()
    prompts = np.random.default_rng(3).integers(0, cfg.vocab, (3, 5))
    toks, _ = tinygpt64.generate(w, prompts, 10, n_layers=2, n_heads=2)
    # recompute: decode one step at a time from a growing prompt, no cache reuse
    cur = prompts.copy()
    for _ in range(10):
        nxt, _ = tinygpt64.generate(w, cur, 1, n_layers=2, n_heads=2)
        cur = nxt
    np.testing.assert_array_equal(toks, cur)


def test_zero_blocks_closed_form():
    cfg, w = small_weights(seed=4, zero_blocks=True)
    prompts = np.random.default_rng(5).integers(0, cfg.vocab, (4, 6))
    toks, _ = tinygpt64.generate(w, prompts, 1, n_layers=2, n_heads=2)
    x = w["tok"][prompts[:, -1]].astype(np.float64) + w["pos"][5]
    d = x - x.mean(1, keepdims=True)
    logits = d / np.sqrt((d * d).mean(1, keepdims=True) + 1e-5) @ w["lm"].astype(np.float64)
    np.testing.assert_array_equal(toks[:, -1], np.argmax(logits, 1))


def test_first_divergence_report():
    a = np.array([[1, 2, 3, 4], [1, 2, 3, 4]])
    b = np.array([[1, 2, 3, 5], [1, 2, 3, 4]])
    m = np.array([[0.5, 0.25], [0.5, 0.5]])
    assert tinygpt64.first_divergence(a, b, m, 2) == [(0, 3, 0.25)]
