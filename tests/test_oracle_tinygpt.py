"""Pins the float64 decoder oracle (oracle/tinygpt64.py): its K/V-cache decode equals a full
recompute of the prefix; with the blocks' weights zero the logits have the closed form
LN(tok[id] + pos[t]) Wlm; and hand-set one-layer weights give the closed-form token that fixes
the attention scale 1/sqrt(d_head) and the ReLU."""
import numpy as np
import pytest

import tinygpt_cases
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


@pytest.mark.parametrize("case", ["A", "B"])
def test_scale_and_relu_closed_form(case):
    """Hand-set one-layer weights (tests/tinygpt_cases.py) whose next token is token 0 or 2
    depending on the attention scale 1/sqrt(d_head) and the MLP's ReLU: the float64 model gives
    the closed form's token."""
    D, H, F, V, C = 8, 2, 4, 8, 4
    w = tinygpt_cases.weights(case, D, H, F, V, C)
    toks, margins = tinygpt64.generate(w, tinygpt_cases.prompts(3), 1, n_layers=1, n_heads=H)
    assert (toks[:, -1] == tinygpt_cases.EXPECTED[case]).all()
    assert (margins[:, 0] > 0.01).all()


def test_scale_and_relu_cases_discriminate():
    """The closed form of tests/tinygpt_cases.py: coordinate 0 is 1 + g kappa sigmoid(r) with r =
    s kappa scale_used = scale_used / scale, coordinate 2 is 1.5 (3.5 without the ReLU). Case A
    flips to token 2 for scale 1/sqrt(d_model) (d_head = d_model / 2 here) and without the ReLU;
    case B flips to token 0 with no scale."""
    sig = lambda r: 1.0 / (1.0 + np.exp(-r))  # noqa: E731
    coord0 = {"A": lambda r: 1 + 0.5 / 0.70 * sig(r), "B": lambda r: 1 + 0.5 / 0.80 * sig(r)}
    assert coord0["A"](1.0) > 1.5 and coord0["B"](1.0) < 1.5
    assert coord0["A"](np.sqrt(0.5)) < 1.5          # 1/sqrt(d_model) instead of 1/sqrt(d_head)
    assert coord0["A"](0.5) < 1.5                   # 1/d_head (d_head = 4)
    assert coord0["B"](2.0) > 1.5                   # no scale (scale = 1/2 here)
    assert coord0["A"](1.0) < 3.5                   # without the ReLU coordinate 2 wins


@pytest.mark.parametrize("case,plant", [("A", "scale_d_model"), ("A", "scale_d_head"), ("A", "no_relu"),
                                        ("B", "no_scale")])
def test_planted_mistakes_change_the_token(case, plant):
    """A wrong score scale or a missing ReLU planted in the float64 model changes the closed-form
    cases' token, so the closed form pins both."""
    D, H, F, V, C = 8, 2, 4, 8, 4
    w = tinygpt_cases.weights(case, D, H, F, V, C)
    kw = {"scale_d_model": dict(score_scale=1 / np.sqrt(D)), "scale_d_head": dict(score_scale=1 / (D // H)),
          "no_scale": dict(score_scale=1.0), "no_relu": dict(activation=lambda z: z)}[plant]
    toks, _ = tinygpt64.generate(w, tinygpt_cases.prompts(2), 1, n_layers=1, n_heads=H, **kw)
    assert (toks[:, -1] != tinygpt_cases.EXPECTED[case]).all()
