"""Hand-set one-layer decoder weights whose greedy next token has a closed form that depends on
the attention score scale 1/sqrt(d_head) and on the MLP's ReLU (shared by the float64-model test
and the GPU test).

Prompt [a, b], positions embed to zero, tok[a] = x0 = (+1, +1, -1, -1, ...) and
tok[b] = x1 = (+1, -1, +1, -1, ...): both have mean 0 and variance 1, so LN(x) = kappa * x with
kappa = 1 / sqrt(1 + eps), and x0 . x1 = 0. Head 0, dimension 0 only:
  * q = bias (s, 0, ...) at every position;
  * k_t[0] = LN(x_t) . x1 / D, so k_0[0] = 0 and k_1[0] = kappa;
  * v_t[0] = the same, so v_0[0] = 0 and v_1[0] = kappa;
  * the last query (position 1) sees keys 0 and 1 with scores 0 and s * kappa * scale, so its
    weight on key 1 is p1 = sigmoid(s * kappa * scale), and the head's output is p1 * kappa;
  * Wo[0, 0] = g adds g * kappa * p1 to coordinate 0 of the residual stream.
The MLP has W1 = 0 and b1 = (-1, 0.5, 0, ...): ReLU keeps (0, 0.5); W2 sends hidden 0 to coordinate
2 with weight -2 and hidden 1 with weight +1, so coordinate 2 gains 0.5 (it would gain 2.5 without
the ReLU). The LM head is the identity on the first `vocab` coordinates, and a layernorm keeps the
order of a vector's coordinates, so the next token is the largest coordinate of

    x_final = x1 + (g kappa p1) e_0 + 0.5 e_2,   where x1[0] = x1[2] = 1 and every other x1[j] <= 1.

With s chosen so that s * kappa * scale = 1 (p1 = sigmoid(1) = 0.7311):
  * case "A": g * kappa = 0.5 / 0.70: coordinate 0 is 1.5222 > 1.5, token 0. A smaller scale
    (1/sqrt(d_model), 1/d_head) gives p1 < 0.70 and token 2; dropping the ReLU makes coordinate 2
    3.5 and gives token 2.
  * case "B": g * kappa = 0.5 / 0.80: coordinate 0 is 1.4569 < 1.5, token 2. A larger scale (none,
    or 1/sqrt of a smaller head) gives p1 > 0.80 and token 0.
"""
import numpy as np

A_TOKEN, B_TOKEN = 5, 7
EXPECTED = {"A": 0, "B": 2}


def weights(case, d_model, n_heads, d_mlp, vocab, context, eps=1e-5):
    D = d_model
    assert D % 4 == 0 and vocab <= D and d_mlp >= 2
    scale = 1.0 / np.sqrt(D // n_heads)
    kappa = 1.0 / np.sqrt(1.0 + eps)
    g = {"A": 0.5 / 0.70, "B": 0.5 / 0.80}[case] / kappa
    s = 1.0 / (kappa * scale)
    idx = np.arange(D)
    x0 = np.where(idx % 4 < 2, 1.0, -1.0)
    x1 = np.where(idx % 2 == 0, 1.0, -1.0)
    w = {"tok": np.zeros((vocab, D)), "pos": np.zeros((context, D))}
    w["tok"][A_TOKEN] = x0
    w["tok"][B_TOKEN] = x1
    wqkv = np.zeros((D, 3 * D))
    wqkv[:, D] = x1 / D            # k, head 0, dimension 0
    wqkv[:, 2 * D] = x1 / D        # v, head 0, dimension 0
    bqkv = np.zeros(3 * D)
    bqkv[0] = s                    # q, head 0, dimension 0
    wo = np.zeros((D, D))
    wo[0, 0] = g
    b1 = np.zeros(d_mlp)
    b1[0], b1[1] = -1.0, 0.5
    w2 = np.zeros((d_mlp, D))
    w2[0, 2], w2[1, 2] = -2.0, 1.0
    lm = np.zeros((D, vocab))
    lm[np.arange(vocab), np.arange(vocab)] = 1.0
    w.update({"wqkv0": wqkv, "bqkv0": bqkv, "wo0": wo, "bo0": np.zeros(D), "w10": np.zeros((D, d_mlp)),
              "b10": b1, "w20": w2, "b20": np.zeros(D), "lm": lm})
    return {k: v.astype(np.float32) for k, v in w.items()}


def prompts(batch):
    return np.tile(np.array([[A_TOKEN, B_TOKEN]], np.int32), (batch, 1))
