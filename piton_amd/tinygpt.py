"""TinyGPT: a character-level decoder built from the kernel set, greedy decoding on the MI355X.

The reference has no decoder model; this one is composed from its kernels: the no-affine
layernorm of tests/test_reroll_reduce.py:199-208, the fused dense layer
(examples/nn_kernels.py:23-74, here with strided rows and the residual add fused into the
epilogue), causal attention (examples/attention.py:33-113), ReLU as the only activation, and
the first-index argmax of the digits driver. Architecture (pre-LN):

    x = tok[ids] + pos[t]
    repeat n_layers:  x = x + Wo . Attn(LN(x) Wqkv + bqkv) + bo
                      x = x + W2 . ReLU(LN(x) W1 + b1) + b2
    next = argmax(LN(x_last) Wlm)

Memory layout for MI355X: every activation is position-major, row t*B + b, so the rows of one
position are contiguous: the QKV projection of new tokens writes straight into the K/V cache
(the cache IS each layer's projection output, [context * B, 3 * d_model]), a decode step's rows are one
contiguous block, and attention reads heads through strides. Decoding with the cache runs one
single-query attention per (batch, head) (piton_mi355x_attn_decode); without it every step
recomputes the prefix with the batched flash kernel.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .runtime import mi355x as rt


@dataclass(frozen=True)
class Config:
    vocab: int = 256
    d_model: int = 256
    n_layers: int = 4
    n_heads: int = 4
    d_mlp: int = 1024
    context: int = 256
    eps: float = 1e-5
    init_std: float = 0.02

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads


def init_weights(cfg: Config = Config(), seed: int = 0) -> dict:
    """float32 weights N(0, init_std), biases 0, drawn from numpy's PCG64 in this order: tok,
    pos, then per layer wqkv, wo, w1, w2, then lm."""
    rng = np.random.default_rng(seed)
    D, F, V = cfg.d_model, cfg.d_mlp, cfg.vocab

    def normal(*shape):
        return rng.normal(0.0, cfg.init_std, shape).astype(np.float32)

    w = {"tok": normal(V, D), "pos": normal(cfg.context, D)}
    for i in range(cfg.n_layers):
        w[f"wqkv{i}"] = normal(D, 3 * D)
        w[f"wo{i}"] = normal(D, D)
        w[f"w1{i}"] = normal(D, F)
        w[f"w2{i}"] = normal(F, D)
        w[f"bqkv{i}"] = np.zeros(3 * D, np.float32)
        w[f"bo{i}"] = np.zeros(D, np.float32)
        w[f"b1{i}"] = np.zeros(F, np.float32)
        w[f"b2{i}"] = np.zeros(D, np.float32)
    w["lm"] = normal(D, V)
    return w


def seeded_prompts(batch: int = 64, length: int = 32, vocab: int = 256, seed: int = 1) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, vocab, (batch, length)).astype(np.int32)


class TinyGPT:
    """Device-resident weights and buffers for `batch` sequences of up to cfg.context tokens."""

    def __init__(self, weights: dict, cfg: Config = Config(), batch: int = 64, device="cuda",
                 fused_decode: bool = True):
        """fused_decode: where the shapes allow, a decode step runs each layer's layernorm, QKV
        projection and attention as one piton_mi355x_decode_layer launch (head_dim 64) instead
        of linear_ln + attn_decode, and every forward ends with one piton_mi355x_lm_head_argmax
        launch instead of linear_ln + argmax_rows."""
        self.cfg, self.B = cfg, batch
        self.fused_decode = fused_decode
        self.w = {k: torch.as_tensor(np.ascontiguousarray(v)).to(device) for k, v in weights.items()}
        D, F, V, C = cfg.d_model, cfg.d_mlp, cfg.vocab, cfg.context
        rows = C * batch
        self.x = torch.empty((rows, D), device=device)
        self.h = torch.empty((rows, D), device=device)
        self.att = torch.empty((rows, D), device=device)
        self.mlp = torch.empty((rows, F), device=device)
        # the K/V cache: one [context * B, 3 * d_model] projection output per layer, row t*B + b
        self.qkv = torch.empty((cfg.n_layers, rows, 3 * D), device=device)
        self.logits = torch.empty((batch, V), device=device)
        self.tokens = torch.zeros((C + 1) * batch, dtype=torch.int32, device=device)  # row t*B + b
        self.err = torch.zeros(1, dtype=torch.int32, device=device)
        self._graphs = {}  # (T0, steps, kv_cache) -> captured decode

    def decode_layer_fits(self, n_keys: int) -> bool:
        """Whether a decode step over n_keys cached positions fits the fused decode_layer entry:
        heads of 64, d_model a multiple of 256 up to 1024, at most 256 keys, and every cache
        offset of the launch (rows of 3 d_model floats, n_keys + 3 positions of B rows) within
        31 bits. Other shapes run the separate layernorm, projection and attention launches."""
        D, B = self.cfg.d_model, self.B
        return (self.cfg.head_dim == 64 and D % 256 == 0 and D <= 1024 and n_keys <= 256 and
                (n_keys + 3) * B * 3 * D < 0x7FFFFFFF // 4 - 3 * D)

    # -- one forward over positions [p0, p1) ---------------------------------------------------

    def _forward(self, p0: int, p1: int):
        cfg, B = self.cfg, self.B
        D, F, H, Dh, V = cfg.d_model, cfg.d_mlp, cfg.n_heads, cfg.head_dim, cfg.vocab
        if p0 > 0 and p1 != p0 + 1:
            # checked before any launch: nothing is embedded or written into the caches
            raise ValueError("decode steps take one position at a time")
        n = (p1 - p0) * B
        r0 = p0 * B
        x, h, att, mlp = (t[r0:r0 + n] for t in (self.x, self.h, self.att, self.mlp))
        # a decode step of the fused path embeds its tokens inside layer 0's decode_layer launch
        fused_step = p0 > 0 and self.fused_decode and self.decode_layer_fits(p1)
        if not fused_step:
            rt.embedding(self.tokens[r0:], 1, B, self.w["tok"], self.w["pos"][p0:], x, D, B * D, B, p1 - p0, D, V, 0,
                         self.err)
        scale = 1.0 / float(np.sqrt(Dh))
        # a decode step's products have at most 64 rows: layernorm fuses into the next linear
        # (the same values bit for bit, one launch instead of two)
        fuse_ln = n <= 64 and D % 256 == 0
        for i in range(cfg.n_layers):
            w = lambda k: self.w[f"{k}{i}"]  # noqa: E731
            cache = self.qkv[i]
            qkv = cache[r0:r0 + n]
            if fused_step:
                # a decode step: (layer 0: the embedding,) layernorm, QKV into the cache row and
                # attention in one launch
                emb = dict(ids=self.tokens[r0:r0 + B], tok=self.w["tok"], pos=self.w["pos"][p0], vocab=V,
                           err_flag=self.err) if i == 0 else {}
                rt.decode_layer(x, D, cfg.eps, w("wqkv"), w("bqkv"), cache, 3 * D, att, D, scale, p1, B, H, Dh, D, **emb)
            else:
                if fuse_ln:
                    rt.linear_ln(x, D, cfg.eps, w("wqkv"), w("bqkv"), None, 0, qkv, 3 * D, n, 3 * D, D)
                else:
                    rt.layernorm(x, h, D, cfg.eps, n, D)
                    rt.linear(h, D, w("wqkv"), w("bqkv"), None, 0, qkv, 3 * D, n, 3 * D, D)
            if p0 == 0:
                # prefix: batched causal flash attention over positions [0, p1)
                rt.attn_fwd_batched(cache, cache[:, D:], cache[:, 2 * D:], self.att, scale,
                                    3 * D, Dh, B * 3 * D, 3 * D, Dh, B * 3 * D, 1, 3 * D, Dh, B * 3 * D,
                                    D, Dh, B * D, p1, B, H, Dh, True)
            else:
                if not fused_step:
                    rt.attn_decode(qkv, cache[:, D:], cache[:, 2 * D:], att, scale, 3 * D, Dh, 3 * D, Dh,
                                   B * 3 * D, 3 * D, Dh, B * 3 * D, D, Dh, p1, B, H, Dh)
            rt.linear(att, D, w("wo"), w("bo"), x, D, x, D, n, D, D)
            if fuse_ln:
                rt.linear_ln(x, D, cfg.eps, w("w1"), w("b1"), None, 0, mlp, F, n, F, D, relu=True)
            else:
                rt.layernorm(x, h, D, cfg.eps, n, D)
                rt.linear(h, D, w("w1"), w("b1"), None, 0, mlp, F, n, F, D, relu=True)
            rt.linear(mlp, F, w("w2"), w("b2"), x, D, x, D, n, D, F)
        last = (p1 - 1) * B
        nxt = self.tokens[p1 * B:(p1 + 1) * B]
        if self.fused_decode and D % 256 == 0 and D <= 1024 and V % 4 == 0 and V <= 1024:
            # layernorm, LM head and argmax in one launch
            rt.lm_head_argmax(self.x[last:last + B], D, cfg.eps, self.w["lm"], None, self.logits, V, nxt, B, V, D, V)
            return
        if B <= 64 and D % 256 == 0:
            rt.linear_ln(self.x[last:last + B], D, cfg.eps, self.w["lm"], None, None, 0, self.logits, V, B, V, D)
        else:
            rt.layernorm(self.x[last:last + B], self.h[last:last + B], D, cfg.eps, B, D)
            rt.linear(self.h[last:last + B], D, self.w["lm"], None, None, 0, self.logits, V, B, V, D)
        rt.argmax_rows(self.logits, B, V, V, nxt)

    def _decode(self, T0: int, steps: int, kv_cache: bool):
        self._forward(0, T0)
        for t in range(T0, T0 + steps - 1):
            if kv_cache:
                self._forward(t, t + 1)
            else:
                self._forward(0, t + 1)

    def generate(self, prompts, steps: int, kv_cache: bool = True, graph: bool | None = None) -> np.ndarray:
        """Greedy continuation of int32 prompts [B, T0] by `steps` tokens; returns [B, T0 + steps].

        graph (default: on a GPU): the whole decode (prefill and every step, positions baked in)
        is captured once per (T0, steps, kv_cache) as a HIP graph and replayed on later calls,
        so a step costs no host launches. The capture call runs the decode eagerly first (its
        tokens are the ones returned) and then records it; the prompts are copied in before
        every replay."""
        prompts = np.ascontiguousarray(prompts, np.int32)
        B, T0 = prompts.shape
        if B != self.B or T0 < 1 or T0 + steps > self.cfg.context:
            raise ValueError(f"prompts {prompts.shape} and {steps} steps do not fit batch {self.B}, "
                             f"context {self.cfg.context}")
        use_graph = self.x.is_cuda if graph is None else graph
        self.tokens[:T0 * B].copy_(torch.from_numpy(prompts.T.copy().reshape(-1)))
        self.err.zero_()
        key = (T0, steps, kv_cache)
        if use_graph and key in self._graphs:
            self._graphs[key].replay()
        elif use_graph:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self._decode(T0, steps, kv_cache)
            torch.cuda.current_stream().wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._decode(T0, steps, kv_cache)
            self._graphs[key] = g
        else:
            self._decode(T0, steps, kv_cache)
        out = self.tokens[:(T0 + steps) * B].view(T0 + steps, B).t().contiguous().cpu().numpy()
        if int(self.err.item()):
            raise RuntimeError("a token id outside the vocabulary reached the embedding")
        return out

    def last_logits(self) -> np.ndarray:
        return self.logits.cpu().numpy()
