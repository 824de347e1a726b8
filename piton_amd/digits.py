"""The digits MLP chain on the MI355X: the three dense layers and the argmax of the first ten
logits (examples/digits_model.py:120-139; tests/test_digits_model.py:102-131), in one launch
(mlp3) or one dense launch per layer.

Layers are float32 row-major (w [K, N], b [N]); hidden layers use ReLU. The last layer may be
the reference's 16-wide padded layer or a plain 10-wide one; predictions use the first
`n_classes` logits. The argmax is fused into the last dense entry (first index of the max, the
rule of numpy's argmax).
"""
from __future__ import annotations

import numpy as np
import torch

from .runtime import mi355x as rt

SIZES = (64, 128, 64, 10)


def he_normal_mlp(seed: int = 1729, sizes=SIZES):
    """Random-init weights N(0, 2 / fan_in) and zero biases (examples/digits_model.py:171-174),
    float32, from numpy's PCG64 generator."""
    rng = np.random.default_rng(seed)
    layers = []
    for k, n in zip(sizes[:-1], sizes[1:]):
        w = rng.normal(0.0, np.sqrt(2.0 / k), (k, n)).astype(np.float32)
        layers.append((w, np.zeros(n, np.float32)))
    return layers


def normalize(images) -> np.ndarray:
    """Raw 0..16 pixels to float32 0..1 (examples/digits_model.py:95-102)."""
    images = np.asarray(images)
    if images.ndim not in (1, 2) or images.shape[-1] != 64:
        raise ValueError("Expected shape (64,) or (batch, 64)")
    if not np.all(np.isfinite(images)) or np.any(images < 0) or np.any(images > 16):
        raise ValueError("Raw digit pixels must be finite and in 0..16")
    return np.ascontiguousarray(images, dtype=np.float32) / np.float32(16)


class MLP:
    """Device-resident weights and activation buffers for batches of up to max_batch rows."""

    def __init__(self, layers, max_batch: int, n_classes: int = 10, device="cuda"):
        self.n_classes = n_classes
        self.w = [torch.as_tensor(np.ascontiguousarray(w, np.float32)).to(device) for w, _ in layers]
        self.b = [torch.as_tensor(np.ascontiguousarray(b, np.float32)).to(device) for _, b in layers]
        self.sizes = [self.w[0].shape[0]] + [w.shape[1] for w in self.w]
        self.max_batch = max_batch
        self.h = [torch.empty((max_batch, n), device=device) for n in self.sizes[1:]]
        self.pred = torch.empty(max_batch, dtype=torch.int32, device=device)

    def run(self, x: torch.Tensor, fused: bool = True):
        """Logits [M, N_last] and predictions [M] (int32) for float32 x [M, 64] on the GPU;
        asynchronous on the current stream. A three-layer chain whose sizes fit (even, <= 256)
        runs as one launch (`mlp3`: for the digits network in another k order than the dense
        GEMM, logits equal to the dense launches' within the chain's float32 error bound; for
        other sizes bit for bit); otherwise, or with fused=False, as one dense launch per layer
        with the argmax fused into the last."""
        M = x.shape[0]
        if M > self.max_batch:
            raise ValueError(f"batch {M} exceeds max_batch {self.max_batch}")
        if not x.is_contiguous():
            raise ValueError("x must be contiguous")
        if fused and len(self.w) == 3 and all(n <= 256 for n in self.sizes) and all(n % 2 == 0 for n in self.sizes[:3]):
            out = self.h[-1]
            rt.mlp3(x, M, self.w[0], self.b[0], self.w[1], self.b[1], self.w[2], self.b[2], out, self.pred,
                    self.n_classes)
            return out[:M], self.pred[:M]
        h = x
        last = len(self.w) - 1
        for i, (w, b) in enumerate(zip(self.w, self.b)):
            K, N = w.shape
            y = self.h[i]
            rt.dense(h, w, b, y, M, N, K, add_bias=True, relu=i < last,
                     argmax_out=self.pred if i == last else None, n_classes=self.n_classes if i == last else 0)
            h = y
        return h[:M], self.pred[:M]
