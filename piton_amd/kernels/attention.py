"""Single-head flash attention (examples/attention.py:33-113) and its host helpers (:142-222).

    grid = (cdiv(N_CTX, BLOCK_M), n_heads)
    attn_fwd_kernel[grid](q, k, v, out, 1 / sqrt(d), strides..., N_CTX, HEAD_DIM=d, BLOCK_M=...,
                          BLOCK_N=..., CAUSAL=..., EVEN_N=..., device="mi355x")
"""
from __future__ import annotations

import numpy as np

from .. import jit
from .. import language as tl
from ..jit import cdiv


@jit
def attn_fwd_kernel(Q, K, V, Out, sm_scale,
                    stride_qh, stride_qm, stride_kh, stride_kn, stride_kk,
                    stride_vh, stride_vn, stride_oh, stride_om,
                    N_CTX,
                    HEAD_DIM: tl.constexpr, BLOCK_M: tl.constexpr, BLOCK_N: tl.constexpr,
                    CAUSAL: tl.constexpr, EVEN_N: tl.constexpr):
    """Out = softmax(Q K^T sm_scale) V per head (grid axis 1), causal or not. Q, V, Out rows are
    contiguous with row strides stride_qm / stride_vn / stride_om; K is read through
    (stride_kn, stride_kk) so it may be stored [N, D] or pre-transposed [D, N]. BLOCK_M fixes
    the grid; BLOCK_N and EVEN_N are tiling hints of the reference (EVEN_N is checked). Runs as
    piton_mi355x_attn_fwd."""


def contiguous_strides(head_dim: int, k_layout: str = "nd", n_ctx: int | None = None) -> dict:
    """Row strides of contiguous [N_CTX, HEAD_DIM] Q, V and Out with K stored [N_CTX, HEAD_DIM]
    ("nd") or pre-transposed [HEAD_DIM, N_CTX] ("dn") (examples/attention.py:142-154)."""
    strides = dict(stride_qm=head_dim, stride_vn=head_dim, stride_om=head_dim)
    if k_layout == "nd":
        strides.update(stride_kn=head_dim, stride_kk=1)
    elif k_layout == "dn":
        if n_ctx is None:
            raise ValueError("a transposed K needs n_ctx (its row stride)")
        strides.update(stride_kn=1, stride_kk=n_ctx)
    else:
        raise ValueError(f"k_layout {k_layout!r}: expected 'nd' or 'dn'")
    return strides


def attention_flops(n_ctx, head_dim, causal=False, heads=1) -> float:
    """FLOPs of the two products as Triton tutorial 06 counts them, 4 N^2 D per head, half when
    causal (examples/attention.py:194-197)."""
    return 4.0 * n_ctx * n_ctx * head_dim * heads * (0.5 if causal else 1.0)


def run_attention(q, k, v, causal=False, block_m=64, block_n=32, compiled=None, k_layout="nd", sm_scale=None):
    """attn_fwd_kernel on [N, D] or [H, N, D] float32 q, k, v (numpy or GPU tensors); k_layout
    "dn" passes K pre-transposed ([H, D, N]). Returns (out, record, stats) as
    examples/attention.py:200-222 returns (out, compiled kernel, emulator stats): `out` has the
    type of q, `record` is the launch's LaunchRecord (the kernel's name, grid, entry, signature
    and constants) and `stats` its `last_stats` (the device kernels run with their grids,
    registers and spills, and the launch's FLOPs and bytes). `compiled` is accepted for the
    reference's signature and unused: the device library is built ahead of time, so there is
    no per-shape compile to reuse."""
    del compiled
    import torch
    is_np = isinstance(q, np.ndarray)
    tq, tk, tv = (torch.as_tensor(np.ascontiguousarray(t, np.float32)) if is_np else t for t in (q, k, v))
    if is_np:
        tq, tk, tv = tq.cuda(), tk.cuda(), tv.cuda()
    squeeze = tq.dim() == 2
    if squeeze:
        tq, tk, tv = tq[None], tk[None], tv[None]
    heads, n_ctx, head_dim = tq.shape
    tq, tv = tq.contiguous(), tv.contiguous()
    if k_layout == "dn":
        tk = tk.transpose(1, 2).contiguous()
    else:
        tk = tk.contiguous()
    out = torch.full_like(tq, float("nan"))
    st = contiguous_strides(head_dim, k_layout, n_ctx)
    scale = float(1.0 / np.sqrt(head_dim)) if sm_scale is None else float(sm_scale)
    grid = (cdiv(n_ctx, block_m), heads)
    record = attn_fwd_kernel[grid](tq, tk, tv, out, scale,
                                   n_ctx * head_dim, st["stride_qm"], n_ctx * head_dim, st["stride_kn"],
                                   st["stride_kk"], n_ctx * head_dim, st["stride_vn"], n_ctx * head_dim,
                                   st["stride_om"], n_ctx,
                                   HEAD_DIM=head_dim, BLOCK_M=block_m, BLOCK_N=block_n, CAUSAL=bool(causal),
                                   EVEN_N=n_ctx % block_n == 0, device="mi355x")
    if squeeze:
        out = out[0]
    if is_np:
        torch.cuda.current_stream().synchronize()
        out = out.cpu().numpy()
    return out, record, record.last_stats
