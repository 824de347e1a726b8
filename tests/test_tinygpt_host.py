"""The decoder driver's memory layout on the host: piton_amd/tinygpt.py runs against a host
mirror of the C ABI entries it calls (each reads and writes memory through exactly the
pointers and element strides the driver passes), and must decode the same tokens as the
float64 oracle. A wrong offset or stride in the driver fails here without a GPU."""
import numpy as np
import torch

from oracle import tinygpt64
from piton_amd import tinygpt


def view(t, size, stride):
    return torch.as_strided(t, size, stride, storage_offset=t.storage_offset())


class HostABI:
    """Float64 mirror of the entries the decoder uses, addressing memory as the C ABI does."""

    @staticmethod
    def embedding(ids, ids_sb, ids_st, tok, pos, out, out_sb, out_st, batch, T, d, vocab, pos_offset, err=None):
        i = view(ids, (batch, T), (ids_sb, ids_st)).long()
        o = view(out, (batch, T, d), (out_sb, out_st, 1))
        o.copy_(tok[i] + pos[pos_offset:pos_offset + T][None])

    @staticmethod
    def layernorm(x, out, n, eps, rows, rs):
        xv = view(x, (rows, n), (rs, 1)).double()
        d = xv - xv.mean(1, keepdim=True)
        view(out, (rows, n), (rs, 1)).copy_(d / torch.sqrt((d * d).mean(1, keepdim=True) + eps))

    @staticmethod
    def linear(x, ldx, w, bias, residual, ldr, y, ldy, M, N, K, relu=False):
        r = view(x, (M, K), (ldx, 1)).double() @ w.double()
        if bias is not None:
            r = r + bias.double()
        if relu:
            r = torch.clamp(r, min=0)
        if residual is not None:
            r = r + view(residual, (M, N), (ldr, 1)).double()
        view(y, (M, N), (ldy, 1)).copy_(r)

    @staticmethod
    def attn_fwd_batched(q, k, v, out, scale, s_qb, s_qh, s_qm, s_kb, s_kh, s_kn, s_kk, s_vb, s_vh, s_vn, s_ob,
                         s_oh, s_om, n, batch, heads, dh, causal):
        Q = view(q, (batch, heads, n, dh), (s_qb, s_qh, s_qm, 1)).double()
        Kt = view(k, (batch, heads, n, dh), (s_kb, s_kh, s_kn, s_kk)).double()
        V = view(v, (batch, heads, n, dh), (s_vb, s_vh, s_vn, 1)).double()
        s = Q @ Kt.transpose(-1, -2) * scale
        if causal:
            s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool), 1), float("-inf"))
        view(out, (batch, heads, n, dh), (s_ob, s_oh, s_om, 1)).copy_(torch.softmax(s, -1) @ V)

    @staticmethod
    def attn_decode(q, k, v, out, scale, s_qb, s_qh, s_kb, s_kh, s_kn, s_vb, s_vh, s_vn, s_ob, s_oh, n_keys, batch,
                    heads, dh):
        Q = view(q, (batch, heads, 1, dh), (s_qb, s_qh, 0, 1)).double()
        Kt = view(k, (batch, heads, n_keys, dh), (s_kb, s_kh, s_kn, 1)).double()
        V = view(v, (batch, heads, n_keys, dh), (s_vb, s_vh, s_vn, 1)).double()
        p = torch.softmax(Q @ Kt.transpose(-1, -2) * scale, -1)
        view(out, (batch, heads, dh), (s_ob, s_oh, 1)).copy_((p @ V)[:, :, 0])

    @staticmethod
    def argmax_rows(x, rows, ld, n, out):
        out[:rows].copy_(torch.argmax(view(x, (rows, n), (ld, 1)), 1).int())

    # the fused entries (piton_mi355x_decode_layer, _lm_head_argmax)

    @staticmethod
    def _ln(x, eps):
        d = x - x.mean(1, keepdim=True)
        return d / torch.sqrt((d * d).mean(1, keepdim=True) + eps)

    @staticmethod
    def decode_layer(x, ldx, eps, w, bias, cache, ldc, out, ldo, scale, n_keys, batch, heads, dh, d_model, ids=None,
                     tok=None, pos=None, vocab=0, err_flag=None):
        xv = view(x, (batch, d_model), (ldx, 1))
        if ids is not None:
            xv.copy_(tok[ids.long()] + pos[None])
        y = HostABI._ln(xv.double(), eps) @ w.double()
        if bias is not None:
            y = y + bias.double()
        rows = view(cache, (n_keys, batch, 3 * d_model), (batch * ldc, ldc, 1))
        rows[n_keys - 1].copy_(y)
        q = rows[n_keys - 1, :, :d_model].double().reshape(batch, heads, 1, dh)
        k = rows[:, :, d_model:2 * d_model].double().reshape(n_keys, batch, heads, dh).permute(1, 2, 0, 3)
        v = rows[:, :, 2 * d_model:].double().reshape(n_keys, batch, heads, dh).permute(1, 2, 0, 3)
        p = torch.softmax(q @ k.transpose(-1, -2) * scale, -1)
        view(out, (batch, d_model), (ldo, 1)).copy_((p @ v)[:, :, 0].reshape(batch, d_model))

    @staticmethod
    def linear_ln(x, ldx, eps, w, bias, residual, ldr, y, ldy, M, N, K, relu=False):
        xn = HostABI._ln(view(x, (M, K), (ldx, 1)).double(), eps)
        HostABI.linear(xn.contiguous(), K, w, bias, residual, ldr, y, ldy, M, N, K, relu)

    @staticmethod
    def lm_head_argmax(x, ldx, eps, w, bias, logits, ldl, nxt, M, N, K, n_classes):
        r = HostABI._ln(view(x, (M, K), (ldx, 1)).double(), eps) @ w.double()
        if bias is not None:
            r = r + bias.double()
        if logits is not None:
            view(logits, (M, N), (ldl, 1)).copy_(r)
        nxt[:M].copy_(torch.argmax(r[:, :n_classes], 1).int())


def run_host(monkeypatch, kv_cache, steps=6, batch=3, fused_shapes=False):
    """fused_shapes: d_model 256 in heads of 64 and a vocabulary of 32, so that the decoder takes
    its fused entries (decode_layer with the embedding, lm_head_argmax); otherwise the shapes
    only the separate entries take (heads of 32, a vocabulary of 29)."""
    cfg = (tinygpt.Config(d_model=256, n_heads=4, d_mlp=96, vocab=32, context=24, n_layers=2) if fused_shapes else
           tinygpt.Config(d_model=64, n_heads=2, d_mlp=96, vocab=29, context=24, n_layers=2))
    w = tinygpt.init_weights(cfg, seed=1)
    w = {k: (v * 10 if k.startswith("w") or k == "lm" else v) for k, v in w.items()}  # wide margins
    prompts = tinygpt.seeded_prompts(batch=batch, length=5, vocab=cfg.vocab, seed=2)
    monkeypatch.setattr(tinygpt, "rt", HostABI)
    model = tinygpt.TinyGPT({k: v.astype(np.float64) for k, v in w.items()}, cfg, batch=batch, device="cpu")
    for name in ("x", "h", "att", "mlp", "qkv", "logits"):  # float64 buffers: exact layout check
        setattr(model, name, getattr(model, name).double())
    got = model.generate(prompts, steps, kv_cache=kv_cache)
    want, _ = tinygpt64.generate(w, prompts, steps, n_layers=2, n_heads=cfg.n_heads)
    return got, want


def test_driver_layout_kv_cache(monkeypatch):
    got, want = run_host(monkeypatch, True)
    np.testing.assert_array_equal(got, want)


def test_driver_layout_recompute(monkeypatch):
    got, want = run_host(monkeypatch, False)
    np.testing.assert_array_equal(got, want)


def test_driver_layout_fused_entries(monkeypatch):
    """The same check through the fused entries (their pointers, strides and the cache row a
    decode step writes), with the recompute path as the second opinion."""
    calls = []
    for name in ("decode_layer", "lm_head_argmax"):
        f = getattr(HostABI, name)
        monkeypatch.setattr(HostABI, name, staticmethod(lambda *a, _f=f, _n=name, **k: (calls.append(_n), _f(*a, **k))[1]))
    got, want = run_host(monkeypatch, True, fused_shapes=True)
    np.testing.assert_array_equal(got, want)
    assert {"decode_layer", "lm_head_argmax"} <= set(calls)


def test_fused_decode_only_where_the_entry_takes_the_shape():
    """The fused decode step is chosen only for shapes decode_layer accepts (its limits: heads of
    64, d_model a multiple of 256 up to 1024, at most 256 keys, cache offsets within 31 bits);
    the rest take the separate launches instead of an unsupported-shape error."""
    def model(d_model, n_heads, batch):
        cfg = tinygpt.Config(d_model=d_model, n_heads=n_heads, d_mlp=64, vocab=32, context=8, n_layers=1)
        m = tinygpt.TinyGPT.__new__(tinygpt.TinyGPT)
        m.cfg, m.B = cfg, batch
        return m
    assert model(256, 4, 64).decode_layer_fits(160)
    assert model(1024, 16, 64).decode_layer_fits(256)
    assert not model(256, 4, 64).decode_layer_fits(257)      # more keys than the entry stages
    assert not model(1280, 20, 64).decode_layer_fits(16)     # d_model past 1024
    assert not model(256, 8, 64).decode_layer_fits(16)       # heads of 32
    assert not model(384, 6, 64).decode_layer_fits(16)       # d_model not a multiple of 256
    # cache offsets: (n_keys + 3) positions x B rows x 3 d_model floats past 2 GiB
    assert model(1024, 16, 1024).decode_layer_fits(64)
    assert not model(1024, 16, 1024).decode_layer_fits(256)
