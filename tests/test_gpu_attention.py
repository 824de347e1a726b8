"""Flash attention (examples/attention.py:33-113) on the MI355X against the oracle and the
reference tests' known answers (tests/test_attention.py:42-166).

Bar: relative Frobenius error <= 1e-5 vs float64 (attention.py:180-191) and no larger than
the oracle's; the known answers hold (N = 1, hard attention, V = I, causal prefix invariance,
[N, D] vs pre-transposed K bit-identical)."""
import numpy as np
import pytest
import torch

import oracle
from oracle import fp64
from piton_amd import cdiv
from piton_amd.kernels import attn_fwd_kernel
from piton_amd.kernels.attention import attention_flops, contiguous_strides, run_attention

pytestmark = pytest.mark.gpu
TOL = 1e-5


def qkv(n, d, seed=0, gain=1.0, heads=None):
    rng = np.random.default_rng(seed)
    shape = (n, d) if heads is None else (heads, n, d)
    q, k, v = (rng.standard_normal(shape).astype(np.float32) for _ in range(3))
    return (q * np.float32(gain)).astype(np.float32), k, v


@pytest.mark.parametrize("n,d,causal", [(64, 16, False), (64, 16, True), (64, 32, False), (64, 32, True),
                                        (32, 64, True), (100, 64, False), (100, 64, True), (37, 32, True),
                                        (17, 16, False), (200, 128, True), (1, 64, True)])
def test_matches_float64(n, d, causal):
    q, k, v = qkv(n, d, seed=n + d)
    out = run_attention(q, k, v, causal)[0]
    ref = fp64.attention_reference(q, k, v, causal)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, ref, rtol=0, atol=2e-5)  # tests/test_attention.py:53
    assert fp64.rel_fro(out, ref) <= TOL
    emu = oracle.attention(q, k, v, causal, block_n=16)
    assert fp64.rel_fro(out, ref) <= max(fp64.rel_fro(emu, ref), 2e-7)


def test_config_shape_causal_1024():
    """BH = 32, N = 1024, d = 64, causal: float64 on every head, the oracle on one head."""
    q, k, v = qkv(1024, 64, seed=4, heads=32)
    tq, tk, tv = (torch.from_numpy(t).cuda() for t in (q, k, v))
    out, record, stats = run_attention(tq, tk, tv, causal=True)
    out = out.cpu().numpy()
    # (out, record, stats), as examples/attention.py:200-222 returns (out, compiled, stats)
    assert record.name == "attn_fwd_kernel" and record.grid == (16, 32) and record.last_stats is stats
    assert record.constants["CAUSAL"] is True and record.constants["HEAD_DIM"] == 64
    assert stats["flops"] == attention_flops(1024, 64, True, 32)
    assert stats["launches"] and all(x["scratch_bytes"] == 0 for x in stats["launches"])
    ref = fp64.attention_reference(q, k, v, True)
    err = fp64.rel_fro(out, ref)
    assert err <= TOL, err
    emu = oracle.attention(q[:1], k[:1], v[:1], True, block_n=32)
    assert fp64.rel_fro(out[:1], ref[:1]) <= fp64.rel_fro(emu, ref[:1])


@pytest.mark.parametrize("heads,n,d", [(40, 1056, 64), (72, 1000, 32), (24, 2080, 64)])
def test_many_causal_groups_take_the_single_group_grid(heads, n, d):
    """Causal launches with more query-group pairs than two per CU run one group per
    workgroup (three waves per SIMD) instead of pairs; ragged N leaves a partial last block.
    Same tolerance as the config shape, and the pairing must not change any bits: a prefix of
    the heads (few enough to be paired) gives the same output for those heads."""
    q, k, v = qkv(n, d, seed=heads + n, heads=heads)
    tq, tk, tv = (torch.from_numpy(t).cuda() for t in (q, k, v))
    out = run_attention(tq, tk, tv, causal=True)[0].cpu().numpy()
    ref = fp64.attention_reference(q, k, v, True)
    assert fp64.rel_fro(out, ref) <= TOL
    np.testing.assert_allclose(out, ref, rtol=0, atol=2e-5)
    few = run_attention(tq[:2].contiguous(), tk[:2].contiguous(), tv[:2].contiguous(), causal=True)[0]
    few = few.cpu().numpy()
    np.testing.assert_array_equal(few, out[:2])


def test_single_key_returns_v():
    q, k, v = qkv(1, 64, seed=9)
    out = run_attention(q, k, v, causal=False)[0]
    np.testing.assert_allclose(out, v, rtol=2 ** -22, atol=0)


def test_hard_attention_retrieves_values():
    """tests/test_attention.py:108-121: each query matches one key by 1000 / sqrt(d); every
    other weight underflows to 0 and the match gets exp2(0) = 1, so the output is the matched
    value row up to the final normalisation."""
    n = d = 32
    rng = np.random.default_rng(3)
    perm = rng.permutation(n)
    k = np.eye(n, dtype=np.float32)
    q = (1000.0 * np.eye(n, dtype=np.float32)[perm]).astype(np.float32)
    v = rng.standard_normal((n, d)).astype(np.float32)
    out = run_attention(q, k, v, causal=False)[0]
    np.testing.assert_array_max_ulp(out, v[perm], maxulp=2)


def test_causal_rows_ignore_future_keys():
    """tests/test_attention.py:124-137: new keys and values after position 31 leave rows 0-31
    bit-identical."""
    n, d = 48, 16
    q, k, v = qkv(n, d, seed=8)
    a = run_attention(q, k, v, causal=True)[0]
    k2, v2 = k.copy(), v.copy()
    rng = np.random.default_rng(9)
    k2[32:] = rng.standard_normal((n - 32, d)) * 10
    v2[32:] = rng.standard_normal((n - 32, d)) * 10
    b = run_attention(q, k2, v2, causal=True)[0]
    np.testing.assert_array_equal(a[:32].view(np.uint32), b[:32].view(np.uint32))
    np.testing.assert_array_max_ulp(a[0], v[0], maxulp=2)
    assert not np.array_equal(a[32:], b[32:])


def test_identity_values_give_the_attention_matrix():
    n = d = 64
    q, k, _ = qkv(n, d, seed=6)
    eye = np.eye(n, dtype=np.float32)
    p = run_attention(q, k, eye, causal=True)[0]
    assert (p[np.triu_indices(n, 1)] == 0).all()
    np.testing.assert_allclose(p.sum(axis=1), 1.0, atol=1e-6)


def test_causal_prefix_is_bit_identical():
    q, k, v = qkv(256, 64, seed=7)
    full = run_attention(q, k, v, causal=True)[0]
    for m in (1, 31, 33, 100, 129):
        part = run_attention(q[:m], k[:m], v[:m], causal=True)[0]
        np.testing.assert_array_equal(part, full[:m])


def test_k_layouts_bit_identical():
    q, k, v = qkv(96, 64, seed=8, heads=3)
    nd = run_attention(q, k, v, causal=True, k_layout="nd")[0]
    dn = run_attention(q, k, v, causal=True, k_layout="dn")[0]
    np.testing.assert_array_equal(nd, dn)


def test_multihead_runtime_strides_padded_rows():
    """Heads through stride_*h and a padded query row stride (tests/test_attention.py:83-97)."""
    H, n, d = 3, 50, 32
    q, k, v = qkv(n, d, seed=10, heads=H)
    Q = np.zeros((H, n, d + 3), np.float32); Q[:, :, :d] = q
    O = np.full((H, n + 2, d + 5), -3.0, np.float32)
    tQ, tK, tV, tO = (torch.from_numpy(t).cuda() for t in (Q, k, v, O))
    st = contiguous_strides(d, "nd")
    attn_fwd_kernel[(cdiv(n, 16), H)](tQ, tK, tV, tO, float(1 / np.sqrt(d)), n * (d + 3), d + 3, n * d,
                                      st["stride_kn"], st["stride_kk"], n * d, d, (n + 2) * (d + 5), d + 5, n,
                                      HEAD_DIM=d, BLOCK_M=16, BLOCK_N=16, CAUSAL=True, EVEN_N=False,
                                      device="mi355x")
    torch.cuda.synchronize()
    got = tO.cpu().numpy()
    ref = fp64.attention_reference(q, k, v, True)
    assert fp64.rel_fro(got[:, :n, :d], ref) <= TOL
    assert (got[:, n:, :] == -3.0).all() and (got[:, :, d:] == -3.0).all()


def test_large_scores_stay_finite():
    """tests/test_attention.py:149-155: scores of +-100 stay finite (atol 2e-5)."""
    q, k, v = qkv(48, 16, seed=4, gain=25.0)
    out = run_attention(q, k, v, causal=False)[0]
    assert np.isfinite(out).all()
    ref = fp64.attention_reference(q, k, v, False)
    np.testing.assert_allclose(out, ref, rtol=0, atol=2e-5)
    assert fp64.rel_fro(out, ref) <= TOL
