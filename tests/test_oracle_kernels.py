"""Pins the oracle's kernels (oracle/oracle.c) against the reference tests' known answers and
tolerances and against what the mathematics fixes: dyadic inputs are exact in any order, a
round-toward-zero chain never exceeds the exact value in magnitude for positive data, a hand
derived 16-lane reduction distinguishes the lowering's butterfly from any other order, and
the digits model reaches its recorded accuracy (1,743 of 1,797)."""
import hashlib
import os

import numpy as np
import pytest

import oracle
from oracle import fp64

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "digits")
rng = np.random.default_rng(11)


# -- matmul / dense (examples/kernels.py:18-57, examples/nn_kernels.py:23-74) -----------------

@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (72, 100, 64), (40, 70, 36), (16, 128, 32)])
def test_matmul_reference_shapes(M, N, K):
    """tests/test_kernels.py:41-50: rtol / atol 1e-4 vs numpy."""
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    np.testing.assert_allclose(oracle.matmul(a, b), a @ b, rtol=1e-4, atol=1e-4)


def test_matmul_dyadic_exact_and_strided():
    a = (rng.integers(-4, 5, (40, 36)) / 4).astype(np.float32)
    b = (rng.integers(-4, 5, (36, 70)) / 4).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul(a, b), a @ b)
    big = np.zeros((36, 80), np.float32)
    big[:, :70] = b
    np.testing.assert_array_equal(oracle.matmul(a, big[:, :70]), a @ b)          # padded ldb
    np.testing.assert_array_equal(oracle.matmul(a, np.asfortranarray(b)), a @ b)  # stride_bk = 1


def test_matmul_truncates_toward_zero():
    """Positive data: every partial sum and product is truncated, so the chain never exceeds
    the exact value, and it falls short by about K/2 ulp (a round-to-nearest chain would be
    unbiased)."""
    a = rng.uniform(0, 1, (32, 512)).astype(np.float32)
    b = rng.uniform(0, 1, (512, 48)).astype(np.float32)
    c = oracle.matmul(a, b).astype(np.float64)
    ref = fp64.matmul(a, b)
    assert (c <= ref).all()
    bias = np.mean((ref - c) / ref)
    assert 1e-6 < bias < 512 * 2.0 ** -23


def test_matmul_fast_equals_exact():
    a = rng.uniform(-1, 1, (33, 300)).astype(np.float32)
    b = rng.uniform(-1, 1, (300, 77)).astype(np.float32)
    a[0, :10] = 0.0
    b[:, 0] = -0.0
    np.testing.assert_array_equal(oracle.matmul_fast(a, b, threads=3).view(np.uint32),
                                  oracle.matmul(a, b).view(np.uint32))


@pytest.mark.parametrize("m,n,k,add_bias,relu", [(8, 64, 64, True, True), (9, 17, 11, True, False),
                                                 (3, 10, 7, False, True), (1, 16, 8, False, False)])
def test_dense_dyadic_bit_exact(m, n, k, add_bias, relu):
    """tests/test_nn_kernels.py:37-61."""
    r = np.random.default_rng(340 + m)
    x = r.integers(-4, 5, (m, k)).astype(np.float32) / np.float32(4)
    w = r.integers(-4, 5, (k, n)).astype(np.float32) / np.float32(4)
    bias = r.integers(-8, 9, n).astype(np.float32) / np.float32(4)
    want = x @ w + (bias if add_bias else 0)
    if relu:
        want = np.maximum(want, np.float32(0))
    np.testing.assert_array_equal(oracle.dense(x, w, bias if add_bias else None, relu), want)


# -- reductions (lower.py:3911-4063) ---------------------------------------------------------

def test_sum_follows_the_lane_butterfly():
    """16 lanes, x0 = 1 and x1..x15 = 2^-24. By hand through s = 8, 4, 2, 1 with truncation:
    lanes holding 1 gain 2^-23, 3 * 2^-23, then 7 * 2^-23, so the result is 1 + 7 * 2^-23.
    A sequential sum gives 1, the exact sum is 1 + 7.5 * 2^-23 and rounding to nearest
    gives 1 + 8 * 2^-23."""
    x = np.full(16, 2.0 ** -24, np.float32)
    x[0] = 1.0
    assert oracle.row_reduce(x, "sum")[0] == np.float32(1 + 7 * 2.0 ** -23)
    # with two registers the lanes fold first: lane 0 = 1 + 2^-24 -> 1 (truncated)
    y = np.zeros(32, np.float32)
    y[0], y[16] = 1.0, 2.0 ** -24
    assert oracle.row_reduce(y, "sum")[0] == np.float32(1.0)


def test_max_reduction_specials():
    x = rng.standard_normal((4, 64)).astype(np.float32)
    x[1, 5] = np.nan
    x[2, :] = -np.inf
    x[3, 7] = np.float32(np.array(0xFFC00000, np.uint32).view(np.float32))  # -NaN orders lowest
    m = oracle.row_reduce(x, "max")
    assert m[0] == x[0].max() and np.isnan(m[1]) and np.isneginf(m[2])
    assert m[3] == np.delete(x[3], 7).max()


# -- softmax (examples/kernels.py:60-76) -------------------------------------------------------

@pytest.mark.parametrize("rows,cols,block", [(4, 64, 64), (3, 100, 128), (5, 16, 16), (40, 128, 128), (2, 1000, 1024),
                                             (3, 1823, 2048)])
def test_softmax_matches_float64(rows, cols, block):
    """tests/test_kernels.py:16-22 (rtol 2e-5, atol 1e-6); tests/test_reroll_reduce.py:177-185."""
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 4
    got = oracle.softmax(x, cols, block)
    np.testing.assert_allclose(got, fp64.softmax(x), rtol=2e-5, atol=1e-6)
    # truncated sums make the divisor small, so rows sum slightly above 1: by <= ~n ulp
    sums = got.astype(np.float64).sum(1)
    assert (sums >= 1 - 1e-6).all() and (sums <= 1 + 2e-6 + cols * 2.0 ** -23).all()


def test_softmax_special_rows():
    """+inf entry, all -inf row, +NaN entry: whole row NaN as numpy; a -inf entry in a finite
    row is exactly 0; a -NaN entry becomes 0 and the rest of the row is a normal softmax
    (fmax orders -NaN lowest)."""
    x = rng.standard_normal((6, 64)).astype(np.float32)
    x[0, 3] = np.inf
    x[1, :] = -np.inf
    x[2, 9] = np.nan
    x[3, 0] = -np.inf
    x[4, 1] = np.array(0xFFC00000, np.uint32).view(np.float32)
    got = oracle.softmax(x, 64, 64)
    assert np.isnan(got[0]).all() and np.isnan(got[1]).all() and np.isnan(got[2]).all()
    assert got[3, 0] == 0.0 and np.isfinite(got[3]).all()
    assert got[4, 1] == 0.0
    np.testing.assert_allclose(np.delete(got[4], 1), fp64.softmax(np.delete(x[4], 1)[None])[0], rtol=2e-5, atol=1e-6)


def test_softmax_masked_columns_untouched():
    x = rng.standard_normal((3, 200)).astype(np.float32)
    got = oracle.softmax(x, 200, 128)
    assert np.isnan(got[:, 128:]).all()
    np.testing.assert_allclose(got[:, :128], fp64.softmax(x[:, :128]), rtol=2e-5, atol=1e-6)


# -- attention (examples/attention.py:33-113) --------------------------------------------------

def qkv(n, d, seed, heads=None, gain=1.0):
    r = np.random.default_rng(seed)
    shape = (n, d) if heads is None else (heads, n, d)
    q, k, v = (r.standard_normal(shape).astype(np.float32) for _ in range(3))
    return (q * np.float32(gain)).astype(np.float32), k, v


@pytest.mark.parametrize("n,d,block_n,causal", [(64, 16, 16, False), (64, 16, 16, True), (64, 32, 32, False),
                                                (64, 32, 32, True), (32, 64, 16, True), (37, 32, 16, True),
                                                (17, 16, 16, False)])
def test_attention_matches_float64(n, d, block_n, causal):
    """tests/test_attention.py:42-55, 72-80: atol 2e-5 vs float64, ragged N included."""
    q, k, v = qkv(n, d, n + d)
    np.testing.assert_allclose(oracle.attention(q, k, v, causal, block_n=block_n),
                               fp64.attention_reference(q, k, v, causal), rtol=0, atol=2e-5)


def test_attention_single_key_and_layouts():
    q, k, v = qkv(1, 64, 3)
    out = oracle.attention(q, k, v, False)
    # N = 1: softmax weight 1, then x / 1.0 -> within 2 ulp (tests/test_attention.py:72-80)
    ulps = np.abs(np.abs(out).view(np.int32) - np.abs(v).view(np.int32))
    assert (ulps <= 2).all()
    q, k, v = qkv(32, 32, 11)
    nd = oracle.attention(q, k, v, False, block_n=16)
    dn = oracle.attention(q, np.ascontiguousarray(k.T), v, False, block_n=16, k_layout="dn")
    np.testing.assert_array_equal(nd.view(np.uint32), dn.view(np.uint32))  # tests/test_attention.py:100-105


def test_hard_attention_retrieves_values():
    """tests/test_attention.py:108-121: each query matches one key by 1000 / sqrt(d); every
    other weight flushes to 0, the match gets exp2(0) = 1, and only the division by l = 1
    rounds (2 ulp toward zero)."""
    n = d = 32
    r = np.random.default_rng(3)
    perm = r.permutation(n)
    k = np.eye(n, dtype=np.float32)
    q = (1000.0 * np.eye(n, dtype=np.float32)[perm]).astype(np.float32)
    v = r.standard_normal((n, d)).astype(np.float32)
    out = oracle.attention(q, k, v, False, block_n=16)
    np.testing.assert_array_max_ulp(out, v[perm], maxulp=2)


def test_causal_rows_ignore_future_keys():
    """tests/test_attention.py:124-137: changing keys and values after position 31 leaves rows
    0-31 bit-identical; row 0 equals V[0] up to the division by 1."""
    n, d = 48, 16
    q, k, v = qkv(n, d, 8)
    a = oracle.attention(q, k, v, True, block_n=16)
    k2, v2 = k.copy(), v.copy()
    r = np.random.default_rng(9)
    k2[32:] = r.standard_normal((n - 32, d)) * 10
    v2[32:] = r.standard_normal((n - 32, d)) * 10
    b = oracle.attention(q, k2, v2, True, block_n=16)
    np.testing.assert_array_equal(a[:32].view(np.uint32), b[:32].view(np.uint32))
    np.testing.assert_array_max_ulp(a[0], v[0], maxulp=2)
    assert not np.array_equal(a[32:], b[32:])


def test_attention_large_scores_stay_finite():
    """tests/test_attention.py:149-155: scores of +-100 stay finite and within atol 2e-5."""
    q, k, v = qkv(48, 16, 4, gain=25.0)
    out = oracle.attention(q, k, v, False, block_n=16)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, fp64.attention_reference(q, k, v, False), rtol=0, atol=2e-5)


def test_identity_values_give_the_attention_matrix():
    """tests/test_attention.py:158-166: with V = I the output is the attention matrix: exactly
    0 above the diagonal when causal, rows summing to 1."""
    q, k, _ = qkv(32, 32, 12)
    eye = np.eye(32, dtype=np.float32)
    p = oracle.attention(q, k, eye, True, block_n=16)
    np.testing.assert_allclose(p, fp64.attention_reference(q, k, eye, True), rtol=0, atol=2e-5)
    np.testing.assert_array_equal(p[np.triu_indices(32, 1)], 0)
    np.testing.assert_allclose(p.sum(axis=1), 1, atol=1e-5)


# -- layernorm (tests/test_reroll_reduce.py:199-231) ---------------------------------------------

@pytest.mark.parametrize("block,n", [(256, 256), (256, 200), (128, 100), (128, 127)])
def test_layernorm_matches_float64(block, n):
    x = (rng.standard_normal((3, block)) * 2 + 1).astype(np.float32)
    out = oracle.layernorm(x, n, 1e-5, block)
    np.testing.assert_allclose(out[:, :n], fp64.layernorm(x, n), rtol=1e-4, atol=1e-4)
    assert np.isnan(out[:, n:]).all()


def test_add_is_fadd():
    x, y = rng.standard_normal(1000).astype(np.float32), rng.standard_normal(1000).astype(np.float32)
    np.testing.assert_array_equal(oracle.add(x, y).view(np.uint32), oracle.fadd(x, y).view(np.uint32))


# -- digits (examples/digits_model.py, tests/test_digits_model.py) --------------------------------

def test_digits_fixtures_are_the_reference_artifacts():
    """SHA-256s recorded for the artifacts (examples/data/digits/metadata.json)."""
    want = {"dataset.npz": "43742f8917d76413fdfe477f067cfd0670f3a7e3bcf8a05c0b96b01f0a650545",
            "model.npz": "482253c59cfc35ef340b5638293d594ffc62171622a20ab39ff93276b00e9684"}
    for name, digest in want.items():
        assert hashlib.sha256(open(os.path.join(GOLDEN, name), "rb").read()).hexdigest() == digest
    labels = np.load(os.path.join(GOLDEN, "dataset.npz"))["test_labels"]
    np.testing.assert_array_equal(np.bincount(labels), [178, 182, 177, 183, 181, 182, 181, 179, 174, 180])


def test_digits_model_known_accuracy_within_bounds():
    """The three-layer chain in the emulator's arithmetic: 1,743 of 1,797 correct
    (tests/test_digits_model.py:57-70) and every logit inside the propagated bound
    (tests/test_digits_model.py:84-131)."""
    data = np.load(os.path.join(GOLDEN, "dataset.npz"))
    model = np.load(os.path.join(GOLDEN, "model.npz"))
    chain = [(model[f"w{i}"], model[f"b{i}"], i < 3) for i in (1, 2, 3)]
    x = data["test_images"].astype(np.float32) / np.float32(16)
    logits = oracle.mlp_forward(x, chain)
    ref, bound = fp64.mlp_with_bounds(x, chain)
    assert (np.abs(logits - ref) <= bound).all()
    assert (logits[:, 10:] == 0).all()
    pred = oracle.argmax_rows(logits, 10)
    assert int((pred == data["test_labels"]).sum()) == 1743
    np.testing.assert_array_equal(pred, np.argmax(ref[:, :10], axis=1))


def test_argmax_rule():
    x = np.array([[1, 3, 3, 0], [np.nan, 5, np.nan, 1], [2, 2, 2, 2], [-1, -5, np.inf, np.inf]], np.float32)
    np.testing.assert_array_equal(oracle.argmax_rows(x), np.argmax(x, axis=1))


# -- input recipes (pi/runtime/piton_rt.h:60-67; perf/test_perf_suite.py:18-24) --------------------

def test_lcg_twin():
    s, ref = 99, []
    for _ in range(5):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        ref.append(s)
    np.testing.assert_array_equal(fp64.lcg_u32(5, 99), np.array(ref, np.uint32))
    s, floats = 12345, []
    for _ in range(257):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        floats.append(np.float32(s >> 8) * np.float32(1.0 / 8388608.0) - np.float32(1.0))
    np.testing.assert_array_equal(fp64.lcg_floats(257, 12345), np.array(floats, np.float32))
