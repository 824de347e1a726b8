"""The oracle against the reference's own QPU emulator, bit for bit.

tests/golden/emulator/*.npz hold inputs and outputs of the reference's strict emulator
(written by tests/golden/make_emulator_vectors.py, which imports the reference where its
checkout exists): one-op math kernels over seeded and special values
(piton/backend/lower.py: exp/exp2 :2716-2797, division :633-764, rsqrt/sqrt :766-795, 2899-2939),
softmax_kernel rows with +inf / all -inf / -inf / NaN rows and rows of 1000-1823 columns at
BLOCK_SIZE 1024 / 2048 (examples/kernels.py:60-76), the
tutorial matmul (examples/kernels.py:18-57), row layernorm (tests/test_reroll_reduce.py:199-208) and
add_kernel (examples/kernels.py:6-15), attention through run_attention
(examples/attention.py:200-222) and the digits MLP's three dense_layer_kernel launches (He-normal
weights, raw [0, 16] pixels, 64 -> 128 -> 64 -> 10) for 96 images and for all
1,797 (examples/nn_kernels.py:23-74). Every output must equal the oracle's bits (NaN equals NaN)."""
import os

import numpy as np
import pytest

import oracle
from piton_amd import digits

G = os.path.join(os.path.dirname(__file__), "golden", "emulator")


def load(name):
    return np.load(os.path.join(G, f"{name}.npz"))


def assert_bits(got, want):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert got.shape == want.shape
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    bad = np.flatnonzero(~same.ravel())
    assert bad.size == 0, f"{bad.size} of {same.size} differ, first at {bad[:5]}: " \
                          f"{got.ravel()[bad[:5]]} vs {want.ravel()[bad[:5]]}"


@pytest.mark.parametrize("name,fn", [("exp", oracle.exp), ("exp2", oracle.exp2), ("rsqrt", oracle.rsqrt),
                                     ("sqrt", oracle.sqrt)])
def test_unary_math(name, fn):
    m = load("math")
    assert_bits(fn(m[f"{name}_x"]), m[f"{name}_y"])


def test_one_over_is_division():
    """`1.0 / x` lowers to the division (a * recip(b) with its NaN rules): 1 / -inf is +0 there
    (the multiply's zero is +0), while recip alone keeps the sign."""
    m = load("math")
    x = m["recip_x"]
    assert_bits(oracle.fdiv(np.ones_like(x), x), m["recip_y"])


def test_division():
    m = load("math")
    assert_bits(oracle.fdiv(m["fdiv_x"], m["fdiv_y"]), m["fdiv_out"])


@pytest.mark.parametrize("j", range(4))
def test_division_by_a_uniform(j):
    m = load("math")
    x = m["fdiv_uniform_x"]
    s = np.full_like(x, m[f"fdiv_uniform_s{j}"])
    assert_bits(oracle.fdiv_uniform(x, s), m[f"fdiv_uniform_out{j}"])


@pytest.mark.parametrize("i", range(4))
def test_softmax_rows(i):
    s = load("softmax")
    rows, cols, block, stride = (int(v) for v in s[f"case{i}_shape"])
    x, want = s[f"case{i}_x"], s[f"case{i}_y"]
    got = np.asarray(oracle.softmax(x, cols, block))
    assert_bits(got[:, :cols], want[:, :cols])
    assert (want[:, cols:] == np.float32(-7.0)).all()  # the kernel leaves the rest of the row


def test_softmax_special_value_rows():
    """NaN, -NaN, +inf, -inf, -0, +0 and denormal entries (tests/test_reroll_reduce.py:157-174)
    and rows whose only special entry is a -NaN: the emulator makes a -NaN entry exactly 0 and
    the rest of its row a normal softmax (fmax orders -NaN lowest, the ALUs read it as -inf)."""
    s = load("softmax_specials")
    rows, cols, block, _ = (int(v) for v in s["shape"])
    x, want = s["x"], s["y"]
    assert_bits(np.asarray(oracle.softmax(x, cols, block)), want)
    assert np.isnan(want[[0, 1, 5, 6, 7]]).all() and np.isfinite(want[[2, 3, 4, 8, 9, 10, 11]]).all()
    assert want[8, 0] == 0 and want[9, 130] == 0 and want[10, 255] == 0 and (want[11, 40:42] == 0).all()


@pytest.mark.parametrize("i", range(3))
def test_softmax_long_rows(i):
    """BLOCK_SIZE 1024 (n_cols 1000, 1023) and 2048 (n_cols 1823, the config's non-power-of-two
    row), built with the reduction reroll on (tests/test_reroll_reduce.py:37-44)."""
    s = load("softmax_long")
    rows, cols, block, _ = (int(v) for v in s[f"case{i}_shape"])
    assert_bits(np.asarray(oracle.softmax(s[f"case{i}_x"], cols, block)), s[f"case{i}_y"])


@pytest.mark.parametrize("i", range(4))
def test_layernorm_rows(i):
    """The layernorm kernel of tests/test_reroll_reduce.py:199-208 at (BLOCK, n) = (256, 256),
    (256, 200), (128, 100), (128, 127); columns past n stay as the emulator left them (NaN)."""
    m = load("layernorm")
    rows, n, block = (int(v) for v in m[f"case{i}_shape"])
    assert_bits(oracle.layernorm(m[f"case{i}_x"], n, 1e-5, block), m[f"case{i}_y"])


def test_add():
    m = load("layernorm")
    assert_bits(oracle.add(m["add_x"], m["add_y"]), m["add_out"])


@pytest.mark.parametrize("i", range(2))
def test_matmul(i):
    m = load("matmul")
    assert_bits(oracle.matmul(m[f"case{i}_a"], m[f"case{i}_b"]), m[f"case{i}_c"])


@pytest.mark.parametrize("i", range(3))
def test_attention(i):
    a = load("attention")
    got = oracle.attention(a[f"case{i}_q"], a[f"case{i}_k"], a[f"case{i}_v"], bool(a[f"case{i}_causal"]), block_n=16)
    assert_bits(got, a[f"case{i}_o"])


def test_digits_mlp_logits_and_predictions():
    m = load("mlp")
    layers = digits.he_normal_mlp(seed=1729)
    chain = [(w, b, i < 2) for i, (w, b) in enumerate(layers)]
    logits = oracle.mlp_forward(m["x"], chain)
    assert_bits(logits, m["h3"])
    np.testing.assert_array_equal(oracle.argmax_rows(logits, 10), m["pred"])


def test_digits_mlp_all_1797_images():
    """The emulator's three dense launches over every one of the 1,797 test images."""
    m = load("mlp_full")
    x = np.load(os.path.join(os.path.dirname(__file__), "golden", "digits", "dataset.npz"))["test_images"]
    chain = [(w, b, i < 2) for i, (w, b) in enumerate(digits.he_normal_mlp(seed=1729))]
    logits = oracle.mlp_forward(x.astype(np.float32), chain)
    assert_bits(logits, m["logits"])
    np.testing.assert_array_equal(oracle.argmax_rows(logits, 10), m["pred"])
