"""Pins the oracle's restated math sequences (piton/backend/lower.py: exp/exp2 :2716-2797,
recip/fdiv/fdiv_uniform :633-764, rsqrt/sqrt :766-795, 2899-2939) by the reference's own
accuracy tests and special values (tests/test_tiles.py:158-228), the reference's known answer
for x / 1.0 (tests/test_attention.py:25-27), and the claim that fdiv_uniform gives fdiv's
bits (lower.py:736-739). A dropped polynomial term, a wrong constant or a wrong special-case
rule fails one of these; the last-bit agreement of the sequences with the emulator itself is
pinned separately by the emulator's own outputs (tests/test_oracle_emulator_vectors.py)."""
import numpy as np
import pytest

import oracle

rng = np.random.default_rng(7)
FLT_MIN = np.float32(1.17549435e-38)

# tests/test_tiles.py:172-174
EXPLOG_SPECIALS = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0, 2.0, 0.5, 88.7, 88.73,
                            -87.3, -87.4, -103.9, -150, 127.9, 128.0, 1e30, -1e30, 3.4e38, 1.17549435e-38],
                           np.float32)
# tests/test_tiles.py:203-204
DIV_SPECIALS = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0, 4.0, 2.0 ** 127, 3.4e38,
                         1.2e-38, 0.25, -4.0, 9.0], np.float32)


def flushed(ref):
    ref = ref.astype(np.float32)
    ref[np.abs(ref) < FLT_MIN] = 0.0
    return ref


@pytest.mark.parametrize("base2", [False, True])
def test_exp_accuracy_and_specials(base2):
    """tests/test_tiles.py:177-192: within rtol 3e-7 of float64, specials included."""
    lo, hi = (-125, 127) if base2 else (-87, 88)
    x = np.concatenate([rng.uniform(lo, hi, 20000).astype(np.float32), EXPLOG_SPECIALS])
    got = oracle.exp2(x) if base2 else oracle.exp(x)
    with np.errstate(all="ignore"):
        ref = flushed((np.exp2 if base2 else np.exp)(x.astype(np.float64)))
    np.testing.assert_allclose(got, ref, rtol=3e-7, atol=0, equal_nan=True)


def test_exp_exact_points():
    assert oracle.exp(np.float32(0.0)) == 1.0 and oracle.exp2(np.float32(0.0)) == 1.0
    assert oracle.exp2(np.float32(10.0)) == 1024.0  # integer powers are exact: r = 0, q = 1
    assert oracle.exp(np.float32(-np.inf)) == 0.0 and np.isposinf(oracle.exp(np.float32(np.inf)))
    assert np.isposinf(oracle.exp2(np.float32(128.0))) and oracle.exp2(np.float32(-150.0)) == 0.0


def test_exp_is_monotone_on_a_dense_grid():
    x = np.linspace(-20, 20, 200001).astype(np.float32)
    e = oracle.exp(x)
    assert (np.diff(e.astype(np.float64)) >= 0).all()


@pytest.mark.parametrize("F", ["div", "rsqrt", "sqrt"])
def test_div_sqrt_accuracy_and_specials(F):
    """tests/test_tiles.py:207-228: within rtol 4e-7 of float64, specials included. (For
    |b| >= 2^126 the restatement flushes 1/b to 0, as the lowering does, so the numerators
    paired with the special divisors stay below 2 in magnitude.)"""
    y = np.exp(rng.uniform(-80, 80, 20000)).astype(np.float32)
    if F == "div":
        y *= rng.choice([-1, 1], len(y)).astype(np.float32)
    y = np.concatenate([y, DIV_SPECIALS])
    x = rng.standard_normal(len(y)).astype(np.float32)
    x[-len(DIV_SPECIALS):] = np.clip(x[-len(DIV_SPECIALS):], -1.5, 1.5)
    got = {"div": lambda: oracle.fdiv(x, y), "rsqrt": lambda: oracle.rsqrt(y), "sqrt": lambda: oracle.sqrt(y)}[F]()
    with np.errstate(all="ignore"):
        y64 = y.astype(np.float64)
        ref = flushed({"div": x / y64, "rsqrt": 1 / np.sqrt(y64), "sqrt": np.sqrt(y64)}[F])
    np.testing.assert_allclose(got, ref, rtol=4e-7, atol=0, equal_nan=True)


def test_division_special_rules():
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    f = lambda a, b: oracle.fdiv(np.float32(a), np.float32(b))  # noqa: E731
    assert np.isnan(f(0.0, 0.0)) and np.isnan(f(inf, inf)) and np.isnan(f(nan, 2.0)) and np.isnan(f(2.0, nan))
    assert np.isposinf(f(3.0, 0.0)) and np.isneginf(f(3.0, -0.0)) and np.isneginf(f(-3.0, 0.0))
    assert f(3.0, inf) == 0.0 and f(-3.0, inf) == 0.0
    assert np.isnan(f(1e-40, 0.0))  # a denormal numerator is 0: 0 / 0


def test_x_over_one_lands_two_ulp_toward_zero():
    """tests/test_attention.py:25-27: 'PIton's x / y is within 2 ulp (x / 1.0 lands 2 ulp
    toward zero)'."""
    x = rng.uniform(-100, 100, 10000).astype(np.float32)
    got = oracle.fdiv(x, np.float32(1.0))
    ulps = (np.abs(x).view(np.int32) - np.abs(got).view(np.int32))
    assert (ulps >= 0).all() and (ulps <= 2).all() and (ulps == 2).mean() > 0.5


def test_fdiv_uniform_gives_fdiv_bits():
    a = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 100, DIV_SPECIALS, DIV_SPECIALS])
    b = np.concatenate([np.exp(rng.uniform(-80, 80, 5000)).astype(np.float32), DIV_SPECIALS,
                        DIV_SPECIALS[::-1]])
    for bb in (b, np.full_like(a, np.float32(3.0)), np.full_like(a, np.float32(0.0)), np.full_like(a, np.inf),
               np.full_like(a, np.nan)):
        np.testing.assert_array_equal(oracle.fdiv(a, bb).view(np.uint32), oracle.fdiv_uniform(a, bb).view(np.uint32))


def test_recip_specials():
    vals = np.array([0.0, -0.0, np.inf, -np.inf, 2.0 ** 126, -(2.0 ** 127), 1e-40, np.nan], np.float32)
    r = oracle.recip(vals)
    assert np.isposinf(r[0]) and np.isneginf(r[1])
    assert r[2].view(np.uint32) == 0 and r[3].view(np.uint32) == 0x80000000
    assert r[4] == 0.0 and r[5].view(np.uint32) == 0x80000000
    assert np.isposinf(r[6]) and np.isnan(r[7])


def test_sqrt_specials():
    vals = np.array([-1.0, 0.0, -0.0, np.inf, np.nan, 1e-40, 4.0], np.float32)
    s = oracle.sqrt(vals)
    assert np.isnan(s[0]) and s[1] == 0 and s[2].view(np.uint32) == 0x80000000
    assert np.isposinf(s[3]) and np.isnan(s[4]) and s[5] == 0.0
    assert abs(s[6] - 2.0) <= 2 * np.spacing(np.float32(2.0))
