"""Pins the oracle's scalar arithmetic (oracle/qpu_float.h), the emulator's float rules
(piton/qpu/emulator.py:139-235), against exact rational arithmetic truncated toward zero and
against the rules' own special cases. A wrong rounding direction, a missed flush, or a
swapped operand in the inf + (-inf) rule fails here."""
from fractions import Fraction

import numpy as np
import pytest

import oracle

F32_MIN = Fraction(2) ** -126
TWO128 = Fraction(2) ** 128


def f32(bits):
    return np.array(bits, np.uint32).view(np.float32)


def read_operand(x: np.float32):
    """The ALU's reading of an operand (emulator.py:173-178): denormal -> +0, inf/NaN -> inf
    of its sign."""
    b = int(np.float32(x).view(np.uint32))
    e = (b >> 23) & 0xFF
    if e == 255:
        return None, (-1 if b >> 31 else 1)  # infinity with sign
    if e == 0:
        return (Fraction(0) if (b & 0x7FFFFF) else Fraction(float(x))), 0
    return Fraction(float(x)), 0


def truncate(r: Fraction) -> np.float32:
    """Textbook truncation of an exact value to float32, with the QPU's flush and overflow."""
    if abs(r) >= TWO128:
        return np.float32(np.inf if r > 0 else -np.inf)
    c = np.float32(float(r))
    while abs(Fraction(float(c))) > abs(r):
        c = np.nextafter(c, np.float32(0))
    while True:
        up = np.nextafter(c, np.float32(np.inf if r > 0 else -np.inf))
        if np.isfinite(up) and abs(Fraction(float(up))) <= abs(r):
            c = up
        else:
            break
    if abs(Fraction(float(c))) < F32_MIN:
        return np.float32(0.0)
    return c


def exact_add(a, b):
    (fa, ia), (fb, ib) = read_operand(a), read_operand(b)
    if ib:
        return np.float32(np.inf * ib)
    if ia:
        return np.float32(np.inf * ia)
    return truncate(fa + fb)


def exact_mul(a, b):
    (fa, ia), (fb, ib) = read_operand(a), read_operand(b)
    if (ia and fb == 0) or (ib and fa == 0):
        return np.float32(0.0)
    if ia or ib:
        sa = ia or (1 if (fa > 0 or (fa == 0 and not np.signbit(a))) else -1)
        sb = ib or (1 if (fb > 0 or (fb == 0 and not np.signbit(b))) else -1)
        return np.float32(np.inf * sa * sb)
    return truncate(fa * fb)


def samples(n, seed):
    rng = np.random.default_rng(seed)
    mant = rng.uniform(1, 2, n) * rng.choice([-1, 1], n)
    a = (mant * 2.0 ** rng.integers(-30, 30, n)).astype(np.float32)
    # b: nearby magnitudes (cancellation, carries) and far ones (sticky bits)
    rel = rng.choice([0, 1, 2], n)
    b = np.where(rel == 0, -a * (1 + rng.uniform(-1e-6, 1e-6, n)),
                 np.where(rel == 1, a * rng.uniform(-3, 3, n), a * 2.0 ** rng.integers(-40, 40, n))).astype(np.float32)
    return a, b


def test_fadd_is_exact_sum_truncated():
    a, b = samples(3000, 1)
    got = oracle.fadd(a, b)
    want = np.array([exact_add(x, y) for x, y in zip(a, b)], np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fmul_is_exact_product_truncated():
    a, b = samples(3000, 2)
    got = oracle.fmul(a, b)
    want = np.array([exact_mul(x, y) for x, y in zip(a, b)], np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_underflow_and_overflow_edges():
    tiny = np.float32(2.0 ** -126)
    big = np.float32(3.0e38)
    a = np.array([tiny, tiny, big, big, -big, np.float32(1.5 * 2.0 ** -126)], np.float32)
    b = np.array([np.float32(0.5), -tiny, big, np.float32(2.0), big, np.float32(-2.0 ** -126)], np.float32)
    np.testing.assert_array_equal(oracle.fmul(a[:2], b[:2]).view(np.uint32), [0, 0])  # below 2^-126 -> +0
    assert oracle.fadd(a[1], b[1]).view(np.uint32) == 0                              # x + (-x) = +0
    assert np.isposinf(oracle.fadd(a[2], b[2]))                                       # >= 2^128 -> inf
    assert np.isposinf(oracle.fmul(a[3], b[3]))
    assert oracle.fadd(a[4], b[4]).view(np.uint32) == 0
    # 1.5 * 2^-126 - 2^-126 = 2^-127: a denormal result flushes to +0
    assert oracle.fadd(a[5], b[5]).view(np.uint32) == 0


def test_special_operand_rules():
    inf, nan = np.float32(np.inf), np.float32(np.nan)
    den = f32(0x00000001)
    negnan = f32(0xFFC00000)
    # NaN operands read as infinities of their sign
    assert np.isposinf(oracle.fadd(nan, np.float32(1)))
    assert np.isneginf(oracle.fadd(negnan, np.float32(1)))
    # inf + (-inf) is the second operand
    assert np.isneginf(oracle.fadd(inf, -inf)) and np.isposinf(oracle.fadd(-inf, inf))
    # fsub negates the second operand first: -inf - (-inf) = +inf
    assert np.isposinf(oracle.fsub(-inf, -inf))
    # 0 * inf = +0, both orders and signs
    for x, y in ((0.0, inf), (inf, 0.0), (-0.0, -inf), (-inf, 0.0), (den, inf)):
        assert oracle.fmul(np.float32(x), np.float32(y)).view(np.uint32) == 0
    # denormal operands read as +0; zero results are +0
    assert oracle.fadd(den, den).view(np.uint32) == 0
    assert oracle.fmul(np.float32(-3), np.float32(0)).view(np.uint32) == 0
    assert oracle.fadd(np.float32(-0.0), np.float32(-0.0)).view(np.uint32) == 0


def test_fmax_fmin_order_by_sign_magnitude_bits():
    vals = f32([0x7FC00000, 0xFFC00000, 0x7F800000, 0xFF800000, 0x00000000, 0x80000000, 0x00000001, 0x80000001,
                0x3F800000, 0xBF800000])
    # +NaN largest, then +inf; -NaN smallest; -0 and negative denormals count as positive
    assert oracle.fmax(vals[0], vals[2]).view(np.uint32) == 0x7FC00000
    assert oracle.fmax(vals[1], vals[3]).view(np.uint32) == 0xFF800000
    assert oracle.fmax(vals[5], vals[4]).view(np.uint32) == 0x00000000   # equal keys: the second operand
    assert oracle.fmax(vals[4], vals[5]).view(np.uint32) == 0x80000000
    assert oracle.fmax(vals[7], vals[4]).view(np.uint32) == 0x80000001   # key 1 > key 0
    assert oracle.fmin(vals[9], vals[8]).view(np.uint32) == 0xBF800000
    assert oracle.fmax(vals[9], np.float32(0)).view(np.uint32) == 0       # ReLU of -1


@pytest.mark.parametrize("x,want", [(2.7, 2), (-2.7, 0xFFFFFFFE), (0.5, 0), (2.0 ** 40, 0), (-(2.0 ** 31), 0x80000000),
                                    (np.inf, 0), (np.nan, 0), (1e-40, 0)])
def test_ftoi_truncates_and_wraps(x, want):
    assert int(oracle.ftoi(np.float32(x))) == want


def test_itof_truncates():
    ints = np.array([16777217, -16777217, 2 ** 31 - 1, -(2 ** 31), 0, 7], np.int32)
    got = oracle.itof(ints)
    want = np.array([truncate(Fraction(int(i))) for i in ints], np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
