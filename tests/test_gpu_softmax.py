"""Fused row softmax (examples/kernels.py:60-76) on the MI355X against the oracle.

Bar: relative Frobenius error <= 1e-5 vs float64 over finite rows and no larger than the
oracle's (the emulator's arithmetic); the NaN pattern of rows with special values matches
numpy's, except that a -NaN entry is 0 and leaves its row finite, as in the emulator; columns
past min(n_cols, BLOCK_SIZE) are never written."""
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import fp64
from piton_amd import next_power_of_2
from piton_amd.kernels import softmax_kernel
from piton_amd.runtime import mi355x as rt

pytestmark = pytest.mark.gpu
TOL = 1e-5
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "emulator")


def run(x, n_cols=None, block=None, out=None):
    rows, stride = x.shape
    n_cols = stride if n_cols is None else n_cols
    block = block or next_power_of_2(n_cols)
    if out is None:
        out = torch.full_like(x, float("nan"))
    softmax_kernel[(rows,)](out, x, x.stride(0), out.stride(0), n_cols, BLOCK_SIZE=block, device="mi355x")
    torch.cuda.synchronize()
    return out


def check(got, x, n_cols, block=None):
    n = min(n_cols, block or n_cols)
    ref = fp64.softmax(x, n_cols, block)
    finite = np.isfinite(ref[:, :n]).all(axis=1)
    np.testing.assert_array_equal(np.isnan(got[:, :n]), np.isnan(ref[:, :n]))
    err = fp64.rel_fro(got[finite, :n], ref[finite, :n])
    assert err <= TOL, err
    return err


@pytest.mark.parametrize("rows,cols,block", [(4, 64, 64), (3, 100, 128), (5, 16, 16), (7, 1, 1), (2, 3, 4)])
def test_reference_shapes(rows, cols, block):
    rng = np.random.default_rng(42 + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    got = run(torch.from_numpy(x).cuda(), cols, block).cpu().numpy()
    check(got, x, cols, block)
    emu = oracle.softmax(x, cols, block)
    ref = fp64.softmax(x, cols, block)
    assert fp64.rel_fro(got, ref) <= max(fp64.rel_fro(emu, ref), 1e-7)


@pytest.mark.parametrize("n", [1024, 4096, 1823])
def test_benchmark_shapes_with_special_rows(n):
    """4096 rows x n of N(0,1)*4 with a +inf entry, a -inf entry, an all -inf row and a NaN
    entry in a few rows; rows of 1823 are not 16-byte aligned."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((4096, n)) * 4).astype(np.float32)
    x[3, 17] = np.inf
    x[5, n - 1] = -np.inf
    x[9, :] = -np.inf
    x[11, 2] = np.nan
    got = run(torch.from_numpy(x).cuda()).cpu().numpy()
    check(got, x, n)
    assert np.isnan(got[3]).all() and np.isnan(got[9]).all() and np.isnan(got[11]).all()
    assert got[5, n - 1] == 0.0
    finite_rows = np.isfinite(x).all(axis=1)
    np.testing.assert_allclose(got[finite_rows].astype(np.float64).sum(axis=1), 1.0, rtol=0, atol=2e-6)
    # the oracle's error on a sample of finite rows bounds the GPU's there
    sample = np.flatnonzero(finite_rows)[:64]
    emu = oracle.softmax(x[sample], n)
    ref = fp64.softmax(x[sample])
    assert fp64.rel_fro(got[sample], ref) <= fp64.rel_fro(emu, ref)


NEG_NAN = np.array([0xFFC00000], np.uint32).view(np.float32)[0]


def neg_nan_as_ninf(x):
    """The emulator's reading of a -NaN operand (piton/qpu/emulator.py:173-177, 201-205): -inf."""
    x = np.array(x, np.float32)
    x[np.isnan(x) & np.signbit(x)] = -np.inf
    return x


def test_special_value_rows_match_the_emulator():
    """The emulator's own output on NaN, -NaN, +inf, -inf, -0, +0 and denormal rows
    (tests/test_reroll_reduce.py:157-174; fixture written by the reference's emulator): the same
    NaN pattern, exact zeros where it has them, and finite rows within the tolerance of float64
    applied to the emulator's reading of the operands and no worse than the emulator there."""
    s = np.load(os.path.join(GOLDEN, "softmax_specials.npz"))
    x, want = s["x"], s["y"]
    rows, cols = x.shape
    got = run(torch.from_numpy(x).cuda(), cols, cols).cpu().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(got == 0, want == 0)
    fin = np.isfinite(want).all(axis=1)
    ref = fp64.softmax(neg_nan_as_ninf(x[fin]))
    assert fp64.rel_fro(got[fin], ref) <= max(fp64.rel_fro(want[fin], ref), 1e-7)


@pytest.mark.parametrize("n", [1024, 4096, 1823, 2048, 6001, 20000])
def test_negative_nan_entries(n):
    """A -NaN entry is exactly 0 and the rest of its row a normal softmax, in every row kernel
    (one wave per row, persistent waves, one workgroup per row, three passes), as in the
    oracle; a +NaN entry still makes its row NaN."""
    rng = np.random.default_rng(n + 5)
    x = (rng.standard_normal((6, n)) * 4).astype(np.float32)
    x[0, 0] = NEG_NAN
    x[1, n - 1] = NEG_NAN
    x[2, n // 3] = NEG_NAN
    x[2, n // 2] = NEG_NAN
    x[3, 7] = NEG_NAN
    x[3, 8] = np.nan
    got = run(torch.from_numpy(x).cuda()).cpu().numpy()
    assert got[0, 0] == 0 and got[1, n - 1] == 0 and got[2, n // 3] == 0 and got[2, n // 2] == 0
    assert np.isnan(got[3]).all() and not np.isnan(got[[0, 1, 2, 4, 5]]).any()
    ref = fp64.softmax(neg_nan_as_ninf(x[:3]))
    assert fp64.rel_fro(got[:3], ref) <= TOL
    emu = np.asarray(oracle.softmax(x[:3], n))
    np.testing.assert_array_equal(emu == 0, got[:3] == 0)
    assert fp64.rel_fro(got[:3], ref) <= max(fp64.rel_fro(emu, ref), 1e-7)


def test_block_smaller_than_row_and_untouched_columns():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, 300)).astype(np.float32)
    got = run(torch.from_numpy(x).cuda(), 300, 128).cpu().numpy()
    check(got, x, 300, 128)
    assert np.isnan(got[:, 128:]).all()


@pytest.mark.parametrize("in_stride,out_stride,n", [(1823, 1823, 1823), (1825, 1830, 1823), (37, 41, 33),
                                                    (4096, 4099, 4000)])
def test_row_strides_and_alignments(in_stride, out_stride, n):
    rows = 33
    rng = np.random.default_rng(in_stride)
    xin = torch.from_numpy(rng.standard_normal((rows, in_stride)).astype(np.float32)).cuda()
    out = torch.full((rows, out_stride), -5.0, device="cuda")
    rt.softmax(out, xin, in_stride, out_stride, n, rows, next_power_of_2(n))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    x = xin.cpu().numpy()
    check(got[:, :n], x[:, :n], n)
    assert (got[:, n:] == -5.0).all()


@pytest.mark.parametrize("n", [2048, 2047, 4093, 6000, 6001, 10000, 10001, 16384, 16385, 20000])
def test_row_lengths_of_every_kernel(n):
    """Lengths that take each workgroup-per-row variant (2, 4, 8, 16 chunks per thread;
    aligned and not) and the three-pass kernel for rows past 16K columns; one row holds a
    +inf, one a -inf."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((5, n)) * 3).astype(np.float32)
    x[1, n // 2] = np.inf
    x[2, 0] = -np.inf
    got = run(torch.from_numpy(x).cuda()).cpu().numpy()
    check(got, x, n)
    assert np.isnan(got[1]).all() and got[2, 0] == 0.0


def test_in_place():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 1000)).astype(np.float32)
    t = torch.from_numpy(x).cuda()
    run(t, out=t)
    check(t.cpu().numpy(), x, 1000)


def test_numpy_launch():
    x = np.random.default_rng(4).standard_normal((3, 100)).astype(np.float32)
    y = np.zeros_like(x)
    softmax_kernel[(3,)](y, x, 100, 100, 100, BLOCK_SIZE=128, device="mi355x")
    check(y, x, 100)
