"""The perf suite's primitives (perf/suite.py:148-351) on the MI355X through the launch surface,
with the suite's inputs (the LCG of piton_rt.h, scaled per case) and its tolerances: each
float case passes |got - want| <= atol + rtol |want| against float64, integer cases and
data movement are exact."""
import numpy as np
import pytest
import torch

from oracle.fp64 import lcg_u32
from piton_amd import cdiv
from piton_amd.kernels import (copy_kernel, fma_kernel, idiv_kernel, log_kernel, mul_kernel, row_max_kernel,
                               row_sum_kernel, scaled_relu_kernel, sfu_kernel, transpose_kernel)
from piton_amd.runtime import mi355x as rt

pytestmark = pytest.mark.gpu
VEC = 262144  # the suite's "pi" vector length (perf/suite.py:143)
MAT = 256     # and matrix side


class Inputs:
    """The suite's buffer recipe (perf/suite.py:71-101): seeds 1000003 * k for k = 2, 3, ...;
    floats = lcg_float * (hi - lo)/2 + (hi + lo)/2 in float32; ints = (int32) lcg >> shift | mask."""

    def __init__(self):
        self.k = 1

    def _seed(self):
        self.k += 1
        return 1000003 * self.k

    def floats(self, n, lo=-1.0, hi=1.0):
        u = lcg_u32(n, self._seed())
        f = (u >> np.uint32(8)).astype(np.float32) * np.float32(1.0 / 8388608.0) - np.float32(1.0)
        return f * np.float32((hi - lo) / 2) + np.float32((hi + lo) / 2)

    def ints(self, n, shift=0, or_mask=0):
        return (lcg_u32(n, self._seed()).view(np.int32) >> shift) | np.int32(or_mask)


def within(got, want, rtol, atol):
    got = np.asarray(got, np.float64)
    assert np.isfinite(got).all()
    err = np.abs(got - want)
    bad = np.flatnonzero(err > atol + rtol * np.abs(want))
    assert bad.size == 0, f"{bad.size} outside tolerance, worst {err.max():.3g} at {int(err.argmax())}"


ELEMENTWISE = [  # name, kernel, inputs, lo, hi, extra args, reference, rtol, atol
    ("copy", copy_kernel, 1, -1, 1, {}, lambda x: x, 1e-6, 1e-6),
    ("mul", mul_kernel, 2, -1, 1, {}, lambda x, y: x * y, 1e-6, 1e-6),
    ("fma", fma_kernel, 2, -1, 1, {"alpha": 1.5}, lambda x, y: x * 1.5 + y, 1e-6, 1e-6),
    ("scaled_relu", scaled_relu_kernel, 1, -1, 1, {"alpha": 0.5}, lambda x: np.where(x > 0, x * 0.5, 0.0), 1e-6,
     1e-6),
    ("exp", sfu_kernel, 1, -8, 8, {"OP": 4}, np.exp, 4e-6, 1e-30),
    ("exp2", sfu_kernel, 1, -8, 8, {"OP": 0}, np.exp2, 4e-6, 1e-30),
    ("log", log_kernel, 1, 0.01, 100, {}, np.log, 4e-6, 4e-7),
    ("log2", sfu_kernel, 1, 0.01, 100, {"OP": 1}, np.log2, 4e-6, 4e-7),
    ("recip", sfu_kernel, 1, 0.01, 100, {"OP": 2}, lambda x: 1.0 / x, 4e-6, 1e-30),
    ("rsqrt", sfu_kernel, 1, 0.01, 100, {"OP": 3}, lambda x: 1.0 / np.sqrt(x), 4e-6, 1e-30),
    ("sqrt", sfu_kernel, 1, 0.01, 100, {"OP": 5}, np.sqrt, 4e-6, 1e-30),
]


@pytest.mark.parametrize("case", ELEMENTWISE, ids=[c[0] for c in ELEMENTWISE])
@pytest.mark.parametrize("n", [VEC, VEC + 3])
def test_elementwise_suite_cases(case, n):
    name, kernel, n_in, lo, hi, extra, ref, rtol, atol = case
    g = Inputs()
    xs = [g.floats(n, lo, hi) for _ in range(n_in)]
    out = np.full(n, np.nan, np.float32)
    names = ("x_ptr", "y_ptr")[:n_in]
    kernel[(cdiv(n, 256),)](**dict(zip(names, xs)), out_ptr=out, n=n, **extra, BLOCK=256, device="mi355x")
    within(out, ref(*[x.astype(np.float64) for x in xs]), rtol, atol)


def test_elementwise_unaligned_views_and_tails():
    """Tensor views one float past an allocation start (no 16-byte vectors) and odd lengths."""
    g = Inputs()
    base = torch.from_numpy(g.floats(1001, 0.01, 100)).cuda()
    x = base[1:]
    out = torch.full((1001,), -1.0, device="cuda")
    rt.sfu(x, out[1:], 1000, 5)
    rt.fma(x, x, out[:999], 999, 2.0)
    torch.cuda.synchronize()
    xn = base.cpu().numpy()[1:].astype(np.float64)
    got = out.cpu().numpy()
    within(got[:999], xn[:999] * 3.0, 1e-6, 1e-6)
    within(got[999:], np.sqrt(xn[998:]), 4e-6, 1e-30)


def test_idiv_truncates_like_c():
    g = Inputs()
    x = g.ints(VEC)
    y = g.ints(VEC, shift=8, or_mask=1)  # nonzero, varied size (perf/suite.py:178-185)
    q = np.full(VEC, -1, np.int32)
    r = np.full(VEC, -1, np.int32)
    idiv_kernel[(cdiv(VEC, 256),)](x, y, q, r, VEC, BLOCK=256, device="mi355x")
    x64, y64 = x.astype(np.int64), y.astype(np.int64)
    want_q = np.sign(x64) * np.sign(y64) * (np.abs(x64) // np.abs(y64))
    np.testing.assert_array_equal(q, want_q.astype(np.int32))
    np.testing.assert_array_equal(r, (x64 - want_q * y64).astype(np.int32))


@pytest.mark.parametrize("kernel,op,rtol", [(row_sum_kernel, np.sum, 1e-5), (row_max_kernel, np.max, 0.0)])
@pytest.mark.parametrize("m", [MAT, 1000])
def test_row_reductions(kernel, op, rtol, m):
    g = Inputs()
    x = g.floats(m * m).reshape(m, m)
    out = np.full(m, np.nan, np.float32)
    kernel[(m // 4,)](x, out, m, m, BLOCK_M=4, BLOCK_N=8, device="mi355x")
    within(out, op(x.astype(np.float64), axis=1), rtol, 1e-5)


def test_row_reduction_reads_whole_chunks_like_the_reference():
    """n_cols = 70 with BLOCK_N = 64 reads 128 columns of each row (kernels.py:92-95)."""
    x = np.arange(4 * 130, dtype=np.float32).reshape(4, 130) * np.float32(0.01)
    out = np.zeros(4, np.float32)
    row_sum_kernel[(1,)](x, out, 70, 130, BLOCK_M=4, BLOCK_N=64, device="mi355x")
    within(out, x[:, :128].astype(np.float64).sum(axis=1), 1e-5, 1e-5)


@pytest.mark.parametrize("rows,cols,pad", [(MAT, MAT, 0), (100, 37, 3), (1, 300, 0), (513, 64, 1),
                                           (260, 132, 4), (64, 8, 0), (4, 4100, 8), (1028, 196, 12)])
def test_transpose_exact(rows, cols, pad):
    g = Inputs()
    x = np.zeros((rows, cols + pad), np.float32)
    x[:, :cols] = g.floats(rows * cols).reshape(rows, cols)
    out = np.full((cols, rows + pad), -7.0, np.float32)
    transpose_kernel[(cdiv(rows, 16) * cdiv(cols, 16),)](x, out, rows, cols, cols + pad, rows + pad, BLOCK_M=16,
                                                        BLOCK_N=16, device="mi355x")
    np.testing.assert_array_equal(out[:, :rows], x[:, :cols].T)
    assert (out[:, rows:] == -7.0).all()


def test_wrong_grids_are_refused():
    x = np.zeros(1000, np.float32)
    with pytest.raises(ValueError, match="grid"):
        copy_kernel[(3,)](x, x.copy(), 1000, BLOCK=256, device="mi355x")
