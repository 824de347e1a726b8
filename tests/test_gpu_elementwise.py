"""add_kernel (examples/kernels.py:6-15) and the row layernorm_kernel
(tests/test_reroll_reduce.py:199-208) on the MI355X, through the reference's launch surface.

Bar:
  * add: bit-exact with numpy's float32 `x + y` (one correctly rounded add), never further from
    the exact float64 sum than the oracle's round-toward-zero add, and a 16-float guard band of
    7.0 past n left untouched (tests/test_vector_add.py:12-21);
  * layernorm: within rtol/atol 1e-4 of float64 (tests/test_reroll_reduce.py:226-230), relative
    Frobenius error <= 1e-5 and no larger than the oracle's (whose bits equal the emulator's on
    the golden rows), and every column past n still NaN.
"""
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle
from oracle import fp64
from piton_amd import cdiv
from piton_amd.kernels import add_kernel, layernorm_kernel

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "emulator")


def _check_add(x, y, got):
    np.testing.assert_array_equal(got, x + y)
    exact = x.astype(np.float64) + y.astype(np.float64)
    rtz = oracle.add(x, y).astype(np.float64)
    assert (np.abs(got.astype(np.float64) - exact) <= np.abs(rtz - exact)).all()


@pytest.mark.parametrize("n,block", [(64, 64), (1000, 64), (4096, 256), (37, 16), (16, 16), (2048 * 256, 256)])
def test_add_guard_band_numpy(n, block):
    """numpy arguments: copied in and out, as the emulator does."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal(n).astype(np.float32)
    y = rng.standard_normal(n).astype(np.float32)
    out = np.full(n + 16, 7.0, dtype=np.float32)
    grid = lambda meta: (cdiv(n, meta["BLOCK_SIZE"]),)  # noqa: E731
    add_kernel[grid](x, y, out, n, BLOCK_SIZE=block, device="mi355x")
    _check_add(x, y, out[:n])
    assert np.all(out[n:] == 7.0)


@pytest.mark.parametrize("n,offset", [(2048 * 256, 0), (1027, 0), (1027, 1), (5, 3), (4099, 2)])
def test_add_tensors(n, offset):
    """Device tensors, including views that start off a 16-byte boundary (the scalar path)."""
    rng = np.random.default_rng(n + offset)
    x = (rng.standard_normal(n) * 8).astype(np.float32)
    y = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    tx = torch.zeros(n + 8, device="cuda")
    ty = torch.zeros(n + 8, device="cuda")
    tx[offset:offset + n] = torch.from_numpy(x).cuda()
    ty[offset:offset + n] = torch.from_numpy(y).cuda()
    buf = torch.full((n + offset + 16,), 7.0, device="cuda")
    add_kernel[(cdiv(n, 256),)](tx[offset:], ty[offset:], buf[offset:], n, BLOCK_SIZE=256, device="mi355x")
    torch.cuda.synchronize()
    got = buf.cpu().numpy()
    _check_add(x, y, got[offset:offset + n])
    assert np.all(got[:offset] == 7.0) and np.all(got[offset + n:] == 7.0)


def test_add_golden_values():
    """The golden add inputs (seeded values and specials): the GPU's add is IEEE round to
    nearest, so it equals numpy; where the exact sum is representable it equals the emulator's
    bits as well."""
    g = np.load(os.path.join(GOLDEN, "layernorm.npz"))
    x, y, emu = g["add_x"], g["add_y"], g["add_out"]
    out = np.full(x.size + 16, 7.0, np.float32)
    add_kernel[(cdiv(x.size, 64),)](x, y, out, x.size, BLOCK_SIZE=64, device="mi355x")
    with np.errstate(invalid="ignore", over="ignore"):
        want = x + y
    finite = np.isfinite(x) & np.isfinite(y)
    np.testing.assert_array_equal(out[:x.size][finite], want[finite])
    tiny = np.float32(2.0 ** -126)
    normal = lambda v: (v == 0) | (np.abs(v) >= tiny)  # noqa: E731  (the emulator flushes denormals)
    exact = finite & normal(x) & normal(y) & (np.abs(want) >= tiny)
    exact &= np.array([bool(e) and Fraction(float(a)) + Fraction(float(b)) == Fraction(float(w))
                       for e, a, b, w in zip(exact, x, y, want)])
    assert exact.sum() > 100
    np.testing.assert_array_equal(out[:x.size][exact], emu[exact])
    assert np.all(out[x.size:] == 7.0)


def _layernorm_ref(x, n, eps=1e-5):
    xs = x[:, :n].astype(np.float64)
    d = xs - xs.mean(axis=1, keepdims=True)
    return d / np.sqrt((d * d).mean(axis=1, keepdims=True) + eps)


def _check_layernorm(x, n, block, out):
    ref = _layernorm_ref(x, n)
    np.testing.assert_allclose(out[:, :n], ref, rtol=1e-4, atol=1e-4)
    assert np.isnan(out[:, n:]).all()
    err = fp64.rel_fro(out[:, :n], ref)
    orc = oracle.layernorm(x, n, 1e-5, block)
    assert err <= 1e-5 and err <= fp64.rel_fro(orc[:, :n], ref), err


@pytest.mark.parametrize("i", range(4))
def test_layernorm_golden_rows(i):
    """The golden rows at (BLOCK, n) = (256, 256), (256, 200), (128, 100), (128, 127): the launch
    form with n < BLOCK writes only the first n columns of each BLOCK-wide row."""
    g = np.load(os.path.join(GOLDEN, "layernorm.npz"))
    rows, n, block = (int(v) for v in g[f"case{i}_shape"])
    x = g[f"case{i}_x"]
    out = np.full(rows * block, np.nan, np.float32)
    layernorm_kernel[(rows,)](x.ravel(), out, n, 1e-5, BLOCK=block, device="mi355x")
    out = out.reshape(rows, block)
    _check_layernorm(x, n, block, out)
    emu = g[f"case{i}_y"]
    assert fp64.rel_fro(out[:, :n], _layernorm_ref(x, n)) <= fp64.rel_fro(emu[:, :n], _layernorm_ref(x, n))


@pytest.mark.parametrize("rows,n,block", [(2048, 256, 256), (64, 256, 256), (7, 1000, 1024), (5, 33, 64)])
def test_layernorm_tensors(rows, n, block):
    """Device tensors; 2048 x 256 is the decoder's prefill shape (64 sequences x 32 tokens)."""
    rng = np.random.default_rng(rows * 7 + n)
    x = (rng.standard_normal((rows, block)) * 2 + 1).astype(np.float32)
    tx = torch.from_numpy(x).cuda()
    tout = torch.full((rows, block), float("nan"), device="cuda")
    layernorm_kernel[(rows,)](tx, tout, n, 1e-5, BLOCK=block, device="mi355x")
    torch.cuda.synchronize()
    _check_layernorm(x, n, block, tout.cpu().numpy())


def test_layernorm_block_smaller_than_n():
    """With BLOCK < n the kernel reads and writes only the first BLOCK columns of each row (the
    reference's mask is offs < n over offs < BLOCK)."""
    rows, block, n = 4, 128, 300
    rng = np.random.default_rng(5)
    x = rng.standard_normal((rows, block)).astype(np.float32)
    out = np.full(rows * block, np.nan, np.float32)
    layernorm_kernel[(rows,)](x.ravel(), out, n, 1e-5, BLOCK=block, device="mi355x")
    _check_layernorm(x, block, block, out.reshape(rows, block))
