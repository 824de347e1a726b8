"""Fused dense layers and the digits MLP (examples/nn_kernels.py:23-74,
examples/digits_model.py:120-139) on the MI355X against the oracle.

Bar: dyadic inputs bit-exact (tests/test_nn_kernels.py:37-61); argmax predictions bit-exact
against the oracle's (the emulator's arithmetic), each certified by its top-2 margin against the
propagated error bounds (examples/digits_reference.py:14-55); the trained model's known accuracy
(1,743 of 1,797, tests/test_digits_model.py:57-70)."""
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import fp64
from piton_amd import cdiv, digits
from piton_amd.kernels import dense_layer_kernel, dense_tiles
from piton_amd.runtime import mi355x as rt

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "digits")


def run_dense(x, w, bias, relu, add_bias=True):
    """dense_layer_kernel[grid] with the reference's tiles and a sentinel suffix catching
    stores past M*N (tests/test_nn_kernels.py:14-34)."""
    m, k = x.shape
    n = w.shape[1]
    bm, bn, bk = dense_tiles(n)
    storage = torch.full((m * n + 32,), -1234.5, device="cuda")
    tx, tw, tb = (torch.from_numpy(t).cuda() for t in (x, w, bias))
    dense_layer_kernel[(cdiv(m, bm) * cdiv(n, bn),)](tx, tw, tb, storage, m, N=n, K=k, BLOCK_SIZE_M=bm,
                                                     BLOCK_SIZE_N=bn, BLOCK_SIZE_K=bk, GROUP_SIZE_M=1,
                                                     ADD_BIAS=add_bias, RELU=relu, device="mi355x")
    torch.cuda.synchronize()
    s = storage.cpu().numpy()
    assert (s[m * n:] == np.float32(-1234.5)).all()
    return s[:m * n].reshape(m, n)


@pytest.mark.parametrize("m,n,k,add_bias,relu", [(8, 64, 64, True, True), (9, 17, 11, True, False),
                                                 (3, 10, 7, False, True), (1, 16, 8, False, False),
                                                 (1797, 128, 64, True, True), (1797, 10, 64, True, False)])
def test_dense_dyadic_bit_exact(m, n, k, add_bias, relu):
    rng = np.random.default_rng(340 + m)
    x = rng.integers(-4, 5, (m, k)).astype(np.float32) / np.float32(4)
    w = rng.integers(-4, 5, (k, n)).astype(np.float32) / np.float32(4)
    bias = rng.integers(-8, 9, n).astype(np.float32) / np.float32(4)
    got = run_dense(x, w, bias, relu, add_bias)
    expected = x @ w
    if add_bias:
        expected += bias
    if relu:
        expected = np.maximum(expected, np.float32(0))
    np.testing.assert_array_equal(got, expected)
    np.testing.assert_array_equal(got, oracle.dense(x, w, bias if add_bias else None, relu))


def test_network_64_128_64_16():
    rng = np.random.default_rng(340)
    x = rng.uniform(-1, 1, (3, 64)).astype(np.float32)
    ref = x.astype(np.float64)
    for i, (k, n) in enumerate(((64, 128), (128, 64), (64, 16))):
        w = rng.normal(0, 0.1, (k, n)).astype(np.float32)
        b = rng.normal(0, 0.1, n).astype(np.float32)
        x = run_dense(x, w, b, relu=i < 2)
        ref = fp64.dense(ref, w, b, relu=i < 2)
        np.testing.assert_allclose(x, ref, rtol=2e-4, atol=2e-5)
    np.testing.assert_array_equal(np.argmax(x[:, :10], 1), np.argmax(ref[:, :10], 1))


def _chain_check(images, layers, n_classes=10):
    """GPU logits and predictions for images (float32) vs the oracle and certified margins."""
    mlp = digits.MLP(layers, max_batch=len(images), n_classes=n_classes)
    x = torch.from_numpy(np.ascontiguousarray(images, np.float32)).cuda()
    logits, pred = mlp.run(x)
    torch.cuda.synchronize()
    logits, pred = logits.cpu().numpy(), pred.cpu().numpy()
    chain = [(w, b, i < len(layers) - 1) for i, (w, b) in enumerate(layers)]
    emu_logits = oracle.mlp_forward(images, chain)
    emu_pred = oracle.argmax_rows(emu_logits, n_classes)
    ref, bound_rtz = fp64.mlp_with_bounds(images, chain, unit=2.0 ** -23)
    # the GPU's float32 chain, any faithful rounding per operation (<= 1 ulp)
    _, bound_rn = fp64.mlp_with_bounds(images, chain, unit=2.0 ** -23)
    assert (np.abs(emu_logits - ref) <= bound_rtz).all()
    assert (np.abs(logits - ref) <= bound_rn).all()
    top, certified = fp64.certified_argmax(ref, bound_rtz + bound_rn, n_classes)
    np.testing.assert_array_equal(pred, oracle.argmax_rows(logits, n_classes))
    mismatch = np.flatnonzero(pred != emu_pred)
    assert not np.isin(mismatch, np.flatnonzero(certified)).any(), "a certified prediction differs"
    return pred, emu_pred, certified


def test_config_random_init_unnormalised_pixels():
    """Config: He-normal weights, zero biases, the 1,797 UCI test images as raw [0, 16] floats."""
    images = np.load(os.path.join(GOLDEN, "dataset.npz"))["test_images"].astype(np.float32)
    layers = digits.he_normal_mlp(seed=1729)
    pred, emu_pred, certified = _chain_check(images, layers)
    np.testing.assert_array_equal(pred, emu_pred)
    assert certified.mean() > 0.95  # worst-case bounds; the rest must still agree bit for bit
    # the reference emulator's own predictions for this batch (tests/golden/emulator/mlp_full.npz)
    emulator = np.load(os.path.join(os.path.dirname(__file__), "golden", "emulator", "mlp_full.npz"))
    np.testing.assert_array_equal(pred, emulator["pred"])


def test_trained_model_known_accuracy():
    data = np.load(os.path.join(GOLDEN, "dataset.npz"))
    model = np.load(os.path.join(GOLDEN, "model.npz"))
    layers = [(model[f"w{i}"], model[f"b{i}"]) for i in (1, 2, 3)]
    images = digits.normalize(data["test_images"])
    pred, emu_pred, _ = _chain_check(images, layers, n_classes=10)
    np.testing.assert_array_equal(pred, emu_pred)
    assert int((pred == data["test_labels"]).sum()) == 1743


def test_ragged_batches_reuse_buffers():
    layers = digits.he_normal_mlp(seed=3)
    mlp = digits.MLP(layers, max_batch=1800)
    rng = np.random.default_rng(12864)
    for m in (1, 8, 9, 1797):
        x = rng.integers(0, 17, (m, 64)).astype(np.float32)
        logits, pred = mlp.run(torch.from_numpy(x).cuda())
        torch.cuda.synchronize()
        chain = [(w, b, i < 2) for i, (w, b) in enumerate(layers)]
        ref = fp64.mlp_with_bounds(x, chain)[0]
        np.testing.assert_allclose(logits.cpu().numpy(), ref, rtol=2e-4, atol=2e-4)


@pytest.mark.parametrize("m,sizes", [(1797, (64, 128, 64, 10)), (1797, (64, 128, 64, 16)), (33, (64, 128, 64, 10)),
                                     (1, (64, 128, 64, 10)), (16, (64, 128, 64, 16)), (70, (32, 256, 96, 40))])
def test_one_launch_chain_against_three_dense_launches(m, sizes):
    """mlp3 (the whole chain in one launch) against the three dense launches. The digits sizes
    run 16-row tiles on 16x16x4 MFMAs, whose k order differs from the dense GEMM's: both chains'
    logits lie within the float32 error bounds of the float64 chain, they agree to 2e-6 relative,
    and their predictions agree wherever the bounds certify the top logit. Other sizes run the
    dense GEMM's MFMA chains in its k order: the same logits and predictions bit for bit."""
    layers = digits.he_normal_mlp(seed=m + sizes[-1], sizes=sizes)
    layers = [(w, np.random.default_rng(i).normal(0, 0.1, b.shape).astype(np.float32)) for i, (w, b) in enumerate(layers)]
    n_classes = min(10, sizes[-1])
    mlp = digits.MLP(layers, max_batch=m, n_classes=n_classes)
    xh = np.random.default_rng(m).integers(0, 17, (m, sizes[0])).astype(np.float32)
    x = torch.from_numpy(xh).cuda()
    lf, pf = (t.clone() for t in mlp.run(x, fused=True))
    (launch,) = rt.last_launches()
    ll, pl = (t.clone() for t in mlp.run(x, fused=False))
    torch.cuda.synchronize()
    lf, ll, pf, pl = lf.cpu().numpy(), ll.cpu().numpy(), pf.cpu().numpy(), pl.cpu().numpy()
    assert launch["scratch_bytes"] == 0
    if sizes[:3] == (64, 128, 64):
        assert launch["kernel"].startswith("mlp3_rows16_kernel") and launch["grid"][0] == -(-m // 16), launch
        chain = [(w, b, i < 2) for i, (w, b) in enumerate(layers)]
        ref, bound = fp64.mlp_with_bounds(xh, chain, unit=2.0 ** -23)
        assert (np.abs(lf - ref) <= bound).all() and (np.abs(ll - ref) <= bound).all()
        assert fp64.rel_fro(lf, ll) <= 2e-6
        _, certified = fp64.certified_argmax(ref, 2 * bound, n_classes)
        np.testing.assert_array_equal(pf[certified], pl[certified])
        np.testing.assert_array_equal(pf, oracle.argmax_rows(lf, n_classes))
    else:
        assert launch["kernel"] == "mlp3_kernel", launch
        np.testing.assert_array_equal(lf, ll)
        np.testing.assert_array_equal(pf, pl)


def test_one_launch_chain_unaligned_input_takes_the_general_kernel():
    """Digits input rows that are not 16-byte aligned take the 32-row kernel, whose logits equal
    the dense launches' bit for bit."""
    layers = digits.he_normal_mlp(seed=5)
    mlp = digits.MLP(layers, max_batch=40)
    xh = np.random.default_rng(5).integers(0, 17, (40 * 64 + 1,)).astype(np.float32)
    x = torch.from_numpy(xh).cuda()[1:].view(40, 64)
    lf, pf = (t.clone() for t in mlp.run(x, fused=True))
    (launch,) = rt.last_launches()
    ll, pl = (t.clone() for t in mlp.run(x, fused=False))
    torch.cuda.synchronize()
    assert launch["kernel"] == "mlp3_kernel", launch
    np.testing.assert_array_equal(lf.cpu().numpy(), ll.cpu().numpy())
    np.testing.assert_array_equal(pf.cpu().numpy(), pl.cpu().numpy())


def test_one_launch_chain_refuses_unsupported_sizes():
    w = [torch.zeros(s, device="cuda") for s in ((64, 300), (300, 64), (64, 10))]
    x = torch.zeros((4, 64), device="cuda")
    with pytest.raises(rt.MI355XError):
        rt.mlp3(x, 4, w[0], None, w[1], None, w[2], None, torch.zeros((4, 10), device="cuda"), None, 10)


def test_argmax_rows_wide_rows_across_lanes():
    """Rows longer than a wave: ties between lanes go to the first index, the first NaN wins
    wherever it sits, an all -inf row gives 0, row strides are honoured."""
    rng = np.random.default_rng(9)
    rows, n, ld = 9, 1000, 1003
    x = rng.standard_normal((rows, ld)).astype(np.float32)
    x[1, 700] = x[1, 70] = 50.0            # tie across lanes and passes
    x[2, 999] = np.nan
    x[3, 5] = np.nan
    x[3, 900] = np.nan
    x[4, :] = -np.inf
    x[5, 64] = x[5, 128] = x[5, 1] = 99.0  # same lane, three passes
    x[6, n:] = 1e9                         # past n: never looked at
    tx = torch.from_numpy(x).cuda()
    out = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    rt.argmax_rows(tx, rows, ld, n, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), np.argmax(x[:, :n], axis=1))


def test_argmax_rows_ties_and_nan():
    x = np.array([[1, 3, 3, 0], [np.nan, 5, np.nan, 1], [2, 2, 2, 2], [-1, -5, np.inf, np.inf]], np.float32)
    tx = torch.from_numpy(x).cuda()
    out = torch.empty(4, dtype=torch.int32, device="cuda")
    rt.argmax_rows(tx, 4, 4, 4, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), np.argmax(x, axis=1))
