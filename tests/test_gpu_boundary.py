"""The drop-in boundary on the MI355X: launches made the way the reference's launcher makes them
once INTEGRATION.md's mi355x branch is in place (a JIT object with only the reference's
attributes, the reference's `bind`, the branch before compile()), with numpy arrays (copied in
and out) and device tensors, checked against the oracle; and the per-launch statistics."""
import numpy as np
import pytest
import torch

import oracle
from oracle import fp64
from piton_amd import cdiv
from ref_launch import RefJIT, patched_reference_call, ref_add_kernel, ref_matmul_kernel, ref_softmax_kernel

pytestmark = pytest.mark.gpu


def test_matmul_numpy_through_the_reference_call():
    rng = np.random.default_rng(1)
    M, N, K = 130, 70, 36
    a = (rng.integers(-4, 5, (M, K)) / 4).astype(np.float32)
    b = (rng.integers(-4, 5, (K, N)) / 4).astype(np.float32)
    c = np.full((M, N), -1.0, np.float32)
    rec = patched_reference_call(RefJIT(ref_matmul_kernel), (cdiv(M, 8) * cdiv(N, 64),), a, b, c, M, N, K, K, 1, N,
                                 1, N, 1, BLOCK_SIZE_M=8, BLOCK_SIZE_N=64, BLOCK_SIZE_K=8, GROUP_SIZE_M=8)
    np.testing.assert_array_equal(c, oracle.matmul(a, b))
    (launch,) = rec.last_stats["launches"]
    # a product this small takes the split kernel: 32 x 32 tiles, waves splitting K
    assert launch["kernel"].startswith("gemm_split_kernel") and launch["grid"][0] == cdiv(M, 32) * cdiv(N, 32)
    assert launch["block"][0] in (64, 128, 256) and launch["vgprs"] > 0 and launch["scratch_bytes"] == 0
    assert rec.last_stats["flops"] == 2 * M * N * K


def test_matmul_tensors_whole_tiles_take_the_direct_kernel(monkeypatch):
    """2048^3 has as many 128 x 128 tiles as the chip has CUs: the register-direct kernel."""
    monkeypatch.setenv("PITON_MI355X_TIMING", "1")
    g = torch.Generator(device="cuda").manual_seed(3)
    n = 2048
    a = torch.rand((n, n), device="cuda", generator=g)
    b = torch.rand((n, n), device="cuda", generator=g)
    c = torch.empty((n, n), device="cuda")
    rec = patched_reference_call(RefJIT(ref_matmul_kernel), (cdiv(n, 128) ** 2,), a, b, c, n, n, n, n, 1, n, 1, n,
                                 1, BLOCK_SIZE_M=128, BLOCK_SIZE_N=128, BLOCK_SIZE_K=32, GROUP_SIZE_M=8)
    torch.cuda.synchronize()
    assert rec.last_stats["launches"][0]["kernel"].startswith("gemm_direct_kernel")
    assert rec.last_stats["elapsed_us"] > 0
    ref = fp64.matmul(a.cpu().numpy(), b.cpu().numpy())
    assert fp64.rel_fro(c.cpu().numpy(), ref) <= 1e-5


def test_softmax_and_add_through_the_reference_call():
    rng = np.random.default_rng(2)
    rows, n = 33, 1823
    x = (rng.standard_normal((rows, n)) * 4).astype(np.float32)
    y = np.full((rows, n), 9.0, np.float32)
    patched_reference_call(RefJIT(ref_softmax_kernel), (rows,), y, x, n, n, n, BLOCK_SIZE=2048)
    err = fp64.rel_fro(y, fp64.softmax(x))
    assert err <= 1e-5 and err <= fp64.rel_fro(oracle.softmax(x, n, 2048), fp64.softmax(x))
    tx = torch.from_numpy(x.ravel()).cuda()
    out = torch.full((rows * n + 16,), 7.0, device="cuda")
    rec = patched_reference_call(RefJIT(ref_add_kernel), lambda m: (cdiv(rows * n, m["BLOCK_SIZE"]),), tx, tx, out,
                                 rows * n, BLOCK_SIZE=1024)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got[:rows * n], x.ravel() + x.ravel())
    assert (got[rows * n:] == 7.0).all()
    assert [l["kernel"] for l in rec.last_stats["launches"]] == ["add_vec4_kernel", "add_scalar_kernel"]
