"""Grouped matmul (examples/kernels.py:18-57) on the MI355X against the oracle.

Bar: bit-exact on dyadic inputs (every product and partial sum exact, so any order gives the
same bits; tests/test_nn_kernels.py:37-61 style); otherwise relative Frobenius error <= 1e-5
vs float64 and no larger than the oracle's (the emulator's round-toward-zero chain)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from oracle import fp64
from piton_amd import cdiv
from piton_amd.kernels import matmul_kernel
from piton_amd.runtime import mi355x as rt

pytestmark = pytest.mark.gpu
TOL = 1e-5


def run(a, b, c=None, group=8, block=(64, 64, 16)):
    """matmul_kernel[grid] on torch tensors, with the reference's argument list."""
    M, K = a.shape
    N = b.shape[1]
    if c is None:
        c = torch.full((M, N), -1.0, device="cuda")
    grid = (cdiv(M, block[0]) * cdiv(N, block[1]),)
    matmul_kernel[grid](a, b, c, M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0),
                        c.stride(1), BLOCK_SIZE_M=block[0], BLOCK_SIZE_N=block[1], BLOCK_SIZE_K=block[2],
                        GROUP_SIZE_M=group, device="mi355x")
    torch.cuda.synchronize()
    return c


def dyadic(rng, shape):
    return (rng.integers(-4, 5, shape) / 4).astype(np.float32)


@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (72, 100, 64), (40, 70, 36), (16, 128, 32), (1, 1, 1),
                                   (129, 257, 33), (300, 129, 515)])
def test_dyadic_bit_exact(M, N, K):
    rng = np.random.default_rng(M * 1000 + N + K)
    a, b = dyadic(rng, (M, K)), dyadic(rng, (K, N))
    c = run(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()).cpu().numpy()
    np.testing.assert_array_equal(c, oracle.matmul(a, b))
    np.testing.assert_array_equal(c, a @ b)


@pytest.mark.parametrize("n", [512, 1024])
def test_square_uniform(n):
    rng = np.random.default_rng(n)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    c = run(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()).cpu().numpy()
    ref = fp64.matmul(a, b)
    emu = oracle.matmul_fast(a, b, threads=8)
    err, err_emu = fp64.rel_fro(c, ref), fp64.rel_fro(emu, ref)
    assert err <= TOL, err
    assert err <= err_emu, (err, err_emu)


def test_4096_sampled_rows():
    """At the benchmark size the float64 check runs on 64 sampled rows of C (the kernel
    computes them in tiles shared with every other row)."""
    n = 4096
    g = torch.Generator(device="cuda").manual_seed(7)
    a = torch.rand((n, n), device="cuda", generator=g) * 2 - 1
    b = torch.rand((n, n), device="cuda", generator=g) * 2 - 1
    c = run(a, b)
    rows = np.random.default_rng(1).choice(n, 64, replace=False)
    an, bn = a.cpu().numpy(), b.cpu().numpy()
    ref = fp64.matmul(an[rows], bn)
    got = c.cpu().numpy()[rows]
    emu = oracle.matmul_fast(an[rows], bn, threads=8)
    assert fp64.rel_fro(got, ref) <= TOL
    assert fp64.rel_fro(got, ref) <= fp64.rel_fro(emu, ref)


@pytest.mark.parametrize("layout", ["padded", "b_transposed", "a_transposed", "odd_strides"])
def test_ragged_runtime_strides(layout):
    """The ragged 1000 x 1800 x 700 case with runtime strides in four layouts: within 1e-5 of
    float64 and no further from it than the oracle on sampled rows; C's padding must stay
    untouched (a guard band: the masked store)."""
    M, N, K = 1000, 1800, 700
    rng = np.random.default_rng(5)
    a_np = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b_np = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    if layout == "padded":
        A = torch.zeros((M, K + 4), device="cuda"); A[:, :K] = torch.from_numpy(a_np)
        B = torch.zeros((K, N + 4), device="cuda"); B[:, :N] = torch.from_numpy(b_np)
        a, b = A[:, :K], B[:, :N]
    elif layout == "b_transposed":
        a = torch.from_numpy(a_np).cuda()
        b = torch.from_numpy(np.ascontiguousarray(b_np.T)).cuda().t()  # stride_bk = 1
    elif layout == "a_transposed":
        a = torch.from_numpy(np.ascontiguousarray(a_np.T)).cuda().t()  # stride_am = 1
        b = torch.from_numpy(b_np).cuda()
    else:  # lda = 703, ldb = 1805: rows not 16-byte aligned -> scalar loaders
        A = torch.zeros((M, K + 3), device="cuda"); A[:, :K] = torch.from_numpy(a_np)
        B = torch.zeros((K, N + 5), device="cuda"); B[:, :N] = torch.from_numpy(b_np)
        a, b = A[:, :K], B[:, :N]
    C = torch.full((M + 2, N + 7), -7.0, device="cuda")
    c = C[:M, :N]
    run(a, b, c)
    Cn = C.cpu().numpy()
    ref = fp64.matmul(a_np, b_np)
    assert fp64.rel_fro(Cn[:M, :N], ref) <= TOL
    assert (Cn[M:, :] == -7.0).all() and (Cn[:, N:] == -7.0).all()
    # no further from float64 than the oracle (the emulator's round-toward-zero chain) on 64
    # sampled rows, the first and last included
    rows = np.concatenate([[0, M - 1], np.random.default_rng(2).choice(np.arange(1, M - 1), 62, replace=False)])
    emu = oracle.matmul_fast(np.ascontiguousarray(a_np[rows]), b_np, threads=8)
    assert fp64.rel_fro(Cn[rows, :N], ref[rows]) <= fp64.rel_fro(emu, ref[rows])


def test_numpy_arrays_copy_in_copy_out():
    """numpy arguments: copied to the device and every array copied back (launcher.py:209-211)."""
    rng = np.random.default_rng(3)
    a, b = dyadic(rng, (40, 36)), dyadic(rng, (36, 70))
    c = np.full((40, 70), -1.0, np.float32)
    a0, b0 = a.copy(), b.copy()
    matmul_kernel[(cdiv(40, 8) * cdiv(70, 64),)](a, b, c, 40, 70, 36, 36, 1, 70, 1, 70, 1, BLOCK_SIZE_M=8,
                                                 BLOCK_SIZE_N=64, BLOCK_SIZE_K=4, GROUP_SIZE_M=4,
                                                 device="mi355x")
    np.testing.assert_array_equal(c, a @ b)
    np.testing.assert_array_equal(a, a0)
    np.testing.assert_array_equal(b, b0)


@pytest.mark.parametrize("M,N,K,pad", [(256, 384, 96, (4, 8, 3)), (128, 128, 32, (0, 0, 0)), (384, 128, 2080, (8, 4, 1)),
                                       (256, 384, 128, (4, 8, 3)), (128, 128, 64, (0, 0, 0)),
                                       (384, 256, 2112, (8, 4, 1))])
def test_whole_tile_shapes_with_padded_rows(M, N, K, pad):
    """Shapes whose tiles are all whole (M, N multiples of 128): the register-direct kernel for
    K % 64 == 0 with at least as many tiles as CUs (its last prefetch reloads the last K tile),
    the split kernel otherwise. Padded row strides of A, B and C (NaN in the padding) must not
    leak into the product or past C's rows."""
    rng = np.random.default_rng(M + N + K)
    a = dyadic(rng, (M, K))
    b = dyadic(rng, (K, N))
    A = torch.zeros((M, K + pad[0]), device="cuda")
    B = torch.zeros((K, N + pad[1]), device="cuda")
    C = torch.full((M, N + pad[2]), -7.0, device="cuda")
    A[:, :K] = torch.from_numpy(a).cuda()
    A[:, K:] = float("nan")
    B[:, :N] = torch.from_numpy(b).cuda()
    B[:, N:] = float("nan")
    run(A[:, :K], B[:, :N], C[:, :N])
    got = C.cpu().numpy()
    np.testing.assert_array_equal(got[:, :N], a @ b)
    assert (got[:, N:] == -7.0).all()


@pytest.mark.parametrize("group", [1, 3, 8, 64, 2 ** 31 - 1])
def test_group_order_does_not_change_bits(group):
    """Any GROUP_SIZE_M, up to the largest int32 (a group taller than the tile rows orders the
    tiles as one group of all of them), gives the same bits."""
    g = torch.Generator(device="cuda").manual_seed(11)
    a = torch.rand((700, 500), device="cuda", generator=g)
    b = torch.rand((500, 900), device="cuda", generator=g)
    base = run(a, b, group=8)
    other = run(a, b, group=group)
    assert torch.equal(base, other)


@pytest.mark.parametrize("group", [1, 3, 7, 64, 2 ** 31 - 1])
def test_group_order_across_generation_launches(group):
    """4096 x 4096 x 64 runs as two launches of 256 wide tiles whose logical ids continue from
    one launch to the next (tile0): any GROUP_SIZE_M orders the tiles differently across the
    launches and gives the same bits, every element written once (C prefilled with NaN)."""
    g = torch.Generator(device="cuda").manual_seed(13)
    a = torch.rand((4096, 64), device="cuda", generator=g)
    b = torch.rand((64, 4096), device="cuda", generator=g)

    def mm(group_m):
        c = torch.full((4096, 4096), float("nan"), device="cuda")
        rt.matmul(a, b, c, 4096, 4096, 64, 64, 1, 4096, 1, 4096, 1, group_m)
        torch.cuda.synchronize()
        return c

    base, other = mm(8), mm(group)
    assert not torch.isnan(other).any()
    assert torch.equal(base, other)


@pytest.mark.parametrize("group", [1, 3, 64, 2 ** 31 - 1])
def test_group_order_does_not_change_bits_whole_tiles(group):
    g = torch.Generator(device="cuda").manual_seed(12)
    a = torch.rand((640, 256), device="cuda", generator=g)
    b = torch.rand((256, 896), device="cuda", generator=g)
    assert torch.equal(run(a, b, group=8), run(a, b, group=group))


def _sweep_shape(rng, kind):
    if kind == 0:  # whole tiles, K % 64 == 0: the register-direct kernel
        return int(rng.integers(1, 5)) * 128, int(rng.integers(1, 5)) * 128, int(rng.integers(1, 11)) * 64
    if kind == 1:  # whole tiles, K % 32 == 0: the direct kernel or the LDS kernel's whole-tile form
        return int(rng.integers(1, 5)) * 128, int(rng.integers(1, 5)) * 128, int(rng.integers(1, 21)) * 32
    return tuple(int(rng.integers(1, 400)) for _ in range(3))  # ragged edges


def test_seeded_large_whole_tile_sweep():
    """16 seeded whole-tile shapes past one generation of tiles (the register-direct kernel in
    one launch per generation, 128 x 128 or 128 x 256 tiles), each operand row- or column-major
    with padded strides, random GROUP_SIZE_M: 48 sampled rows of every C within the float32
    bound of the float64 product, and C's padding columns untouched."""
    rng = np.random.default_rng(2027)
    for case in range(16):
        M, N = (int(rng.integers(8, 33)) * 128 for _ in range(2))
        K = int(rng.integers(1, 9)) * 64
        a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
        b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
        lay = int(rng.integers(0, 4))
        pad = int(rng.integers(0, 3)) * 4
        A, B = _nan_padded(a, lay & 1, pad), _nan_padded(b, lay & 2, pad)
        C = torch.full((M, N + 4), -7.0, device="cuda")
        group = int(rng.choice([1, 3, 8, 2 ** 31 - 1]))
        rt.matmul(A, B, C, M, N, K, A.stride(0), A.stride(1), B.stride(0), B.stride(1), N + 4, 1, group)
        kernel = rt.last_launches()[0]["kernel"]
        torch.cuda.synchronize()
        rows = rng.choice(M, 48, replace=False)
        got = C[torch.from_numpy(rows).cuda()].cpu().numpy()
        ref = fp64.matmul(a[rows], b)
        bound = (K + 2) * 2.0 ** -24 * (np.abs(a[rows]).astype(np.float64) @ np.abs(b).astype(np.float64))
        assert not (np.abs(got[:, :N] - ref) > bound).any(), (case, M, N, K, lay, pad, group, kernel)
        assert (got[:, N:] == -7.0).all(), (case, kernel)


def test_seeded_shape_sweep_against_float64():
    """48 seeded shapes and layouts in one process (whole tiles for the register-direct and the
    LDS kernels, ragged edges, padded rows, A or B stored transposed); every element within the
    worst-case bound of a float32 contraction in any order, |C - C64| <= (K + 2) u sum_k |A||B|,
    u = 2^-24."""
    rng = np.random.default_rng(2026)
    for case in range(48):
        kind = case % 4
        M, N, K = _sweep_shape(rng, kind)
        a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
        b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
        pad_a = int(rng.integers(0, 3)) * 4 if kind < 2 else int(rng.integers(0, 5))
        pad_b = int(rng.integers(0, 3)) * 4 if kind < 2 else int(rng.integers(0, 5))
        if kind == 3 and case % 8 == 3:  # A stored transposed: element (m, k) at k * M + m
            A = torch.from_numpy(np.ascontiguousarray(a.T)).cuda().t()
        else:
            A = torch.zeros((M, K + pad_a), device="cuda")
            A[:, :K] = torch.from_numpy(a).cuda()
            A = A[:, :K]
        if kind == 3 and case % 8 == 7:  # B stored transposed
            B = torch.from_numpy(np.ascontiguousarray(b.T)).cuda().t()
        else:
            B = torch.zeros((K, N + pad_b), device="cuda")
            B[:, :N] = torch.from_numpy(b).cuda()
            B = B[:, :N]
        got = run(A, B).cpu().numpy()
        ref = fp64.matmul(a, b)
        bound = (K + 2) * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
        bad = np.abs(got - ref) > bound
        assert not bad.any(), (case, M, N, K, pad_a, pad_b, int(bad.sum()))


LAYOUTS = ["row-major", "A transposed", "B transposed", "both transposed"]


def _stored(x, transposed):
    """x (rows x cols) on the GPU, row-major or stored transposed (element (r, c) at c * rows + r)."""
    if transposed:
        return torch.from_numpy(np.ascontiguousarray(x.T)).cuda().t()
    return torch.from_numpy(x).cuda()


@pytest.mark.parametrize("M,N,K,family", [(256, 384, 192, "gemm_split_kernel"),
                                          (2048, 4096, 128, "gemm_direct_kernel")])
def test_every_layout_gives_the_same_bits(M, N, K, family):
    """Row- or column-major A and B: the register-direct kernel (whole 128 x 128 tiles, K % 64 ==
    0, at least as many tiles as CUs) and the split kernel (fewer tiles) take every layout, and
    each lane supplies the same k at each MFMA step whichever operand is contiguous, so all four
    layouts give identical bits, within the float32 bound of the float64 product."""
    rng = np.random.default_rng(M + N + K)
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    ref = fp64.matmul(a, b)
    bound = (K + 2) * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    out = {}
    for i, name in enumerate(LAYOUTS):
        A, B = _stored(a, i & 1), _stored(b, i & 2)
        C = torch.full((M, N), -1.0, device="cuda")
        rt.matmul(A, B, C, M, N, K, A.stride(0), A.stride(1), B.stride(0), B.stride(1), N, 1)
        kernel = rt.last_launches()[0]["kernel"]
        torch.cuda.synchronize()
        out[name] = C.cpu().numpy()
        assert kernel.startswith(family), (name, kernel)
        assert not (np.abs(out[name] - ref) > bound).any(), name
    for name in LAYOUTS[1:]:
        np.testing.assert_array_equal(out[name], out[LAYOUTS[0]], err_msg=name)


@pytest.mark.parametrize("b_transposed", [False, True])
def test_generations_run_as_separate_launches(b_transposed):
    """4096 x 4096 C on 256 CUs runs as two launches of 256 tiles of 128 x 256, one per CU each;
    C from A's first 3072 rows as three launches of 256 tiles of 128 x 128 (384 wide tiles would
    take two launches, the second half empty); C from its last 1024 rows as one launch of 256
    tiles of 128 x 128. Each row tile of C depends on its rows of A alone and each element's k
    order is the same in every form, so C equals the two parts stacked, bit for bit."""
    M = N = 4096
    K = 128
    g = torch.Generator(device="cuda").manual_seed(21)
    A = torch.rand((M, K), device="cuda", generator=g) * 2 - 1
    Bs = torch.rand((N, K) if b_transposed else (K, N), device="cuda", generator=g) * 2 - 1
    s_bk, s_bn = (1, K) if b_transposed else (N, 1)

    def mm(a):
        c = torch.full((a.shape[0], N), -1.0, device="cuda")
        rt.matmul(a, Bs, c, a.shape[0], N, K, K, 1, s_bk, s_bn, N, 1, 8)
        launches = [(l["kernel"], l["grid"][0]) for l in rt.last_launches()]
        torch.cuda.synchronize()
        return c, launches

    c, launches = mm(A)
    top, l_top = mm(A[:3072])
    bottom, l_bottom = mm(A[3072:])
    if rt.device_info()["cu_count"] == 256:
        assert [grid for _, grid in launches] == [256] * 2, launches
        assert all(k.startswith("gemm_direct_kernel<true,") and k.endswith("DNB_WIDE>") for k, _ in launches)
        assert [grid for _, grid in l_top] == [256] * 3 and [grid for _, grid in l_bottom] == [256]
        assert all(k.endswith(", DNB>") for k, _ in l_top + l_bottom), (l_top, l_bottom)
    assert torch.equal(c, torch.cat([top, bottom]))
    rows = np.random.default_rng(2).choice(M, 48, replace=False)
    a_np = A.cpu().numpy()[rows]
    b_np = (Bs.t() if b_transposed else Bs).cpu().numpy()
    ref = fp64.matmul(a_np, b_np)
    bound = (K + 2) * 2.0 ** -24 * (np.abs(a_np).astype(np.float64) @ np.abs(b_np).astype(np.float64))
    assert not (np.abs(c.cpu().numpy()[rows] - ref) > bound).any()


@pytest.mark.parametrize("M", [2048, 1024])
def test_dense_and_linear_epilogues_in_generation_launches(M):
    """The bias, ReLU and residual epilogue in the register-direct kernel's one-launch-per-
    generation forms: 2048 x 4096 (512 tiles of 128 x 128, so one launch of 256 wide tiles) and
    1024 x 4096 (256 tiles, one launch of 128 x 128 tiles). Dyadic inputs: every product and sum
    is exact, so the result equals numpy's bit for bit."""
    N, K = 4096, 64
    rng = np.random.default_rng(M + 5)
    a, b, bias = dyadic(rng, (M, K)), dyadic(rng, (K, N)), dyadic(rng, (N,))
    res = dyadic(rng, (M, N))
    x, w, tb, tr = (torch.from_numpy(v).cuda() for v in (a, b, bias, res))
    y = torch.full((M, N), -7.0, device="cuda")
    rt.dense(x, w, tb, y, M, N, K, add_bias=True, relu=True)
    dense_launches = [(l["kernel"], l["grid"][0]) for l in rt.last_launches()]
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), np.maximum(a @ b + bias, 0))
    y.fill_(-7.0)
    rt.linear(x, K, w, tb, tr, N, y, N, M, N, K, relu=False)
    linear_launches = [(l["kernel"], l["grid"][0]) for l in rt.last_launches()]
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), a @ b + bias + res)
    if rt.device_info()["cu_count"] == 256:
        for launches in (dense_launches, linear_launches):
            assert len(launches) == 1 and launches[0][1] == 256, launches
            assert launches[0][0].startswith("gemm_direct_kernel<true,"), launches
            assert launches[0][0].endswith("DNB_WIDE>" if M == 2048 else ", DNB>"), launches


def _nan_padded(x, transposed, pad):
    """x (rows x cols) on the GPU in storage whose padding holds NaN: row-major with rows of
    cols + pad floats, or stored transposed with columns of rows + pad floats."""
    r, c = x.shape
    if transposed:
        full = torch.full((c, r + pad), float("nan"), device="cuda")
        full[:, :r] = torch.from_numpy(np.ascontiguousarray(x.T)).cuda()
        return full[:, :r].t()
    full = torch.full((r, c + pad), float("nan"), device="cuda")
    full[:, :c] = torch.from_numpy(x).cuda()
    return full[:, :c]


@pytest.mark.parametrize("M,N,K", [(1000, 1800, 700), (100, 72, 36), (129, 257, 516), (256, 256, 64)])
def test_split_kernel_layouts_with_nan_padding(M, N, K):
    """Shapes that give the direct kernel too few tiles, or ragged edges, take the split kernel in
    every layout of A and B; the K tail (k >= K inside the last tile of 32) reads as zero, so
    NaN in the storage's padding, which a tail load of an unmasked operand would read, never
    reaches C. Every element within the float32 bound of the float64 product."""
    rng = np.random.default_rng(M * 7 + N + K)
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    ref = fp64.matmul(a, b)
    bound = (K + 2) * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    for i, name in enumerate(LAYOUTS):
        for pad in (0, 4, 3):
            if pad == 3 and i & 2:
                continue  # a column-major B is loaded in 16-byte chunks: columns 16-byte aligned
            A, B = _nan_padded(a, i & 1, pad), _nan_padded(b, i & 2, pad)
            C = torch.full((M, N), -1.0, device="cuda")
            rt.matmul(A, B, C, M, N, K, A.stride(0), A.stride(1), B.stride(0), B.stride(1), N, 1)
            kernel = rt.last_launches()[0]["kernel"]
            torch.cuda.synchronize()
            got = C.cpu().numpy()
            assert kernel.startswith("gemm_split_kernel"), (name, pad, kernel)
            assert np.isfinite(got).all(), (name, pad, kernel)
            assert not (np.abs(got - ref) > bound).any(), (name, pad, kernel)


@pytest.mark.parametrize("K", [128, 96])
def test_negative_row_stride_through_the_c_abi(K):
    """The C entry takes any strides: A addressed from its last row with row stride -K (a
    row-reversed view) on a whole-tile shape gives the product of the reversed rows."""
    M, N = 256, 256
    rng = np.random.default_rng(K)
    a = dyadic(rng, (M, K))
    b = dyadic(rng, (K, N))
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    tc = torch.full((M, N), -1.0, device="cuda")
    last_row = ctypes.c_void_p(ta.data_ptr() + (M - 1) * K * 4)
    rt._call("piton_mi355x_matmul", last_row, rt._ptr(tb), rt._ptr(tc), M, N, K, -K, 1, N, 1, N, 1, 8, rt._stream())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(tc.cpu().numpy(), a[::-1] @ b)


def test_empty_and_k_zero():
    a = torch.zeros((5, 0), device="cuda")
    b = torch.zeros((0, 7), device="cuda")
    c = torch.full((5, 7), 3.0, device="cuda")
    rt.matmul(a, b, c, 5, 7, 0, 0, 1, 7, 1, 7, 1)
    torch.cuda.synchronize()
    assert (c == 0).all()
    rt.matmul(a, b, c, 0, 7, 0, 0, 1, 7, 1, 7, 1)  # nothing to do


def test_out_of_storage_strides_are_rejected():
    a = torch.zeros((8, 8), device="cuda")
    with pytest.raises(ValueError):
        rt.matmul(a, a, a, 8, 8, 9, 8, 1, 8, 1, 8, 1)


# shapes that give the register-direct kernel fewer 128 x 128 tiles than CUs, or ragged edges:
# the split kernel (64 x 64 or 32 x 32 workgroup tiles, waves splitting K)
# (1000, 1800, 700), (1024, 2048, 256), (900, 1500, 260) and (2048, 768, 256) take the wide 64 x 128 tile
# (A row-major, B row-major)
SPLIT_SHAPES = [(512, 512, 512, 0, 0), (1024, 1024, 1024, 0, 0), (1000, 1800, 700, 3, 5), (1000, 1800, 700, 4, 8),
                (130, 70, 33, 0, 0), (2048, 768, 256, 0, 0), (77, 300, 1, 0, 0), (300, 1, 5000, 0, 0),
                (257, 129, 97, 1, 2), (1024, 2048, 256, 0, 0), (900, 1500, 260, 4, 3)]


@pytest.mark.parametrize("M,N,K,pad_a,pad_b", SPLIT_SHAPES)
def test_split_kernel_dyadic_with_nan_padding(M, N, K, pad_a, pad_b):
    """Dyadic inputs (every product and sum exact: any order gives the same bits) with NaN in
    the row padding of A and B: the K tail of A and the columns of B past N never reach a
    stored element, and C's padding (a guard band) stays untouched."""
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    a, b = dyadic(rng, (M, K)), dyadic(rng, (K, N))
    A = torch.full((M, K + pad_a), float("nan"), device="cuda")
    B = torch.full((K, N + pad_b), float("nan"), device="cuda")
    A[:, :K] = torch.from_numpy(a).cuda()
    B[:, :N] = torch.from_numpy(b).cuda()
    C = torch.full((M + 1, N + 3), -7.0, device="cuda")
    rt.matmul(A, B, C, M, N, K, K + pad_a, 1, N + pad_b, 1, N + 3, 1, 8)
    (launch,) = rt.last_launches()
    torch.cuda.synchronize()
    got = C.cpu().numpy()
    np.testing.assert_array_equal(got[:M, :N], a @ b)
    assert (got[M:] == -7.0).all() and (got[:, N:] == -7.0).all()
    assert launch["kernel"].startswith("gemm_split_kernel"), launch
    wide = (M, N, K) in ((1000, 1800, 700), (1024, 2048, 256), (900, 1500, 260), (2048, 768, 256))
    assert launch["kernel"].startswith("gemm_split_kernel<2, 4, 4,") == wide, launch
    assert launch["block"][0] in (64, 128, 256) and launch["scratch_bytes"] == 0


@pytest.mark.parametrize("M,N,K,pad_a,pad_b", SPLIT_SHAPES[:4])
def test_split_kernel_uniform_against_float64_and_oracle(M, N, K, pad_a, pad_b):
    rng = np.random.default_rng(K)
    a = rng.uniform(-1, 1, (M, K + pad_a)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N + pad_b)).astype(np.float32)
    C = torch.empty((M, N), device="cuda")
    rt.matmul(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), C, M, N, K, K + pad_a, 1, N + pad_b, 1, N, 1, 8)
    got = C.cpu().numpy()
    ref = fp64.matmul(a[:, :K], b[:, :N])
    assert fp64.rel_fro(got, ref) <= TOL
    rows = np.random.default_rng(0).choice(M, 64, replace=False)
    emu = oracle.matmul_fast(np.ascontiguousarray(a[rows, :K]), np.ascontiguousarray(b[:, :N]), threads=8)
    assert fp64.rel_fro(got[rows], ref[rows]) <= fp64.rel_fro(emu, ref[rows])


@pytest.mark.parametrize("ldb,split", [(64, False), (96, True)])
def test_row_major_b_with_overlapping_rows(ldb, split):
    """B row-major with rows closer together than N floats (a strided view whose rows overlap):
    the split kernel relies on B's rows past K lying past the end of B for its K tail, which
    overlapping rows break, so such a B takes the LDS kernel and its masks; rows N apart keep
    the split kernel. Either way within the float32 bound of float64 over the view's values."""
    M, N, K = 200, 96, 100  # K % 32 != 0: a partial last K tile
    rng = np.random.default_rng(ldb)
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    store = rng.uniform(-1, 1, (K - 1) * ldb + N).astype(np.float32)
    b = np.lib.stride_tricks.as_strided(store, (K, N), (4 * ldb, 4))
    ref = fp64.matmul(a, np.ascontiguousarray(b))
    bound = (K + 2) * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    A, B = torch.from_numpy(a).cuda(), torch.from_numpy(store).cuda()
    C = torch.full((M, N), -1.0, device="cuda")
    rt.matmul(A, B, C, M, N, K, K, 1, ldb, 1, N, 1, 8)
    (launch,) = rt.last_launches()
    torch.cuda.synchronize()
    assert launch["kernel"].startswith("gemm_split_kernel") == split, launch
    assert not (np.abs(C.cpu().numpy() - ref) > bound).any()


def test_split_kernel_group_order_and_repeatability():
    g = torch.Generator(device="cuda").manual_seed(21)
    a = torch.rand((1000, 700), device="cuda", generator=g)
    b = torch.rand((700, 1800), device="cuda", generator=g)
    base = run(a, b, group=8)
    for group in (1, 5, 2 ** 31 - 1, 8):
        assert torch.equal(run(a, b, group=group), base)


@pytest.mark.parametrize("a_off,lda", [(1, 700), (2, 703), (3, 701), (1, 64)])
def test_split_kernel_unaligned_base_and_rows(a_off, lda):
    """A starting 1-3 floats past a 16-byte boundary, rows of any length: each lane reads the
    aligned 16-byte chunks around its values and selects them in registers; dyadic inputs give
    numpy's bits, with NaN before A, between its rows and after it."""
    M, N, K = 333, 200, min(lda, 77 if lda == 64 else 650)
    rng = np.random.default_rng(a_off * 1000 + lda)
    a, b = dyadic(rng, (M, K)), dyadic(rng, (K, N))
    store = torch.full((a_off + M * lda + 8,), float("nan"), device="cuda")
    A = store[a_off:a_off + M * lda].view(M, lda)
    A[:, :K] = torch.from_numpy(a).cuda()
    B = torch.from_numpy(b).cuda()
    C = torch.full((M, N), -7.0, device="cuda")
    rt.matmul(A, B, C, M, N, K, lda, 1, N, 1, N, 1, 8)
    (launch,) = rt.last_launches()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(C.cpu().numpy(), a @ b)
    assert launch["kernel"].startswith("gemm_split_kernel<") and ", A_ROW, false, " in launch["kernel"], launch
