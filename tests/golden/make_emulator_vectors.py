"""Golden vectors of the reference's QPU emulator, for pinning the oracle bit for bit.

Imports the reference from /root/reference (run only where that checkout exists; nothing here
is imported by the tests, and only the vectors are committed), runs small kernels on its strict
emulator and writes their inputs and outputs to tests/golden/emulator/*.npz:

    python tests/golden/make_emulator_vectors.py

  math.npz      exp, exp2, x / y, 1 / y, x / s (s uniform), rsqrt, sqrt over seeded values and
                special values, one op per kernel (the way tests/test_tiles.py:158-228 builds
                its accuracy kernels)
  softmax.npz   softmax_kernel (examples/kernels.py:60-76) rows, including +inf, all -inf,
                -inf entries and NaN rows
  matmul.npz    matmul_kernel (examples/kernels.py:18-57) at 64^3 and ragged 40 x 70 x 36
  attention.npz attn_fwd_kernel (examples/attention.py:67-113) through run_attention
                (examples/attention.py:200-222), causal and not
  mlp.npz       dense_layer_kernel (examples/nn_kernels.py:23-74) three times with the
                launch of tests/test_nn_kernels.py:14-34, on the digits MLP (He-normal weights from
                seed 1729, raw 0..16 pixels) for the first 96 test images, every layer's output
  mlp_full.npz  the same chain's logits and predictions for all 1,797 test images
                (`--full-mlp`, about half an hour of emulation)
  layernorm.npz row layernorm (the kernel of tests/test_reroll_reduce.py:199-208) at BLOCK 256
                and 128, and add_kernel's x + y (`--layernorm`)
  softmax_specials.npz  softmax_kernel (BLOCK 256) over rows of special values: NaN, -NaN,
                +inf, -inf, -0, +0 and denormals in the first register, alone and mixed with
                N(0, 1) entries (the pattern of tests/test_reroll_reduce.py:157-174, plus rows
                with only a -NaN entry) (`--softmax-specials`)
  softmax_long.npz  softmax_kernel rows at BLOCK_SIZE 1024 and 2048 (n_cols 1000, 1023, 1823),
                which compile only with the reduction reroll of piton/reroll.py switched on
                (PITON_REROLL_REDUCE=1, the build of tests/test_reroll_reduce.py:37-44)
                (`--softmax-long`)

The kernels below are written for this script in the reference's language; no reference source
is copied anywhere.
"""
from __future__ import annotations

import os
import sys
import time

import numpy as np

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "emulator")
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))  # this repository (seeded weights)
sys.path.insert(0, os.path.join(REF, "examples"))
sys.path.insert(0, REF)

import piton  # noqa: E402
import piton.compiler as pc  # noqa: E402
import piton.language as tl  # noqa: E402
from piton.runtime.launcher import run_emulator  # noqa: E402


@piton.jit
def unary_k(x_ptr, o_ptr, n, F: tl.constexpr, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    x = tl.load(x_ptr + offs, mask=m, other=1.0)
    if F == 0:
        y = tl.exp(x)
    elif F == 1:
        y = tl.exp2(x)
    elif F == 2:
        y = tl.rsqrt(x)
    elif F == 3:
        y = tl.sqrt(x)
    else:
        y = 1.0 / x
    tl.store(o_ptr + offs, y, mask=m)


@piton.jit
def div_k(x_ptr, y_ptr, o_ptr, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    x = tl.load(x_ptr + offs, mask=m, other=1.0)
    y = tl.load(y_ptr + offs, mask=m, other=1.0)
    tl.store(o_ptr + offs, x / y, mask=m)


@piton.jit
def div_uniform_k(x_ptr, o_ptr, n, s, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    x = tl.load(x_ptr + offs, mask=m, other=1.0)
    tl.store(o_ptr + offs, x / s, mask=m)


@piton.jit
def rownorm_k(x_ptr, out_ptr, n, eps, BLOCK: tl.constexpr):
    row = tl.program_id(0)
    cols = tl.arange(0, BLOCK)
    live = cols < n
    v = tl.load(x_ptr + row * BLOCK + cols, mask=live, other=0.0)
    mu = tl.sum(v, axis=0) / n
    c = tl.where(live, v - mu, 0.0)
    s2 = tl.sum(c * c, axis=0) / n
    tl.store(out_ptr + row * BLOCK + cols, c / tl.sqrt(s2 + eps), mask=live)


@piton.jit
def add_k(x_ptr, y_ptr, o_ptr, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    tl.store(o_ptr + offs, tl.load(x_ptr + offs, mask=m) + tl.load(y_ptr + offs, mask=m), mask=m)


SPECIALS = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0, 2.0, 0.5, 4.0, 9.0, 88.7, 88.73, -87.3,
                     -87.4, -103.9, -150.0, 127.9, 128.0, 1e30, -1e30, 3.4e38, 1.17549435e-38, 1.2e-38, 2.0 ** 127,
                     1e-45, -1e-45], np.float32)


def math_vectors(rng):
    out = {}
    x = np.concatenate([rng.uniform(-87, 88, 1000), rng.uniform(-30, 30, 1000)]).astype(np.float32)
    x = np.concatenate([x, SPECIALS])
    for f, name, inp in ((0, "exp", x), (1, "exp2", np.concatenate([rng.uniform(-125, 127, 1000).astype(np.float32),
                                                                          SPECIALS])),
                         (2, "rsqrt", np.concatenate([np.exp(rng.uniform(-80, 80, 1500)).astype(np.float32),
                                                      SPECIALS])),
                         (3, "sqrt", np.concatenate([np.exp(rng.uniform(-80, 80, 1500)).astype(np.float32),
                                                     SPECIALS])),
                         (4, "recip", np.concatenate([(np.exp(rng.uniform(-80, 80, 1500)) *
                                                       rng.choice([-1, 1], 1500)).astype(np.float32), SPECIALS]))):
        o = np.zeros_like(inp)
        unary_k[(piton.cdiv(len(inp), 128),)](inp, o, len(inp), F=f, BLOCK=128)
        out[f"{name}_x"], out[f"{name}_y"] = inp, o
    y = np.concatenate([(np.exp(rng.uniform(-80, 80, 1500)) * rng.choice([-1, 1], 1500)).astype(np.float32), SPECIALS])
    xn = np.concatenate([rng.standard_normal(1500).astype(np.float32), rng.permutation(SPECIALS)])
    o = np.zeros_like(y)
    div_k[(piton.cdiv(len(y), 128),)](xn, y, o, len(y), BLOCK=128)
    out["fdiv_x"], out["fdiv_y"], out["fdiv_out"] = xn, y, o
    for j, s in enumerate((3.0, -0.7, 1e-20, 6.5e35)):
        o = np.zeros_like(xn)
        div_uniform_k[(piton.cdiv(len(xn), 128),)](xn, o, len(xn), float(s), BLOCK=128)
        out[f"fdiv_uniform_s{j}"], out[f"fdiv_uniform_out{j}"] = np.float32(s), o
    out["fdiv_uniform_x"] = xn
    return out


def softmax_vectors(rng):
    import kernels as K
    out = {}
    cases = [(4, 64, 64), (3, 100, 128), (5, 16, 16), (2, 200, 256)]
    for i, (rows, cols, block) in enumerate(cases):
        stride = cols + 3
        x = (rng.standard_normal((rows, stride)) * 4).astype(np.float32)
        if i == 0:
            x[1, 5] = np.inf
            x[2, :] = -np.inf
            x[3, 7] = -np.inf
            x[3, 9] = -np.inf
        if i == 1:
            x[1, 50] = np.nan
        y = np.full((rows, stride), np.float32(-7.0))
        K.softmax_kernel[(rows,)](y, x, stride, stride, cols, BLOCK_SIZE=block)
        out[f"case{i}_x"], out[f"case{i}_y"] = x, y
        out[f"case{i}_shape"] = np.array([rows, cols, block, stride], np.int64)
    out["n_cases"] = np.int64(len(cases))
    return out


def matmul_vectors(rng):
    import kernels as K
    from piton.runtime.launcher import Launcher
    out = {}
    for i, (M, N, Kd) in enumerate([(64, 64, 64), (40, 70, 36)]):
        a = rng.uniform(-1, 1, (M, Kd)).astype(np.float32)
        b = rng.uniform(-1, 1, (Kd, N)).astype(np.float32)
        c = np.full((M, N), -1.0, np.float32)
        grid = (piton.cdiv(M, 8) * piton.cdiv(N, 64),)
        Launcher(K.matmul_kernel, grid, {})(a, b, c, M, N, Kd, Kd, 1, N, 1, N, 1, BLOCK_SIZE_M=8, BLOCK_SIZE_N=64,
                                            BLOCK_SIZE_K=4, GROUP_SIZE_M=4)
        out[f"case{i}_a"], out[f"case{i}_b"], out[f"case{i}_c"] = a, b, c
    out["n_cases"] = np.int64(2)
    return out


def attention_vectors(rng):
    import attention as A
    out = {}
    cases = [(2, 64, 16, True), (1, 48, 32, False), (2, 40, 16, True)]
    for i, (H, N, D, causal) in enumerate(cases):
        q, k, v = (rng.standard_normal((H, N, D)).astype(np.float32) for _ in range(3))
        o, _, _ = A.run_attention(q, k, v, causal=causal, block_m=2, block_n=16)
        out[f"case{i}_q"], out[f"case{i}_k"], out[f"case{i}_v"], out[f"case{i}_o"] = q, k, v, o
        out[f"case{i}_causal"] = np.int64(causal)
    out["n_cases"] = np.int64(len(cases))
    return out


def dense_emulator(x, w, bias, relu):
    from nn_kernels import dense_layer_kernel, dense_tiles
    m, k = x.shape
    n = w.shape[1]
    bm, bn, bk = dense_tiles(n)
    grid = ((m + bm - 1) // bm * ((n + bn - 1) // bn),)
    constants = dict(N=n, K=k, BLOCK_SIZE_M=bm, BLOCK_SIZE_N=bn, BLOCK_SIZE_K=bk, GROUP_SIZE_M=1, ADD_BIAS=True,
                     RELU=relu)
    signature = dict.fromkeys(("x_ptr", "w_ptr", "bias_ptr", "y_ptr"), "*fp32")
    signature["M"] = "i32"
    compiled = pc.compile(dense_layer_kernel, signature, constants, grid=grid, num_stages=2)
    y = np.full(m * n, np.float32(-1234.5), np.float32)
    run_emulator(compiled, grid, dict(x_ptr=np.ascontiguousarray(x), w_ptr=w, bias_ptr=bias, y_ptr=y, M=m),
                 strict=True)
    return y.reshape(m, n)


def mlp_vectors():
    from piton_amd import digits
    data = np.load(os.path.join(HERE, "digits", "dataset.npz"))
    x = data["test_images"][:96].astype(np.float32)
    layers = digits.he_normal_mlp(seed=1729)
    h = x
    out = {"x": x}
    for i, (w, b) in enumerate(layers):
        h = dense_emulator(h, w, b, relu=i < 2)
        out[f"h{i + 1}"] = h
    out["pred"] = np.argmax(h[:, :10], axis=1).astype(np.int32)
    return out


def mlp_full_vectors():
    from piton_amd import digits
    x = np.load(os.path.join(HERE, "digits", "dataset.npz"))["test_images"].astype(np.float32)
    h = x
    for i, (w, b) in enumerate(digits.he_normal_mlp(seed=1729)):
        h = dense_emulator(h, w, b, relu=i < 2)
    return {"logits": h, "pred": np.argmax(h[:, :10], axis=1).astype(np.int32)}


def softmax_long_vectors(rng):
    from kernels import softmax_kernel
    os.environ["PITON_REROLL_REDUCE"] = "1"
    sig = {"output_ptr": "*fp32", "input_ptr": "*fp32", "input_row_stride": "i32", "output_row_stride": "i32",
           "n_cols": "i32"}
    out = {}
    cases = [(2, 1000, 1024), (2, 1023, 1024), (2, 1823, 2048)]
    done = 0
    for rows, cols, block in cases:
        try:
            ck = pc.compile(softmax_kernel, sig, {"BLOCK_SIZE": block}, grid=(rows,))
        except Exception as e:  # a build the reference cannot make is recorded, not faked
            print(f"softmax BLOCK {block} n_cols {cols}: no build ({type(e).__name__}: {e})", flush=True)
            continue
        x = (rng.standard_normal((rows, cols)) * 4).astype(np.float32)
        y = np.full(rows * cols, np.float32(-7.0))
        run_emulator(ck, (rows,), {"output_ptr": y, "input_ptr": x.ravel().copy(), "input_row_stride": cols,
                                   "output_row_stride": cols, "n_cols": cols})
        out[f"case{done}_x"], out[f"case{done}_y"] = x, y.reshape(rows, cols)
        out[f"case{done}_shape"] = np.array([rows, cols, block, cols], np.int64)
        done += 1
    out["n_cases"] = np.int64(done)
    return out


def softmax_specials_vectors(rng):
    """softmax_kernel at BLOCK 256 on 12 rows of 256: the special-value rows of
    tests/test_reroll_reduce.py:157-174 and four rows whose only special entry is a -NaN (first,
    middle, last column; two of them)."""
    import kernels as K
    rows, block = 12, 256
    neg_nan = np.array([0xFFC00000], np.uint32).view(np.float32)[0]
    x = rng.standard_normal((rows, block)).astype(np.float32)
    x[0, :8] = np.array([np.nan, neg_nan, np.inf, -np.inf, -0.0, 0.0, 1e-40, -1e-40], np.float32)
    x[1, 3] = np.inf
    x[2, 0] = -np.inf
    x[3, :] = -0.0
    x[4, 0] = 1e-40
    x[4, 17] = -1e-40
    x[5, 16] = np.nan
    x[6, :] = -np.inf
    x[7, 255] = np.nan
    x[8, 0] = neg_nan
    x[9, 130] = neg_nan
    x[10, 255] = neg_nan
    x[11, 40] = neg_nan
    x[11, 41] = neg_nan
    y = np.full((rows, block), np.float32(-7.0))
    K.softmax_kernel[(rows,)](y, x, block, block, block, BLOCK_SIZE=block)
    return {"x": x, "y": y, "shape": np.array([rows, block, block, block], np.int64)}


def layernorm_vectors(rng):
    """Row layernorm without affine (the kernel of tests/test_reroll_reduce.py:199-208) over 3 rows
    at (BLOCK, n) = (256, 256), (256, 200), (128, 100), (128, 127), built the way that test builds
    it (reduction reroll on; store slots 1 at BLOCK 256, 0 with a 360-instruction cache
    threshold at 128), and add_kernel's x + y over seeded and special values."""
    import piton.reroll as reroll
    os.environ["PITON_REROLL_REDUCE"] = "1"
    sig = {"x_ptr": "*fp32", "out_ptr": "*fp32", "n": "i32", "eps": "fp32"}
    out, done, rows = {}, 0, 3
    for block, n, slots in ((256, 256, "1"), (256, 200, "1"), (128, 100, "0"), (128, 127, "0")):
        os.environ["PITON_STORE_SLOTS"] = slots
        saved = reroll.ICACHE_INSTRUCTIONS
        if block == 128:
            reroll.ICACHE_INSTRUCTIONS = 360
        try:
            ck = pc.compile(rownorm_k, sig, {"BLOCK": block}, grid=(4,))
        except Exception as e:  # a build the reference cannot make is recorded, not faked
            print(f"layernorm BLOCK {block} n {n}: no build ({type(e).__name__}: {e})", flush=True)
            continue
        finally:
            reroll.ICACHE_INSTRUCTIONS = saved
        x = (rng.standard_normal((rows, block)) * 2 + 1).astype(np.float32)
        y = np.full(rows * block, np.nan, np.float32)
        run_emulator(ck, (rows,), {"x_ptr": x.ravel().copy(), "out_ptr": y, "n": n, "eps": 1e-5})
        out[f"case{done}_x"], out[f"case{done}_y"] = x, y.reshape(rows, block)
        out[f"case{done}_shape"] = np.array([rows, n, block], np.int64)
        done += 1
    out["n_cases"] = np.int64(done)
    os.environ.pop("PITON_STORE_SLOTS", None)
    xa = np.concatenate([(rng.standard_normal(1000) * 10).astype(np.float32), SPECIALS])
    ya = np.concatenate([rng.standard_normal(1000).astype(np.float32), rng.permutation(SPECIALS)])
    oa = np.zeros_like(xa)
    add_k[(piton.cdiv(len(xa), 128),)](xa, ya, oa, len(xa), BLOCK=128)
    out["add_x"], out["add_y"], out["add_out"] = xa, ya, oa
    return out


def main():
    os.makedirs(OUT, exist_ok=True)
    if "--softmax-long" in sys.argv:
        t0 = time.time()
        np.savez_compressed(os.path.join(OUT, "softmax_long.npz"), **softmax_long_vectors(np.random.default_rng(7)))
        print(f"softmax_long: {time.time() - t0:.1f} s", flush=True)
        return
    if "--softmax-specials" in sys.argv:
        t0 = time.time()
        np.savez_compressed(os.path.join(OUT, "softmax_specials.npz"),
                            **softmax_specials_vectors(np.random.default_rng(13)))
        print(f"softmax_specials: {time.time() - t0:.1f} s", flush=True)
        return
    if "--layernorm" in sys.argv:
        t0 = time.time()
        np.savez_compressed(os.path.join(OUT, "layernorm.npz"), **layernorm_vectors(np.random.default_rng(11)))
        print(f"layernorm: {time.time() - t0:.1f} s", flush=True)
        return
    if "--full-mlp" in sys.argv:
        t0 = time.time()
        np.savez_compressed(os.path.join(OUT, "mlp_full.npz"), **mlp_full_vectors())
        print(f"mlp_full: {time.time() - t0:.1f} s", flush=True)
        return
    rng = np.random.default_rng(20261201)
    for name, make in (("math", lambda: math_vectors(rng)), ("softmax", lambda: softmax_vectors(rng)),
                       ("matmul", lambda: matmul_vectors(rng)), ("attention", lambda: attention_vectors(rng)),
                       ("mlp", mlp_vectors)):
        t0 = time.time()
        vec = make()
        np.savez_compressed(os.path.join(OUT, f"{name}.npz"), **vec)
        print(f"{name}: {len(vec)} arrays, {time.time() - t0:.1f} s", flush=True)


if __name__ == "__main__":
    main()
