"""The oracle: TEST INFRASTRUCTURE ONLY.

A CPU restatement of the reference's own path for the hot kernels, used as the checker by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg. The product package
(piton_amd) never imports, links or calls anything here, and nothing here is measured as the
product.

Two halves:
  * liboracle.so (oracle.c + qpu_float.h): the emulator's round-toward-zero float32 semantics
    (piton/qpu/emulator.py:139-235) and the kernels' operation order (piton/backend/lower.py
    dot :3761-3877, reductions :3911-4063, exp :2716-2797, recip/fdiv :633-764, rsqrt/sqrt
    :766-795, 2899-2939), wrapped below;
  * fp64.py: the float64 host references the reference validates against (numpy).

Pinning (each function's checks live in tests/test_oracle*.py): the scalar ALU rules against
exact rational arithmetic truncated toward zero; matmul/dense against dyadic inputs (exact,
bit-for-bit), fp64 tolerances and the one-sided truncation bound; exp/exp2/recip/fdiv/sqrt/
rsqrt against float64 within the reference's tolerances plus special values; softmax and
attention against float64 plus the reference tests' known answers; layernorm against float64;
the digits MLP against the reference's known accuracy on its committed model and data. And
bit for bit against the reference's own emulator: golden vectors of exp, exp2, division, division
by a uniform, 1/x, rsqrt, sqrt (seeded and special values), softmax rows (with +inf, all -inf,
-inf and NaN rows), the tutorial matmul, attention and the digits MLP (He-normal weights, raw pixels), written by running the
reference's emulator (tests/golden/emulator, tests/test_oracle_emulator_vectors.py).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import fp64  # noqa: F401  (re-exported: oracle.fp64.*)

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile beside this file; returns its path."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        for name in ("fadd", "fsub", "fmul", "fmax", "fmin", "fdiv", "fdiv_uniform"):
            getattr(L, "oracle_" + name).argtypes = [_u32p, _u32p, _u32p, _i64]
        for name in ("ftoi", "itof", "exp", "exp2", "recip", "rsqrt", "sqrt"):
            getattr(L, "oracle_" + name).argtypes = [_u32p, _u32p, _i64]
        L.oracle_row_reduce.argtypes = [_u32p, _i64, _i64, _i32, _i32, _u32p]
        L.oracle_matmul.argtypes = [_u32p, _u32p, _u32p] + [_i64] * 11
        L.oracle_matmul_fast.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i32]
        L.oracle_dense.argtypes = [_u32p, _u32p, _u32p, _u32p, _i64, _i64, _i64, _i32, _i32]
        L.oracle_softmax.argtypes = [_u32p, _u32p, _i64, _i64, _i64, _i64, _i32]
        L.oracle_attention.argtypes = [_u32p, _u32p, _u32p, _u32p, ctypes.c_uint32] + [_i64] * 11 + \
            [_i32, _i32, _i32, _i64, _i64]
        L.oracle_layernorm.argtypes = [_u32p, _u32p, _i64, ctypes.c_uint32, _i64, _i64, _i32]
        L.oracle_add.argtypes = [_u32p, _u32p, _u32p, _i64]
        L.oracle_argmax_rows.argtypes = [_f32p, _i64, _i64, _i32, _i32p]
        _lib = L
    return _lib


def _bits(x) -> np.ndarray:
    """float32 (or uint32 bit patterns) -> contiguous uint32 bits."""
    x = np.asarray(x)
    if x.dtype == np.uint32:
        return np.ascontiguousarray(x)
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def _p(x, t=_u32p):
    return x.ctypes.data_as(t)


def _binary(name, a, b):
    a, b = np.broadcast_arrays(_bits(a), _bits(b))
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    out = np.empty(a.shape, np.uint32)
    getattr(lib(), "oracle_" + name)(_p(a), _p(b), _p(out), a.size)
    return out.view(np.float32)


def _unary(name, a, raw=False):
    a = _bits(a)
    out = np.empty(a.shape, np.uint32)
    getattr(lib(), "oracle_" + name)(_p(a), _p(out), a.size)
    return out if raw else out.view(np.float32)


# -- scalar ALU (emulator.py:139-235) ---------------------------------------------------------
def fadd(a, b): return _binary("fadd", a, b)
def fsub(a, b): return _binary("fsub", a, b)
def fmul(a, b): return _binary("fmul", a, b)
def fmax(a, b): return _binary("fmax", a, b)
def fmin(a, b): return _binary("fmin", a, b)
def ftoi(a): return _unary("ftoi", a, raw=True)
def itof(a): return _unary("itof", np.asarray(a, np.int32).view(np.uint32))


# -- lowered math (lower.py) ------------------------------------------------------------------
def exp(a): return _unary("exp", a)
def exp2(a): return _unary("exp2", a)
def recip(a): return _unary("recip", a)
def fdiv(a, b): return _binary("fdiv", a, b)
def fdiv_uniform(a, b): return _binary("fdiv_uniform", a, b)
def rsqrt(a): return _unary("rsqrt", a)
def sqrt(a): return _unary("sqrt", a)


def row_reduce(x, kind: str):
    """tl.sum / tl.max over the last axis of a [rows, L] float32 array, in the lowering's
    order (register fold then 16-lane butterfly)."""
    x = _bits(np.atleast_2d(x))
    out = np.empty(x.shape[0], np.uint32)
    lib().oracle_row_reduce(_p(x), x.shape[0], x.shape[1], x.shape[1], {"sum": 0, "max": 1}[kind], _p(out))
    return out.view(np.float32)


# -- kernels ----------------------------------------------------------------------------------
def matmul(a, b, rows=None):
    """matmul_kernel's result (examples/kernels.py:18-57) for float32 A [M,K] (any strides),
    B [K,N]; rows = (row0, row1) restricts the rows computed (others are NaN)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    r0, r1 = rows if rows is not None else (0, M)
    c = np.full((M, N), np.nan, np.float32)
    # element strides of the (possibly strided) views, through a bits view of the base
    ab, bb = a.view(np.uint32), b.view(np.uint32)
    sa = [s // 4 for s in ab.strides]
    sb = [s // 4 for s in bb.strides]
    ptr_a = ctypes.cast(ab.ctypes.data, _u32p)
    ptr_b = ctypes.cast(bb.ctypes.data, _u32p)
    cb = c.view(np.uint32)
    lib().oracle_matmul(ptr_a, ptr_b, _p(cb), M, N, K, sa[0], sa[1], sb[0], sb[1], N, 1, r0, r1)
    return c


def matmul_fast(a, b, rows=None, threads: int = 1):
    """The same bits as matmul() for finite inputs (host FPU in round-toward-zero mode,
    vectorised, `threads` OpenMP threads); contiguous A and B."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    M, K = a.shape
    N = b.shape[1]
    r0, r1 = rows if rows is not None else (0, M)
    c = np.full((M, N), np.nan, np.float32)
    lib().oracle_matmul_fast(_p(a, _f32p), _p(b, _f32p), _p(c, _f32p), N, K, r0, r1, int(threads))
    return c


def dense(x, w, bias=None, relu=False):
    """dense_layer_kernel (examples/nn_kernels.py:23-74): [ReLU](X W [+ b])."""
    x = _bits(x)
    w = _bits(w)
    M, K = x.shape
    N = w.shape[1]
    b = _bits(bias if bias is not None else np.zeros(N, np.float32))
    y = np.empty((M, N), np.uint32)
    lib().oracle_dense(_p(x), _p(w), _p(b), _p(y), M, N, K, int(bias is not None), int(bool(relu)))
    return y.view(np.float32)


def softmax(x, n_cols=None, block=None, out=None):
    """softmax_kernel (examples/kernels.py:60-76) over [rows, stride] float32 x; returns out
    (a copy of `out`, or NaN-filled) with columns < min(n_cols, block) written."""
    x = _bits(np.atleast_2d(x))
    rows, stride = x.shape
    n_cols = stride if n_cols is None else int(n_cols)
    block = block or (1 << max(0, n_cols - 1).bit_length())
    o = np.full(x.shape, np.nan, np.float32) if out is None else np.array(out, np.float32, copy=True)
    ob = o.view(np.uint32)
    lib().oracle_softmax(_p(ob), _p(x), stride, stride, n_cols, rows, int(block))
    return o


def attention(q, k, v, causal=False, sm_scale=None, block_n=16, rows=None, k_layout="nd"):
    """attn_fwd_kernel (examples/attention.py:67-113) for float32 [N, D] or [H, N, D] q, k, v
    (k pre-transposed [H, D, N] when k_layout == "dn"); rows = (q0, q1) limits the query rows
    computed (others NaN)."""
    q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
    squeeze = q.ndim == 2
    if squeeze:
        q, k, v = q[None], k[None], v[None]
    H, N, D = q.shape
    if block_n < 16 or block_n % 16:
        raise ValueError("the restatement covers BLOCK_N >= 16, a multiple of 16")
    if k_layout == "nd":
        s_kh, s_kn, s_kk = N * D, D, 1
    else:
        s_kh, s_kn, s_kk = D * N, 1, N
    scale = np.float32(1.0 / np.sqrt(D) if sm_scale is None else sm_scale)
    out = np.full(q.shape, np.nan, np.float32)
    q0, q1 = rows if rows is not None else (0, N)
    bq, bk, bv, bo = (t.view(np.uint32) for t in (q, k, v, out))
    lib().oracle_attention(_p(bq), _p(bk), _p(bv), _p(bo), int(scale.view(np.uint32)),
                           N * D, D, s_kh, s_kn, s_kk, N * D, D, N * D, D, N, H, D, int(block_n),
                           int(bool(causal)), q0, q1)
    return out[0] if squeeze else out


def layernorm(x, n=None, eps=1e-5, block=None):
    """layernorm_kernel (tests/test_reroll_reduce.py:199-208) over rows of `block` elements."""
    x = _bits(np.atleast_2d(x))
    rows, ld = x.shape
    block = block or ld
    n = ld if n is None else int(n)
    out = np.full(x.shape, np.nan, np.float32)
    lib().oracle_layernorm(_p(x), _p(out.view(np.uint32)), n, int(np.float32(eps).view(np.uint32)),
                           rows, ld, int(block))
    return out


def add(x, y):
    """add_kernel (examples/kernels.py:6-15)."""
    x, y = _bits(x), _bits(y)
    out = np.empty(x.shape, np.uint32)
    lib().oracle_add(_p(x), _p(y), _p(out), x.size)
    return out.view(np.float32)


def argmax_rows(x, n=None):
    """First index of the row maximum over the first n columns (numpy's argmax rule)."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    n = x.shape[1] if n is None else int(n)
    out = np.empty(x.shape[0], np.int32)
    lib().oracle_argmax_rows(_p(x, _f32p), x.shape[0], x.shape[1], n, _p(out, _i32p))
    return out


def mlp_forward(x, layers):
    """The digits chain of three dense launches (tests/test_digits_model.py:102-131):
    layers = [(w, b, relu), ...]; returns the last layer's output."""
    h = np.asarray(x, np.float32)
    for w, b, relu in layers:
        h = dense(h, w, b, relu=relu)
    return h
