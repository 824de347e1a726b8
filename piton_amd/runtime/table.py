"""The one mapping from the reference's kernels to libpiton_mi355x.so's entries.

For every kernel of the launch surface: its parameter list (the reference kernel's), the C entry
it runs as, the entry's arguments as expressions over the kernel's parameters and the launch
grid, the canonical grid (the cover `kernel[grid](...)` must use), checks, and the algorithmic
work of one launch. The launcher (piton_amd.runtime.launcher) evaluates the expressions in
Python at launch time; the AOT emitter (piton_amd.aot) renders the same expressions as C in a
generated launcher. Neither keeps a mapping of its own.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable


class Arr:
    """An array argument named by its kernel parameter (resolved to a device pointer at call)."""
    __slots__ = ("name",)

    def __init__(self, name):
        self.name = name


def cdiv(a, b):
    return (a + b - 1) // b


# -- expressions over the kernel's parameters and the grid -------------------------------------
# .py(env): the value, env = parameters (values and constants) plus "grid" (three ints);
# .c(sub): C source, sub(name) = the C expression of parameter `name`.

class Expr:
    def __mul__(self, other):
        return Mul(self, other)


class P(Expr):
    """A scalar parameter, converted by `conv` (int, float, bool)."""

    def __init__(self, name, conv=int):
        self.name, self.conv = name, conv

    def py(self, env):
        return self.conv(env[self.name])

    def c(self, sub):
        return sub(self.name)


class Ptr(Expr):
    """An array parameter."""

    def __init__(self, name):
        self.name = name

    def py(self, env):
        return Arr(self.name)

    def c(self, sub):
        return sub(self.name)


class Null(Expr):
    def __init__(self, ctype):
        self.ctype = ctype

    def py(self, env):
        return None

    def c(self, sub):
        return f"({self.ctype})0"


class Lit(Expr):
    def __init__(self, v):
        self.v = v

    def py(self, env):
        return self.v

    def c(self, sub):
        return str(int(self.v))


class GridDim(Expr):
    def __init__(self, axis):
        self.axis = axis

    def py(self, env):
        return int(env["grid"][self.axis])

    def c(self, sub):
        return f"(long long)g{'xyz'[self.axis]}"


class _Bin(Expr):
    op = ""

    def __init__(self, a, b):
        self.a, self.b = a, b

    def c(self, sub):
        return f"({self.a.c(sub)} {self.op} {self.b.c(sub)})"


class Mul(_Bin):
    op = "*"

    def py(self, env):
        return self.a.py(env) * self.b.py(env)


class Mod(_Bin):
    op = "%"

    def py(self, env):
        return self.a.py(env) % self.b.py(env)


class Eq(_Bin):
    op = "=="

    def py(self, env):
        return self.a.py(env) == self.b.py(env)


class Or(_Bin):
    op = "||"

    def py(self, env):
        return bool(self.a.py(env)) or bool(self.b.py(env))


class Not(Expr):
    def __init__(self, a):
        self.a = a

    def py(self, env):
        return not self.a.py(env)

    def c(self, sub):
        return f"(!{self.a.c(sub)})"


class Cdiv(_Bin):
    def py(self, env):
        return cdiv(self.a.py(env), self.b.py(env))

    def c(self, sub):
        a, b = self.a.c(sub), self.b.c(sub)
        return f"(({a} + {b} - 1) / {b})"


class Min(_Bin):
    def py(self, env):
        return min(self.a.py(env), self.b.py(env))

    def c(self, sub):
        a, b = self.a.c(sub), self.b.c(sub)
        return f"({a} < {b} ? {a} : {b})"


class Select(Expr):
    def __init__(self, cond, a, b):
        self.cond, self.a, self.b = cond, a, b

    def py(self, env):
        return self.a.py(env) if self.cond.py(env) else self.b.py(env)

    def c(self, sub):
        return f"({self.cond.c(sub)} ? {self.a.c(sub)} : {self.b.c(sub)})"


@dataclass
class KernelSpec:
    params: tuple                 # the reference kernel's parameter names, in order
    entry: str                    # C entry piton_mi355x_<entry> (and piton_amd.runtime.mi355x.<entry>)
    call: tuple                   # the entry's arguments before the stream, as expressions
    grid: tuple                   # canonical grid: an expression per axis, None = any
    reference: str                # the reference kernel (file:line)
    checks: tuple = ()            # (expression that must hold, message)
    work: Callable = field(default=lambda env: {})  # algorithmic flops / bytes of one launch

    def args(self, env):
        return tuple(e.py(env) for e in self.call)

    def expected_grid(self, env):
        return tuple(None if g is None else int(g.py(env)) for g in self.grid)


def _mm_work(env):
    M, N, K = int(env["M"]), int(env["N"]), int(env["K"])
    return {"flops": 2 * M * N * K, "bytes": 4 * (M * K + K * N + M * N)}


def _softmax_work(env):
    cols = min(int(env["n_cols"]), int(env["BLOCK_SIZE"]))
    return {"bytes": 8 * int(env["grid"][0]) * cols}


def _attn_work(env):
    n, d, h = int(env["N_CTX"]), int(env["HEAD_DIM"]), int(env["grid"][1])
    return {"flops": int(4 * n * n * d * h * (0.5 if env["CAUSAL"] else 1.0)), "bytes": 16 * n * d * h}


def _dense_work(env):
    w = _mm_work(env)
    w["bytes"] += 4 * int(env["N"]) if env["ADD_BIAS"] else 0
    return w


def _map(entry, ptrs, scalars=(), ref=""):
    """An elementwise primitive: grid (cdiv(n, BLOCK),), arguments (pointers..., n, scalars...)."""
    params = (*ptrs, "n", *(s for s, _ in scalars), "BLOCK")
    return KernelSpec(params, entry, (*(Ptr(p) for p in ptrs), P("n"), *(P(s, conv) for s, conv in scalars)),
                      (Cdiv(P("n"), P("BLOCK")), Lit(1), Lit(1)), ref,
                      work=lambda env: {"bytes": 4 * len(ptrs) * int(env["n"])})


def _row(entry, ref):
    # the reference reads whole BLOCK_N chunks of each row, unmasked (kernels.py:92-95)
    return KernelSpec(("x_ptr", "out_ptr", "n_cols", "stride", "BLOCK_M", "BLOCK_N"), entry,
                      (Ptr("x_ptr"), Ptr("out_ptr"), GridDim(0) * P("BLOCK_M"),
                       Cdiv(P("n_cols"), P("BLOCK_N")) * P("BLOCK_N"), P("stride")),
                      (None, Lit(1), Lit(1)), ref,
                      work=lambda env: {"bytes": 4 * int(env["grid"][0]) * int(env["BLOCK_M"])
                                        * (cdiv(int(env["n_cols"]), int(env["BLOCK_N"])) * int(env["BLOCK_N"]) + 1)})


_TILES = Cdiv(P("M"), P("BLOCK_SIZE_M")) * Cdiv(P("N"), P("BLOCK_SIZE_N"))

KERNELS = {
    "matmul_kernel": KernelSpec(
        ("a_ptr", "b_ptr", "c_ptr", "M", "N", "K", "stride_am", "stride_ak", "stride_bk", "stride_bn", "stride_cm",
         "stride_cn", "BLOCK_SIZE_M", "BLOCK_SIZE_N", "BLOCK_SIZE_K", "GROUP_SIZE_M"),
        "matmul",
        (Ptr("a_ptr"), Ptr("b_ptr"), Ptr("c_ptr"), P("M"), P("N"), P("K"), P("stride_am"), P("stride_ak"),
         P("stride_bk"), P("stride_bn"), P("stride_cm"), P("stride_cn"), P("GROUP_SIZE_M")),
        (_TILES, Lit(1), Lit(1)), "examples/kernels.py:18-57", work=_mm_work),
    "softmax_kernel": KernelSpec(
        ("output_ptr", "input_ptr", "input_row_stride", "output_row_stride", "n_cols", "BLOCK_SIZE"),
        "softmax",
        (Ptr("output_ptr"), Ptr("input_ptr"), P("input_row_stride"), P("output_row_stride"), P("n_cols"),
         GridDim(0), P("BLOCK_SIZE")),
        (None, Lit(1), Lit(1)), "examples/kernels.py:60-76", work=_softmax_work),
    "attn_fwd_kernel": KernelSpec(
        ("Q", "K", "V", "Out", "sm_scale", "stride_qh", "stride_qm", "stride_kh", "stride_kn", "stride_kk",
         "stride_vh", "stride_vn", "stride_oh", "stride_om", "N_CTX", "HEAD_DIM", "BLOCK_M", "BLOCK_N", "CAUSAL",
         "EVEN_N"),
        "attn_fwd",
        (Ptr("Q"), Ptr("K"), Ptr("V"), Ptr("Out"), P("sm_scale", float), P("stride_qh"), P("stride_qm"),
         P("stride_kh"), P("stride_kn"), P("stride_kk"), P("stride_vh"), P("stride_vn"), P("stride_oh"),
         P("stride_om"), P("N_CTX"), GridDim(1), P("HEAD_DIM"), P("CAUSAL", bool)),
        (Cdiv(P("N_CTX"), P("BLOCK_M")), None, Lit(1)), "examples/attention.py:67-113",
        checks=((Or(Not(P("EVEN_N", bool)), Eq(Mod(P("N_CTX"), P("BLOCK_N")), Lit(0))),
                 "EVEN_N promises N_CTX % BLOCK_N == 0"),),
        work=_attn_work),
    "dense_layer_kernel": KernelSpec(
        ("x_ptr", "w_ptr", "bias_ptr", "y_ptr", "M", "N", "K", "BLOCK_SIZE_M", "BLOCK_SIZE_N", "BLOCK_SIZE_K",
         "GROUP_SIZE_M", "ADD_BIAS", "RELU"),
        "dense",
        (Ptr("x_ptr"), Ptr("w_ptr"), Select(P("ADD_BIAS", bool), Ptr("bias_ptr"), Null("const float *")),
         Ptr("y_ptr"), P("M"), P("N"), P("K"), P("ADD_BIAS", bool), P("RELU", bool), Null("int32_t *"), Lit(0)),
        (_TILES, Lit(1), Lit(1)), "examples/nn_kernels.py:23-74", work=_dense_work),
    "add_kernel": KernelSpec(
        ("x_ptr", "y_ptr", "output_ptr", "n_elements", "BLOCK_SIZE"), "add",
        (Ptr("x_ptr"), Ptr("y_ptr"), Ptr("output_ptr"), P("n_elements")),
        (Cdiv(P("n_elements"), P("BLOCK_SIZE")), Lit(1), Lit(1)), "examples/kernels.py:6-15",
        work=lambda env: {"flops": int(env["n_elements"]), "bytes": 12 * int(env["n_elements"])}),
    "layernorm_kernel": KernelSpec(
        ("x_ptr", "out_ptr", "n", "eps", "BLOCK"), "layernorm",
        (Ptr("x_ptr"), Ptr("out_ptr"), Min(P("n"), P("BLOCK")), P("eps", float), GridDim(0), P("BLOCK")),
        (None, Lit(1), Lit(1)), "tests/test_reroll_reduce.py:199-208",
        work=lambda env: {"bytes": 8 * int(env["grid"][0]) * min(int(env["n"]), int(env["BLOCK"]))}),
    "copy_kernel": _map("copy", ("x_ptr", "out_ptr"), ref="examples/primitive_kernels.py"),
    "mul_kernel": _map("mul", ("x_ptr", "y_ptr", "out_ptr"), ref="examples/elementwise.py"),
    "fma_kernel": _map("fma", ("x_ptr", "y_ptr", "out_ptr"), (("alpha", float),), ref="examples/elementwise.py"),
    "scaled_relu_kernel": _map("scaled_relu", ("x_ptr", "out_ptr"), (("alpha", float),),
                               ref="examples/primitive_kernels.py"),
    "sfu_kernel": _map("sfu", ("x_ptr", "out_ptr"), (("OP", int),), ref="examples/sfu_tests.py"),
    "log_kernel": _map("log", ("x_ptr", "out_ptr"), ref="examples/primitive_kernels.py"),
    "idiv_kernel": _map("idiv", ("x_ptr", "y_ptr", "q_ptr", "r_ptr"), ref="examples/kernels.py:79-85"),
    "row_sum_kernel": _row("row_sum", "examples/kernels.py:88-96"),
    "row_max_kernel": _row("row_max", "examples/primitive_kernels.py:41-50"),
    "transpose_kernel": KernelSpec(
        ("x_ptr", "out_ptr", "n_rows", "n_cols", "stride_x", "stride_out", "BLOCK_M", "BLOCK_N"), "transpose",
        (Ptr("x_ptr"), Ptr("out_ptr"), P("n_rows"), P("n_cols"), P("stride_x"), P("stride_out")),
        (Cdiv(P("n_rows"), P("BLOCK_M")) * Cdiv(P("n_cols"), P("BLOCK_N")), Lit(1), Lit(1)),
        "examples/primitive_kernels.py:53-67",
        work=lambda env: {"bytes": 8 * int(env["n_rows"]) * int(env["n_cols"])}),
}
