"""The perf suite's primitives (perf/suite.py:323-351) on the launch surface: the reference's
parameter lists, each running as one libpiton_mi355x.so entry (`kernel[grid](...,
device="mi355x")`). The BLOCK constexprs fix the grid the reference launches with; the device
tiles are the library's own."""
from .. import jit
from .. import language as tl


@jit
def copy_kernel(x_ptr, out_ptr, n, BLOCK: tl.constexpr):
    """out = x over n elements; grid (cdiv(n, BLOCK),). Runs as piton_mi355x_copy."""


@jit
def mul_kernel(x_ptr, y_ptr, out_ptr, n, BLOCK: tl.constexpr):
    """out = x * y; grid (cdiv(n, BLOCK),). Runs as piton_mi355x_mul."""


@jit
def fma_kernel(x_ptr, y_ptr, out_ptr, n, alpha, BLOCK: tl.constexpr):
    """out = x * alpha + y; grid (cdiv(n, BLOCK),). Runs as piton_mi355x_fma."""


@jit
def scaled_relu_kernel(x_ptr, out_ptr, n, alpha, BLOCK: tl.constexpr):
    """out = x > 0 ? x * alpha : 0; grid (cdiv(n, BLOCK),). Runs as piton_mi355x_scaled_relu."""


@jit
def sfu_kernel(x_ptr, out_ptr, n, OP: tl.constexpr, BLOCK: tl.constexpr):
    """out = exp2 / log2 / 1/x / rsqrt / exp / sqrt of x for OP 0..5; grid (cdiv(n, BLOCK),).
    Runs as piton_mi355x_sfu."""


@jit
def log_kernel(x_ptr, out_ptr, n, BLOCK: tl.constexpr):
    """out = ln(x); grid (cdiv(n, BLOCK),). Runs as piton_mi355x_log."""


@jit
def idiv_kernel(x_ptr, y_ptr, q_ptr, r_ptr, n, BLOCK: tl.constexpr):
    """int32 q = x // y, r = x % y truncating toward zero; grid (cdiv(n, BLOCK),). Runs as
    piton_mi355x_idiv."""


@jit
def row_sum_kernel(x_ptr, out_ptr, n_cols, stride, BLOCK_M: tl.constexpr, BLOCK_N: tl.constexpr):
    """out[r] = sum of the row's columns 0 .. cdiv(n_cols, BLOCK_N) * BLOCK_N - 1 (the reference
    reads whole BLOCK_N chunks, unmasked), BLOCK_M rows per program; grid (rows / BLOCK_M,).
    Runs as piton_mi355x_row_sum."""


@jit
def row_max_kernel(x_ptr, out_ptr, n_cols, stride, BLOCK_M: tl.constexpr, BLOCK_N: tl.constexpr):
    """As row_sum_kernel with max, starting from -FLT_MAX. Runs as piton_mi355x_row_max."""


@jit
def transpose_kernel(x_ptr, out_ptr, n_rows, n_cols, stride_x, stride_out, BLOCK_M: tl.constexpr,
                     BLOCK_N: tl.constexpr):
    """out[c, r] = x[r, c], masked to n_rows x n_cols; grid (cdiv(n_rows, BLOCK_M) *
    cdiv(n_cols, BLOCK_N),). Runs as piton_mi355x_transpose."""
