"""Tutorial kernels: add (examples/kernels.py:6-15), grouped matmul (:18-57), fused row
softmax (:60-76), and the row layernorm of tests/test_reroll_reduce.py:199-208."""
from .. import jit
from .. import language as tl


@jit
def add_kernel(x_ptr, y_ptr, output_ptr, n_elements, BLOCK_SIZE: tl.constexpr):
    """output[i] = x[i] + y[i] for i < n_elements; grid (cdiv(n_elements, BLOCK_SIZE),).
    Runs as piton_mi355x_add."""


@jit
def matmul_kernel(a_ptr, b_ptr, c_ptr, M, N, K, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn,
                  BLOCK_SIZE_M: tl.constexpr, BLOCK_SIZE_N: tl.constexpr, BLOCK_SIZE_K: tl.constexpr,
                  GROUP_SIZE_M: tl.constexpr):
    """C = A B through six element strides, grouped-M tile order; grid
    (cdiv(M, BLOCK_SIZE_M) * cdiv(N, BLOCK_SIZE_N),). The BLOCK_SIZE_* constexprs fix the
    grid; the device tiles are the library's own. Runs as piton_mi355x_matmul."""


@jit
def softmax_kernel(output_ptr, input_ptr, input_row_stride, output_row_stride, n_cols, BLOCK_SIZE: tl.constexpr):
    """Row softmax over the first min(n_cols, BLOCK_SIZE) columns, one row per program; grid
    (n_rows,). Runs as piton_mi355x_softmax."""


@jit
def layernorm_kernel(x_ptr, out_ptr, n, eps, BLOCK: tl.constexpr):
    """(x - mean) / sqrt(var + eps) over the first n of each row of BLOCK elements (row stride
    BLOCK), biased variance, no affine; grid (rows,). Runs as piton_mi355x_layernorm."""
