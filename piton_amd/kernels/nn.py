"""Fused dense layer (examples/nn_kernels.py:14-74)."""
from .. import jit
from .. import language as tl


def dense_tiles(output_features):
    """(BM, BN, BK) the reference launches a layer with (examples/nn_kernels.py:14-20); they
    fix the grid of a `dense_layer_kernel[grid]` call."""
    return (4, 64, 4) if output_features >= 64 else (8, 16, 4)


@jit
def dense_layer_kernel(x_ptr, w_ptr, bias_ptr, y_ptr, M, N: tl.constexpr, K: tl.constexpr,
                       BLOCK_SIZE_M: tl.constexpr, BLOCK_SIZE_N: tl.constexpr, BLOCK_SIZE_K: tl.constexpr,
                       GROUP_SIZE_M: tl.constexpr, ADD_BIAS: tl.constexpr, RELU: tl.constexpr):
    """Y[M, N] = [ReLU](X[M, K] W[K, N] [+ bias]) on contiguous row-major storage; grid
    (cdiv(M, BLOCK_SIZE_M) * cdiv(N, BLOCK_SIZE_N),). Runs as piton_mi355x_dense."""
