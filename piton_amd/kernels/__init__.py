"""The kernel set, declared with the reference's signatures so that `kernel[grid](...)` calls
written for PIton run unchanged with device="mi355x". Each kernel's work is done by the HIP
entry its docstring names; the Python body is never executed."""
from .attention import attn_fwd_kernel
from .nn import dense_layer_kernel, dense_tiles
from .primitives import (copy_kernel, fma_kernel, idiv_kernel, log_kernel, mul_kernel, row_max_kernel,
                         row_sum_kernel, scaled_relu_kernel, sfu_kernel, transpose_kernel)
from .tutorial import add_kernel, layernorm_kernel, matmul_kernel, softmax_kernel

__all__ = ["add_kernel", "matmul_kernel", "softmax_kernel", "layernorm_kernel", "dense_layer_kernel",
           "dense_tiles", "attn_fwd_kernel", "copy_kernel", "mul_kernel", "fma_kernel", "scaled_relu_kernel",
           "sfu_kernel", "log_kernel", "idiv_kernel", "row_sum_kernel", "row_max_kernel", "transpose_kernel"]
