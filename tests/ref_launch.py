"""The reference's side of the drop-in boundary, for tests: a JIT object with only the attributes
the reference's JITFunction has, kernels declared as the reference declares them, and the
reference's Launcher.__call__ with the mi355x branch of INTEGRATION.md applied."""
import inspect

from piton_amd import language as tl
from piton_amd.runtime import launcher


class RefJIT:
    """Carries only what the reference's JITFunction has (piton/jit.py:16-25)."""

    def __init__(self, fn):
        self.fn = fn
        self.__name__ = fn.__name__
        self.arg_names = list(inspect.signature(fn).parameters)
        self._cache = {}


def ref_add_kernel(x_ptr, y_ptr, output_ptr, n_elements, BLOCK_SIZE: tl.constexpr):
    pass


def ref_matmul_kernel(a_ptr, b_ptr, c_ptr, M, N, K, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn,
                      BLOCK_SIZE_M: tl.constexpr, BLOCK_SIZE_N: tl.constexpr, BLOCK_SIZE_K: tl.constexpr,
                      GROUP_SIZE_M: tl.constexpr):
    pass


ref_add_kernel.__name__ = "add_kernel"
ref_matmul_kernel.__name__ = "matmul_kernel"


def patched_reference_call(jitfn, grid, *args, **kwargs):
    """Launcher.__call__ of piton/runtime/launcher.py:223-229 up to the resolved grid, then the
    mi355x branch INTEGRATION.md adds before the cache lookup and compile() (:230-237)."""
    kwargs = {k: v for k, v in kwargs.items() if k not in ("num_warps", "num_ctas")}
    signature, constants, values = launcher.bind(jitfn.fn, args, kwargs, getattr(jitfn, "do_not_specialize", ()))
    grid = grid(dict(constants, **values)) if callable(grid) else grid
    grid = tuple(grid) if isinstance(grid, (tuple, list)) else (grid,)
    return launcher.run_mi355x(jitfn, grid, signature, constants, values)


def ref_softmax_kernel(output_ptr, input_ptr, input_row_stride, output_row_stride, n_cols, BLOCK_SIZE: tl.constexpr):
    pass


ref_softmax_kernel.__name__ = "softmax_kernel"
