"""`kernel[grid](*args, device="mi355x")` for PIton kernels (piton/runtime/launcher.py:42-63,
217-245), dispatched to libpiton_mi355x.so.

Arguments follow the reference's conventions: `bind` splits them into signature, constants and
runtime values exactly as PIton does (constexpr-annotated parameters and ints equal to 1 become
constants), so a kernel's arguments are read from `dict(values, **constants)`. Arrays may be
  * torch tensors on the ROCm device (float32 / int32): passed by pointer, the launch is
    asynchronous on torch's current stream, as a GPU Triton launch is;
  * numpy float32 / int32 / uint32 arrays: every array is copied to the device, the kernel
    runs, and every array is copied back, inputs included, before the call returns (the
    emulator's copy-in / copy-out contract, launcher.py:175-180, 209-211).

The kernel is identified by its name and parameter list; the grid must be the kernel's
canonical cover for the given constexprs (any other grid would compute a different set of
tiles in the reference) and is checked.
"""
from __future__ import annotations

import inspect
from dataclasses import dataclass, field

import numpy as np

from ..jit import cdiv
from ..language import constexpr

_DTYPE_SIG = {np.dtype(np.float32): "*fp32", np.dtype(np.int32): "*i32", np.dtype(np.uint32): "*u32"}


def _is_tensor(v) -> bool:
    try:
        import torch
    except ImportError:  # pragma: no cover
        return False
    return isinstance(v, torch.Tensor)


def _sig_of(value):
    """The signature type of a runtime argument (piton/runtime/launcher.py:28-39), plus
    torch tensors."""
    if isinstance(value, np.ndarray):
        if value.dtype not in _DTYPE_SIG:
            raise TypeError(f"unsupported array dtype {value.dtype} (use float32/int32)")
        return _DTYPE_SIG[value.dtype]
    if _is_tensor(value):
        import torch
        sig = {torch.float32: "*fp32", torch.int32: "*i32"}.get(value.dtype)
        if sig is None:
            raise TypeError(f"unsupported tensor dtype {value.dtype} (use float32/int32)")
        return sig
    if isinstance(value, bool):
        return "i1"
    if isinstance(value, (int, np.integer)):
        return "i32"
    if isinstance(value, (float, np.floating)):
        return "fp32"
    raise TypeError(f"unsupported kernel argument {type(value).__name__}")


def bind(fn, args, kwargs, do_not_specialize=()):
    """Split launch arguments into (signature, constants, runtime values), as
    piton/runtime/launcher.py:42-63 does."""
    params = list(inspect.signature(fn).parameters.values())
    bound = inspect.signature(fn).bind_partial(*args, **kwargs)
    signature, constants, values = {}, {}, {}
    for p in params:
        if p.name not in bound.arguments:
            if p.default is inspect.Parameter.empty:
                raise TypeError(f"missing kernel argument '{p.name}'")
            constants[p.name] = p.default.value if isinstance(p.default, constexpr) else p.default
            continue
        v = bound.arguments[p.name]
        ann = p.annotation
        if ann is constexpr or (isinstance(ann, str) and "constexpr" in ann):
            constants[p.name] = v
        elif isinstance(v, (int, np.integer)) and not isinstance(v, bool) and v == 1 \
                and p.name not in do_not_specialize:
            constants[p.name] = 1
        else:
            signature[p.name] = _sig_of(v)
            values[p.name] = v
    return signature, constants, values


@dataclass
class LaunchRecord:
    """What a launch returns (the reference returns its CompiledKernel, launcher.py:245)."""
    name: str
    grid: tuple
    entry: str
    signature: dict
    constants: dict
    last_stats: dict = field(default_factory=dict)


# -- kernel registry: name -> (parameter names, planner) -----------------------------------------
# A planner checks the grid and the constexprs and returns (entry name in mi355x.py, args), where
# Arr(name) stands for the array argument `name`; nothing touches the device before it returns.

class Arr:
    __slots__ = ("name",)

    def __init__(self, name):
        self.name = name


def _grid3(grid):
    return tuple(int(g) for g in grid) + (1,) * (3 - len(grid))


def _expect_grid(name, grid, want):
    if _grid3(grid) != _grid3(want):
        raise ValueError(f"{name}: grid {tuple(grid)} does not cover the kernel's tiles; expected {tuple(want)}")


def _plan_matmul(a, grid):
    M, N, K = int(a["M"]), int(a["N"]), int(a["K"])
    _expect_grid("matmul_kernel", grid, (cdiv(M, a["BLOCK_SIZE_M"]) * cdiv(N, a["BLOCK_SIZE_N"]),))
    return "matmul", (Arr("a_ptr"), Arr("b_ptr"), Arr("c_ptr"), M, N, K, int(a["stride_am"]), int(a["stride_ak"]),
                      int(a["stride_bk"]), int(a["stride_bn"]), int(a["stride_cm"]), int(a["stride_cn"]),
                      int(a["GROUP_SIZE_M"]))


def _plan_softmax(a, grid):
    g = _grid3(grid)
    if g[1] != 1 or g[2] != 1:
        raise ValueError(f"softmax_kernel: grid {tuple(grid)} must be (n_rows,)")
    return "softmax", (Arr("output_ptr"), Arr("input_ptr"), int(a["input_row_stride"]), int(a["output_row_stride"]),
                       int(a["n_cols"]), g[0], int(a["BLOCK_SIZE"]))


def _plan_attn(a, grid):
    n_ctx, heads = int(a["N_CTX"]), _grid3(grid)[1]
    _expect_grid("attn_fwd_kernel", grid, (cdiv(n_ctx, a["BLOCK_M"]), heads))
    if a["EVEN_N"] and n_ctx % int(a["BLOCK_N"]):
        raise ValueError("attn_fwd_kernel: EVEN_N promises N_CTX % BLOCK_N == 0")
    return "attn_fwd", (Arr("Q"), Arr("K"), Arr("V"), Arr("Out"), float(a["sm_scale"]), int(a["stride_qh"]),
                        int(a["stride_qm"]), int(a["stride_kh"]), int(a["stride_kn"]), int(a["stride_kk"]),
                        int(a["stride_vh"]), int(a["stride_vn"]), int(a["stride_oh"]), int(a["stride_om"]), n_ctx,
                        heads, int(a["HEAD_DIM"]), bool(a["CAUSAL"]))


def _plan_dense(a, grid):
    M, N, K = int(a["M"]), int(a["N"]), int(a["K"])
    _expect_grid("dense_layer_kernel", grid, (cdiv(M, a["BLOCK_SIZE_M"]) * cdiv(N, a["BLOCK_SIZE_N"]),))
    add_bias = bool(a["ADD_BIAS"])
    return "dense", (Arr("x_ptr"), Arr("w_ptr"), Arr("bias_ptr") if add_bias else None, Arr("y_ptr"), M, N, K,
                     add_bias, bool(a["RELU"]))


def _plan_add(a, grid):
    n = int(a["n_elements"])
    _expect_grid("add_kernel", grid, (cdiv(n, a["BLOCK_SIZE"]),))
    return "add", (Arr("x_ptr"), Arr("y_ptr"), Arr("output_ptr"), n)


def _plan_layernorm(a, grid):
    g = _grid3(grid)
    if g[1] != 1 or g[2] != 1:
        raise ValueError(f"layernorm_kernel: grid {tuple(grid)} must be (rows,)")
    block = int(a["BLOCK"])
    return "layernorm", (Arr("x_ptr"), Arr("out_ptr"), min(int(a["n"]), block), float(a["eps"]), g[0], block)


def _plan_map(entry, ptrs, scalars=()):
    """An elementwise primitive: grid (cdiv(n, BLOCK),), arguments (pointers..., n, scalars...)."""
    def plan(a, grid):
        n = int(a["n"])
        _expect_grid(entry + "_kernel", grid, (cdiv(n, a["BLOCK"]),))
        return entry, (*[Arr(p) for p in ptrs], n, *[conv(a[s]) for s, conv in scalars])
    return plan


def _plan_row_reduce(entry):
    def plan(a, grid):
        g = _grid3(grid)
        if g[1] != 1 or g[2] != 1:
            raise ValueError(f"{entry}_kernel: grid {tuple(grid)} must be (rows / BLOCK_M,)")
        # the reference reads whole BLOCK_N chunks of each row, unmasked (kernels.py:92-95)
        cols = cdiv(int(a["n_cols"]), a["BLOCK_N"]) * int(a["BLOCK_N"])
        return entry, (Arr("x_ptr"), Arr("out_ptr"), g[0] * int(a["BLOCK_M"]), cols, int(a["stride"]))
    return plan


def _plan_transpose(a, grid):
    n_rows, n_cols = int(a["n_rows"]), int(a["n_cols"])
    _expect_grid("transpose_kernel", grid, (cdiv(n_rows, a["BLOCK_M"]) * cdiv(n_cols, a["BLOCK_N"]),))
    return "transpose", (Arr("x_ptr"), Arr("out_ptr"), n_rows, n_cols, int(a["stride_x"]), int(a["stride_out"]))


REGISTRY = {
    "matmul_kernel": (("a_ptr", "b_ptr", "c_ptr", "M", "N", "K", "stride_am", "stride_ak", "stride_bk",
                       "stride_bn", "stride_cm", "stride_cn", "BLOCK_SIZE_M", "BLOCK_SIZE_N", "BLOCK_SIZE_K",
                       "GROUP_SIZE_M"), _plan_matmul),
    "softmax_kernel": (("output_ptr", "input_ptr", "input_row_stride", "output_row_stride", "n_cols",
                        "BLOCK_SIZE"), _plan_softmax),
    "attn_fwd_kernel": (("Q", "K", "V", "Out", "sm_scale", "stride_qh", "stride_qm", "stride_kh", "stride_kn",
                         "stride_kk", "stride_vh", "stride_vn", "stride_oh", "stride_om", "N_CTX", "HEAD_DIM",
                         "BLOCK_M", "BLOCK_N", "CAUSAL", "EVEN_N"), _plan_attn),
    "dense_layer_kernel": (("x_ptr", "w_ptr", "bias_ptr", "y_ptr", "M", "N", "K", "BLOCK_SIZE_M", "BLOCK_SIZE_N",
                            "BLOCK_SIZE_K", "GROUP_SIZE_M", "ADD_BIAS", "RELU"), _plan_dense),
    "add_kernel": (("x_ptr", "y_ptr", "output_ptr", "n_elements", "BLOCK_SIZE"), _plan_add),
    "layernorm_kernel": (("x_ptr", "out_ptr", "n", "eps", "BLOCK"), _plan_layernorm),
    "copy_kernel": (("x_ptr", "out_ptr", "n", "BLOCK"), _plan_map("copy", ("x_ptr", "out_ptr"))),
    "mul_kernel": (("x_ptr", "y_ptr", "out_ptr", "n", "BLOCK"), _plan_map("mul", ("x_ptr", "y_ptr", "out_ptr"))),
    "fma_kernel": (("x_ptr", "y_ptr", "out_ptr", "n", "alpha", "BLOCK"),
                   _plan_map("fma", ("x_ptr", "y_ptr", "out_ptr"), (("alpha", float),))),
    "scaled_relu_kernel": (("x_ptr", "out_ptr", "n", "alpha", "BLOCK"),
                           _plan_map("scaled_relu", ("x_ptr", "out_ptr"), (("alpha", float),))),
    "sfu_kernel": (("x_ptr", "out_ptr", "n", "OP", "BLOCK"), _plan_map("sfu", ("x_ptr", "out_ptr"), (("OP", int),))),
    "log_kernel": (("x_ptr", "out_ptr", "n", "BLOCK"), _plan_map("log", ("x_ptr", "out_ptr"))),
    "idiv_kernel": (("x_ptr", "y_ptr", "q_ptr", "r_ptr", "n", "BLOCK"),
                    _plan_map("idiv", ("x_ptr", "y_ptr", "q_ptr", "r_ptr"))),
    "row_sum_kernel": (("x_ptr", "out_ptr", "n_cols", "stride", "BLOCK_M", "BLOCK_N"), _plan_row_reduce("row_sum")),
    "row_max_kernel": (("x_ptr", "out_ptr", "n_cols", "stride", "BLOCK_M", "BLOCK_N"), _plan_row_reduce("row_max")),
    "transpose_kernel": (("x_ptr", "out_ptr", "n_rows", "n_cols", "stride_x", "stride_out", "BLOCK_M", "BLOCK_N"),
                         _plan_transpose),
}


def lookup(jitfn):
    """The planner of a kernel, matched by name and parameter list."""
    entry = REGISTRY.get(jitfn.__name__)
    if entry is None:
        raise NotImplementedError(f"no mi355x kernel for {jitfn.__name__!r}; this backend provides "
                                  f"{sorted(REGISTRY)}")
    params, planner = entry
    if tuple(jitfn.arg_names) != params:
        raise NotImplementedError(f"{jitfn.__name__}{tuple(jitfn.arg_names)} does not match the mi355x "
                                  f"kernel's parameters {params}")
    return planner


def plan(jitfn, grid, constants, values):
    """(entry, args) of a launch, with every host-side check done."""
    return lookup(jitfn)(dict(values, **constants), grid)


def run_mi355x(jitfn, grid, signature, constants, values) -> LaunchRecord:
    """Launch on the MI355X library: stage numpy arrays, call the entry, copy arrays back."""
    entry, args = plan(jitfn, grid, constants, values)
    import torch

    from . import mi355x as rt
    staged = {}
    for name, v in values.items():
        if isinstance(v, np.ndarray):
            flat = np.ascontiguousarray(v).reshape(-1)
            staged[name] = torch.from_numpy(flat.view(np.int32) if v.dtype == np.uint32 else flat).to("cuda")
    resolved = [(staged.get(x.name, values.get(x.name)) if isinstance(x, Arr) else x) for x in args]
    getattr(rt, entry)(*resolved)
    if staged:
        torch.cuda.current_stream().synchronize()
        for name, dev in staged.items():
            v = values[name]
            v[...] = dev.cpu().numpy().view(v.dtype).reshape(v.shape)
    return LaunchRecord(jitfn.__name__, tuple(grid), "piton_mi355x_" + entry, signature, constants)


class Launcher:
    def __init__(self, jitfn, grid, extra_constants=None):
        self.jitfn = jitfn
        self.grid = grid
        self.extra_constants = dict(extra_constants or {})

    def __call__(self, *args, device: str = "mi355x", num_stages: int = 2, **kwargs):
        fn = self.jitfn.fn
        for k in ("num_warps", "num_ctas"):
            kwargs.pop(k, None)
        signature, constants, values = bind(fn, args, kwargs, getattr(self.jitfn, "do_not_specialize", ()))
        constants.update(self.extra_constants)
        grid = self.grid(dict(constants, **values)) if callable(self.grid) else self.grid
        grid = tuple(grid) if isinstance(grid, (tuple, list)) else (grid,)
        if device == "mi355x":
            rec = run_mi355x(self.jitfn, grid, signature, constants, values)
            rec.last_stats = {"num_stages": num_stages}
            return rec
        raise ValueError(f"unknown device {device!r}")
