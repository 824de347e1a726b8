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
import os
from dataclasses import dataclass, field

import numpy as np

from ..language import constexpr
from .table import KERNELS, Arr, KernelSpec

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
    """What a launch returns (the reference returns its CompiledKernel with `last_stats` set from
    the emulator's counters, launcher.py:238-245). `last_stats` holds:
      * "launches": the device kernels the entry ran, each with its grid, block, LDS bytes,
        vector registers and spill bytes (piton_mi355x_last_launches);
      * "flops" / "bytes": the launch's algorithmic work (what the reference kernel computes,
        read once and written once), the figures a roofline is computed from;
      * "elapsed_us": the launch's time from HIP events around it, when PITON_MI355X_TIMING=1
        (the call then waits for the launch);
      * "num_stages": as passed."""
    name: str
    grid: tuple
    entry: str
    signature: dict
    constants: dict
    last_stats: dict = field(default_factory=dict)


REGISTRY = KERNELS  # kernel name -> KernelSpec (piton_amd.runtime.table)


def lookup(jitfn) -> KernelSpec:
    """The spec of a kernel, matched by name and parameter list."""
    spec = KERNELS.get(jitfn.__name__)
    if spec is None:
        raise NotImplementedError(f"no mi355x kernel for {jitfn.__name__!r}; this backend provides "
                                  f"{sorted(KERNELS)}")
    if tuple(jitfn.arg_names) != spec.params:
        raise NotImplementedError(f"{jitfn.__name__}{tuple(jitfn.arg_names)} does not match the mi355x "
                                  f"kernel's parameters {spec.params}")
    return spec


def _grid3(grid):
    return tuple(int(g) for g in grid) + (1,) * (3 - len(grid))


def _env(grid, constants, values):
    env = dict(values, **constants)
    env["grid"] = _grid3(grid)
    return env


def plan(jitfn, grid, constants, values):
    """(entry, args) of a launch, with every host-side check done: the grid must be the kernel's
    canonical cover (any other grid would compute a different set of tiles in the reference)."""
    spec = lookup(jitfn)
    env = _env(grid, constants, values)
    want = spec.expected_grid(env)
    if any(w is not None and w != g for w, g in zip(want, env["grid"])):
        shown = tuple("any" if w is None else w for w in want)
        raise ValueError(f"{jitfn.__name__}: grid {tuple(grid)} does not cover the kernel's tiles; expected {shown}")
    for cond, msg in spec.checks:
        if not cond.py(env):
            raise ValueError(f"{jitfn.__name__}: {msg}")
    return spec.entry, spec.args(env)


def _timing() -> bool:
    return os.environ.get("PITON_MI355X_TIMING", "") not in ("", "0")


def run_mi355x(jitfn, grid, signature, constants, values) -> LaunchRecord:
    """Launch on the MI355X library: stage numpy arrays, call the entry, copy arrays back.

    `jitfn` needs only what the reference's JITFunction carries (piton/jit.py:16-25): `__name__`
    and `arg_names`; `signature`, `constants` and `values` are what the reference's `bind`
    returns for the launch (launcher.py:42-63) and `grid` the resolved grid tuple."""
    entry, args = plan(jitfn, grid, constants, values)
    import torch

    from . import mi355x as rt
    dev = rt.staging_device()
    staged = {}
    for name, v in values.items():
        if isinstance(v, np.ndarray):
            flat = np.ascontiguousarray(v).reshape(-1)
            staged[name] = torch.from_numpy(flat.view(np.int32) if v.dtype == np.uint32 else flat).to(dev)
    resolved = [(staged.get(x.name, values.get(x.name)) if isinstance(x, Arr) else x) for x in args]
    timed = _timing()
    if timed:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
    getattr(rt, entry)(*resolved)
    if timed:
        e1.record()  # right behind the launch: the host work below is not in the interval
    stats = {"launches": rt.last_launches(), **lookup(jitfn).work(_env(grid, constants, values))}
    if timed:
        e1.synchronize()
        stats["elapsed_us"] = e0.elapsed_time(e1) * 1e3
    if staged:
        rt.synchronize()
        for name, t in staged.items():
            v = values[name]
            v[...] = t.cpu().numpy().view(v.dtype).reshape(v.shape)
    return LaunchRecord(jitfn.__name__, tuple(grid), "piton_mi355x_" + entry, signature, constants, stats)


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
            rec.last_stats["num_stages"] = num_stages
            return rec
        raise ValueError(f"unknown device {device!r}")
