"""`@jit`: a Triton-style decorator around a kernel function (piton/jit.py:1-41)."""
from __future__ import annotations

import inspect


def cdiv(a, b):
    """Ceiling division (piton/jit.py:8-9)."""
    return (a + b - 1) // b


def next_power_of_2(n):
    """Smallest power of two >= n (piton/jit.py:12-13)."""
    return 1 << (int(n) - 1).bit_length()


class JITFunction:
    """A kernel: its Python function is the signature (parameter names, `constexpr`
    annotations and defaults) of a kernel in the device library; it is never executed."""

    _piton_jit = True

    def __init__(self, fn):
        self.fn = fn
        self.__name__ = fn.__name__
        self.__doc__ = fn.__doc__
        self.arg_names = list(inspect.signature(fn).parameters)
        self._cache = {}

    def __call__(self, *args, **kwargs):
        raise RuntimeError("@piton.jit kernels are launched with kernel[grid](...)")

    def __getitem__(self, grid):
        from .runtime.launcher import Launcher
        return Launcher(self, grid)

    def __repr__(self):
        return f"JITFunction({self.__name__})"


def jit(fn=None, **_kwargs):
    """Decorator, with or without keyword options (accepted and ignored, piton/jit.py:36-39)."""
    if fn is None:
        return lambda f: JITFunction(f)
    return JITFunction(fn)
