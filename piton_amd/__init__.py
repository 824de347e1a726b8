"""piton_amd: PIton's data-parallel kernel set on AMD MI355X (gfx950).

The launch surface is PIton's own (piton/__init__.py:3-6, piton/jit.py, piton/runtime/
launcher.py): `@jit` kernels launched as `kernel[grid](*args, device="mi355x", ...)`. Below it,
instead of PIton's compiler and QPU emulator, every launch is a ctypes call into
libpiton_mi355x.so, a library of hand-written gfx950 HIP kernels (piton_amd/csrc), on
PyTorch-ROCm device memory and streams.
"""
from . import language
from .jit import JITFunction, cdiv, jit, next_power_of_2

__all__ = ["jit", "JITFunction", "language", "cdiv", "next_power_of_2"]
