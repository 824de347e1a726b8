"""`import piton_amd.language as tl`: the names a kernel definition needs at definition time
(piton/language/core.py:17-52): the `constexpr` marker, the dtype names and
CompilationError. Kernel bodies are not executed on this backend, so tensor builtins are not
provided."""
from __future__ import annotations


class CompilationError(Exception):
    pass


class constexpr:
    """Marker for compile-time arguments (`BLOCK: tl.constexpr`), and a wrapper whose
    `.value` is a default's value (piton/language/core.py:45-52)."""

    def __init__(self, value=None):
        self.value = value.value if isinstance(value, constexpr) else value

    def __repr__(self):
        return f"constexpr[{self.value!r}]"


class dtype:
    def __init__(self, name: str, supported: bool = True):
        self.name = name
        self.supported = supported

    def __repr__(self):
        return self.name


float32 = dtype("fp32")
int32 = dtype("i32")
uint32 = dtype("u32")
int1 = dtype("i1")
bool_ = int1
float16 = dtype("fp16", False)
bfloat16 = dtype("bf16", False)
float64 = dtype("fp64", False)
int8 = dtype("int8", False)
int16 = dtype("int16", False)
int64 = dtype("int64", False)
uint8 = dtype("uint8", False)
