"""Ahead-of-time C launchers over libpiton_mi355x.so (piton/tools/compile.py:1-15, 55-172).

    python -m piton_amd.aot examples/kernels.py --kernel-name matmul_kernel \\
        --signature "a_ptr=*fp32,b_ptr=*fp32,c_ptr=*fp32,M=i32,N=i32,K=i32,stride_am=i32,stride_bk=i32,stride_cm=i32" \\
        --constants "stride_ak=1,stride_bn=1,stride_cn=1,BLOCK_SIZE_M=128,BLOCK_SIZE_N=128,BLOCK_SIZE_K=32,GROUP_SIZE_M=8" \\
        --out-name matmul -o build/

writes build/matmul.h and build/matmul.c: a typed argument struct and launchers, so C and
C++ programs call a specialised kernel without Python, as the reference's AOT path gives
bare-metal programs on the Pi:

    matmul_args_t args = { .a_ptr = A, ..., .M = 4096, ... };      // device pointers
    int32_t rc = matmul_launch(&args, gx, 1, 1, stream);           // asynchronous, a status
    int32_t rc = matmul_launch_us(&args, gx, 1, 1, &usec);         // synchronous, timed

The kernel is named by its file and function (a `@jit` function of this package's launch
surface, or any function with the same name and parameter list); `--signature` lists the
runtime arguments with their types (`*fp32`, `*i32`, `*u32`, `i32`, `u32`, `fp32`, `i1`) and
`--constants` the specialised ones. The launcher checks the grid against the kernel's
canonical cover (the rule `kernel[grid](...)` applies) and returns PITON_EINVAL (-1) for any
other grid, then calls the library entry with the struct fields and the constants folded in.
Compile the .c with any C compiler: `-I include -I /opt/rocm/include -D__HIP_PLATFORM_AMD__`,
link `-lpiton_mi355x -lamdhip64`.
"""
from __future__ import annotations

import argparse
import importlib.util
import inspect
import os
import sys

from .runtime import table

C_TYPES = {"*fp32": "float *", "*i32": "int32_t *", "*u32": "uint32_t *", "i32": "int32_t", "u32": "uint32_t",
           "fp32": "float", "i1": "int32_t"}


# The kernel -> entry mapping is piton_amd.runtime.table's, the one the launcher evaluates at run
# time; here its expressions are rendered as C.
KERNELS = table.KERNELS


def _parse_kv(text: str) -> dict:
    out = {}
    for item in filter(None, (t.strip() for t in text.split(","))):
        k, v = item.split("=", 1)
        k, v = k.strip(), v.strip()
        if v in ("True", "False"):
            out[k] = v == "True"
            continue
        try:
            out[k] = int(v, 0)
        except ValueError:
            try:
                out[k] = float(v)
            except ValueError:
                out[k] = v
    return out


def _literal(v) -> str:
    if isinstance(v, bool):
        return "1" if v else "0"
    if isinstance(v, int):
        return f"{v}LL"
    if isinstance(v, float):
        return f"{v!r}f" if "e" in repr(v) or "." in repr(v) else f"{v!r}.0f"
    raise TypeError(f"constant {v!r}: expected an int, float or bool")


def load_kernel(path: str, name: str):
    """The function `name` of the Python file at `path`; a file inside a package (directories
    with __init__.py) is imported by its dotted name, so its relative imports work."""
    path = os.path.abspath(path)
    parts = [os.path.splitext(os.path.basename(path))[0]]
    d = os.path.dirname(path)
    while os.path.exists(os.path.join(d, "__init__.py")):
        parts.insert(0, os.path.basename(d))
        d = os.path.dirname(d)
    if len(parts) > 1:
        if d not in sys.path:
            sys.path.insert(0, d)
        mod = importlib.import_module(".".join(parts))
    else:
        spec = importlib.util.spec_from_file_location(parts[0], path)
        mod = importlib.util.module_from_spec(spec)
        sys.path.insert(0, os.path.dirname(path))
        spec.loader.exec_module(mod)
    return getattr(mod, name)


def _params_of(kernel) -> tuple:
    fn = getattr(kernel, "fn", kernel)
    return tuple(inspect.signature(fn).parameters)


def emit_c(kernel_name: str, params: tuple, signature: dict, constants: dict, out_name: str) -> tuple:
    """(header, source) of the launcher of `kernel_name` specialised on `constants`."""
    spec = KERNELS.get(kernel_name)
    if spec is None:
        raise NotImplementedError(f"no mi355x kernel for {kernel_name!r}; this backend provides {sorted(KERNELS)}")
    if tuple(params) != spec.params:
        raise NotImplementedError(f"{kernel_name}{tuple(params)} does not match the mi355x kernel's parameters "
                                  f"{spec.params}")
    both = set(signature) & set(constants)
    if both:
        raise ValueError(f"{sorted(both)} given both as runtime arguments and constants")
    missing = [p for p in params if p not in signature and p not in constants]
    if missing:
        raise TypeError(f"missing kernel argument(s) {missing}: give each a --signature type or a --constants value")
    for n, t in signature.items():
        if t not in C_TYPES:
            raise TypeError(f"{n}: unsupported type {t!r} (one of {sorted(C_TYPES)})")

    def sub(p: str) -> str:
        return f"args->{p}" if p in signature else _literal(constants[p])

    sym = out_name
    guard = f"{sym.upper()}_H"
    h = [f"// Generated by piton_amd.aot from kernel `{kernel_name}` for libpiton_mi355x.so (gfx950).",
         f"// constants: {', '.join(f'{k}={v}' for k, v in constants.items()) or '(none)'}",
         f"#ifndef {guard}", f"#define {guard}", "", "#include <stdint.h>", "",
         "#ifdef __cplusplus", 'extern "C" {', "#endif", "",
         "// Pointer arguments are device pointers (hipMalloc'd, or torch tensors' data_ptr()).",
         "typedef struct {"]
    for n, t in signature.items():
        h.append(f"    {C_TYPES[t]}{'' if C_TYPES[t].endswith('*') else ' '}{n};   // {t}")
    if not signature:
        h.append("    int32_t _unused;")
    h += [f"}} {sym}_args_t;", "",
          "// Launches on `stream` (a hipStream_t; NULL = the default stream) without waiting. Returns",
          "// 0, or a negative status: -1 for a grid other than the kernel's canonical cover (and for",
          "// the library's own argument checks), -2 unsupported, -3 HIP error, -4 no device; the",
          "// library's message is piton_mi355x_last_error().",
          f"int32_t {sym}_launch(const {sym}_args_t *args, unsigned gx, unsigned gy, unsigned gz, void *stream);",
          "",
          "// Launches on the default stream, waits, and stores the elapsed microseconds in *usec.",
          f"int32_t {sym}_launch_us(const {sym}_args_t *args, unsigned gx, unsigned gy, unsigned gz, "
          "uint32_t *usec);", "",
          "#ifdef __cplusplus", "}", "#endif", "", "#endif", ""]

    gchecks = [f"(long long)g{axis} != (long long){g.c(sub)}" for axis, g in zip("xyz", spec.grid) if g is not None]
    c = [f'#include "{sym}.h"', "", "#include <hip/hip_runtime_api.h>", "", '#include "piton_mi355x.h"', "",
         f"int32_t {sym}_launch(const {sym}_args_t *args, unsigned gx, unsigned gy, unsigned gz, void *stream) {{",
         "    (void)args;"]
    if gchecks:
        c.append(f"    if ({' || '.join(gchecks)}) return PITON_EINVAL;")
    if len(gchecks) < 3:
        c.append("    (void)gx; (void)gy; (void)gz;")
    for cond, _msg in spec.checks:
        c.append(f"    if (!{cond.c(sub)}) return PITON_EINVAL;")
    call = ", ".join(e.c(sub) for e in spec.call)
    c += [f"    return piton_mi355x_{spec.entry}({call}, stream);", "}", "",
          f"int32_t {sym}_launch_us(const {sym}_args_t *args, unsigned gx, unsigned gy, unsigned gz, "
          "uint32_t *usec) {",
          "    hipEvent_t e0, e1;",
          "    if (hipEventCreate(&e0) != hipSuccess) return PITON_EHIP;",
          "    if (hipEventCreate(&e1) != hipSuccess) { (void)hipEventDestroy(e0); return PITON_EHIP; }",
          "    int32_t rc = hipEventRecord(e0, 0) == hipSuccess ? PITON_OK : PITON_EHIP;",
          f"    if (rc == PITON_OK) rc = {sym}_launch(args, gx, gy, gz, 0);",
          "    if (rc == PITON_OK && hipEventRecord(e1, 0) != hipSuccess) rc = PITON_EHIP;",
          "    if (rc == PITON_OK && hipEventSynchronize(e1) != hipSuccess) rc = PITON_EHIP;",
          "    float ms = 0.f;",
          "    if (rc == PITON_OK && hipEventElapsedTime(&ms, e0, e1) != hipSuccess) rc = PITON_EHIP;",
          "    if (rc == PITON_OK && usec) *usec = (uint32_t)(ms * 1000.0f + 0.5f);",
          "    (void)hipEventDestroy(e0);",
          "    (void)hipEventDestroy(e1);",
          "    return rc;", "}", ""]
    return "\n".join(h), "\n".join(c)


def main(argv=None):
    ap = argparse.ArgumentParser(description="C launchers for a kernel of libpiton_mi355x.so")
    ap.add_argument("path", help="python file containing the kernel")
    ap.add_argument("--kernel-name", "-n", required=True)
    ap.add_argument("--signature", "-s", default="", help="name=type,... for runtime arguments")
    ap.add_argument("--constants", "-c", default="", help="name=value,... specialised arguments")
    ap.add_argument("--out-name", default=None)
    ap.add_argument("-o", "--out-dir", default=".")
    args = ap.parse_args(argv)
    kernel = load_kernel(args.path, args.kernel_name)
    name = args.out_name or args.kernel_name
    h, c = emit_c(args.kernel_name, _params_of(kernel), _parse_kv(args.signature), _parse_kv(args.constants), name)
    os.makedirs(args.out_dir, exist_ok=True)
    for ext, text in ((".h", h), (".c", c)):
        with open(os.path.join(args.out_dir, name + ext), "w") as f:
            f.write(text)
    print(os.path.join(args.out_dir, name + ".h"))
    print(os.path.join(args.out_dir, name + ".c"))


if __name__ == "__main__":
    main()
