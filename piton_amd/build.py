"""Builds libpiton_mi355x.so (gfx950) from piton_amd/csrc/*.hip with hipcc, in-tree.

    python -m piton_amd.build [--verbose]

Each source compiles to an object in piton_amd/_build/ in parallel, then they link into
piton_amd/lib/libpiton_mi355x.so. Every call compiles again (the build is the check that the
sources build); objects whose source and headers are older than the object are reused only
when `incremental=True`.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libpiton_mi355x.so")
ARCH = "gfx950"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm toolchain required to build libpiton_mi355x.so)")
    return path


COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Wall", "-Wno-unused-result",
    # packed FP32 instructions are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-I", os.path.join(ROOT, "include"),
]


def _newer(src: str, obj: str, deps) -> bool:
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(p) > t for p in [src, *deps])


def build(verbose: bool = False, incremental: bool = False, extra_flags=(), obj_dir: str = OBJ,
          lib: str = LIB) -> str:
    """Compiles every csrc/*.hip for gfx950 into obj_dir and links `lib` (by default the product
    library; piton_amd.phase_trace builds its traced copy beside it with its own paths)."""
    os.makedirs(obj_dir, exist_ok=True)
    os.makedirs(os.path.dirname(lib), exist_ok=True)
    cc = hipcc()
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    deps = glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(ROOT, "include", "*.h"))
    flags = COMMON_FLAGS + list(extra_flags)

    def compile_one(src):
        obj = os.path.join(obj_dir, os.path.basename(src)[:-4] + ".o")
        if incremental and not _newer(src, obj, deps):
            return obj, ""
        cmd = [cc, *flags, "-c", src, "-o", obj + ".tmp"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{r.stderr[-6000:]}")
        os.replace(obj + ".tmp", obj)
        return obj, r.stderr

    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(compile_one, srcs))
    if verbose:
        for obj, err in results:
            if err.strip():
                print(f"--- {os.path.basename(obj)}\n{err}")
    objs = [o for o, _ in results]
    tmp = lib + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-Wl,-rpath,/opt/rocm/lib", "-Wl,--no-undefined"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--incremental", action="store_true")
    ap.add_argument("--resource-usage", action="store_true",
                    help="print each kernel's registers, LDS and occupancy")
    a = ap.parse_args()
    extra = ["-Rpass-analysis=kernel-resource-usage"] if a.resource_usage else []
    print(build(verbose=a.verbose or a.resource_usage, incremental=a.incremental, extra_flags=extra))
