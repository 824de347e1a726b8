"""The AOT C launchers (piton_amd/aot.py; piton/tools/compile.py:55-172 is the reference's):
generated headers and sources compile as C, the grid check refuses other covers before any
device call, the launch reaches the library, and on a GPU a C launcher computes what the
Python launch surface computes."""
import ctypes
import os
import shutil
import subprocess

import pytest

from piton_amd import aot
from piton_amd.runtime import mi355x

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = "/opt/rocm"
GCC = shutil.which("gcc")
pytestmark = pytest.mark.skipif(GCC is None, reason="gcc not found")

MATMUL_SIG = ("a_ptr=*fp32,b_ptr=*fp32,c_ptr=*fp32,M=i32,N=i32,K=i32,stride_am=i32,stride_bk=i32,stride_cm=i32")
MATMUL_CONST = "stride_ak=1,stride_bn=1,stride_cn=1,BLOCK_SIZE_M=128,BLOCK_SIZE_N=128,BLOCK_SIZE_K=32,GROUP_SIZE_M=8"

SPECS = {
    "matmul_kernel": (MATMUL_SIG, MATMUL_CONST),
    "softmax_kernel": ("output_ptr=*fp32,input_ptr=*fp32,input_row_stride=i32,output_row_stride=i32,n_cols=i32",
                       "BLOCK_SIZE=1024"),
    "attn_fwd_kernel": ("Q=*fp32,K=*fp32,V=*fp32,Out=*fp32,sm_scale=fp32,stride_qh=i32,stride_qm=i32,stride_kh=i32,"
                        "stride_kn=i32,stride_vh=i32,stride_vn=i32,stride_oh=i32,stride_om=i32,N_CTX=i32",
                        "stride_kk=1,HEAD_DIM=64,BLOCK_M=32,BLOCK_N=32,CAUSAL=True,EVEN_N=False"),
    "dense_layer_kernel": ("x_ptr=*fp32,w_ptr=*fp32,bias_ptr=*fp32,y_ptr=*fp32,M=i32",
                           "N=128,K=64,BLOCK_SIZE_M=4,BLOCK_SIZE_N=64,BLOCK_SIZE_K=4,GROUP_SIZE_M=1,ADD_BIAS=True,"
                           "RELU=True"),
    "add_kernel": ("x_ptr=*fp32,y_ptr=*fp32,output_ptr=*fp32,n_elements=i32", "BLOCK_SIZE=1024"),
    "layernorm_kernel": ("x_ptr=*fp32,out_ptr=*fp32,n=i32,eps=fp32", "BLOCK=256"),
    "fma_kernel": ("x_ptr=*fp32,y_ptr=*fp32,out_ptr=*fp32,n=i32,alpha=fp32", "BLOCK=256"),
    "sfu_kernel": ("x_ptr=*fp32,out_ptr=*fp32,n=i32", "OP=4,BLOCK=256"),
    "idiv_kernel": ("x_ptr=*i32,y_ptr=*i32,q_ptr=*i32,r_ptr=*i32,n=i32", "BLOCK=256"),
    "row_sum_kernel": ("x_ptr=*fp32,out_ptr=*fp32,n_cols=i32,stride=i32", "BLOCK_M=4,BLOCK_N=64"),
    "transpose_kernel": ("x_ptr=*fp32,out_ptr=*fp32,n_rows=i32,n_cols=i32,stride_x=i32,stride_out=i32",
                         "BLOCK_M=16,BLOCK_N=16"),
}
KERNEL_FILES = {"matmul_kernel": "tutorial.py", "softmax_kernel": "tutorial.py", "add_kernel": "tutorial.py",
                "layernorm_kernel": "tutorial.py", "attn_fwd_kernel": "attention.py", "dense_layer_kernel": "nn.py",
                "fma_kernel": "primitives.py", "sfu_kernel": "primitives.py", "idiv_kernel": "primitives.py",
                "row_sum_kernel": "primitives.py", "transpose_kernel": "primitives.py"}


def generate(tmp, kernel, name):
    sig, const = SPECS[kernel]
    path = os.path.join(ROOT, "piton_amd", "kernels", KERNEL_FILES[kernel])
    aot.main([path, "--kernel-name", kernel, "--signature", sig, "--constants", const, "--out-name", name,
              "-o", str(tmp)])
    return os.path.join(tmp, name + ".c")


def cflags():
    return ["-std=c99", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
            "-I", os.path.join(ROCM, "include")]


def link_flags():
    lib = os.path.dirname(mi355x.library_path())
    return ["-L", lib, "-Wl,-rpath," + lib, "-lpiton_mi355x", "-L", os.path.join(ROCM, "lib"),
            "-Wl,-rpath," + os.path.join(ROCM, "lib"), "-lamdhip64"]


@pytest.mark.parametrize("kernel", sorted(SPECS))
def test_generated_sources_compile_as_c(tmp_path, kernel):
    src = generate(tmp_path, kernel, kernel.replace("_kernel", ""))
    r = subprocess.run([GCC, *cflags(), "-c", src, "-o", str(tmp_path / "x.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    header = open(src[:-2] + ".h").read()
    assert "_args_t;" in header and "_launch(" in header and "_launch_us(" in header


def test_grid_check_and_dispatch_without_a_device(tmp_path):
    """A C program: a wrong grid is refused (-1) before the library is called; the canonical
    grid reaches the library, which reports no device (-4) in a container without a GPU."""
    if not os.path.exists(mi355x.library_path()):
        pytest.skip("libpiton_mi355x.so not built")
    src = generate(tmp_path, "matmul_kernel", "matmul")
    main = tmp_path / "main.c"
    main.write_text("""
#include <stdio.h>
#include "matmul.h"
int main(void) {
    matmul_args_t a = {0};
    /* placeholders that pass the library's null and alignment checks; nothing reads them,
       since the device check comes first */
    a.a_ptr = (float *)64; a.b_ptr = (float *)128; a.c_ptr = (float *)192;
    a.M = 1000; a.N = 300; a.K = 64; a.stride_am = 64; a.stride_bk = 300; a.stride_cm = 300;
    printf("%d %d\\n", matmul_launch(&a, 7, 1, 1, 0), matmul_launch(&a, 24, 1, 1, 0));
    return 0;
}
""")
    exe = tmp_path / "main"
    r = subprocess.run([GCC, *cflags(), "-I", str(tmp_path), str(main), src, "-o", str(exe), *link_flags()],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    env = dict(os.environ, HIP_VISIBLE_DEVICES="")  # no device, whatever the host has
    out = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert out.returncode == 0, out.stderr
    wrong, right = map(int, out.stdout.split())
    assert wrong == -1  # cdiv(1000, 128) * cdiv(300, 128) = 8 * 3 = 24 programs, not 7
    assert right == -4


def test_bad_specifications_are_refused():
    params = aot.KERNELS["add_kernel"]["params"]
    with pytest.raises(TypeError, match="missing"):
        aot.emit_c("add_kernel", params, {"x_ptr": "*fp32"}, {}, "x")
    with pytest.raises(TypeError, match="unsupported type"):
        aot.emit_c("add_kernel", params, {"x_ptr": "*fp64", "y_ptr": "*fp32", "output_ptr": "*fp32",
                                          "n_elements": "i32"}, {"BLOCK_SIZE": 4}, "x")
    with pytest.raises(ValueError, match="both"):
        aot.emit_c("add_kernel", params, {"x_ptr": "*fp32", "y_ptr": "*fp32", "output_ptr": "*fp32",
                                          "n_elements": "i32"}, {"BLOCK_SIZE": 4, "n_elements": 3}, "x")
    with pytest.raises(NotImplementedError):
        aot.emit_c("nope_kernel", params, {}, {}, "x")


@pytest.mark.gpu
def test_c_launchers_compute_what_the_launch_surface_computes(tmp_path):
    """matmul and softmax through generated C launchers (built into a shared object, called
    with device pointers) equal the ctypes launch of the same library bit for bit."""
    import torch
    srcs = [generate(tmp_path, "matmul_kernel", "matmul"), generate(tmp_path, "softmax_kernel", "softmax")]
    so = tmp_path / "liblaunchers.so"
    r = subprocess.run([GCC, *cflags(), "-fPIC", "-shared", *srcs, "-o", str(so), *link_flags()],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    L = ctypes.CDLL(str(so))
    M, N, K = 300, 200, 72
    g = torch.Generator(device="cuda").manual_seed(3)
    a, b = torch.rand((M, K), device="cuda", generator=g), torch.rand((K, N), device="cuda", generator=g)
    c_aot, c_ref = torch.zeros((M, N), device="cuda"), torch.zeros((M, N), device="cuda")

    class MatmulArgs(ctypes.Structure):
        _fields_ = [("a_ptr", ctypes.c_void_p), ("b_ptr", ctypes.c_void_p), ("c_ptr", ctypes.c_void_p),
                    ("M", ctypes.c_int32), ("N", ctypes.c_int32), ("K", ctypes.c_int32),
                    ("stride_am", ctypes.c_int32), ("stride_bk", ctypes.c_int32), ("stride_cm", ctypes.c_int32)]

    args = MatmulArgs(a.data_ptr(), b.data_ptr(), c_aot.data_ptr(), M, N, K, K, N, N)
    usec = ctypes.c_uint32(0)
    torch.cuda.synchronize()
    assert L.matmul_launch_us(ctypes.byref(args), 3 * 2, 1, 1, ctypes.byref(usec)) == 0
    mi355x.matmul(a, b, c_ref, M, N, K, K, 1, N, 1, N, 1, 8)
    torch.cuda.synchronize()
    assert torch.equal(c_aot, c_ref)
    assert usec.value >= 0

    class SoftmaxArgs(ctypes.Structure):
        _fields_ = [("output_ptr", ctypes.c_void_p), ("input_ptr", ctypes.c_void_p),
                    ("input_row_stride", ctypes.c_int32), ("output_row_stride", ctypes.c_int32),
                    ("n_cols", ctypes.c_int32)]

    x = torch.randn((64, 1000), device="cuda", generator=g)
    y_aot, y_ref = torch.zeros_like(x), torch.zeros_like(x)
    sargs = SoftmaxArgs(y_aot.data_ptr(), x.data_ptr(), 1000, 1000, 1000)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.softmax_launch(ctypes.byref(sargs), 64, 1, 1, stream) == 0
    mi355x.softmax(y_ref, x, 1000, 1000, 1000, 64, 1024)
    torch.cuda.synchronize()
    assert torch.equal(y_aot, y_ref)
    assert L.softmax_launch(ctypes.byref(sargs), 64, 2, 1, stream) == -1
