"""The AOT C launchers (piton_amd/aot.py; piton/tools/compile.py:55-172 is the reference's):
generated headers and sources compile as C, the grid check refuses other covers before any
device call, the launch reaches the library, and on a GPU the C launchers' results match float64
and the oracle at config shapes."""
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
                       "BLOCK_SIZE=2048"),
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
    params = aot.KERNELS["add_kernel"].params
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


def _launchers(tmp_path, kernels):
    srcs = [generate(tmp_path, k, k.replace("_kernel", "")) for k in kernels]
    so = tmp_path / "liblaunchers.so"
    r = subprocess.run([GCC, *cflags(), "-fPIC", "-shared", *srcs, "-o", str(so), *link_flags()],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return ctypes.CDLL(str(so))


def _struct(kernel):
    """The ctypes twin of a generated <name>_args_t (fields in --signature order)."""
    sig, _ = SPECS[kernel]
    ctype = {"*fp32": ctypes.c_void_p, "*i32": ctypes.c_void_p, "i32": ctypes.c_int32, "fp32": ctypes.c_float}
    fields = [(n, ctype[t]) for n, t in (item.split("=") for item in sig.split(","))]
    return type(kernel + "_args", (ctypes.Structure,), {"_fields_": fields})


@pytest.mark.gpu
def test_c_launchers_against_the_oracle(tmp_path):
    """Config shapes through generated C launchers, called with device pointers: the ragged
    1000 x 1800 x 700 matmul with padded row strides, softmax over 1823 columns (BLOCK_SIZE
    2048), causal attention, and the dense layer; each checked against float64 and the oracle
    (the emulator's arithmetic), and bit-identical to the ctypes launch of the same library."""
    import numpy as np
    import torch

    import oracle
    from oracle import fp64
    L = _launchers(tmp_path, ["matmul_kernel", "softmax_kernel", "attn_fwd_kernel", "dense_layer_kernel"])
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rng = np.random.default_rng(11)

    # matmul, ragged with padded strides (lda 703, ldb 1805, ldc 1807)
    M, N, K, lda, ldb, ldc = 1000, 1800, 700, 703, 1805, 1807
    a = rng.uniform(-1, 1, (M, lda)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, ldb)).astype(np.float32)
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    tc, tc2 = (torch.full((M, ldc), -3.0, device="cuda") for _ in range(2))
    args = _struct("matmul_kernel")(ta.data_ptr(), tb.data_ptr(), tc.data_ptr(), M, N, K, lda, ldb, ldc)
    assert L.matmul_launch(ctypes.byref(args), 8 * 15, 1, 1, stream) == 0
    assert L.matmul_launch(ctypes.byref(args), 8 * 15 + 1, 1, 1, stream) == -1
    mi355x.matmul(ta, tb, tc2, M, N, K, lda, 1, ldb, 1, ldc, 1, 8)
    torch.cuda.synchronize()
    assert torch.equal(tc, tc2)
    c = tc.cpu().numpy()
    assert (c[:, N:] == -3.0).all()
    ref = fp64.matmul(a[:, :K], b[:, :N])
    assert fp64.rel_fro(c[:, :N], ref) <= 1e-5
    rows = slice(0, 64)
    orc = np.asarray(oracle.matmul_fast(np.ascontiguousarray(a[rows, :K]), np.ascontiguousarray(b[:, :N])))
    assert fp64.rel_fro(c[rows, :N], ref[rows]) <= fp64.rel_fro(orc, ref[rows])

    # softmax, 1823 columns
    x = (rng.standard_normal((257, 1823)) * 4).astype(np.float32)
    tx = torch.from_numpy(x).cuda()
    ty, ty2 = torch.zeros_like(tx), torch.zeros_like(tx)
    sargs = _struct("softmax_kernel")(ty.data_ptr(), tx.data_ptr(), 1823, 1823, 1823)
    assert L.softmax_launch(ctypes.byref(sargs), 257, 1, 1, stream) == 0
    mi355x.softmax(ty2, tx, 1823, 1823, 1823, 257, 2048)
    torch.cuda.synchronize()
    assert torch.equal(ty, ty2)
    err = fp64.rel_fro(ty.cpu().numpy(), fp64.softmax(x))
    assert err <= 1e-5 and err <= fp64.rel_fro(oracle.softmax(x, 1823, 2048), fp64.softmax(x))

    # causal attention, 4 heads x 256 x 64
    H, Nc, D = 4, 256, 64
    q, k, v = (rng.standard_normal((H, Nc, D)).astype(np.float32) for _ in range(3))
    tq, tk, tv = (torch.from_numpy(t).cuda() for t in (q, k, v))
    to = torch.zeros_like(tq)
    at = _struct("attn_fwd_kernel")(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), to.data_ptr(), 0.125, Nc * D, D,
                                    Nc * D, D, Nc * D, D, Nc * D, D, Nc)
    assert L.attn_fwd_launch(ctypes.byref(at), Nc // 32, H, 1, stream) == 0
    torch.cuda.synchronize()
    ref = fp64.attention_reference(q, k, v, True, 0.125)
    err = fp64.rel_fro(to.cpu().numpy(), ref)
    assert err <= 1e-5 and err <= fp64.rel_fro(oracle.attention(q, k, v, True, 0.125, block_n=32), ref)

    # dense + bias + ReLU (N = 128, K = 64 specialised), dyadic inputs: bit-exact
    m = 1797
    xd = (rng.integers(-4, 5, (m, 64)) / 4).astype(np.float32)
    wd = (rng.integers(-4, 5, (64, 128)) / 4).astype(np.float32)
    bd = (rng.integers(-8, 9, 128) / 4).astype(np.float32)
    txd, twd, tbd = (torch.from_numpy(t).cuda() for t in (xd, wd, bd))
    yd = torch.zeros((m, 128), device="cuda")
    dargs = _struct("dense_layer_kernel")(txd.data_ptr(), twd.data_ptr(), tbd.data_ptr(), yd.data_ptr(), m)
    assert L.dense_layer_launch(ctypes.byref(dargs), (m + 3) // 4 * 2, 1, 1, stream) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(yd.cpu().numpy(), oracle.dense(xd, wd, bd, True))

    usec = ctypes.c_uint32(0)
    assert L.matmul_launch_us(ctypes.byref(args), 8 * 15, 1, 1, ctypes.byref(usec)) == 0 and usec.value > 0
