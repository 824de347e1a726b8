"""The drop-in boundary on any host: the C ABI library loads and exports every entry its
header declares, rejects bad arguments before touching a device, reports a missing device;
the launch surface binds arguments as PIton does (piton/runtime/launcher.py:42-63) and
checks grids before anything reaches the device."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest
import torch

import piton_amd
from piton_amd import language as tl
from piton_amd.kernels import attn_fwd_kernel, matmul_kernel, softmax_kernel
from piton_amd.runtime import launcher, mi355x
from ref_launch import RefJIT, patched_reference_call, ref_add_kernel, ref_matmul_kernel

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_entries():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        names += re.findall(r"PITON_API\s+[\w\s\*]+?\b(piton_mi355x_\w+)\s*\(", open(h).read())
    return sorted(set(names))


def test_library_exports_every_declared_entry():
    lib = mi355x.lib()
    names = declared_entries()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) >= set(mi355x.SIGNATURES)
    assert lib.piton_mi355x_abi_version() == mi355x.ABI_VERSION


def header_prototypes():
    """entry name -> list of parameter C types, parsed from include/*.h."""
    protos = {}
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for name, params in re.findall(r"PITON_API\s+[\w\s\*]+?\b(piton_mi355x_\w+)\s*\(([^)]*)\)", text):
            params = " ".join(params.split())
            protos[name] = [] if params == "void" else [p.strip() for p in params.split(",")]
    return protos


def _ctype_of(decl: str):
    decl = decl.replace("const ", "")
    if "*" in decl:
        return "ptr"
    t = decl.split()[0]
    return {"int64_t": "i64", "int32_t": "i32", "float": "f32"}[t]


def test_ctypes_signatures_match_the_header():
    protos = header_prototypes()
    names = {ctypes.c_void_p: "ptr", ctypes.c_int64: "i64", ctypes.c_int32: "i32", ctypes.c_float: "f32"}
    for entry, argtypes in mi355x.SIGNATURES.items():
        want = [_ctype_of(p) for p in protos[entry]]
        got = [names.get(a, "ptr") for a in argtypes]
        assert got == want, entry


def _raw():
    return mi355x.lib()


def test_invalid_arguments_fail_before_any_device_call():
    L = _raw()
    null = ctypes.c_void_p(0)
    rc = L.piton_mi355x_matmul(null, null, null, -1, 4, 4, 4, 1, 4, 1, 4, 1, 8, null)
    assert rc == mi355x.EINVAL and b"negative" in L.piton_mi355x_last_error()
    rc = L.piton_mi355x_matmul(null, null, null, 4, 4, 4, 4, 1, 4, 1, 4, 1, 0, null)
    assert rc == mi355x.EINVAL and b"GROUP_SIZE_M" in L.piton_mi355x_last_error()
    rc = L.piton_mi355x_softmax(null, null, 8, 8, 8, 4, 0, null)
    assert rc == mi355x.EINVAL
    rc = L.piton_mi355x_attn_fwd(null, null, null, null, 1.0, *([0] * 9), 16, 1, 48, 0, null)
    assert rc == mi355x.EUNSUPPORTED and b"HEAD_DIM" in L.piton_mi355x_last_error()
    rc = L.piton_mi355x_dense(null, null, null, null, 4, 4, 4, 1, 0, null, 0, null)
    assert rc == mi355x.EINVAL
    rc = L.piton_mi355x_layernorm(null, null, 0, 1e-5, 1, 1, null)
    assert rc == mi355x.EINVAL
    rc = L.piton_mi355x_layernorm(null, null, 9000, 1e-5, 0, 9000, null)
    assert rc == mi355x.EUNSUPPORTED


def test_size_checks_do_not_wrap():
    """Extents whose products overflow 64 bits are refused, not wrapped past the grid and offset
    checks (host buffers stand in for device ones: the checks run before any device call)."""
    L = _raw()
    null = ctypes.c_void_p(0)
    buf = np.zeros(4096, np.float32)
    p = ctypes.c_void_p(buf.ctypes.data)
    assert buf.ctypes.data % 16 == 0
    big = 1 << 40
    # heads x query groups: 2^62 heads x 2 groups
    rc = L.piton_mi355x_attn_fwd(p, p, p, p, 1.0, *([0] * 9), 64, 1 << 62, 64, 1, null)
    assert rc == mi355x.EUNSUPPORTED and b"exceed one grid" in L.piton_mi355x_last_error()
    # tiles: 2^34 x 2^34
    rc = L.piton_mi355x_transpose(p, p, big, big, big, big, null)
    assert rc == mi355x.EUNSUPPORTED and b"too large" in L.piton_mi355x_last_error()
    # cache offsets: (1 + 3) x 2^40 rows x 2^40 floats
    rc = L.piton_mi355x_decode_layer(p, 256, 1e-5, p, null, p, big, p, 256, 0.125, 1, big, 4, 64, 256,
                                     null, null, null, 0, null, null)
    assert rc == mi355x.EUNSUPPORTED and b"2 GiB" in L.piton_mi355x_last_error()


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device path")
def test_no_device_is_reported():
    with pytest.raises(mi355x.MI355XError) as e:
        mi355x.device_info()
    assert e.value.code == mi355x.ENODEV
    L = _raw()
    null = ctypes.c_void_p(0)
    # valid arguments, nothing to do, still needs a device
    assert L.piton_mi355x_add(null, null, null, 0, null) == mi355x.ENODEV


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(mi355x, "_lib", None)
    monkeypatch.setenv("PITON_MI355X_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="not built"):
        mi355x.lib()


# -- launch surface --------------------------------------------------------------------------------

def test_jit_surface():
    assert piton_amd.cdiv(10, 4) == 3 and piton_amd.next_power_of_2(1823) == 2048
    with pytest.raises(RuntimeError):
        matmul_kernel(1, 2)

    @piton_amd.jit
    def k(x_ptr, n, BLOCK: tl.constexpr = 4):
        pass

    assert k.arg_names == ["x_ptr", "n", "BLOCK"]
    assert repr(tl.constexpr(3)) == "constexpr[3]"


def test_bind_specialises_ones_and_constexprs():
    a = np.zeros((4, 4), np.float32)
    sig, const, vals = launcher.bind(matmul_kernel.fn, (a, a, a, 4, 4, 4, 4, 1, 4, 1, 4, 1),
                                     dict(BLOCK_SIZE_M=8, BLOCK_SIZE_N=8, BLOCK_SIZE_K=4, GROUP_SIZE_M=1))
    assert const["stride_ak"] == 1 and "stride_ak" not in vals
    assert const["GROUP_SIZE_M"] == 1 and const["BLOCK_SIZE_M"] == 8
    assert sig["a_ptr"] == "*fp32" and sig["M"] == "i32"
    with pytest.raises(TypeError):
        launcher.bind(matmul_kernel.fn, (a,), {})
    with pytest.raises(TypeError):
        launcher.bind(softmax_kernel.fn, (a.astype(np.float64), a, 4, 4, 4), dict(BLOCK_SIZE=4))


def test_plans_check_grids_before_the_device():
    a = np.zeros((4, 4), np.float32)
    args = (a, a, a, 4, 4, 4, 4, 1, 4, 1, 4, 1)
    kw = dict(BLOCK_SIZE_M=2, BLOCK_SIZE_N=2, BLOCK_SIZE_K=4, GROUP_SIZE_M=1)
    with pytest.raises(ValueError, match="grid"):
        matmul_kernel[(3,)](*args, **kw)
    _, const, vals = launcher.bind(matmul_kernel.fn, args, kw)
    entry, plan = launcher.plan(matmul_kernel, (4,), const, vals)
    assert entry == "matmul" and plan[3:6] == (4, 4, 4) and plan[7] == 1
    with pytest.raises(ValueError, match="EVEN_N"):
        attn_fwd_kernel[(1, 1)](a, a, a, a, 0.5, 16, 4, 16, 4, 1, 16, 4, 16, 4, 3, HEAD_DIM=4, BLOCK_M=4, BLOCK_N=2,
                                CAUSAL=True, EVEN_N=True)
    with pytest.raises(ValueError, match="unknown device"):
        softmax_kernel[(4,)](a, a, 4, 4, 4, BLOCK_SIZE=4, device="emu")


def test_unknown_kernels_are_refused():
    @piton_amd.jit
    def mandelbrot_kernel(out_ptr, x0, y0, step, width, max_iter, BLOCK: tl.constexpr):
        pass

    with pytest.raises(NotImplementedError):
        mandelbrot_kernel[(1,)](np.zeros(4, np.int32), -0.5, 0.0, 0.01, 4, 10, BLOCK=4)

    @piton_amd.jit
    def matmul_kernel(a_ptr, b_ptr, c_ptr, M, N, K):  # same name, other parameters
        pass

    with pytest.raises(NotImplementedError):
        launcher.lookup(matmul_kernel)


def test_tensor_checks():
    t = torch.zeros(16)
    with pytest.raises(ValueError, match="GPU"):
        mi355x.check_tensor("x", t)
    with pytest.raises(TypeError):
        mi355x.check_tensor("x", t.double())
    assert mi355x._span((4, 10), (3, 1)) == 32 and mi355x._span((0, 5)) == -1


# -- the reference-side hunks driven on any host ------------------------------------

@pytest.fixture
def host_entries(monkeypatch):
    """The library's entries replaced by host computations on CPU tensors, so that the binding,
    grid check, staging and copy-back run on a machine without a GPU."""
    calls = []

    def add(x, y, out, n):
        calls.append(("add", x, y, out, n))
        out[:n] = x[:n] + y[:n]

    def matmul(a, b, c, M, N, K, s_am, s_ak, s_bk, s_bn, s_cm, s_cn, group):
        calls.append(("matmul", M, N, K, s_am, s_ak, s_bk, s_bn, s_cm, s_cn, group))
        A = torch.as_strided(a, (M, K), (s_am, s_ak))
        B = torch.as_strided(b, (K, N), (s_bk, s_bn))
        torch.as_strided(c, (M, N), (s_cm, s_cn)).copy_(A @ B)

    monkeypatch.setattr(mi355x, "staging_device", lambda: "cpu")
    monkeypatch.setattr(mi355x, "synchronize", lambda: None)
    monkeypatch.setattr(mi355x, "last_launches", lambda: [{"kernel": "host"}])
    monkeypatch.setattr(mi355x, "add", add)
    monkeypatch.setattr(mi355x, "matmul", matmul)
    return calls


def test_reference_jit_object_with_numpy_arguments(host_entries):
    """numpy arrays are copied in and every array is copied back (launcher.py:175-180, 209-211);
    the grid is a callable of the launch's meta-parameters."""
    k = RefJIT(ref_add_kernel)
    n = 37
    x = np.arange(n, dtype=np.float32)
    y = np.full(n, 0.5, np.float32)
    out = np.full(n + 16, 7.0, np.float32)
    rec = patched_reference_call(k, lambda meta: (piton_amd.cdiv(n, meta["BLOCK_SIZE"]),), x, y, out, n,
                                 BLOCK_SIZE=16)
    np.testing.assert_array_equal(out[:n], x + y)
    assert (out[n:] == 7.0).all()
    np.testing.assert_array_equal(x, np.arange(n, dtype=np.float32))
    name, tx, ty, tout, nn = host_entries[0]
    assert name == "add" and nn == n and tx.device.type == "cpu" and tout.numel() == n + 16
    assert rec.entry == "piton_mi355x_add" and rec.grid == (3,) and rec.signature["x_ptr"] == "*fp32"
    assert rec.last_stats["bytes"] == 12 * n and rec.last_stats["launches"] == [{"kernel": "host"}]


def test_reference_jit_object_with_tensors_and_unit_strides(host_entries):
    """Tensor arguments pass through by reference; strides equal to 1 arrive as constants and
    still reach the entry; the grid is checked before the entry is called."""
    k = RefJIT(ref_matmul_kernel)
    M, N, K = 5, 7, 3
    a = torch.arange(M * K, dtype=torch.float32).reshape(M, K)
    b = torch.ones(K, N)
    c = torch.zeros(M, N)
    kw = dict(BLOCK_SIZE_M=4, BLOCK_SIZE_N=4, BLOCK_SIZE_K=4, GROUP_SIZE_M=8, num_warps=4)
    args = (a, b, c, M, N, K, K, 1, N, 1, N, 1)
    with pytest.raises(ValueError, match="grid"):
        patched_reference_call(k, (3,), *args, **kw)
    assert host_entries == []
    rec = patched_reference_call(k, (4,), *args, **kw)
    assert host_entries[0] == ("matmul", M, N, K, K, 1, N, 1, N, 1, 8)
    torch.testing.assert_close(c, a @ b)
    assert rec.constants["stride_ak"] == 1 and rec.last_stats["flops"] == 2 * M * N * K


def test_reference_sig_of_rejects_other_tensor_dtypes():
    k = RefJIT(ref_add_kernel)
    x = torch.zeros(4, dtype=torch.float64)
    with pytest.raises(TypeError, match="tensor dtype"):
        patched_reference_call(k, (1,), x, x, x, 4, BLOCK_SIZE=4)
