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
