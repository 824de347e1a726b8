"""ctypes binding of libpiton_mi355x.so and the Python entries over it.

Loading order matters on ROCm: torch is imported first, so the library's libamdhip64.so.7
dependency resolves to the HIP runtime torch already loaded (one runtime per process, shared
device memory and streams).

Every entry takes torch tensors already on the GPU (float32 / int32), checks dtype, device
and that the elements the kernel addresses lie inside each tensor's storage, then launches
on torch's current stream. A missing library or a failed call raises; there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG = os.path.dirname(_HERE)
DEFAULT_LIB = os.path.join(_PKG, "lib", "libpiton_mi355x.so")

ABI_VERSION = 1
OK, EINVAL, EUNSUPPORTED, EHIP, ENODEV = 0, -1, -2, -3, -4

_lock = threading.Lock()
_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


class DeviceInfo(ctypes.Structure):
    _fields_ = [("cu_count", ctypes.c_int32), ("max_clock_khz", ctypes.c_int32),
                ("mem_clock_khz", ctypes.c_int32), ("mem_bus_width", ctypes.c_int32),
                ("hbm_bytes", ctypes.c_int64), ("lds_per_cu", ctypes.c_int32),
                ("l2_bytes", ctypes.c_int32), ("wavefront_size", ctypes.c_int32),
                ("xcd_count", ctypes.c_int32), ("arch", ctypes.c_char * 64)]


class LaunchInfo(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_char * 96), ("grid", ctypes.c_uint32 * 3), ("block", ctypes.c_uint32 * 3),
                ("lds_bytes", ctypes.c_uint32), ("vgprs", ctypes.c_int32), ("scratch_bytes", ctypes.c_uint32)]


# entry name -> argtypes (every entry returns int32)
SIGNATURES = {
    "piton_mi355x_device_info": [ctypes.POINTER(DeviceInfo)],
    "piton_mi355x_last_launches": [ctypes.POINTER(LaunchInfo), _i32, ctypes.POINTER(_i32)],
    "piton_mi355x_matmul": [_p, _p, _p] + [_i64] * 9 + [_i32, _p],
    "piton_mi355x_softmax": [_p, _p] + [_i64] * 5 + [_p],
    "piton_mi355x_attn_fwd": [_p, _p, _p, _p, _f32] + [_i64] * 11 + [_i32, _i32, _p],
    "piton_mi355x_dense": [_p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _p, _i32, _p],
    "piton_mi355x_add": [_p, _p, _p, _i64, _p],
    "piton_mi355x_layernorm": [_p, _p, _i64, _f32, _i64, _i64, _p],
    "piton_mi355x_argmax_rows": [_p, _i64, _i64, _i64, _p, _p],
    "piton_mi355x_embedding": [_p, _i64, _i64, _p, _p, _p] + [_i64] * 7 + [_p, _p],
    "piton_mi355x_linear": [_p, _i64, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64, _i32, _p],
    "piton_mi355x_linear_ln": [_p, _i64, _f32, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64, _i32, _p],
    "piton_mi355x_mlp3": [_p, _i64] + [_p] * 6 + [_i64] * 4 + [_p, _p, _i32, _p],
    "piton_mi355x_attn_fwd_batched": [_p, _p, _p, _p, _f32] + [_i64] * 16 + [_i32, _i32, _p],
    "piton_mi355x_attn_decode": [_p, _p, _p, _p, _f32] + [_i64] * 13 + [_i32, _p],
    "piton_mi355x_decode_layer": [_p, _i64, _f32, _p, _p, _p, _i64, _p, _i64, _f32, _i64, _i64, _i64, _i32, _i64,
                                  _p, _p, _p, _i64, _p, _p],
    "piton_mi355x_lm_head_argmax": [_p, _i64, _f32, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i32, _p],
    "piton_mi355x_copy": [_p, _p, _i64, _p],
    "piton_mi355x_mfma_probe": [_p, _i64, _i32, _p],
    "piton_mi355x_mul": [_p, _p, _p, _i64, _p],
    "piton_mi355x_fma": [_p, _p, _p, _i64, _f32, _p],
    "piton_mi355x_scaled_relu": [_p, _p, _i64, _f32, _p],
    "piton_mi355x_sfu": [_p, _p, _i64, _i32, _p],
    "piton_mi355x_log": [_p, _p, _i64, _p],
    "piton_mi355x_idiv": [_p, _p, _p, _p, _i64, _p],
    "piton_mi355x_row_sum": [_p, _p, _i64, _i64, _i64, _p],
    "piton_mi355x_row_max": [_p, _p, _i64, _i64, _i64, _p],
    "piton_mi355x_transpose": [_p, _p, _i64, _i64, _i64, _i64, _p],
}


class MI355XError(RuntimeError):
    """A failed library call: .code is the status (-1 .. -4), the message the library's."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


def library_path() -> str:
    return os.environ.get("PITON_MI355X_LIB", DEFAULT_LIB)


def lib():
    """The loaded library (loaded once). Raises RuntimeError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = library_path()
            if not os.path.exists(path):
                raise RuntimeError(f"{path} is not built: run `python -m piton_amd.build` "
                                   "(or __graft_entry__.build()) first")
            L = ctypes.CDLL(path)
            L.piton_mi355x_abi_version.restype = ctypes.c_int32
            L.piton_mi355x_abi_version.argtypes = []
            L.piton_mi355x_last_error.restype = ctypes.c_char_p
            L.piton_mi355x_last_error.argtypes = []
            for name, argtypes in SIGNATURES.items():
                f = getattr(L, name)
                f.argtypes = argtypes
                f.restype = ctypes.c_int32
            v = L.piton_mi355x_abi_version()
            if v != ABI_VERSION:
                raise RuntimeError(f"{path} has ABI {v}, expected {ABI_VERSION}")
            _lib = L
    return _lib


def _call(name: str, *args) -> None:
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != OK:
        msg = L.piton_mi355x_last_error().decode(errors="replace")
        if rc == EINVAL:
            raise ValueError(f"{name}: {msg}")
        raise MI355XError(rc, f"{name}: {msg}")


def device_info() -> dict:
    info = DeviceInfo()
    _call("piton_mi355x_device_info", ctypes.byref(info))
    d = {k: getattr(info, k) for k, _ in DeviceInfo._fields_}
    d["arch"] = info.arch.decode()
    return d


def last_launches() -> list:
    """The kernel launches of this thread's last entry call: kernel name, grid, block, LDS bytes
    per workgroup, vector registers and spill bytes per lane."""
    infos = (LaunchInfo * 8)()
    n = ctypes.c_int32(0)
    _call("piton_mi355x_last_launches", infos, 8, ctypes.byref(n))
    return [{"kernel": i.kernel.decode(), "grid": tuple(i.grid), "block": tuple(i.block), "lds_bytes": i.lds_bytes,
             "vgprs": i.vgprs, "scratch_bytes": i.scratch_bytes} for i in infos[:min(n.value, 8)]]


def staging_device() -> str:
    """Where numpy arguments of a launch are copied before the call."""
    return "cuda"


def synchronize() -> None:
    """Waits for the work queued on torch's current stream."""
    torch.cuda.current_stream().synchronize()


# -- argument checks ---------------------------------------------------------------------------

def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _avail(t: torch.Tensor) -> int:
    """Elements from t's first element to the end of its storage."""
    return t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()


def check_tensor(name: str, t, dtype=torch.float32, max_offset: int | None = None, allow_none=False):
    """t must be a GPU tensor of `dtype` whose storage holds element offsets 0..max_offset."""
    if t is None:
        if allow_none:
            return None
        raise ValueError(f"{name}: a tensor is required")
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: tensor on {t.device}, expected a ROCm GPU tensor")
    if max_offset is not None and max_offset >= 0 and max_offset >= _avail(t):
        raise ValueError(f"{name}: the kernel addresses element {max_offset} but the storage holds "
                         f"{_avail(t)} from the tensor's start")
    return t


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _span(*pairs) -> int:
    """Largest element offset sum((n_i - 1) * stride_i) of an access pattern; -1 if empty."""
    off = 0
    for n, s in pairs:
        if n <= 0:
            return -1
        if s < 0:
            raise ValueError("negative strides are not supported")
        off += (n - 1) * s
    return off


# -- entries -------------------------------------------------------------------------------------

def matmul(a, b, c, M, N, K, s_am, s_ak, s_bk, s_bn, s_cm, s_cn, group_size_m=8):
    """C = A B (matmul_kernel, examples/kernels.py:18-57) on torch tensors."""
    check_tensor("a", a, max_offset=_span((M, s_am), (K, s_ak)))
    check_tensor("b", b, max_offset=_span((K, s_bk), (N, s_bn)))
    check_tensor("c", c, max_offset=_span((M, s_cm), (N, s_cn)))
    _call("piton_mi355x_matmul", _ptr(a), _ptr(b), _ptr(c), M, N, K, s_am, s_ak, s_bk, s_bn, s_cm, s_cn,
          int(group_size_m), _stream())


def softmax(out, inp, in_row_stride, out_row_stride, n_cols, n_rows, block_size):
    """softmax_kernel (examples/kernels.py:60-76) over n_rows rows."""
    n = min(int(n_cols), int(block_size))
    check_tensor("input", inp, max_offset=_span((n_rows, in_row_stride), (n, 1)))
    check_tensor("output", out, max_offset=_span((n_rows, out_row_stride), (n, 1)))
    _call("piton_mi355x_softmax", _ptr(out), _ptr(inp), in_row_stride, out_row_stride, n_cols, n_rows,
          int(block_size), _stream())


def attn_fwd(q, k, v, out, sm_scale, s_qh, s_qm, s_kh, s_kn, s_kk, s_vh, s_vn, s_oh, s_om, n_ctx, heads,
             head_dim, causal):
    """attn_fwd_kernel (examples/attention.py:67-113) for `heads` heads."""
    check_tensor("Q", q, max_offset=_span((heads, s_qh), (n_ctx, s_qm), (head_dim, 1)))
    check_tensor("K", k, max_offset=_span((heads, s_kh), (n_ctx, s_kn), (head_dim, s_kk)))
    check_tensor("V", v, max_offset=_span((heads, s_vh), (n_ctx, s_vn), (head_dim, 1)))
    check_tensor("Out", out, max_offset=_span((heads, s_oh), (n_ctx, s_om), (head_dim, 1)))
    _call("piton_mi355x_attn_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(out), float(sm_scale), s_qh, s_qm, s_kh,
          s_kn, s_kk, s_vh, s_vn, s_oh, s_om, n_ctx, heads, int(head_dim), int(bool(causal)), _stream())


def dense(x, w, bias, y, M, N, K, add_bias=True, relu=False, argmax_out=None, n_classes=0):
    """dense_layer_kernel (examples/nn_kernels.py:23-74): Y = [ReLU](X W [+ b]), with an
    optional per-row argmax over the first n_classes outputs."""
    check_tensor("x", x, max_offset=M * K - 1)
    check_tensor("w", w, max_offset=K * N - 1)
    check_tensor("bias", bias, max_offset=N - 1, allow_none=not add_bias)
    check_tensor("y", y, max_offset=M * N - 1)
    check_tensor("argmax", argmax_out, dtype=torch.int32, max_offset=M - 1, allow_none=True)
    _call("piton_mi355x_dense", _ptr(x), _ptr(w), _ptr(bias if add_bias else None), _ptr(y), M, N, K,
          int(bool(add_bias)), int(bool(relu)), _ptr(argmax_out), int(n_classes), _stream())


def add(x, y, out, n):
    """add_kernel (examples/kernels.py:6-15)."""
    for name, t in (("x", x), ("y", y), ("output", out)):
        check_tensor(name, t, max_offset=n - 1)
    _call("piton_mi355x_add", _ptr(x), _ptr(y), _ptr(out), n, _stream())


def layernorm(x, out, n, eps, rows, row_stride):
    """layernorm_kernel (tests/test_reroll_reduce.py:199-208)."""
    check_tensor("x", x, max_offset=_span((rows, row_stride), (n, 1)))
    check_tensor("out", out, max_offset=_span((rows, row_stride), (n, 1)))
    _call("piton_mi355x_layernorm", _ptr(x), _ptr(out), n, float(eps), rows, row_stride, _stream())


def argmax_rows(x, rows, ld, n, out):
    check_tensor("x", x, max_offset=_span((rows, ld), (n, 1)))
    check_tensor("out", out, dtype=torch.int32, max_offset=rows - 1)
    _call("piton_mi355x_argmax_rows", _ptr(x), rows, ld, n, _ptr(out), _stream())


def embedding(ids, ids_sb, ids_st, tok, pos, out, out_sb, out_st, batch, T, d_model, vocab, pos_offset,
              err_flag=None):
    """out[b, t, :] = tok[ids[b, t]] + pos[pos_offset + t] through element strides."""
    check_tensor("ids", ids, dtype=torch.int32, max_offset=_span((batch, ids_sb), (T, ids_st)))
    check_tensor("tok", tok, max_offset=vocab * d_model - 1)
    check_tensor("pos", pos, max_offset=(pos_offset + T) * d_model - 1)
    check_tensor("out", out, max_offset=_span((batch, out_sb), (T, out_st), (d_model, 1)))
    check_tensor("err_flag", err_flag, dtype=torch.int32, max_offset=0, allow_none=True)
    _call("piton_mi355x_embedding", _ptr(ids), ids_sb, ids_st, _ptr(tok), _ptr(pos), _ptr(out), out_sb, out_st, batch,
          T, d_model, vocab, pos_offset, _ptr(err_flag), _stream())


def linear(x, ldx, w, bias, residual, ldr, y, ldy, M, N, K, relu=False):
    """Y = [ReLU](X W [+ b]) [+ R] over strided rows (the decoder's projections)."""
    check_tensor("x", x, max_offset=_span((M, ldx), (K, 1)))
    check_tensor("w", w, max_offset=K * N - 1)
    check_tensor("bias", bias, max_offset=N - 1, allow_none=True)
    check_tensor("residual", residual, max_offset=_span((M, ldr), (N, 1)), allow_none=True)
    check_tensor("y", y, max_offset=_span((M, ldy), (N, 1)))
    _call("piton_mi355x_linear", _ptr(x), ldx, _ptr(w), _ptr(bias), _ptr(residual), ldr, _ptr(y), ldy, M, N, K,
          int(bool(relu)), _stream())


def linear_ln(x, ldx, eps, w, bias, residual, ldr, y, ldy, M, N, K, relu=False):
    """Y = [ReLU](LN(X) W [+ b]) [+ R]: layernorm then linear in one launch, bit-identical to the
    two (M <= 64, K % 256 == 0, 16-byte X rows; else MI355XError with status -2)."""
    check_tensor("x", x, max_offset=_span((M, ldx), (K, 1)))
    check_tensor("w", w, max_offset=K * N - 1)
    check_tensor("bias", bias, max_offset=N - 1, allow_none=True)
    check_tensor("residual", residual, max_offset=_span((M, ldr), (N, 1)), allow_none=True)
    check_tensor("y", y, max_offset=_span((M, ldy), (N, 1)))
    _call("piton_mi355x_linear_ln", _ptr(x), ldx, float(eps), _ptr(w), _ptr(bias), _ptr(residual), ldr, _ptr(y), ldy,
          M, N, K, int(bool(relu)), _stream())


def mlp3(x, M, w1, b1, w2, b2, w3, b3, logits, pred, n_classes):
    """Three dense layers (ReLU on the first two) and the argmax of the first n_classes logits
    in one launch; logits equal three dense() calls bit for bit. x [M, K0] contiguous."""
    k0, n1 = w1.shape
    n2, n3 = w2.shape[1], w3.shape[1]
    if w2.shape[0] != n1 or w3.shape[0] != n2:
        raise ValueError(f"mlp3: layer shapes {tuple(w1.shape)}, {tuple(w2.shape)}, {tuple(w3.shape)} do not chain")
    check_tensor("x", x, max_offset=M * k0 - 1)
    for name, w, n in (("w1", w1, n1), ("w2", w2, n2), ("w3", w3, n3)):
        if not w.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        check_tensor(name, w, max_offset=w.numel() - 1)
    for name, b, n in (("b1", b1, n1), ("b2", b2, n2), ("b3", b3, n3)):
        check_tensor(name, b, max_offset=n - 1, allow_none=True)
    check_tensor("logits", logits, max_offset=M * n3 - 1, allow_none=True)
    check_tensor("pred", pred, dtype=torch.int32, max_offset=M - 1, allow_none=True)
    _call("piton_mi355x_mlp3", _ptr(x), M, _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2), _ptr(w3), _ptr(b3), k0, n1, n2,
          n3, _ptr(logits), _ptr(pred), int(n_classes), _stream())


def attn_fwd_batched(q, k, v, out, sm_scale, s_qb, s_qh, s_qm, s_kb, s_kh, s_kn, s_kk, s_vb, s_vh, s_vn, s_ob, s_oh,
                     s_om, n_ctx, batch, heads, head_dim, causal):
    """attn_fwd_kernel over batch x heads."""
    check_tensor("Q", q, max_offset=_span((batch, s_qb), (heads, s_qh), (n_ctx, s_qm), (head_dim, 1)))
    check_tensor("K", k, max_offset=_span((batch, s_kb), (heads, s_kh), (n_ctx, s_kn), (head_dim, s_kk)))
    check_tensor("V", v, max_offset=_span((batch, s_vb), (heads, s_vh), (n_ctx, s_vn), (head_dim, 1)))
    check_tensor("Out", out, max_offset=_span((batch, s_ob), (heads, s_oh), (n_ctx, s_om), (head_dim, 1)))
    _call("piton_mi355x_attn_fwd_batched", _ptr(q), _ptr(k), _ptr(v), _ptr(out), float(sm_scale), s_qb, s_qh, s_qm,
          s_kb, s_kh, s_kn, s_kk, s_vb, s_vh, s_vn, s_ob, s_oh, s_om, n_ctx, batch, heads, int(head_dim),
          int(bool(causal)), _stream())


def attn_decode(q, k, v, out, sm_scale, s_qb, s_qh, s_kb, s_kh, s_kn, s_vb, s_vh, s_vn, s_ob, s_oh, n_keys, batch,
                heads, head_dim):
    """One query per (batch, head) against n_keys cached keys."""
    check_tensor("q", q, max_offset=_span((batch, s_qb), (heads, s_qh), (head_dim, 1)))
    check_tensor("k", k, max_offset=_span((batch, s_kb), (heads, s_kh), (n_keys, s_kn), (head_dim, 1)))
    check_tensor("v", v, max_offset=_span((batch, s_vb), (heads, s_vh), (n_keys, s_vn), (head_dim, 1)))
    check_tensor("out", out, max_offset=_span((batch, s_ob), (heads, s_oh), (head_dim, 1)))
    _call("piton_mi355x_attn_decode", _ptr(q), _ptr(k), _ptr(v), _ptr(out), float(sm_scale), s_qb, s_qh, s_kb, s_kh,
          s_kn, s_vb, s_vh, s_vn, s_ob, s_oh, n_keys, batch, heads, int(head_dim), _stream())


def decode_layer(x, ldx, eps, w, bias, cache, ldc, out, ldo, sm_scale, n_keys, batch, heads, head_dim, d_model,
                 ids=None, tok=None, pos=None, vocab=0, err_flag=None):
    """A decode step's layernorm + QKV projection + cache append + attention for one layer, in
    one launch: cache row (n_keys - 1) * batch + b gets LN(x[b]) W + bias (q | k | v), and
    out[b, h*hd:(h+1)*hd] attends head h's query to keys 0 .. n_keys-1 of the position-major
    cache (rows t * batch + b, k at column d_model + h*hd, v at 2 d_model + h*hd). With ids
    (int32 [batch]), x[b] is first set to tok[ids[b]] + pos (pos: the position's row), as
    embedding() does. Equal to linear_ln + attn_decode to rounding (head_dim 64, d_model =
    heads * 64 a multiple of 256 up to 1024, n_keys <= 256; else MI355XError with status -2)."""
    check_tensor("x", x, max_offset=_span((batch, ldx), (d_model, 1)))
    check_tensor("w", w, max_offset=3 * d_model * d_model - 1)
    check_tensor("bias", bias, max_offset=3 * d_model - 1, allow_none=True)
    check_tensor("cache", cache, max_offset=_span((n_keys * batch, ldc), (3 * d_model, 1)))
    check_tensor("out", out, max_offset=_span((batch, ldo), (d_model, 1)))
    if ids is not None:
        check_tensor("ids", ids, dtype=torch.int32, max_offset=batch - 1)
        check_tensor("tok", tok, max_offset=vocab * d_model - 1)
        check_tensor("pos", pos, max_offset=d_model - 1)
        check_tensor("err_flag", err_flag, dtype=torch.int32, max_offset=0, allow_none=True)
    _call("piton_mi355x_decode_layer", _ptr(x), ldx, float(eps), _ptr(w), _ptr(bias), _ptr(cache), ldc, _ptr(out),
          ldo, float(sm_scale), n_keys, batch, heads, int(head_dim), d_model, _ptr(ids), _ptr(tok), _ptr(pos),
          int(vocab), _ptr(err_flag), _stream())


def lm_head_argmax(x, ldx, eps, w, bias, logits, ldl, next_ids, M, N, K, n_classes):
    """The decoder's last step in one launch, one workgroup per row: logits[m] = LN(x[m]) W
    (+ bias) (logits nullable) and next_ids[m] = numpy's argmax of the first n_classes logits.
    Equal to linear_ln + argmax_rows to rounding (K a multiple of 256 and N of 4, both up to
    1024, 16-byte x rows; else MI355XError with status -2)."""
    check_tensor("x", x, max_offset=_span((M, ldx), (K, 1)))
    check_tensor("w", w, max_offset=K * N - 1)
    check_tensor("bias", bias, max_offset=N - 1, allow_none=True)
    check_tensor("logits", logits, max_offset=_span((M, ldl), (N, 1)), allow_none=True)
    check_tensor("next_ids", next_ids, dtype=torch.int32, max_offset=M - 1)
    _call("piton_mi355x_lm_head_argmax", _ptr(x), ldx, float(eps), _ptr(w), _ptr(bias), _ptr(logits), ldl,
          _ptr(next_ids), M, N, K, int(n_classes), _stream())


# ---- the perf suite's primitives (perf/suite.py:323-351) -----------------------------------

def _elementwise(entry, n, tensors, *scalars):
    for name, t in tensors:
        check_tensor(name, t, max_offset=n - 1)
    _call(entry, *[_ptr(t) for _, t in tensors], n, *scalars, _stream())


def mfma_probe(out, workgroups, iters):
    """Diagnostics (no reference counterpart): workgroups x 4 waves each issue iters x 32 fp32
    32x32x2 MFMAs in two independent chains; the caller times the launch. out: float32, at
    least workgroups * 256 elements."""
    check_tensor("out", out, max_offset=int(workgroups) * 256 - 1)
    _call("piton_mi355x_mfma_probe", _ptr(out), int(workgroups), int(iters), _stream())


def copy(x, out, n):
    """copy_kernel (examples/primitive_kernels.py:12-17)."""
    _elementwise("piton_mi355x_copy", n, (("x", x), ("out", out)))


def mul(x, y, out, n):
    """mul_kernel (examples/elementwise.py:5-9)."""
    _elementwise("piton_mi355x_mul", n, (("x", x), ("y", y), ("out", out)))


def fma(x, y, out, n, alpha):
    """fma_kernel (examples/primitive_kernels.py:20-27): out = x * alpha + y."""
    _elementwise("piton_mi355x_fma", n, (("x", x), ("y", y), ("out", out)), float(alpha))


def scaled_relu(x, out, n, alpha):
    """scaled_relu_kernel (examples/kernels.py:79-85)."""
    _elementwise("piton_mi355x_scaled_relu", n, (("x", x), ("out", out)), float(alpha))


def sfu(x, out, n, op):
    """sfu_kernel (examples/sfu_tests.py:5-22): OP 0 exp2, 1 log2, 2 1/x, 3 1/sqrt, 4 exp, 5 sqrt."""
    _elementwise("piton_mi355x_sfu", n, (("x", x), ("out", out)), int(op))


def log(x, out, n):
    """log_kernel (examples/primitive_kernels.py:70-76)."""
    _elementwise("piton_mi355x_log", n, (("x", x), ("out", out)))


def idiv(x, y, q, r, n):
    """idiv_kernel (examples/primitive_kernels.py:30-38): C-style int32 quotient and remainder."""
    for name, t in (("x", x), ("y", y), ("q", q), ("r", r)):
        check_tensor(name, t, dtype=torch.int32, max_offset=n - 1)
    _call("piton_mi355x_idiv", _ptr(x), _ptr(y), _ptr(q), _ptr(r), n, _stream())


def _row_reduce(entry, x, out, rows, n_cols, stride):
    check_tensor("x", x, max_offset=_span((rows, stride), (n_cols, 1)))
    check_tensor("out", out, max_offset=rows - 1)
    _call(entry, _ptr(x), _ptr(out), rows, n_cols, stride, _stream())


def row_sum(x, out, rows, n_cols, stride):
    """row_sum_kernel (examples/kernels.py:88-96)."""
    _row_reduce("piton_mi355x_row_sum", x, out, rows, n_cols, stride)


def row_max(x, out, rows, n_cols, stride):
    """row_max_kernel (examples/primitive_kernels.py:41-50)."""
    _row_reduce("piton_mi355x_row_max", x, out, rows, n_cols, stride)


def transpose(x, out, n_rows, n_cols, stride_x, stride_out):
    """transpose_kernel (examples/primitive_kernels.py:53-67): out[c, r] = x[r, c]."""
    check_tensor("x", x, max_offset=_span((n_rows, stride_x), (n_cols, 1)))
    check_tensor("out", out, max_offset=_span((n_cols, stride_out), (n_rows, 1)))
    _call("piton_mi355x_transpose", _ptr(x), _ptr(out), n_rows, n_cols, stride_x, stride_out, _stream())
