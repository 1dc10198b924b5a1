"""ctypes bindings of libtg_ffi_core.so: the XLA FFI handlers' logic
(train-gpt_amd/csrc/ffi/tg_ffi_core.h) over a C ABI, for the tests.

An operand goes in as a View (data pointer, element type, shape) exactly as
the XLA layer builds it from a buffer; the scratch allocator XLA hands a
handler is a bump allocator over a caller buffer (Scratch), whose ``used``
field comes back as the bytes the handler took.
"""
import ctypes
import os

import build

BF16, F32, F16, E4M3, OTHER = 0, 1, 2, 16, -1
OK, EINVAL, EHIP, EXHAUSTED = 0, 1, 2, 100


class View(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int),
                ("dims", ctypes.POINTER(ctypes.c_int64)), ("rank", ctypes.c_int)]


class Scratch(ctypes.Structure):
    _fields_ = [("base", ctypes.c_void_p), ("cap", ctypes.c_size_t), ("used", ctypes.c_size_t)]


def view(data, dtype, shape):
    """A View of `shape` at device address `data` (an int, or None for null)."""
    dims = (ctypes.c_int64 * max(len(shape), 1))(*shape)
    v = View(data, dtype, dims, len(shape))
    v._dims = dims   # keep the shape array alive with the view
    return v


_TORCH_CODES = None


def tview(t, dtype=None):
    """A View of a torch tensor; the element type follows the tensor unless given."""
    global _TORCH_CODES
    if _TORCH_CODES is None:
        import torch
        _TORCH_CODES = {torch.bfloat16: BF16, torch.float32: F32, torch.float16: F16,
                        torch.float8_e4m3fn: E4M3, torch.uint8: E4M3}
    return view(t.data_ptr(), _TORCH_CODES.get(t.dtype, OTHER) if dtype is None else dtype, tuple(t.shape))


_V = ctypes.POINTER(View)
_S = ctypes.POINTER(Scratch)
_vp, _i64, _f32p, _msg, _n = ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t
SIGNATURES = {
    "tg_ffi_core_quantize_rows": [_vp, _V, _vp, _f32p, _i64, _msg, _n],
    "tg_ffi_core_quantize_cols": [_vp, _V, _vp, _f32p, _i64, _msg, _n],
    "tg_ffi_core_block_scaled_matmul": [_vp, _S, _V, _V, _vp, _i64, _msg, _n],
    "tg_ffi_core_block_scaled_matmul_bwd_fp8": [_vp, _S, _V, _V, _V, _vp, _vp, _i64, _msg, _n],
    "tg_ffi_core_block_scaled_matmul_bwd_bf16": [_vp, _S, _V, _V, _V, _vp, _vp, _msg, _n],
    "tg_ffi_core_rms_norm": [_vp, _V, _V, _V, ctypes.c_float, _msg, _n],
    "tg_ffi_core_rms_norm_fp8": [_vp, _V, _V, _vp, _vp, _f32p, ctypes.c_float, _i64, _msg, _n],
    "tg_ffi_core_rms_norm_bwd": [_vp, _S, _V, _V, _V, _V, _V, ctypes.c_float, _msg, _n],
    "tg_ffi_core_gemm_fp8_nt": [_vp, _V, _f32p, _V, _f32p, _vp, _i64, _msg, _n],
}

_lib = None


def lib():
    """The shim, built by build.build_ffi_core (loads libtg_fp8.so with it)."""
    global _lib
    if _lib is None:
        if not os.path.exists(build.FFI_CORE_LIB):
            raise RuntimeError(f"{build.FFI_CORE_LIB} is missing: run build.build_ffi_core()")
        L = ctypes.CDLL(build.FFI_CORE_LIB)
        for name, args in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = ctypes.c_int
        _lib = L
    return _lib


def call(name, *args):
    """(code, message) of one shim call; args are everything before msg."""
    buf = ctypes.create_string_buffer(512)
    conv = [ctypes.byref(a) if isinstance(a, (View, Scratch)) else a for a in args]
    rc = getattr(lib(), name)(*conv, buf, len(buf))
    return rc, buf.value.decode()
