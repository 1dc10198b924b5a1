"""ctypes access to the C oracle ``oracle/liboracle.so`` (test infrastructure only)."""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compile tg_oracle.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        L.ora_e4m3fn_encode_range.argtypes = [ctypes.c_uint32, ctypes.c_uint64, vp]
        L.ora_e4m3fn_encode_array.argtypes = [vp, i64, vp]
        for name in ("ora_quantize_rows_f32", "ora_quantize_rows_bf16", "ora_quantize_cols_bf16"):
            getattr(L, name).argtypes = [vp, i64, i64, ctypes.c_int, vp, vp]
        L.ora_rms_norm_quant_bf16.argtypes = [vp, vp, i64, i64, ctypes.c_float, ctypes.c_int, vp, vp, vp]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def encode_range(start: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint8)
    lib().ora_e4m3fn_encode_range(start, count, _p(out))
    return out


def encode_array(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint8)
    lib().ora_e4m3fn_encode_array(_p(v), v.size, _p(out))
    return out


def quantize_rows_bf16(x_u16: np.ndarray, block: int = 128):
    x = np.ascontiguousarray(x_u16, dtype=np.uint16)
    R, C = x.reshape(-1, x.shape[-1]).shape
    q = np.empty((R, C), dtype=np.uint8)
    s = np.empty((R, C // block), dtype=np.float32)
    lib().ora_quantize_rows_bf16(_p(x), R, C, block, _p(q), _p(s))
    return q, s


def quantize_cols_bf16(x_u16: np.ndarray, block: int = 128):
    x = np.ascontiguousarray(x_u16, dtype=np.uint16)
    R, C = x.shape
    q = np.empty((C, R), dtype=np.uint8)
    s = np.empty((C, R // block), dtype=np.float32)
    lib().ora_quantize_cols_bf16(_p(x), R, C, block, _p(q), _p(s))
    return q, s


def rms_norm_quant_bf16(x_u16, g_u16, eps: float, block: int = 128, quant: bool = True):
    x = np.ascontiguousarray(x_u16, dtype=np.uint16)
    g = np.ascontiguousarray(g_u16, dtype=np.uint16)
    D = x.shape[-1]
    R = x.size // D
    y = np.empty((R, D), dtype=np.uint16)
    q = np.empty((R, D), dtype=np.uint8) if quant else None
    s = np.empty((R, D // block), dtype=np.float32) if quant else None
    lib().ora_rms_norm_quant_bf16(_p(x), _p(g), R, D, eps, block, _p(y),
                                  _p(q) if quant else None, _p(s) if quant else None)
    return y, q, s
