"""ctypes binding of libtg_fp8.so (the C ABI declared in include/tg_fp8.h).

torch supplies device memory and the current HIP stream; every computation
runs in the HIP kernels of the library.  There is no fallback: if the library
is missing, or no GPU is present, calls raise.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtg_fp8.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "tg_fp8.h")

TG_OK, TG_EINVAL, TG_EHIP = 0, 1, 2
TG_NOALLOC_SCRATCH_BYTES = 64 << 20     # include/tg_fp8.h
TG_DTYPE_BF16, TG_DTYPE_F32, TG_DTYPE_F16 = 0, 1, 2

_vp, _i64, _int, _f32, _sz = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                              ctypes.c_float, ctypes.c_size_t)

# name -> (restype, argtypes); mirrors include/tg_fp8.h
SIGNATURES = {
    "tg_last_error": (ctypes.c_char_p, []),
    "tg_quantize_rows": (_int, [_vp, _int, _i64, _i64, _int, _vp, _vp, _vp]),
    "tg_quantize_cols": (_int, [_vp, _int, _i64, _i64, _int, _vp, _vp, _vp]),
    "tg_quantize_dual": (_int, [_vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, _vp]),
    "tg_quantize_dual_pair": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp,
                                     _vp, _vp, _int, _vp]),
    "tg_quantize_dual_km": (_int, [_vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, _vp]),
    "tg_quantize_dual_pair_km": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp,
                                        _vp, _vp, _int, _vp]),
    "tg_gemm_fp8_nt": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _int, _i64, _i64, _i64, _int, _vp]),
    "tg_gemm_fp8_nt_km": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _int, _i64, _i64, _i64, _int, _vp]),
    "tg_block_scaled_matmul_workspace": (_sz, [_i64, _i64, _i64, _int]),
    "tg_block_scaled_matmul": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _int, _vp, _sz, _vp]),
    "tg_block_scaled_matmul_noalloc": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _int, _vp]),
    "tg_block_scaled_matmul_bwd_workspace": (_sz, [_i64, _i64, _i64, _int]),
    "tg_block_scaled_matmul_bwd_fp8": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int,
                                              _vp, _sz, _vp]),
    "tg_rms_norm": (_int, [_vp, _vp, _vp, _i64, _i64, _f32, _vp]),
    "tg_rms_norm_ex": (_int, [_vp, _int, _vp, _int, _vp, _i64, _i64, _f32, _vp]),
    "tg_rms_norm_fp8": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _int, _vp]),
    "tg_rms_norm_bwd_workspace": (_sz, [_i64, _i64]),
    "tg_rms_norm_bwd": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _vp, _sz, _vp]),
    "tg_rms_norm_bwd_ex": (_int, [_vp, _int, _vp, _int, _vp, _int, _vp, _vp, _i64, _i64, _f32, _vp,
                                  _sz, _vp]),
    "tg_gemv_fp8": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _i64, _i64, _i64, _int, _vp]),
    "tg_gemv_fp8_rowdot": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _i64, _i64, _i64, _int, _vp]),
    "tg_rms_norm_fp8_gemv": (_int, [_vp, _vp, _vp, _f32, _vp, _vp, _vp, _int, _vp, _i64, _i64, _i64, _vp]),
    "tg_relu2_fp8_gemv": (_int, [_vp, _vp, _vp, _int, _vp, _i64, _i64, _i64, _vp]),
    "tg_gemv_fp8_rowdot_add": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _vp, _i64, _i64, _i64, _int, _vp]),
    "tg_relu2_fp8_gemv_add": (_int, [_vp, _vp, _vp, _int, _vp, _vp, _i64, _i64, _i64, _vp]),
    "tg_quantize_weight_128x128": (_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "tg_gemm_bf16_nt": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "tg_pack_bf16": (_int, [_vp, _int, _i64, _i64, _int, _vp, _i64, _vp]),
    "tg_block_scaled_matmul_bwd_bf16_workspace": (_sz, [_i64, _i64, _i64]),
    "tg_block_scaled_matmul_bwd_bf16": (_int, [_vp, _int, _vp, _int, _vp, _int, _vp, _vp, _i64,
                                               _i64, _i64, _vp, _sz, _vp]),
    "tg_quantize_rows_relu2": (_int, [_vp, _i64, _i64, _int, _vp, _vp, _vp]),
    "tg_add_rms_norm_fp8": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_float,
                                   _int, _vp]),
    "tg_decode_attention": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                   ctypes.c_float, _vp]),
    "tg_logit_cap": (_int, [_vp, _vp, _i64, _f32, _vp]),
    "tg_decode_embed": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "tg_logit_cap_xent_fwd": (_int, [_vp, _vp, _i64, _i64, _f32, _vp, _vp, _vp]),
    "tg_logit_cap_xent_bwd": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _i64, _i64, _f32, _vp, _vp]),
    "tg_selftest_fp8_cvt": (_int, [_vp, _vp]),
    "tg_selftest_divide": (_int, [_vp, _vp]),
}

_lib = None


def lib():
    """Load libtg_fp8.so once (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python train-gpt_amd/build.py` "
                "(the FP8 hot path has no non-HIP implementation)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    """Turn a C-ABI return code into the reference's exception types."""
    if rc == TG_OK:
        return
    msg = lib().tg_last_error().decode(errors="replace")
    if rc == TG_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(msg)


def ptr(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """The current torch stream of t's device, as the C ABI's void* stream."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("the FP8 hot path runs on the GPU only: pass device tensors")


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return TG_DTYPE_BF16
    if t.dtype == torch.float32:
        return TG_DTYPE_F32
    raise TypeError(f"unsupported dtype {t.dtype}")


def norm_dtype_code(t: torch.Tensor) -> int:
    """dtype_code plus float16, which the norm entry points (tg_rms_norm_ex,
    tg_rms_norm_bwd_ex) take and no other entry point does."""
    if t.dtype == torch.float16:
        return TG_DTYPE_F16
    return dtype_code(t)
