"""JAX registration of the XLA FFI handlers in csrc/ffi/tg_xla_ffi.cc.

On ROCm these replace jax.nn.scaled_matmul (/root/reference/fp8.py:70-76) and
the Pallas RMSNorm (/root/reference/kernels.py:87-97, selected at :124-127).
``register()`` loads libtg_xla_ffi.so (built by build.build_xla_ffi where jaxlib
is installed) and registers every handler under its target name; a caller then
invokes ``jax.ffi.ffi_call(target, result_shape_dtypes)(*args, **attrs)``.
The reference's ValueError checks (fp8.py:53-56) stay in Python before the call.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtg_xla_ffi.so")

# jax.ffi target name -> (exported handler symbol, C-ABI entry points it calls)
HANDLERS = {
    "tg_quantize_rows": ("tg_ffi_quantize_rows", ("tg_quantize_rows",)),
    "tg_quantize_cols": ("tg_ffi_quantize_cols", ("tg_quantize_cols",)),
    "tg_block_scaled_matmul": ("tg_ffi_block_scaled_matmul",
                               ("tg_block_scaled_matmul", "tg_quantize_rows", "tg_quantize_cols",
                                "tg_gemm_fp8_nt")),
    "tg_block_scaled_matmul_bwd_fp8": ("tg_ffi_block_scaled_matmul_bwd_fp8",
                                       ("tg_block_scaled_matmul_bwd_fp8",)),
    "tg_block_scaled_matmul_bwd_bf16": ("tg_ffi_block_scaled_matmul_bwd_bf16",
                                        ("tg_block_scaled_matmul_bwd_bf16",)),
    "tg_rms_norm": ("tg_ffi_rms_norm", ("tg_rms_norm_ex",)),
    "tg_rms_norm_fp8": ("tg_ffi_rms_norm_fp8", ("tg_rms_norm_fp8",)),
    "tg_rms_norm_bwd": ("tg_ffi_rms_norm_bwd", ("tg_rms_norm_bwd_ex",)),
    "tg_gemm_fp8_nt": ("tg_ffi_gemm_fp8_nt", ("tg_gemm_fp8_nt",)),
}


def register(lib_path: str = LIB_PATH) -> None:
    """Register every handler with JAX for the ROCm platform (needs jax and the built library)."""
    import jax
    if not os.path.exists(lib_path):
        raise RuntimeError(f"{lib_path} is missing: build it with build.build_xla_ffi() where jaxlib "
                           "is installed")
    lib = ctypes.CDLL(lib_path)
    for target, (symbol, _) in HANDLERS.items():
        jax.ffi.register_ffi_target(target, jax.ffi.pycapsule(getattr(lib, symbol)), platform="ROCM")
