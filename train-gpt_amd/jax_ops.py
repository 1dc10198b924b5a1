"""JAX drop-in for the reference's fp8.py and kernels.py on ROCm (MI355X).

A JAX caller of the reference (model.py:15 calls ``rms_norm`` on jax arrays;
bench_fp8_norm.py / debug_fp8.py call ``block_scaled_matmul``) imports this
module in place of /root/reference/fp8.py and /root/reference/kernels.py.  The
names, arguments, nondiff arguments, error types and texts, output dtypes and
custom-VJP residuals are the reference's; the compute is the XLA FFI handlers
of csrc/ffi/tg_xla_ffi.cc (registered by xla_ffi.register()) over the C ABI
of libtg_fp8.so:

  block_scaled_matmul(a, b, block_k=128)   fp8.py:30-36,101  custom_vjp, nondiff block_k
    forward   -> "tg_block_scaled_matmul"                    fp8.py:50-78
    backward  -> "tg_block_scaled_matmul_bwd_bf16"           fp8.py:85-98 (BACKWARD_MODE "bf16")
              or "tg_block_scaled_matmul_bwd_fp8"            the forward's FP8 composition ("fp8")
  _quantize_to_fp8(x_f32, block_k)         fp8.py:39-47      -> "tg_quantize_rows"
  _rms_norm_pure(x, scale, eps)            kernels.py:30-33  -> "tg_rms_norm"
  rms_norm(x, scale, eps)                  kernels.py:55,101-127 custom_vjp, nondiff eps
    backward  -> "tg_rms_norm_bwd"                           kernels.py:104-118
  rms_norm_fp8(x, scale, eps, block_k)     (additive) fused norm -> FP8, "tg_rms_norm_fp8"

jax / jaxlib are not installed in the image this repository is built in, so
this module is checked there as source only (tests/test_jax_ops.py: every
target it calls is registered with the operand / result / attribute layout its
handler binds); the torch surface (fp8.py, kernels.py) runs the same C ABI
under the GPU tests.
"""
import functools

import jax
import jax.numpy as jnp

import xla_ffi

E4M3_MAX = 448.0              # fp8.py:26
DEFAULT_BLOCK_K = 128         # fp8.py:27

# The backward rule of block_scaled_matmul: "bf16" is the reference's
# straight-through rule (fp8.py:85-98); "fp8" quantizes dY and the transposed
# operands as the forward does and runs both gradients on FP8 MFMA.
BACKWARD_MODE = "fp8"

_registered = False


def _ensure_registered():
    global _registered
    if not _registered:
        xla_ffi.register()
        _registered = True


def _call(target, result_shapes, *args, **attrs):
    _ensure_registered()
    return jax.ffi.ffi_call(target, result_shapes)(*args, **attrs)


def _validate(a, b, block_k):
    *_, K = a.shape
    K_b, _ = b.shape
    if K != K_b:                                                   # fp8.py:53-54
        raise ValueError(f"contracted-dim mismatch: a K={K}, b K={K_b}")
    if K % block_k != 0:                                           # fp8.py:55-56
        raise ValueError(f"K={K} not divisible by block_k={block_k}")


def _operand(x):
    """fp8.py:66,68 quantize astype(float32) values: bf16 and f32 go to the
    handler as they are (bf16 widens to f32 exactly); other float dtypes are
    widened here."""
    return x if x.dtype in (jnp.bfloat16, jnp.float32) else x.astype(jnp.float32)


def _quantize_to_fp8(x_f32, block_k):
    """fp8.py:39-47 along the last axis -> (x_f8 float8_e4m3fn, scales f32)."""
    *lead, K = x_f32.shape
    if K % block_k != 0:
        raise ValueError(f"K={K} not divisible by block_k={block_k}")
    return _call("tg_quantize_rows",
                 (jax.ShapeDtypeStruct(x_f32.shape, jnp.float8_e4m3fn),
                  jax.ShapeDtypeStruct((*lead, K // block_k), jnp.float32)),
                 _operand(x_f32), block_k=int(block_k))


def _fp8_forward(a, b, block_k):
    """fp8.py:50-78: a (..., K), b (K, N) -> bf16 (..., N)."""
    _validate(a, b, block_k)
    *lead, K = a.shape
    N = b.shape[1]
    a2 = _operand(a).reshape(-1, K)
    out = _call("tg_block_scaled_matmul", jax.ShapeDtypeStruct((a2.shape[0], N), jnp.bfloat16),
                a2, _operand(b), block_k=int(block_k))
    return out.reshape(*lead, N)


@functools.partial(jax.custom_vjp, nondiff_argnums=(2,))
def block_scaled_matmul(a, b, block_k=DEFAULT_BLOCK_K):
    """Per-K-tile block-scaled FP8 matmul (fp8.py:30-36)."""
    return _fp8_forward(a, b, block_k)


def _fp8_forward_with_residuals(a, b, block_k):
    """fp8.py:81-82: the residuals are the un-quantized operands."""
    return _fp8_forward(a, b, block_k), (a, b)


def _fp8_backward(block_k, residuals, g):
    """fp8.py:85-98 (BACKWARD_MODE "bf16") or the FP8 rule ("fp8"): returns
    (da as a.dtype, db as b.dtype)."""
    a, b = residuals
    *lead, K = a.shape
    N = b.shape[1]
    a2 = a.reshape(-1, K)
    g2 = g.reshape(-1, N)
    M = a2.shape[0]
    if BACKWARD_MODE == "bf16":
        da, db = _call("tg_block_scaled_matmul_bwd_bf16",
                       (jax.ShapeDtypeStruct((M, K), jnp.bfloat16), jax.ShapeDtypeStruct((K, N), jnp.bfloat16)),
                       _operand(a2), _operand(b), _operand(g2))
    elif BACKWARD_MODE == "fp8":
        da, db = _call("tg_block_scaled_matmul_bwd_fp8",
                       (jax.ShapeDtypeStruct((M, K), jnp.bfloat16), jax.ShapeDtypeStruct((K, N), jnp.bfloat16)),
                       a2.astype(jnp.bfloat16), b.astype(jnp.bfloat16), g2.astype(jnp.bfloat16),
                       block_k=int(block_k))
    else:
        raise ValueError(f"unknown BACKWARD_MODE {BACKWARD_MODE!r} (expected 'fp8' or 'bf16')")
    return da.reshape(*lead, K).astype(a.dtype), db.astype(b.dtype)


block_scaled_matmul.defvjp(_fp8_forward_with_residuals, _fp8_backward)


_NORM_FLOATS = (jnp.bfloat16, jnp.float16, jnp.float32)


def _norm_out_dtype(x, scale):
    """jnp's promotion of x_n (x.dtype) * scale (kernels.py:33)."""
    return jnp.promote_types(x.dtype, scale.dtype)


def _check_norm(x, scale):
    for t in (x, scale):
        if t.dtype not in _NORM_FLOATS:
            raise TypeError(f"rms_norm: x and scale must be bfloat16, float16 or float32, got {x.dtype}, {scale.dtype}")
    D = x.shape[-1]
    if scale.shape != (D,):
        raise ValueError(f"scale must have shape ({D},), got {tuple(scale.shape)}")


def _rms_norm_pure(x, scale, eps):
    """kernels.py:30-33: x (..., D), scale (D,) -> (..., D) in the promoted dtype."""
    _check_norm(x, scale)
    return _call("tg_rms_norm", jax.ShapeDtypeStruct(x.shape, _norm_out_dtype(x, scale)), x, scale,
                 eps=float(eps))


@functools.partial(jax.custom_vjp, nondiff_argnums=(2,))
def rms_norm(x, scale, eps):
    """kernels.py:124-127's rms_norm: the HIP kernel on every backend."""
    return _rms_norm_pure(x, scale, eps)


def _rms_norm_fwd(x, scale, eps):
    """kernels.py:101-102: the residuals are (x, scale)."""
    return _rms_norm_pure(x, scale, eps), (x, scale)


def _rms_norm_bwd(eps, residuals, g):
    """kernels.py:104-118: (grad_x as x.dtype, grad_scale as scale.dtype)."""
    x, scale = residuals
    if g.dtype not in _NORM_FLOATS:
        g = g.astype(jnp.float32)
    return tuple(_call("tg_rms_norm_bwd",
                       (jax.ShapeDtypeStruct(x.shape, x.dtype), jax.ShapeDtypeStruct(scale.shape, scale.dtype)),
                       x, scale, g, eps=float(eps)))


rms_norm.defvjp(_rms_norm_fwd, _rms_norm_bwd)


def _rms_norm_fp8_call(x, scale, eps, block_k):
    if x.dtype != jnp.bfloat16 or scale.dtype != jnp.bfloat16:
        raise TypeError("rms_norm_fp8: x and scale must be bfloat16 (the model's dtype)")
    _check_norm(x, scale)
    *lead, D = x.shape
    if block_k != DEFAULT_BLOCK_K or D % block_k != 0:
        raise ValueError(f"rms_norm_fp8: block_k must be 128 and divide D={D}")
    return _call("tg_rms_norm_fp8",
                 (jax.ShapeDtypeStruct(x.shape, jnp.bfloat16), jax.ShapeDtypeStruct(x.shape, jnp.float8_e4m3fn),
                  jax.ShapeDtypeStruct((*lead, D // block_k), jnp.float32)),
                 x, scale, eps=float(eps), block_k=int(block_k))


@functools.partial(jax.custom_vjp, nondiff_argnums=(2, 3))
def rms_norm_fp8(x, scale, eps, block_k=DEFAULT_BLOCK_K):
    """The norm fused with the quantization of its output (additive; no single
    reference function): (y bf16 (..., D), y_f8 e4m3fn (..., D), y_scales f32
    (..., D / block_k)) from one read of x -- the bytes and scales
    _quantize_to_fp8(y.astype(f32), block_k) gives.  x and scale bf16.  The
    gradient flows through y only (the bytes and scales feed a matmul whose
    own backward differentiates its un-quantized operand), with rms_norm's
    backward (kernels.py:104-118)."""
    return _rms_norm_fp8_call(x, scale, eps, block_k)


def _rms_norm_fp8_fwd(x, scale, eps, block_k):
    return _rms_norm_fp8_call(x, scale, eps, block_k), (x, scale)


def _rms_norm_fp8_bwd(eps, block_k, residuals, cotangents):
    gy = cotangents[0]
    return _rms_norm_bwd(eps, residuals, gy)


rms_norm_fp8.defvjp(_rms_norm_fp8_fwd, _rms_norm_fp8_bwd)
