"""numpy restatement of the reference's RMSNorm (test infrastructure only).

Follows /root/reference/kernels.py:
  * _rms_norm_pure        kernels.py:30-33 (the canonical semantics)
  * rms_norm_gpu _norm_kernel  kernels.py:44-53 (single-rounding variant)
  * _bwd (VJP)             kernels.py:104-118
and the fused norm -> quantize composition
``_quantize_to_fp8(_rms_norm_pure(x, g, eps).astype(f32))`` (kernels.py:30-33
feeding fp8.py:39-47 the way fp8.py:66 would).

Implementation-defined points, fixed here:
  * jnp.mean's f32 reduction order: the sum of the f32 squares is taken in
    float64 (order-free to far below one f32 ulp) and rounded once to f32,
    then divided by D in f32 (jnp.mean = sum / count).
  * lax.rsqrt: correctly rounded f32 (computed as 1/sqrt in float64, rounded).
  * bf16 x bf16 products are exact in f32 and rounded once to bf16 (RNE) per op.
"""
import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16
from .fp8_ref import quantize_fp8


def row_inv_rms(x_bf16: np.ndarray, eps: float):
    """var = mean(f32(x)^2); returns (var f32, r = f32(rsqrt(var + eps)))."""
    x = bf16_to_f32(x_bf16)
    D = x.shape[-1]
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        sq = (x * x).astype(np.float32)                       # kernels.py:31 (x.astype(f32) ** 2)
        ssum = np.sum(sq.astype(np.float64), axis=-1).astype(np.float32)
        var = (ssum / np.float32(D)).astype(np.float32)       # jnp.mean
        v = (var + np.float32(eps)).astype(np.float32)        # var + eps (eps weakly typed)
        r = (1.0 / np.sqrt(v.astype(np.float64))).astype(np.float32)   # lax.rsqrt
    return var, r


def rms_norm_pure(x_bf16: np.ndarray, g_bf16: np.ndarray, eps: float) -> np.ndarray:
    """``_rms_norm_pure`` (kernels.py:30-33) with bf16 x and scale.

    r = bf16(rsqrt(var + eps)); t = bf16(x * r); y = bf16(t * scale).
    Returns y as bf16 bit patterns with x's shape.
    """
    x = bf16_to_f32(x_bf16)
    g = bf16_to_f32(g_bf16)
    _, r = row_inv_rms(x_bf16, eps)
    r_b = bf16_to_f32(f32_to_bf16(r))[..., None]              # .astype(x.dtype), kernels.py:32
    with np.errstate(over="ignore", invalid="ignore"):
        t = bf16_to_f32(f32_to_bf16((x * r_b).astype(np.float32)))   # x * r in bf16
        y = f32_to_bf16((t * g).astype(np.float32))           # x_n * scale, kernels.py:33
    return y


def _round_to(v, dtype):
    """v (f32) rounded to dtype's precision (RNE), returned as f32."""
    if dtype == "bf16":
        return bf16_to_f32(f32_to_bf16(v))
    if dtype == "f16":
        return np.asarray(v, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "f32":
        return np.asarray(v, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype!r}")


def rms_norm_pure_any(x_f32, x_dtype: str, g_f32, eps):
    """``_rms_norm_pure`` (kernels.py:30-33) for any float dtypes, on values.

    x_f32 holds x's values (representable in x_dtype: "bf16", "f16" or "f32"),
    g_f32 the scale's.  r = rsqrt(var + eps) and x_n = x * r are rounded to x's
    dtype; y = x_n * scale in f32 (the caller rounds to bf16 / f16 when both
    operands have that dtype: the product of two such values is exact in f32,
    so one rounding of it is the dtype's own multiply).  Returns y as f32 values.
    """
    x = np.asarray(x_f32, dtype=np.float32)
    g = np.asarray(g_f32, dtype=np.float32)
    D = x.shape[-1]
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        sq = (x * x).astype(np.float32)
        ssum = np.sum(sq.astype(np.float64), axis=-1).astype(np.float32)
        var = (ssum / np.float32(D)).astype(np.float32)
        v = (var + np.float32(eps)).astype(np.float32)
        r = (1.0 / np.sqrt(v.astype(np.float64))).astype(np.float32)[..., None]
        r = _round_to(r, x_dtype)
        t = _round_to((x * r).astype(np.float32), x_dtype)
        return (t * g).astype(np.float32)


def rms_norm_single_rounding(x_bf16, g_bf16, eps):
    """The Pallas kernel's arithmetic (kernels.py:49-53): f32 x * rnorm * scale, one bf16 rounding."""
    x = bf16_to_f32(x_bf16)
    g = bf16_to_f32(g_bf16)
    _, r = row_inv_rms(x_bf16, eps)
    with np.errstate(over="ignore", invalid="ignore"):
        return f32_to_bf16(((x * r[..., None]).astype(np.float32) * g).astype(np.float32))


def rms_norm_fp8(x_bf16, g_bf16, eps, block_k: int = 128):
    """Fused norm -> quantize: (y, q, s) = (rms_norm_pure(x), quantize_fp8(f32(y))).

    No single reference function; this is the composition a caller of
    kernels.py:30-33 followed by fp8.py:66 computes.  Quantization reads the
    bf16-rounded norm output.
    """
    y = rms_norm_pure(x_bf16, g_bf16, eps)
    q, s = quantize_fp8(bf16_to_f32(y), block_k)
    return y, q, s


def rms_norm_vjp(x_bf16, g_bf16, eps, dy_bf16):
    """``_bwd`` (kernels.py:104-118) in float64 on bf16 bit patterns (see rms_norm_vjp_vals)."""
    return rms_norm_vjp_vals(bf16_to_f32(x_bf16), bf16_to_f32(g_bf16), eps, bf16_to_f32(dy_bf16))


def rms_norm_vjp_vals(x_f32, g_f32, eps, dy_f32):
    """``_bwd`` (kernels.py:104-118) in float64 on the operands' values (any dtype).

    normed = x * rsqrt(mean(x^2) + eps); gs = dy * scale;
    grad_x = rnorm * (gs - normed * mean(gs * normed)); grad_scale = sum(dy * normed).
    Returns (grad_x f64, grad_scale f64).
    """
    x = np.asarray(x_f32, dtype=np.float64)
    g = np.asarray(g_f32, dtype=np.float64)
    dy = np.asarray(dy_f32, dtype=np.float64)
    var = np.mean(x * x, axis=-1, keepdims=True)
    rn = 1.0 / np.sqrt(var + eps)
    normed = x * rn
    gs = dy * g
    dot = np.mean(gs * normed, axis=-1, keepdims=True)
    gx = rn * (gs - normed * dot)
    gscale = np.sum((dy * normed).reshape(-1, x.shape[-1]), axis=0)
    return gx, gscale
