"""bf16 <-> f32 bit helpers for the CPU oracle (test infrastructure only).

bf16 tensors are carried as ``numpy.uint16`` bit patterns.  Rounding from f32
is IEEE round-to-nearest-even on the upper 16 bits, which is what XLA's
``convert f32 -> bf16`` and ``astype(jnp.bfloat16)`` do (fp8.py:78,
kernels.py:32).  NaN inputs map to a quiet NaN with the sign kept.
"""
import numpy as np


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    """Widen bf16 bit patterns to f32 (exact)."""
    u16 = np.asarray(u16, dtype=np.uint16)
    return (u16.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round f32 to bf16 bit patterns, round-to-nearest-even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32)
    is_nan = (b & 0x7FFFFFFF) > 0x7F800000
    lsb = (b >> 16) & 1
    r = ((b.astype(np.uint64) + 0x7FFF + lsb) >> 16).astype(np.uint32)
    r = np.where(is_nan, (b >> 16) | 0x40, r)
    return r.astype(np.uint16)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 -> f32 (the value a bf16 tensor would hold)."""
    return bf16_to_f32(f32_to_bf16(x))


def randn_bf16(rng: np.random.Generator, shape, std=1.0, mean=0.0) -> np.ndarray:
    """Seeded normal samples rounded to bf16 (returned as uint16 bits).

    The build's synthetic inputs are drawn in float64 by ``numpy``'s
    ``default_rng``, scaled, cast to f32 and rounded to bf16 by RNE.  The same
    arrays feed the GPU kernels and this oracle.
    """
    v = rng.standard_normal(size=shape) * std + mean
    return f32_to_bf16(v.astype(np.float32))
