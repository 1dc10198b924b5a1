"""numpy restatement of the reference's block-scaled FP8 matmul (test infrastructure only).

Follows /root/reference/fp8.py:
  * E4M3_MAX / DEFAULT_BLOCK_K            fp8.py:26-27
  * _quantize_to_fp8                       fp8.py:39-47
  * _fp8_forward (quantize a, b.T; scaled GEMM; bf16 cast)   fp8.py:50-78
  * _fp8_backward (straight-through bf16)  fp8.py:85-98

Quantized bytes are e4m3fn bit patterns carried as ``numpy.uint8``.
"""
import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16

E4M3_MAX = 448.0          # fp8.py:26
DEFAULT_BLOCK_K = 128     # fp8.py:27
SCALE_FLOOR = np.float32(1e-30)   # fp8.py:44, weakly typed -> f32 0x0DA24260

_TWO_POW_M6_BITS = 0x3C800000     # f32 bits of 2**-6, smallest normal e4m3fn
_MAGIC_SUB = np.float32(16384.0)  # 2**14: its f32 ulp is 2**-9, the e4m3 subnormal step


def e4m3fn_encode(v: np.ndarray) -> np.ndarray:
    """f32 -> OCP e4m3fn bytes, round-to-nearest-even, non-saturating.

    Restates the f32 -> float8_e4m3fn ``astype`` at fp8.py:46 (ml_dtypes
    semantics): bias 7, max finite 448 (0x7E), 0x7F/0xFF are NaN and there is
    no infinity, so |v| rounding above 448 (|v| > 464) and +-inf become NaN
    with the sign kept; subnormals have step 2**-9; -0 encodes to 0x80.
    """
    v = np.ascontiguousarray(v, dtype=np.float32)
    bits = v.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint32)
    a = bits & 0x7FFFFFFF
    # normal range: round the f32 mantissa to 3 bits (RNE) and rebias 127 -> 7
    rnd = (a.astype(np.int64) + 0x7FFFF + ((a >> 20) & 1)) >> 20
    code_n = rnd - (120 << 3)
    # subnormal range: the f32 adder rounds |v| to a multiple of 2**-9 (RNE)
    af = a.view(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        code_s = ((af + _MAGIC_SUB).view(np.uint32).astype(np.int64)
                  - int(_MAGIC_SUB.view(np.uint32)))
    code = np.where(a < _TWO_POW_M6_BITS, code_s, code_n)
    nan = (a > 0x7F800000) | (code > 0x7E) | (a == 0x7F800000)
    code = np.where(nan, 0x7F, code)
    return (code.astype(np.uint32) | sign).astype(np.uint8)


def _e4m3fn_table() -> np.ndarray:
    t = np.zeros(256, dtype=np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            t[c] = np.nan
        elif e == 0:
            t[c] = s * m * 2.0 ** -9
        else:
            t[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3FN_VALUES = _e4m3fn_table()


def e4m3fn_decode(q: np.ndarray) -> np.ndarray:
    """e4m3fn bytes -> f32 (exact)."""
    return E4M3FN_VALUES[np.asarray(q, dtype=np.uint8)]


def quantize_fp8(x_f32: np.ndarray, block_k: int = DEFAULT_BLOCK_K):
    """``_quantize_to_fp8`` (fp8.py:39-47): per-1xblock_k amax scaling.

    amax = max|x| over each block (NaN propagates, as jnp.max does);
    s = max(fl32(amax / 448), fl32(1e-30)) (NaN propagates, as jnp.maximum);
    q = e4m3fn(fl32(x / s)) with an IEEE f32 divide.
    Returns (q uint8 (..., K), scales f32 (..., K/block_k)).
    """
    x = np.asarray(x_f32, dtype=np.float32)
    *lead, K = x.shape
    if K % block_k:
        raise ValueError(f"K={K} not divisible by block_k={block_k}")
    xt = x.reshape(*lead, K // block_k, block_k)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        amax = np.max(np.abs(xt), axis=-1)
        scales = np.maximum(amax / np.float32(E4M3_MAX), SCALE_FLOOR).astype(np.float32)
        xq = (xt / scales[..., None]).astype(np.float32)
    q = e4m3fn_encode(xq).reshape(*lead, K)
    return q, scales


def dequant_gemm_nt(qa, sa, qb, sb, block_k: int = DEFAULT_BLOCK_K) -> np.ndarray:
    """The scaled GEMM of fp8.py:70-76 (``jax.nn.scaled_matmul``), float64.

    out[m, n] = sum_kb sa[m, kb] * sb[n, kb] * sum_{k in kb} dec(qa[m, k]) * dec(qb[n, k])
    qa (M, K), qb (N, K); sa (M, K/bk); sb (N, K/bk).  Computed in float64 so
    it bounds the kernels' f32 accumulation error from above; the summation
    order of the real GEMM is implementation-defined.
    """
    M, K = qa.shape
    N = qb.shape[0]
    nkb = K // block_k
    A = e4m3fn_decode(qa).astype(np.float64).reshape(M, nkb, block_k)
    B = e4m3fn_decode(qb).astype(np.float64).reshape(N, nkb, block_k)
    out = np.zeros((M, N), dtype=np.float64)
    for kb in range(nkb):
        part = A[:, kb, :] @ B[:, kb, :].T
        out += part * (sa[:, kb].astype(np.float64)[:, None] * sb[:, kb].astype(np.float64)[None, :])
    return out


def fp8_forward(a_bf16: np.ndarray, b_bf16: np.ndarray, block_k: int = DEFAULT_BLOCK_K):
    """``_fp8_forward`` (fp8.py:50-78) on bf16 bit-pattern inputs.

    Returns (y_bf16 uint16 (..., N), out_f64 (M, N), (qa, sa), (qbt, sbt)).
    """
    a = bf16_to_f32(a_bf16)
    b = bf16_to_f32(b_bf16)
    *lead, K = a.shape
    K_b, N = b.shape
    if K != K_b:                                          # fp8.py:53-54
        raise ValueError(f"contracted-dim mismatch: a K={K}, b K={K_b}")
    if K % block_k != 0:                                  # fp8.py:55-56
        raise ValueError(f"K={K} not divisible by block_k={block_k}")
    a2 = a.reshape(-1, K)                                 # fp8.py:65
    qa, sa = quantize_fp8(a2, block_k)                    # fp8.py:66
    qbt, sbt = quantize_fp8(np.ascontiguousarray(b.T), block_k)   # fp8.py:68
    out = dequant_gemm_nt(qa, sa, qbt, sbt, block_k)      # fp8.py:70-76
    y = f32_to_bf16(out.astype(np.float32)).reshape(*lead, N)     # fp8.py:77-78
    return y, out, (qa, sa), (qbt, sbt)


def fp8_backward_bf16(a_bf16, b_bf16, g_bf16):
    """Straight-through bf16 backward (fp8.py:85-98), float64 accumulate.

    da = g @ b.T, db = a.T @ g on the bf16 values; returns float64 arrays
    (the kernels round to bf16, fp8.py:96-97).
    """
    a = bf16_to_f32(a_bf16).astype(np.float64)
    b = bf16_to_f32(b_bf16).astype(np.float64)
    g = bf16_to_f32(g_bf16).astype(np.float64)
    K = a.shape[-1]
    N = b.shape[1]
    a2 = a.reshape(-1, K)
    g2 = g.reshape(-1, N)
    return g2 @ b.T, a2.T @ g2


def quantize_fp8_partial(x_f32: np.ndarray, block_k: int = DEFAULT_BLOCK_K):
    """quantize_fp8 along the last axis with a trailing partial block.

    fp8.py:39-47 defines whole blocks only.  A trailing block of K % block_k
    elements is quantized over its valid elements, i.e. as a zero-padded whole
    block (zeros raise no amax and add nothing to a dot product).  Returns
    (q (..., K) uint8, scales (..., ceil(K / block_k)) f32).
    """
    x = np.asarray(x_f32, dtype=np.float32)
    *lead, K = x.shape
    Kp = -(-K // block_k) * block_k
    if Kp == K:
        return quantize_fp8(x, block_k)
    xp = np.zeros((*lead, Kp), dtype=np.float32)
    xp[..., :K] = x
    q, s = quantize_fp8(xp, block_k)
    return q[..., :K], s


def fp8_backward_fp8(a_bf16, b_bf16, g_bf16, block_k: int = DEFAULT_BLOCK_K):
    """FP8 backward: the forward composition reused for both gradients.

    fp8.py:85-98 is a straight-through bf16 backward; the FP8 variant runs
    the same quantize -> scaled GEMM as fp8.py:50-78 on the gradient GEMMs:
      dX = fwd(g, b.T)   -> A = g row-quantized along N, B = b row-quantized along N
      dW = fwd(a.T, g)   -> A = a.T quantized along M, B = g.T quantized along M
    Returns (dx_f64 (M,K), dw_f64 (K,N), operands) where operands holds the
    four quantized (bytes, scales) pairs for bit-exact checks.  When N (dX's
    contraction) or M (dW's) is not a multiple of block_k, the operands are
    zero-padded along it (quantize_fp8_partial's trailing block); the
    operands returned are then those of the padded problem.
    """
    a = bf16_to_f32(a_bf16)
    b = bf16_to_f32(b_bf16)
    g = bf16_to_f32(g_bf16)
    K = a.shape[-1]
    N = b.shape[1]
    a2 = a.reshape(-1, K)
    g2 = g.reshape(-1, N)
    M = a2.shape[0]
    Mp, Np = -(-M // block_k) * block_k, -(-N // block_k) * block_k
    if (Mp, Np) != (M, N):
        a2 = np.pad(a2, ((0, Mp - M), (0, 0)))
        b = np.pad(b, ((0, 0), (0, Np - N)))
        g2 = np.pad(g2, ((0, Mp - M), (0, Np - N)))
    qg, sg = quantize_fp8(g2, block_k)                          # (M, N) along N
    qb, sb = quantize_fp8(b, block_k)                           # (K, N) along N
    qat, sat = quantize_fp8(np.ascontiguousarray(a2.T), block_k)   # (K, M) along M
    qgt, sgt = quantize_fp8(np.ascontiguousarray(g2.T), block_k)   # (N, M) along M
    dx = dequant_gemm_nt(qg, sg, qb, sb, block_k)[:M]
    dw = dequant_gemm_nt(qat, sat, qgt, sgt, block_k)[:, :N]
    ops = {"g_rows": (qg, sg), "b_rows": (qb, sb), "a_cols": (qat, sat), "g_cols": (qgt, sgt)}
    return dx, dw, ops


def quantize_weight_128x128(w_t_f32: np.ndarray, block: int = 128):
    """128x128-tile weight quantization for the pre-quantized GEMV format.

    No reference function (the reference never pre-quantizes weights); this is
    the literal reading of the "per-128x128 fp32 scales on W" configs.  Input
    is W.T (N, K) f32; one scale per (128-row, 128-col) tile:
    s = max(fl32(amax_tile / 448), 1e-30), q = e4m3fn(fl32(w / s)).
    Returns (q (N, K) uint8, s (ceil(N/128), K/128) f32).
    """
    w = np.asarray(w_t_f32, dtype=np.float32)
    N, K = w.shape
    nb = (N + block - 1) // block
    pad = nb * block - N
    wp = np.pad(np.abs(w), ((0, pad), (0, 0)))
    tiles = wp.reshape(nb, block, K // block, block)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        amax = tiles.max(axis=(1, 3))
        s = np.maximum(amax / np.float32(E4M3_MAX), SCALE_FLOOR).astype(np.float32)
        full = np.repeat(np.repeat(s, block, axis=0)[:N], block, axis=1)
        q = e4m3fn_encode((w / full).astype(np.float32))
    return q, s


def gemv_prequant(qx, sx, qw, sw, bn: int, block_k: int = DEFAULT_BLOCK_K) -> np.ndarray:
    """Decode-shape GEMM with a pre-quantized weight (no reference function).

    out[m, n] = sum_kb sx[m, kb] * sw[n // bn, kb] * sum_k dec(qx[m,k]) dec(qw[n,k]),
    float64.  bn = 1: sw is (N, K/128) (the fp8.py:68 layout); bn = 128: sw is
    (ceil(N/128), K/128).
    """
    N = qw.shape[0]
    swf = np.asarray(sw, dtype=np.float32)
    if bn != 1:
        swf = np.repeat(swf, bn, axis=0)[:N]
    return dequant_gemm_nt(qx, sx, qw, swf, block_k)
