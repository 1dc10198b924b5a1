"""Per-block-scaled FP8 matmul on MI355X -- drop-in for the reference's fp8.py.

Same names, arguments, dtypes and errors as /root/reference/fp8.py:
  * E4M3_MAX, DEFAULT_BLOCK_K                       fp8.py:26-27
  * block_scaled_matmul(a, b, block_k=128)          fp8.py:30-36 (custom_vjp -> autograd.Function)
  * _quantize_to_fp8(x_f32, block_k)                fp8.py:39-47
  * _fp8_forward(a, b, block_k)                     fp8.py:50-78
  * _fp8_forward_with_residuals / _fp8_backward     fp8.py:81-98
Arrays are torch device tensors (the reference's are jax.Arrays); the
computation is the HIP kernels of libtg_fp8.so behind include/tg_fp8.h.

Backward modes (``BACKWARD_MODE``):
  * "fp8" (default): dX and dW run through the same quantize -> scaled GEMM
    composition as the forward (g and W quantized along N; X.T and g.T along
    M, all 1x128 blocks), on FP8 MFMA.
  * "bf16": the reference's straight-through rule (fp8.py:85-98): bf16 MFMA
    GEMMs of the un-quantized operands.

Residuals.  In "fp8" mode with bf16 operands whose M and N divide by
block_k, the forward quantizes a and b once each in both directions
(tg_quantize_dual: a along K and a.T along M; b.T along K and b along N) and
keeps the FP8 forms the backward needs (a.T, b) instead of a and b.  The
bytes are those the backward would compute from a and b, so the gradients
are the same bits; each operand is read once instead of twice and the saved
residuals take ~half the memory.

Additive entry points (no reference counterpart): ``quantize_fp8`` (row or
transposed), ``quantize_weight`` (pre-quantized weight format) and
``fp8_gemv`` (decode-shape GEMM on a pre-quantized weight).
"""
import torch

import _tglib as _L

E4M3_MAX = 448.0          # fp8.py:26
DEFAULT_BLOCK_K = 128     # fp8.py:27
BACKWARD_MODE = "fp8"

# block_k = 128 runs the tuned kernels (one scale block per pair of FP8 MFMA K
# steps); any other block size dividing K runs the library's general
# block-size quantizers, then the tuned GEMM for multiples and divisors (>= 16)
# of 128 and a VALU GEMM for the rest.  The fused paths that exist only for
# 128 (the one-read dual quantizers, the kept FP8 residuals, relu^2
# quantization) are taken only at 128.
TUNED_BLOCK_K = 128


def _check_block_k(block_k: int) -> None:
    if not isinstance(block_k, int) or block_k < 1:
        raise ValueError(f"block_k must be a positive integer, got {block_k!r}")


def _check_block_k_tuned(block_k: int, what: str) -> None:
    _check_block_k(block_k)
    if block_k != TUNED_BLOCK_K:
        raise NotImplementedError(f"{what}: block_k={block_k}: this fused kernel exists for block_k=128 only "
                                  "(quantize_fp8 takes any block_k)")


def block_scaled_matmul(a: torch.Tensor, b: torch.Tensor, block_k: int = DEFAULT_BLOCK_K) -> torch.Tensor:
    """Per-K-tile block-scaled FP8 matmul (fp8.py:30-36).

    a: (..., K), b: (K, N) -> (..., N) bf16.  Requires K % block_k == 0.
    """
    return _BlockScaledMatmul.apply(a, b, block_k)


def _quantize_to_fp8(x_f32: torch.Tensor, block_k: int):
    """fp8.py:39-47 along the last axis -> (x_f8 float8_e4m3fn, scales f32)."""
    return quantize_fp8(x_f32, block_k)


def quantize_fp8(x: torch.Tensor, block_k: int = DEFAULT_BLOCK_K, transpose: bool = False):
    """_quantize_to_fp8 of x (..., K) along its last axis, or, with
    transpose=True, of x.T for a 2-D x (R, C) (what fp8.py:68 does to b).

    x may be bf16 or f32 (f32 is what the reference feeds; bf16 values
    widen to f32 exactly).  Returns (q float8_e4m3fn, scales float32).
    """
    _L.require_gpu(x)
    _check_block_k(block_k)
    if transpose:
        if x.dim() != 2:
            raise ValueError("transpose=True needs a 2-D tensor")
        R, C = x.shape
        if R % block_k != 0:
            raise ValueError(f"K={R} not divisible by block_k={block_k}")
        if x.dtype not in (torch.bfloat16, torch.float32):
            x = x.to(torch.float32)
        x = x.contiguous()
        q = torch.empty((C, R), dtype=torch.uint8, device=x.device)
        s = torch.empty((C, R // block_k), dtype=torch.float32, device=x.device)
        _L.check(_L.lib().tg_quantize_cols(_L.ptr(x), _L.dtype_code(x), R, C, block_k,
                                           _L.ptr(q), _L.ptr(s), _L.stream_of(x)))
        return q.view(torch.float8_e4m3fn), s
    *lead, K = x.shape
    if K % block_k != 0:
        raise ValueError(f"K={K} not divisible by block_k={block_k}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.to(torch.float32)
    x2 = x.reshape(-1, K).contiguous()
    R = x2.shape[0]
    q = torch.empty((R, K), dtype=torch.uint8, device=x.device)
    s = torch.empty((R, K // block_k), dtype=torch.float32, device=x.device)
    _L.check(_L.lib().tg_quantize_rows(_L.ptr(x2), _L.dtype_code(x2), R, K, block_k,
                                       _L.ptr(q), _L.ptr(s), _L.stream_of(x2)))
    return q.view(torch.float8_e4m3fn).reshape(*lead, K), s.reshape(*lead, K // block_k)


def quantize_relu2(x: torch.Tensor, block_k: int = DEFAULT_BLOCK_K):
    """_quantize_to_fp8 of bf16(relu(x)^2) along the last axis (model.py:72's
    activation fused with the quantization feeding the next matmul); x bf16."""
    _L.require_gpu(x)
    _check_block_k_tuned(block_k, "quantize_relu2")
    if x.dtype != torch.bfloat16:
        raise TypeError("quantize_relu2: x must be bfloat16")
    K = x.shape[-1]
    if K % block_k:
        raise ValueError(f"K={K} not divisible by block_k={block_k}")
    x2 = x.reshape(-1, K).contiguous()
    R = x2.shape[0]
    q = torch.empty((R, K), dtype=torch.uint8, device=x.device)
    s = torch.empty((R, K // block_k), dtype=torch.float32, device=x.device)
    _L.check(_L.lib().tg_quantize_rows_relu2(_L.ptr(x2), R, K, block_k, _L.ptr(q), _L.ptr(s),
                                             _L.stream_of(x2)))
    return q.view(torch.float8_e4m3fn).reshape(x.shape), s.reshape(*x.shape[:-1], K // block_k)


def _validate(a: torch.Tensor, b: torch.Tensor, block_k: int):
    *leading, K = a.shape
    K_b, N = b.shape
    if K != K_b:                                                   # fp8.py:53-54
        raise ValueError(f"contracted-dim mismatch: a K={K}, b K={K_b}")
    if K % block_k != 0:                                           # fp8.py:55-56
        raise ValueError(f"K={K} not divisible by block_k={block_k}")
    return leading, K, N


def quantize_fp8_dual(x: torch.Tensor, block_k: int = DEFAULT_BLOCK_K):
    """_quantize_to_fp8 (fp8.py:39-47) of a 2-D bf16 x (R, C) along its rows and
    of x.T, from one read of x: returns (q, scales, q_t, scales_t), equal bit for
    bit to quantize_fp8(x) and quantize_fp8(x, transpose=True).  R and C must
    be multiples of block_k (the FP8 backward's dY)."""
    _L.require_gpu(x)
    _check_block_k_tuned(block_k, "quantize_fp8_dual")
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise ValueError("quantize_fp8_dual needs a 2-D bfloat16 tensor")
    R, C = x.shape
    if R % block_k or C % block_k:
        raise ValueError(f"K={R if R % block_k else C} not divisible by block_k={block_k}")
    x = x.contiguous()
    u8, f32 = torch.uint8, torch.float32
    q = torch.empty((R, C), dtype=u8, device=x.device)
    s = torch.empty((R, C // block_k), dtype=f32, device=x.device)
    qt = torch.empty((C, R), dtype=u8, device=x.device)
    st = torch.empty((C, R // block_k), dtype=f32, device=x.device)
    _L.check(_L.lib().tg_quantize_dual(_L.ptr(x), R, C, block_k, _L.ptr(q), _L.ptr(s), _L.ptr(qt),
                                       _L.ptr(st), _L.stream_of(x)))
    e4 = torch.float8_e4m3fn
    return q.view(e4), s, qt.view(e4), st


def quantize_fp8_dual_pair(x0: torch.Tensor, x1: torch.Tensor, block_k: int = DEFAULT_BLOCK_K):
    """quantize_fp8_dual of two tensors in one launch (the forward's a and b,
    fp8.py:66,68, with the backward's forms from the same reads): returns the
    two 4-tuples, bit for bit those of quantize_fp8_dual on each tensor."""
    _L.require_gpu(x0, x1)
    _check_block_k_tuned(block_k, "quantize_fp8_dual_pair")
    xs, outs, args = [], [], []
    for x in (x0, x1):
        if x.dim() != 2 or x.dtype != torch.bfloat16:
            raise ValueError("quantize_fp8_dual_pair needs 2-D bfloat16 tensors")
        R, C = x.shape
        if R % block_k or C % block_k:
            raise ValueError(f"K={R if R % block_k else C} not divisible by block_k={block_k}")
        x = x.contiguous()
        u8, f32 = torch.uint8, torch.float32
        o = (torch.empty((R, C), dtype=u8, device=x.device),
             torch.empty((R, C // block_k), dtype=f32, device=x.device),
             torch.empty((C, R), dtype=u8, device=x.device),
             torch.empty((C, R // block_k), dtype=f32, device=x.device))
        xs.append(x)
        outs.append(o)
        args += [_L.ptr(x), R, C] + [_L.ptr(t) for t in o]
    _L.check(_L.lib().tg_quantize_dual_pair(*args, block_k, _L.stream_of(xs[0])))
    e4 = torch.float8_e4m3fn
    return tuple((q.view(e4), s, qt.view(e4), st) for q, s, qt, st in outs)


def _quantize_dual_km(x: torch.Tensor, block_k: int):
    """quantize_fp8_dual with K-block-major scales (tg_quantize_dual_km): the
    bytes of quantize_fp8_dual, scales stored transposed, (C/bk, R) and (R/bk, C)."""
    R, C = x.shape
    u8, f32 = torch.uint8, torch.float32
    q = torch.empty((R, C), dtype=u8, device=x.device)
    s = torch.empty((C // block_k, R), dtype=f32, device=x.device)
    qt = torch.empty((C, R), dtype=u8, device=x.device)
    st = torch.empty((R // block_k, C), dtype=f32, device=x.device)
    _L.check(_L.lib().tg_quantize_dual_km(_L.ptr(x), R, C, block_k, _L.ptr(q), _L.ptr(s), _L.ptr(qt),
                                          _L.ptr(st), _L.stream_of(x)))
    return q, s, qt, st


def _quantize_dual_pair_km(x0: torch.Tensor, x1: torch.Tensor, block_k: int):
    """quantize_fp8_dual_pair with K-block-major scales (tg_quantize_dual_pair_km)."""
    outs, args = [], []
    u8, f32 = torch.uint8, torch.float32
    for x in (x0, x1):
        R, C = x.shape
        o = (torch.empty((R, C), dtype=u8, device=x.device),
             torch.empty((C // block_k, R), dtype=f32, device=x.device),
             torch.empty((C, R), dtype=u8, device=x.device),
             torch.empty((R // block_k, C), dtype=f32, device=x.device))
        outs.append(o)
        args += [_L.ptr(x), R, C] + [_L.ptr(v) for v in o]
    _L.check(_L.lib().tg_quantize_dual_pair_km(*args, block_k, _L.stream_of(x0)))
    return outs


def _scaled_matmul_km(a_q, a_s_km, b_q, b_s_km):
    """scaled_matmul on K-block-major scales (tg_gemm_fp8_nt_km), bf16 out; the
    same bits as scaled_matmul on the transposed scales."""
    M, K = a_q.shape
    N = b_q.shape[0]
    c = torch.empty((M, N), dtype=torch.bfloat16, device=a_q.device)
    _L.check(_L.lib().tg_gemm_fp8_nt_km(_L.ptr(a_q), _L.ptr(a_s_km), _L.ptr(b_q), _L.ptr(b_s_km), 1,
                                        _L.ptr(c), _L.TG_DTYPE_BF16, M, N, K, DEFAULT_BLOCK_K,
                                        _L.stream_of(a_q)))
    return c


def scaled_matmul(a_q, a_s, b_q, b_s, b_scale_bn: int = 1, out_dtype=torch.bfloat16):
    """The scaled GEMM of fp8.py:70-76 on already-quantized operands ("NT"):
    a_q (M, K), b_q (N, K) e4m3fn; a_s (M, K/bk), b_s (N or ceil(N/128), K/bk)
    f32, where the block size bk = K / a_s.shape[1] (128 unless the operands
    were quantized with another block_k).  Returns (M, N) in out_dtype (bf16 by
    RNE, or f32)."""
    _L.require_gpu(a_q, b_q)
    M, K = a_q.shape
    N = b_q.shape[0]
    if b_q.shape[1] != K:
        raise ValueError(f"contracted-dim mismatch: a K={K}, b K={b_q.shape[1]}")
    nkb = a_s.shape[1] if a_s.dim() == 2 else 0
    if nkb < 1 or K % nkb or b_s.shape[-1] != nkb:
        raise ValueError(f"scales do not tile K={K}: a_s {tuple(a_s.shape)}, b_s {tuple(b_s.shape)}")
    block_k = K // nkb
    c = torch.empty((M, N), dtype=out_dtype, device=a_q.device)
    code = _L.TG_DTYPE_F32 if out_dtype == torch.float32 else _L.TG_DTYPE_BF16
    a_q, b_q = a_q.contiguous(), b_q.contiguous()
    a_s, b_s = a_s.contiguous().float(), b_s.contiguous().float()
    _L.check(_L.lib().tg_gemm_fp8_nt(_L.ptr(a_q), _L.ptr(a_s), _L.ptr(b_q), _L.ptr(b_s),
                                     b_scale_bn, _L.ptr(c), code, M, N, K, block_k,
                                     _L.stream_of(a_q)))
    return c


def _fp8_forward(a: torch.Tensor, b: torch.Tensor, block_k: int) -> torch.Tensor:
    """fp8.py:50-78: quantize a and b.T, scaled GEMM, bf16 output (..., N)."""
    leading, K, N = _validate(a, b, block_k)
    _L.require_gpu(a, b)
    _check_block_k(block_k)
    a_2d = a.reshape(-1, K)
    M = a_2d.shape[0]
    if a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16:
        a_2d = a_2d.contiguous()
        b_c = b.contiguous()
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
        ws_bytes = _L.lib().tg_block_scaled_matmul_workspace(M, N, K, block_k)
        ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=a.device)
        _L.check(_L.lib().tg_block_scaled_matmul(_L.ptr(a_2d), _L.ptr(b_c), _L.ptr(out), M, N, K,
                                                 block_k, _L.ptr(ws), ws_bytes, _L.stream_of(a_2d)))
        return out.reshape(*leading, N)
    a_q, a_s = quantize_fp8(a_2d, block_k)                         # fp8.py:66
    b_q, b_s = quantize_fp8(b, block_k, transpose=True)            # fp8.py:68
    out = scaled_matmul(a_q.view(torch.uint8), a_s, b_q.view(torch.uint8), b_s)   # fp8.py:70-78
    return out.reshape(*leading, N)


def _fp8_forward_with_residuals(a, b, block_k):
    """fp8.py:81-82: the residuals are the un-quantized operands."""
    return _fp8_forward(a, b, block_k), (a, b)


def _fp8_backward(block_k, residuals, g):
    """Gradients of block_scaled_matmul: (da as a.dtype, db as b.dtype).

    BACKWARD_MODE "fp8": da = fwd(g, b.T), db = fwd(a.T, g) through FP8 MFMA.
    N (da's contraction) and M (db's) need not divide by block_k: the operands
    are zero-padded along them to a multiple of block_k.  Zeros change neither
    a block's amax nor any product, so this is the FP8 rule with the last,
    partial block quantized over its valid elements (fp8.py:39-47 defines only
    whole blocks).
    BACKWARD_MODE "bf16": fp8.py:85-98's straight-through rule, da = bf16(g) @
    bf16(b).T and db = bf16(a).T @ bf16(g), each a bf16 MFMA GEMM with fp32
    accumulation rounded once to bf16; block_k is unused, as in the reference.
    """
    a, b = residuals
    *leading, K = a.shape
    _, N = b.shape
    if BACKWARD_MODE == "bf16":
        return _bf16_backward(a, b, g)
    if BACKWARD_MODE != "fp8":
        raise ValueError(f"unknown BACKWARD_MODE {BACKWARD_MODE!r} (expected 'fp8' or 'bf16')")
    _check_block_k(block_k)
    a_2d = a.reshape(-1, K)
    g_2d = g.reshape(-1, N)
    M = a_2d.shape[0]
    _L.require_gpu(a_2d, b, g_2d)
    if M == 0 or N == 0 or K == 0:
        # empty contraction or empty result: the reference's dots give zeros
        return (torch.zeros(a.shape, dtype=a.dtype, device=a.device),
                torch.zeros(b.shape, dtype=b.dtype, device=b.device))
    Mp, Np = -(-M // block_k) * block_k, -(-N // block_k) * block_k
    if (Mp, Np) != (M, N):
        a_p = a_2d.new_zeros((Mp, K))
        a_p[:M] = a_2d
        g_p = g_2d.new_zeros((Mp, Np))
        g_p[:M, :N] = g_2d
        b_p = b.new_zeros((K, Np))
        b_p[:, :N] = b
        da, db = _fp8_backward(block_k, (a_p, b_p), g_p)
        return da[:M].reshape(*leading, K), db[:, :N].contiguous()
    bf = torch.bfloat16
    if a.dtype == bf and b.dtype == bf and g.dtype == bf:
        a_2d, g_2d, b_c = a_2d.contiguous(), g_2d.contiguous(), b.contiguous()
        da = torch.empty((M, K), dtype=bf, device=a.device)
        db = torch.empty((K, N), dtype=bf, device=a.device)
        ws_bytes = _L.lib().tg_block_scaled_matmul_bwd_workspace(M, N, K, block_k)
        ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=a.device)
        _L.check(_L.lib().tg_block_scaled_matmul_bwd_fp8(
            _L.ptr(a_2d), _L.ptr(b_c), _L.ptr(g_2d), _L.ptr(da), _L.ptr(db), M, N, K, block_k,
            _L.ptr(ws), ws_bytes, _L.stream_of(a_2d)))
    else:
        u8 = torch.uint8
        if g_2d.dtype == bf and block_k == TUNED_BLOCK_K:
            qg, sg, qgt, sgt = quantize_fp8_dual(g_2d, block_k)    # g along N and g.T along M
        else:
            qg, sg = quantize_fp8(g_2d, block_k)                   # g along N
            qgt, sgt = quantize_fp8(g_2d, block_k, transpose=True)  # g.T along M
        qb, sb = quantize_fp8(b, block_k)                          # b along N
        da = scaled_matmul(qg.view(u8), sg, qb.view(u8), sb)
        qat, sat = quantize_fp8(a_2d, block_k, transpose=True)     # a.T along M
        db = scaled_matmul(qat.view(u8), sat, qgt.view(u8), sgt)
    return da.reshape(*leading, K).to(a.dtype), db.to(b.dtype)


def _bf16_backward(a, b, g):
    """fp8.py:85-98: straight-through bf16 gradients (da as a.dtype, db as b.dtype)."""
    *leading, K = a.shape
    _, N = b.shape
    a_2d = a.reshape(-1, K).contiguous()
    g_2d = g.reshape(-1, N).contiguous()
    b_c = b.contiguous()
    M = a_2d.shape[0]
    _L.require_gpu(a_2d, b_c, g_2d)
    bf = torch.bfloat16
    da = torch.empty((M, K), dtype=bf, device=a.device)
    db = torch.empty((K, N), dtype=bf, device=a.device)
    ws_bytes = _L.lib().tg_block_scaled_matmul_bwd_bf16_workspace(M, N, K)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=a.device)
    _L.check(_L.lib().tg_block_scaled_matmul_bwd_bf16(
        _L.ptr(a_2d), _L.dtype_code(a_2d), _L.ptr(b_c), _L.dtype_code(b_c), _L.ptr(g_2d),
        _L.dtype_code(g_2d), _L.ptr(da), _L.ptr(db), M, N, K, _L.ptr(ws), ws_bytes,
        _L.stream_of(a_2d)))
    # fp8.py:95-96: .astype(a.dtype) / .astype(b.dtype) of the bf16 results (exact widening)
    return da.reshape(*leading, K).to(a.dtype), db.to(b.dtype)


def _fp8_forward_quantized_residuals(a, b, block_k, need_da, need_db):
    """_fp8_forward with the FP8 operands of the backward kept as residuals.

    a (..., K), b (K, N) bf16, M and N multiples of block_k.  Returns (out,
    (a.T bytes, a.T scales) or None, (b bytes, b scales) or None): a.T along M
    for db = fwd(a.T, g), b along N for da = fwd(g, b.T) -- the operands
    _fp8_backward would quantize from a and b (fp8.py:66,68 on those inputs).
    When both are kept, their scales are K-block-major and each tuple carries a
    third element "km" (the layout tg_gemm_fp8_nt_km reads); the bytes and the
    scale values are the same either way.
    """
    leading, K, N = _validate(a, b, block_k)
    a_2d = a.reshape(-1, K)
    if need_db and need_da:
        # a along K + a.T along M, and b along N + b.T along K: one launch, the
        # scales K-block-major (the residuals' scales too; the backward reads
        # them with the same GEMM), so the returned residuals are tagged "km"
        (qa, sa, qat, sat), (qb, sb, qbt, sbt) = _quantize_dual_pair_km(a_2d.contiguous(), b.contiguous(),
                                                                         block_k)
        out = _scaled_matmul_km(qa, sa, qbt, sbt)                   # fp8.py:70-78
        e4 = torch.float8_e4m3fn
        return out.reshape(*leading, N), (qat.view(e4), sat, "km"), (qb.view(e4), sb, "km")
    if need_db:
        qa, sa, qat, sat = quantize_fp8_dual(a_2d, block_k)    # a along K, a.T along M
        res_a = (qat, sat)
    else:
        (qa, sa), res_a = quantize_fp8(a_2d, block_k), None
    if need_da:
        qb, sb, qbt, sbt = quantize_fp8_dual(b, block_k)       # b along N, b.T along K
        res_b = (qb, sb)
    else:
        (qbt, sbt), res_b = quantize_fp8(b, block_k, transpose=True), None
    u8 = torch.uint8
    out = scaled_matmul(qa.view(u8), sa, qbt.view(u8), sbt)     # fp8.py:70-78
    return out.reshape(*leading, N), res_a, res_b


def _fp8_backward_quantized(block_k, res_a, res_b, g, a_shape, a_dtype, b_dtype):
    """BACKWARD_MODE "fp8" gradients from the kept FP8 residuals (same bits as
    _fp8_backward on the bf16 operands)."""
    N = g.shape[-1]
    g_2d = g.reshape(-1, N)
    u8 = torch.uint8
    km = res_a is not None and len(res_a) == 3
    if km and g_2d.dtype == torch.bfloat16:
        # K-block-major scales throughout: g along N and g.T along M from one read
        qg, sg, qgt, sgt = _quantize_dual_km(g_2d.contiguous(), block_k)
        (qat, sat, _), (qb, sb, _) = res_a, res_b
        da = _scaled_matmul_km(qg, sg, qb.view(u8), sb).reshape(a_shape).to(a_dtype)
        db = _scaled_matmul_km(qat.view(u8), sat, qgt, sgt).to(b_dtype)
        return da, db
    if km:
        # a non-bf16 gradient: its scales come in the reference layout, so the
        # residuals' scales are transposed back to it
        res_a = (res_a[0], res_a[1].t().contiguous())
        res_b = (res_b[0], res_b[1].t().contiguous())
    if g_2d.dtype == torch.bfloat16 and res_a is not None and res_b is not None:
        qg, sg, qgt, sgt = quantize_fp8_dual(g_2d, block_k)      # g along N and g.T along M
    else:
        qg, sg = quantize_fp8(g_2d, block_k) if res_b is not None else (None, None)
        qgt, sgt = quantize_fp8(g_2d, block_k, transpose=True) if res_a is not None else (None, None)
    da = db = None
    if res_b is not None:
        qb, sb = res_b
        da = scaled_matmul(qg.view(u8), sg, qb.view(u8), sb).reshape(a_shape).to(a_dtype)
    if res_a is not None:
        qat, sat = res_a
        db = scaled_matmul(qat.view(u8), sat, qgt.view(u8), sgt).to(b_dtype)
    return da, db


class _BlockScaledMatmul(torch.autograd.Function):
    """custom_vjp of fp8.py:30-36,101 as a torch autograd Function."""

    @staticmethod
    def forward(ctx, a, b, block_k):
        ctx.block_k = block_k
        ctx.quantized = False
        need_da, need_db = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if (BACKWARD_MODE == "fp8" and a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16
                and a.is_cuda and b.is_cuda and b.dim() == 2 and (need_da or need_db)):
            leading, K, N = _validate(a, b, block_k)
            _check_block_k(block_k)
            M = a.numel() // K if K else 0
            if block_k == TUNED_BLOCK_K and M > 0 and N > 0 and M % block_k == 0 and N % block_k == 0:
                out, res_a, res_b = _fp8_forward_quantized_residuals(a, b, block_k, need_da,
                                                                     need_db)
                ctx.quantized = True
                ctx.has_a, ctx.has_b = res_a is not None, res_b is not None
                ctx.km = res_a is not None and len(res_a) == 3      # K-block-major residual scales
                ctx.save_for_backward(*(res_a[:2] if res_a else ()), *(res_b[:2] if res_b else ()))
                ctx.a_shape, ctx.a_dtype, ctx.b_dtype = a.shape, a.dtype, b.dtype
                return out
        out, (ra, rb) = _fp8_forward_with_residuals(a, b, block_k)
        ctx.save_for_backward(ra, rb)
        return out

    @staticmethod
    def backward(ctx, g):
        if ctx.quantized:
            if BACKWARD_MODE != "fp8":
                raise RuntimeError("BACKWARD_MODE changed between forward and backward: this "
                                   "graph kept FP8 residuals for the 'fp8' backward")
            saved = list(ctx.saved_tensors)
            tag = ("km",) if ctx.km else ()
            res_a = (saved.pop(0), saved.pop(0), *tag) if ctx.has_a else None
            res_b = (saved.pop(0), saved.pop(0), *tag) if ctx.has_b else None
            da, db = _fp8_backward_quantized(ctx.block_k, res_a, res_b, g, ctx.a_shape,
                                             ctx.a_dtype, ctx.b_dtype)
            return da, db, None
        a, b = ctx.saved_tensors
        da, db = _fp8_backward(ctx.block_k, (a, b), g)
        return da, db, None


class _BlockScaledMatmulPrequant(torch.autograd.Function):
    """block_scaled_matmul whose left operand arrives already quantized.

    a_q / a_s must be _quantize_to_fp8(a) (for example the bytes and scales
    kernels.rms_norm_fp8 writes together with its bf16 output a), so the
    forward skips fp8.py:66's quantization of a; the residuals and the
    backward are block_scaled_matmul's (fp8.py:81-98), on the un-quantized a.
    """

    @staticmethod
    def forward(ctx, a, a_q, a_s, b, block_k):
        leading, K, N = _validate(a, b, block_k)
        _L.require_gpu(a, b)
        _check_block_k(block_k)
        b_q, b_s = quantize_fp8(b, block_k, transpose=True)                 # fp8.py:68
        out = scaled_matmul(a_q.reshape(-1, K).view(torch.uint8), a_s.reshape(-1, K // block_k),
                            b_q.view(torch.uint8), b_s)                        # fp8.py:70-78
        ctx.save_for_backward(a, b)
        ctx.block_k = block_k
        return out.reshape(*leading, N)

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        da, db = _fp8_backward(ctx.block_k, (a, b), g)
        return da, None, None, db, None


def block_scaled_matmul_prequant(a, a_q, a_s, b, block_k: int = DEFAULT_BLOCK_K):
    """a @ b through FP8 with a's quantization (a_q, a_s) supplied by the caller."""
    return _BlockScaledMatmulPrequant.apply(a, a_q, a_s, b, block_k)


class _Bf16Matmul(torch.autograd.Function):
    """A bf16 matmul on the bf16 MFMA GEMM: out = bf16(a @ b) with fp32
    accumulation (the `x @ w_out` logits projection that model.py:95-96 and
    bench_fp8_norm.py:117-118 keep in bf16); the backward is the
    straight-through rule of fp8.py:85-98."""

    @staticmethod
    def forward(ctx, a, b):
        *lead, K = a.shape
        K_b, N = b.shape
        if K != K_b:
            raise ValueError(f"contracted-dim mismatch: a K={K}, b K={K_b}")
        if K % 64:
            raise ValueError(f"K={K} must be a multiple of 64 for the bf16 GEMM")
        _L.require_gpu(a, b)
        a2 = a.reshape(-1, K).to(torch.bfloat16).contiguous()
        M = a2.shape[0]
        bt = torch.empty((N, K), dtype=torch.bfloat16, device=a.device)         # b.T, packed
        _L.check(_L.lib().tg_pack_bf16(_L.ptr(b.contiguous()), _L.dtype_code(b), K, N, 1, _L.ptr(bt), K,
                                       _L.stream_of(a2)))
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
        _L.check(_L.lib().tg_gemm_bf16_nt(_L.ptr(a2), _L.ptr(bt), _L.ptr(out), M, N, K,
                                          _L.stream_of(a2)))
        ctx.save_for_backward(a, b)
        return out.reshape(*lead, N)

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        return _bf16_backward(a, b, g)


def bf16_matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """bf16 a (..., K) @ b (K, N) -> bf16 (..., N) on the bf16 MFMA GEMM (autograd-aware)."""
    return _Bf16Matmul.apply(a, b)


# ---------------------------------------------------------------------------
# Pre-quantized weights and decode-shape GEMM (no reference counterpart).
# ---------------------------------------------------------------------------
def quantize_weight(w: torch.Tensor, layout: str = "128x1"):
    """Quantize W (K, N) once into (w_q (N, K) e4m3fn, w_s f32, bn).

    layout "128x1": per (128-K block, column) scales, w_s (N, K/128) -- the
    scales fp8.py:68 computes every call.  layout "128x128": one scale per
    128x128 tile, w_s (ceil(N/128), K/128).
    """
    _L.require_gpu(w)
    if layout == "128x1":
        q, s = quantize_fp8(w, DEFAULT_BLOCK_K, transpose=True)
        return q, s, 1
    if layout != "128x128":
        raise ValueError("layout must be '128x1' or '128x128'")
    K, N = w.shape
    if K % 128:
        raise ValueError(f"K={K} not divisible by block_k=128")
    w = w.to(torch.bfloat16).contiguous()
    q = torch.empty((N, K), dtype=torch.uint8, device=w.device)
    s = torch.empty(((N + 127) // 128, K // 128), dtype=torch.float32, device=w.device)
    _L.check(_L.lib().tg_quantize_weight_128x128(_L.ptr(w), K, N, _L.ptr(q), _L.ptr(s),
                                                 _L.stream_of(w)))
    return q.view(torch.float8_e4m3fn), s, 128


class QuantizedWeight:
    """A weight W (K, N) quantized once and kept across calls and in checkpoints.

    fp8.py:68 re-quantizes W on every forward; this keeps the e4m3fn bytes of
    W.T (N, K) and their fp32 scales in the layout the scaled GEMM and the
    decode GEMV consume, so a frozen or inference weight is quantized once:
      layout "128x1":   scales (N, K/128), bn = 1 -- bit-identical to what
                        fp8.py:68 computes on every call;
      layout "128x128": scales (ceil(N/128), K/128), bn = 128.
    Checkpoints are safetensors files (tensors "q" as float8_e4m3fn and
    "scales" as float32, metadata format/bn/block_k/K/N): the reference's
    pickled checkpoints (train_modal.py:403-410) would execute code on load,
    safetensors does not.
    """

    FORMAT = "tg-fp8-weight-v1"

    def __init__(self, q: torch.Tensor, scales: torch.Tensor, bn: int,
                 block_k: int = DEFAULT_BLOCK_K):
        if bn not in (1, 128):
            raise ValueError("bn must be 1 or 128")
        _check_block_k_tuned(block_k, "QuantizedWeight")
        if q.dim() != 2 or scales.dim() != 2:
            raise ValueError("q and scales must be 2-D")
        N, K = q.shape
        want = (N if bn == 1 else (N + 127) // 128, K // block_k)
        if K % block_k or tuple(scales.shape) != want:
            raise ValueError(f"scales shape {tuple(scales.shape)} does not match q {tuple(q.shape)} "
                             f"with bn={bn} (expected {want})")
        self.q = q.view(torch.float8_e4m3fn) if q.dtype == torch.uint8 else q
        self.scales = scales.to(torch.float32)
        self.bn = bn
        self.block_k = block_k

    @classmethod
    def from_weight(cls, w: torch.Tensor, layout: str = "128x1") -> "QuantizedWeight":
        q, s, bn = quantize_weight(w, layout)
        return cls(q, s, bn)

    @property
    def shape(self):
        """(K, N) of the weight this was quantized from."""
        return (self.q.shape[1], self.q.shape[0])

    def to(self, device) -> "QuantizedWeight":
        return QuantizedWeight(self.q.to(device), self.scales.to(device), self.bn, self.block_k)

    def matmul(self, x: torch.Tensor, exact: bool = False) -> torch.Tensor:
        """x (..., K) -> bf16 (..., N): fp8.py:66's quantization of x, then the
        scaled GEMM (or, for at most 64 rows, the decode GEMV) on the kept W.
        exact: use the MFMA GEMV for 1-2 rows too (the GEMM's block arithmetic,
        bit for bit) instead of the faster VALU one."""
        *lead, K = x.shape
        if K != self.shape[0]:
            raise ValueError(f"contracted-dim mismatch: a K={K}, b K={self.shape[0]}")
        M = 1
        for d in lead:
            M *= d
        if 0 < M <= 64:
            return fp8_gemv(x, self.q, self.scales, self.bn, self.block_k, exact=exact)
        a_q, a_s = quantize_fp8(x.reshape(-1, K), self.block_k)
        out = scaled_matmul(a_q.view(torch.uint8), a_s, self.q.view(torch.uint8), self.scales,
                            b_scale_bn=self.bn)
        return out.reshape(*lead, self.shape[1])

    def matmul_prequant(self, x_q: torch.Tensor, x_s: torch.Tensor, exact: bool = False) -> torch.Tensor:
        """Already-quantized rows (x_q (M, K) e4m3fn, x_s (M, K/128) f32, e.g. from
        kernels.rms_norm_fp8) times the kept W -> bf16 (M, N): the decode GEMV for
        at most 64 rows (exact as in matmul), the scaled GEMM above."""
        M, K = x_q.shape
        if K != self.shape[0]:
            raise ValueError(f"contracted-dim mismatch: a K={K}, b K={self.shape[0]}")
        xq = x_q.view(torch.uint8).contiguous()
        xs = x_s.contiguous().float()
        if 0 < M <= 64:
            out = torch.empty((M, self.shape[1]), dtype=torch.bfloat16, device=x_q.device)
            _gemv_prequant(xq, xs, self.q.view(torch.uint8), self.scales, self.bn, out, self.block_k,
                           exact)
            return out
        return scaled_matmul(xq, xs, self.q.view(torch.uint8), self.scales, b_scale_bn=self.bn)

    def matmul_rms_norm(self, x: torch.Tensor, gamma: torch.Tensor, eps: float,
                        delta: torch.Tensor = None, xout: torch.Tensor = None) -> torch.Tensor:
        """The norm that feeds this weight, fused with the GEMV, for 1-16 rows
        (tg_rms_norm_fp8_gemv): out (M, N) bf16 = the FP8 rows of
        rms_norm(x [+ delta]) (kernels.py:30-33, fp8.py:39-47) times the kept W.
        With delta, xout (M, K) receives the residual sum bf16(x + delta); it
        must not overlap x or delta.  Same bits as kernels.rms_norm_fp8 /
        add_rms_norm_fp8 followed by matmul_prequant (the VALU GEMV for 1-2
        rows, K <= 4096; the MFMA GEMV for 3-16 rows, K <= 2560)."""
        K, N = self.shape
        if x.dim() != 2 or x.shape[1] != K or x.dtype != torch.bfloat16:
            raise ValueError(f"matmul_rms_norm: x must be bf16 (M, {K})")
        if gamma.shape != (K,) or gamma.dtype != torch.bfloat16:
            raise ValueError(f"matmul_rms_norm: gamma must be bf16 ({K},)")
        if delta is not None:
            if delta.shape != x.shape or delta.dtype != torch.bfloat16:
                raise ValueError("matmul_rms_norm: delta must be bf16 with x's shape")
            if xout is None or xout.shape != x.shape or xout.dtype != torch.bfloat16 or not xout.is_contiguous():
                raise ValueError("matmul_rms_norm: with delta, xout must be a contiguous bf16 tensor of x's shape")
        _L.require_gpu(x, self.q)
        x = x.contiguous()
        d = delta.contiguous() if delta is not None else None
        out = torch.empty((x.shape[0], N), dtype=torch.bfloat16, device=x.device)
        _L.check(_L.lib().tg_rms_norm_fp8_gemv(
            _L.ptr(x), _L.ptr(d) if d is not None else None, _L.ptr(gamma.contiguous()), float(eps),
            _L.ptr(xout) if d is not None else None, _L.ptr(self.q.view(torch.uint8)), _L.ptr(self.scales),
            self.bn, _L.ptr(out), x.shape[0], N, K, _L.stream_of(x)))
        return out

    def matmul_relu2(self, u: torch.Tensor) -> torch.Tensor:
        """FP8 rows of bf16(relu(u)^2) (model.py:72) times the kept W, fused, for
        1-2 rows (tg_relu2_fp8_gemv); the same bits as quantize_relu2 followed by
        matmul_prequant (the VALU GEMV)."""
        K, N = self.shape
        if u.dim() != 2 or u.shape[1] != K or u.dtype != torch.bfloat16:
            raise ValueError(f"matmul_relu2: u must be bf16 (M, {K})")
        _L.require_gpu(u, self.q)
        u = u.contiguous()
        out = torch.empty((u.shape[0], N), dtype=torch.bfloat16, device=u.device)
        _L.check(_L.lib().tg_relu2_fp8_gemv(_L.ptr(u), _L.ptr(self.q.view(torch.uint8)), _L.ptr(self.scales),
                                            self.bn, _L.ptr(out), u.shape[0], N, K, _L.stream_of(u)))
        return out

    def _check_resid(self, x, resid, out, who):
        M, N = x.shape[0], self.shape[1]
        if resid.shape != (M, N) or resid.dtype != torch.bfloat16 or not resid.is_contiguous():
            raise ValueError(f"{who}: resid must be a contiguous bf16 ({M}, {N}) tensor")
        if out is None:
            return torch.empty_like(resid)
        if out.shape != resid.shape or out.dtype != torch.bfloat16 or not out.is_contiguous():
            raise ValueError(f"{who}: out must be a contiguous bf16 tensor of resid's shape")
        return out

    def matmul_prequant_add(self, x_q: torch.Tensor, x_s: torch.Tensor, resid: torch.Tensor,
                            out: torch.Tensor = None) -> torch.Tensor:
        """The residual add of model.py:75-76 fused into the GEMV of its term, 1-2
        rows: out = bf16(resid + matmul_prequant(x_q, x_s)) (tg_gemv_fp8_rowdot_add,
        the same bits as the bf16 tensor add after the VALU GEMV).  out may be
        resid itself (in place); by default a new tensor."""
        M, K = x_q.shape
        if K != self.shape[0]:
            raise ValueError(f"contracted-dim mismatch: a K={K}, b K={self.shape[0]}")
        if not 1 <= M <= 2 or K > ROWDOT_MAX_K:
            raise ValueError(f"matmul_prequant_add: 1-2 rows with K <= {ROWDOT_MAX_K}")
        out = self._check_resid(x_q, resid, out, "matmul_prequant_add")
        _L.require_gpu(x_q, self.q)
        xq = x_q.view(torch.uint8).contiguous()
        xs = x_s.contiguous().float()
        _L.check(_L.lib().tg_gemv_fp8_rowdot_add(
            _L.ptr(xq), _L.ptr(xs), _L.ptr(self.q.view(torch.uint8)), _L.ptr(self.scales), self.bn,
            _L.ptr(resid), _L.ptr(out), M, self.shape[1], K, self.block_k, _L.stream_of(xq)))
        return out

    def matmul_relu2_add(self, u: torch.Tensor, resid: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
        """out = bf16(resid + matmul_relu2(u)) for 1-2 rows (tg_relu2_fp8_gemv_add):
        model.py:72-76's MLP down projection and residual add in one launch, the
        same bits as matmul_relu2 followed by the bf16 tensor add.  out may be
        resid itself."""
        K, N = self.shape
        if u.dim() != 2 or u.shape[1] != K or u.dtype != torch.bfloat16 or not 1 <= u.shape[0] <= 2:
            raise ValueError(f"matmul_relu2_add: u must be bf16 (1 or 2, {K})")
        out = self._check_resid(u, resid, out, "matmul_relu2_add")
        _L.require_gpu(u, self.q)
        u = u.contiguous()
        _L.check(_L.lib().tg_relu2_fp8_gemv_add(_L.ptr(u), _L.ptr(self.q.view(torch.uint8)), _L.ptr(self.scales),
                                                self.bn, _L.ptr(resid), _L.ptr(out), u.shape[0], N, K,
                                                _L.stream_of(u)))
        return out

    def state_dict(self):
        return {"q": self.q, "scales": self.scales}

    def metadata(self):
        K, N = self.shape
        return {"format": self.FORMAT, "bn": str(self.bn), "block_k": str(self.block_k),
                "K": str(K), "N": str(N)}

    def save(self, path: str) -> None:
        from safetensors.torch import save_file
        save_file({k: v.detach().contiguous().cpu() for k, v in self.state_dict().items()}, path,
                  metadata=self.metadata())

    @classmethod
    def load(cls, path: str, device="cpu") -> "QuantizedWeight":
        from safetensors import safe_open
        with safe_open(path, framework="pt", device="cpu") as f:
            meta = f.metadata() or {}
            if meta.get("format") != cls.FORMAT:
                raise ValueError(f"{path}: not a {cls.FORMAT} file (format={meta.get('format')!r})")
            q, s = f.get_tensor("q"), f.get_tensor("scales")
        w = cls(q, s, int(meta["bn"]), int(meta["block_k"]))
        if w.shape != (int(meta["K"]), int(meta["N"])):
            raise ValueError(f"{path}: shape metadata {meta['K']}x{meta['N']} does not match the tensors")
        return w.to(device)


ROWDOT_MAX_K = 16384


def _gemv_prequant(xq, xs, wq, ws, bn, out, block_k, exact):
    """out (M, N) = GEMV of quantized rows xq (M, K) u8, xs on W (wq (N, K) u8, ws).
    1-2 rows take tg_gemv_fp8_rowdot (VALU dot products) unless exact, which
    keeps tg_gemv_fp8 (the GEMM's MFMA block arithmetic, bit for bit)."""
    M, K = xq.shape
    N = wq.shape[0]
    fn = (_L.lib().tg_gemv_fp8_rowdot if (M <= 2 and K <= ROWDOT_MAX_K and not exact)
          else _L.lib().tg_gemv_fp8)
    _L.check(fn(_L.ptr(xq), _L.ptr(xs), _L.ptr(wq), _L.ptr(ws), bn, _L.ptr(out), M, N, K, block_k,
                _L.stream_of(xq)))


def fp8_gemv(x: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, w_scale_bn: int = 1,
             block_k: int = DEFAULT_BLOCK_K, exact: bool = False) -> torch.Tensor:
    """Decode-shape GEMM: x (..., K) bf16 (M = prod(...) <= 64 rows) times a
    pre-quantized weight (w_q (N, K), w_s) -> (..., N) bf16.  For 1-2 rows the
    VALU kernel is used unless exact (see _gemv_prequant)."""
    _L.require_gpu(x, w_q)
    _check_block_k_tuned(block_k, "fp8_gemv")
    *lead, K = x.shape
    N = w_q.shape[0]
    if w_q.shape[1] != K:
        raise ValueError(f"contracted-dim mismatch: x K={K}, w K={w_q.shape[1]}")
    x_q, x_s = quantize_fp8(x.reshape(-1, K), block_k)
    M = x_q.shape[0]
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _gemv_prequant(x_q.view(torch.uint8), x_s, w_q.view(torch.uint8).contiguous(), w_s.contiguous(),
                   w_scale_bn, out, block_k, exact)
    return out.reshape(*lead, N)
