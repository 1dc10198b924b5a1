"""RMSNorm on MI355X -- drop-in for the reference's kernels.py.

Same names and arguments as /root/reference/kernels.py:
  * _rms_norm_pure(x, scale, eps)     kernels.py:30-33 (the canonical semantics)
  * rms_norm(x, scale, eps)           kernels.py:55-127 (custom_vjp; backend-selected)
Both run the gfx950 kernel tg_rms_norm with _rms_norm_pure's arithmetic:
r = bf16(rsqrt(mean(x^2) + eps)), y = bf16(bf16(x * r) * scale).  Like the
reference they accept f32 as well (tg_rms_norm_ex): r and x * r are then
rounded in x's dtype and the output has the promoted dtype of x and scale.  The
reference selects its Pallas kernel when jax.default_backend() == "gpu"
(kernels.py:124-127), which would pick the CUDA-only Mosaic path on ROCm; here
the HIP kernel is the only implementation.

Additive (no single reference function): ``rms_norm_fp8(x, scale, eps,
block_k)`` returns the bf16 norm output together with its e4m3fn bytes and
1x128 fp32 scales from one read of x -- what ``_quantize_to_fp8`` of the norm
output (fp8.py:66) would produce.

The backward is the reference's custom VJP (kernels.py:104-118) as the HIP
kernel tg_rms_norm_bwd: dx = bf16(rnorm * (gs - normed * mean(gs * normed)))
and dscale = bf16(sum over rows of dy * normed), with gs = dy * scale; the
dscale sum runs in a fixed order, so it is the same on every call.
"""
import torch

import _tglib as _L


_FLOATS = (torch.bfloat16, torch.float16, torch.float32)


def _prep(x: torch.Tensor, scale: torch.Tensor, bf16_only: bool = True):
    _L.require_gpu(x, scale)
    if bf16_only and (x.dtype != torch.bfloat16 or scale.dtype != torch.bfloat16):
        raise TypeError("rms_norm_fp8: x and scale must be bfloat16 (the model's dtype)")
    if x.dtype not in _FLOATS or scale.dtype not in _FLOATS:
        raise TypeError(f"rms_norm: x and scale must be bfloat16, float16 or float32, got {x.dtype}, {scale.dtype}")
    D = x.shape[-1]
    if scale.shape != (D,):
        raise ValueError(f"scale must have shape ({D},), got {tuple(scale.shape)}")
    return x.reshape(-1, D).contiguous(), scale.contiguous(), D


def _out_dtype(x: torch.Tensor, scale: torch.Tensor):
    """jnp's promotion of x_n (x.dtype) * scale: the common dtype, else f32
    (bf16 with f16 promotes to f32, as in torch)."""
    return x.dtype if x.dtype == scale.dtype else torch.float32


def _rms_norm_pure(x: torch.Tensor, scale: torch.Tensor, eps: float) -> torch.Tensor:
    """kernels.py:30-33 on the GPU: x (..., D), scale (D,), bf16, f16 or f32 -> (..., D) in the promoted dtype."""
    x2, g, D = _prep(x, scale, bf16_only=False)
    y = torch.empty(x2.shape, dtype=_out_dtype(x, scale), device=x.device)
    # bf16 x and scale with D % 8 == 0 (D <= 16384) take the fast kernel inside
    _L.check(_L.lib().tg_rms_norm_ex(_L.ptr(x2), _L.norm_dtype_code(x2), _L.ptr(g), _L.norm_dtype_code(g),
                                     _L.ptr(y), x2.shape[0], D, float(eps), _L.stream_of(x2)))
    return y.reshape(x.shape)


def rms_norm_fp8(x: torch.Tensor, scale: torch.Tensor, eps: float, block_k: int = 128):
    """Fused RMSNorm -> FP8 quantize.

    Returns (y bf16 (..., D), y_f8 float8_e4m3fn (..., D), y_scales f32 (..., D/block_k)),
    where (y_f8, y_scales) == _quantize_to_fp8(y.astype(f32), block_k) bit for bit.
    Differentiable in y (the backward is rms_norm's, kernels.py:104-118); the
    bytes and scales carry no gradient.
    """
    return _RMSNormFP8.apply(x, scale, eps, block_k)


def add_rms_norm_fp8(x: torch.Tensor, delta: torch.Tensor, scale: torch.Tensor, eps: float,
                     block_k: int = 128, inplace: bool = False, want_y: bool = False):
    """Residual add fused with the next norm -> FP8 quantize (model.py:75-76 then
    74/76's norm): x_out = bf16(x + delta), y = rms_norm(x_out), (y_f8, y_s) =
    _quantize_to_fp8(y).  Returns (x_out, y_f8, y_s, y or None); with
    inplace=True x_out is x itself.  Inference only (no autograd)."""
    x2, g, D = _prep(x, scale)
    if D % block_k:
        raise ValueError(f"K={D} not divisible by block_k={block_k}")
    if delta.shape != x.shape or delta.dtype != torch.bfloat16:
        raise ValueError("add_rms_norm_fp8: delta must be bf16 with x's shape")
    if inplace and not x.is_contiguous():
        raise ValueError("add_rms_norm_fp8: inplace needs a contiguous x")
    d2 = delta.reshape(-1, D).contiguous()
    R = x2.shape[0]
    xo = x2 if inplace else torch.empty_like(x2)
    y = torch.empty_like(x2) if want_y else None
    q = torch.empty((R, D), dtype=torch.uint8, device=x.device)
    s = torch.empty((R, D // block_k), dtype=torch.float32, device=x.device)
    _L.check(_L.lib().tg_add_rms_norm_fp8(_L.ptr(x2), _L.ptr(d2), _L.ptr(g), _L.ptr(xo),
                                          _L.ptr(y) if y is not None else None, _L.ptr(q), _L.ptr(s),
                                          R, D, float(eps), block_k, _L.stream_of(x2)))
    lead = x.shape[:-1]
    return (xo.reshape(x.shape), q.view(torch.float8_e4m3fn).reshape(x.shape),
            s.reshape(*lead, D // block_k), y.reshape(x.shape) if y is not None else None)


def _rms_norm_fp8_fwd(x: torch.Tensor, scale: torch.Tensor, eps: float, block_k: int):
    x2, g, D = _prep(x, scale)
    if D % block_k:
        raise ValueError(f"K={D} not divisible by block_k={block_k}")
    R = x2.shape[0]
    y = torch.empty_like(x2)
    q = torch.empty((R, D), dtype=torch.uint8, device=x.device)
    s = torch.empty((R, D // block_k), dtype=torch.float32, device=x.device)
    _L.check(_L.lib().tg_rms_norm_fp8(_L.ptr(x2), _L.ptr(g), _L.ptr(y), _L.ptr(q), _L.ptr(s), R, D,
                                      float(eps), block_k, _L.stream_of(x2)))
    lead = x.shape[:-1]
    return (y.reshape(x.shape), q.view(torch.float8_e4m3fn).reshape(x.shape),
            s.reshape(*lead, D // block_k))


def _rms_norm_bwd(x: torch.Tensor, scale: torch.Tensor, eps: float, g: torch.Tensor):
    """kernels.py:104-118: (grad_x as x.dtype, grad_scale as scale.dtype)."""
    x2, sc, D = _prep(x, scale, bf16_only=False)
    if g.dtype not in _FLOATS:
        g = g.to(torch.float32)
    g2 = g.reshape(-1, D).contiguous()
    R = x2.shape[0]
    dx = torch.empty_like(x2)
    dscale = torch.empty((D,), dtype=scale.dtype, device=x.device)
    ws_bytes = _L.lib().tg_rms_norm_bwd_workspace(R, D)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=x.device)
    # all-bf16 operands with D % 8 == 0 take tg_rms_norm_bwd's kernels inside
    _L.check(_L.lib().tg_rms_norm_bwd_ex(
        _L.ptr(x2), _L.norm_dtype_code(x2), _L.ptr(sc), _L.norm_dtype_code(sc), _L.ptr(g2), _L.norm_dtype_code(g2),
        _L.ptr(dx), _L.ptr(dscale), R, D, float(eps), _L.ptr(ws), ws_bytes, _L.stream_of(x2)))
    return dx.reshape(x.shape), dscale


class _RMSNormFP8(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, scale, eps, block_k):
        y, q, s = _rms_norm_fp8_fwd(x, scale, eps, block_k)
        ctx.save_for_backward(x, scale)
        ctx.eps = eps
        ctx.mark_non_differentiable(q, s)
        return y, q, s

    @staticmethod
    def backward(ctx, gy, gq, gs):
        x, scale = ctx.saved_tensors
        dx, dscale = _rms_norm_bwd(x, scale, ctx.eps, gy)
        return dx, dscale, None, None


class _RMSNorm(torch.autograd.Function):
    """custom_vjp of kernels.py:55,101-120: the saved residuals are (x, scale),
    and the backward recomputes normed from x (kernels.py:102-106)."""

    @staticmethod
    def forward(ctx, x, scale, eps):
        ctx.save_for_backward(x, scale)
        ctx.eps = eps
        return _rms_norm_pure(x, scale, eps)

    @staticmethod
    def backward(ctx, g):
        x, scale = ctx.saved_tensors
        dx, dscale = _rms_norm_bwd(x, scale, ctx.eps, g)
        return dx, dscale, None


def rms_norm(x: torch.Tensor, scale: torch.Tensor, eps: float) -> torch.Tensor:
    """kernels.py:124-127's rms_norm: the HIP kernel on every backend."""
    return _RMSNorm.apply(x, scale, eps)
