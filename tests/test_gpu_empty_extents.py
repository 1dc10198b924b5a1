"""Empty extents through the C ABI on the GPU: a gradient that sums over an
empty axis is the zero array, written in full; everything else is a no-op.

The reference's dots and sums give these results for empty operands
(`g @ b.T` over N = 0, `a.T @ g` over M = 0 in fp8.py:85-98; `sum(dy *
normed, axis=0)` over zero rows in kernels.py:104-118).  Each output is
filled with 3.0 first, so a kernel that skips the write is caught.
"""
import ctypes

import pytest
import torch

import _tglib as L
import fp8

pytestmark = pytest.mark.gpu

NUL = ctypes.c_void_p(0)


def _ws(dev, n=256):
    return torch.empty(max(n, 256), dtype=torch.uint8, device=dev)


def test_fp8_backward_zero_tokens_zero_fills_db(dev):
    """M = 0: da is empty (null is accepted), db = a.T @ g over no rows = 0."""
    K, N = 256, 384
    b = torch.ones((K, N), dtype=torch.bfloat16, device=dev)
    db = torch.full((K, N), 3.0, dtype=torch.bfloat16, device=dev)
    ws = _ws(dev, L.lib().tg_block_scaled_matmul_bwd_workspace(0, N, K, 128))
    L.check(L.lib().tg_block_scaled_matmul_bwd_fp8(NUL, L.ptr(b), NUL, NUL, L.ptr(db), 0, N, K, 128,
                                                   L.ptr(ws), ws.numel(), L.stream_of(b)))
    torch.cuda.synchronize()
    assert torch.all(db == 0)


def test_fp8_backward_zero_width_zero_fills_da(dev):
    """N = 0: db is empty, da = g @ b.T over no columns = 0."""
    M, K = 128, 256
    a = torch.ones((M, K), dtype=torch.bfloat16, device=dev)
    da = torch.full((M, K), 3.0, dtype=torch.bfloat16, device=dev)
    L.check(L.lib().tg_block_scaled_matmul_bwd_fp8(L.ptr(a), NUL, NUL, L.ptr(da), NUL, M, 0, K, 128,
                                                   NUL, 0, L.stream_of(a)))
    torch.cuda.synchronize()
    assert torch.all(da == 0)


def test_fp8_backward_empty_needs_the_gradient_it_writes(dev):
    rc = L.lib().tg_block_scaled_matmul_bwd_fp8(NUL, NUL, NUL, NUL, NUL, 0, 128, 256, 128, NUL, 0, NUL)
    assert rc == L.TG_EINVAL and L.lib().tg_last_error().endswith(b"null pointer")


@pytest.mark.parametrize("dim", [256, 2048, 6144])   # the row kernel's widths and the general one
def test_norm_backward_zero_rows_gives_zero_dscale(dev, dim):
    scale = torch.ones(dim, dtype=torch.bfloat16, device=dev)
    dscale = torch.full((dim,), 3.0, dtype=torch.bfloat16, device=dev)
    ws = _ws(dev, L.lib().tg_rms_norm_bwd_workspace(0, dim))
    L.check(L.lib().tg_rms_norm_bwd(NUL, L.ptr(scale), NUL, NUL, L.ptr(dscale), 0, dim, 1e-6, L.ptr(ws),
                                    ws.numel(), L.stream_of(scale)))
    torch.cuda.synchronize()
    assert torch.all(dscale == 0)


def test_norm_backward_ex_zero_rows_gives_zero_dscale_in_scale_dtype(dev):
    dim = 1000                                        # not a multiple of 8: the general kernels
    scale = torch.ones(dim, dtype=torch.float32, device=dev)
    dscale = torch.full((dim,), 3.0, dtype=torch.float32, device=dev)
    ws = _ws(dev, L.lib().tg_rms_norm_bwd_workspace(0, dim))
    L.check(L.lib().tg_rms_norm_bwd_ex(NUL, L.TG_DTYPE_BF16, L.ptr(scale), L.TG_DTYPE_F32, NUL,
                                       L.TG_DTYPE_BF16, NUL, L.ptr(dscale), 0, dim, 1e-6, L.ptr(ws),
                                       ws.numel(), L.stream_of(scale)))
    torch.cuda.synchronize()
    assert torch.all(dscale == 0)


def test_weight_128x128_of_zero_columns(dev):
    """W (K, 0): an empty quantized weight, no launch."""
    w = torch.zeros((256, 0), dtype=torch.bfloat16, device=dev)
    q, s, bn = fp8.quantize_weight(w, "128x128")
    assert q.shape == (0, 256) and s.shape == (0, 2) and bn == 128
    assert L.lib().tg_quantize_weight_128x128(NUL, 256, 0, NUL, NUL, NUL) == L.TG_OK
