"""GPU parity of the block-scaled FP8 GEMM (fp8.py:50-78) and its VJP.

Bar (north star): bit-exact quantized operands; GEMM outputs within 1e-2
max-abs-normalised error of the oracle (float64 dequant GEMM of the same
quantized operands, fp8_ref.dequant_gemm_nt); the bf16 output is the RNE of
the f32 accumulator.  The f32 output is held much tighter, to F32_TOL.
Measured on gfx950 (C3-like data, K = 256 .. 2048, both tile paths): the f32
output is 1.5e-5 .. 1.9e-5 of max|ref| away from the float64 oracle, while a
CPU emulation of the same promotion with exactly rounded block sums stays at
7e-8 .. 1.8e-7, so the error is the FP8 MFMA's own block summation (it does
not round the exact 128-product sum once).  F32_TOL = 5e-5 sits above that
with margin and far below what a scale applied to the wrong row, column or
K block produces (one block of 16 off by 1% already moves the output by
~1e-3 of max|ref|).  Structured operands with power-of-two scales give exact
known answers on the persistent 256 x 256 tile path.  The error against a
plain bf16 matmul is printed.
"""
import numpy as np
import pytest
import torch

import fp8
from helpers import maxabs_rel, same_scales, to_dev, u8
from oracle import bf16 as ob
from oracle import fp8_ref

pytestmark = pytest.mark.gpu

TOL = 1e-2
F32_TOL = 5e-5


def _gemm(qa, sa, qb, sb, dev, bn=1, out=torch.bfloat16):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return fp8.scaled_matmul(t(qa), t(sa), t(qb), t(sb), b_scale_bn=bn, out_dtype=out)


def test_ones_known_answer(dev):
    """debug_fp8.py:104-109: ones(4,128) @ ones(128,4) == 128."""
    a = torch.ones((4, 128), dtype=torch.bfloat16, device=dev)
    b = torch.ones((128, 4 * 2), dtype=torch.bfloat16, device=dev)
    y = fp8.block_scaled_matmul(a, b)
    assert torch.all(y.float() == 128.0)


def test_layout_known_answer(dev):
    """Asymmetric operands catch transposed fragments: c[m, n] = (m + 1) * (n + 1) * 128 / 448^2 * 448^2."""
    M, N, K = 48, 40, 256
    qa = np.full((M, K), 0x38, np.uint8)          # e4m3 1.0
    qb = np.full((N, K), 0x38, np.uint8)
    sa = np.repeat((np.arange(M, dtype=np.float32) + 1)[:, None], K // 128, axis=1)
    sb = np.repeat((np.arange(N, dtype=np.float32) + 1)[:, None], K // 128, axis=1)
    sb[:, 1] *= 2
    c = _gemm(qa, sa, qb, sb, dev, out=torch.float32).cpu().numpy()
    ref = fp8_ref.dequant_gemm_nt(qa, sa, qb, sb)
    np.testing.assert_allclose(c, ref, rtol=1e-6)


@pytest.mark.parametrize("M,N,K", [(1, 8, 128), (17, 40, 256), (130, 200, 384), (256, 256, 512),
                                   # below 128 large tiles: the short-K ring kernel with 128 x 192
                                   # tiles (C1; 1, 5 and 6 K blocks: no tail / a tail of 2 after a
                                   # round of 3 stages), 128 x 128 (2048^2 on 256 CUs), 128 x 64 (few
                                   # rows: 1 tile row over many CUs; 5 and 18 K blocks against 6
                                   # stages) and N % 8 != 0 (element stores instead of staged rows)
                                   (300, 136, 1024), (2048, 3072, 768), (2048, 3072, 640), (2048, 3072, 128),
                                   (2048, 2048, 256), (128, 6912, 2304), (640, 768, 640), (257, 1001, 640),
                                   # >= 128 tiles of 256 x 256: the large-tile kernel, with ragged
                                   # M / N edges and odd / even numbers of K blocks
                                   (2100, 4000, 384), (4096, 4096, 256), (3000, 2900, 640),
                                   # more tiles than CUs: workgroups loop over 1-2 tiles, the next
                                   # tile's first K block loaded during the current one's last;
                                   # one K block per tile, and an odd count with N % 8 != 0
                                   (5000, 5000, 128), (4300, 4404, 384)])
def test_scaled_gemm_random(dev, M, N, K):
    rng = np.random.default_rng(M * 7 + N)
    a = ob.bf16_to_f32(ob.randn_bf16(rng, (M, K)))
    b = ob.bf16_to_f32(ob.randn_bf16(rng, (N, K), std=0.02))
    qa, sa = fp8_ref.quantize_fp8(a)
    qb, sb = fp8_ref.quantize_fp8(b)
    ref = fp8_ref.dequant_gemm_nt(qa, sa, qb, sb)
    assert maxabs_rel(_gemm(qa, sa, qb, sb, dev), ref) <= TOL
    c32 = _gemm(qa, sa, qb, sb, dev, out=torch.float32).cpu().numpy()
    assert maxabs_rel(c32, ref) <= F32_TOL
    # the bf16 output is the RNE of the f32 accumulator (fp8.py:78)
    c16 = _gemm(qa, sa, qb, sb, dev).view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(c16, ob.f32_to_bf16(c32))


@pytest.mark.parametrize("M,N,K", [(96, 300, 512), (4300, 4400, 384)])
def test_scaled_gemm_weight_tiles_128x128(dev, M, N, K):
    rng = np.random.default_rng(21 + M)
    a = ob.bf16_to_f32(ob.randn_bf16(rng, (M, K)))
    w_t = ob.bf16_to_f32(ob.randn_bf16(rng, (N, K), std=0.02))
    qa, sa = fp8_ref.quantize_fp8(a)
    qw, sw = fp8_ref.quantize_weight_128x128(w_t)
    c = _gemm(qa, sa, qw, sw, dev, bn=128, out=torch.float32)
    assert maxabs_rel(c, fp8_ref.gemv_prequant(qa, sa, qw, sw, bn=128)) <= F32_TOL


def _structured_operands(M, N, K, bn):
    """Exact known answer with row-, column- and K-block-dependent scales.

    Bytes: qa[m, k] = 1.0 for even k, 2.0 for odd k; qb[n, k] = 1.0 or 2.0 by
    (k // 2) % 2, so every 128-wide block sums to 32 * (1 + 2 + 2 + 4) = 288
    only if A and B fragments pair the same K positions.  Scales are powers
    of two that differ per row, column (or 128-column group) and K block:
    every product and partial sum is exact in f32, so the f32 output equals
    288 * (sa @ sb.T) exactly.
    """
    k = np.arange(K)
    qa = np.broadcast_to(np.where(k % 2 == 0, 0x38, 0x40).astype(np.uint8), (M, K)).copy()
    qb = np.broadcast_to(np.where((k // 2) % 2 == 0, 0x38, 0x40).astype(np.uint8), (N, K)).copy()
    nkb = K // 128
    kb = np.arange(nkb)
    sa = np.exp2(((np.arange(M)[:, None] * 7 + kb[None, :] * 3) % 5) - 2).astype(np.float32)
    rows_b = N if bn == 1 else (N + 127) // 128
    sb = np.exp2(((np.arange(rows_b)[:, None] * 5 + kb[None, :] * 11) % 7) - 3).astype(np.float32)
    sb_full = sb if bn == 1 else np.repeat(sb, 128, axis=0)[:N]
    want = 288.0 * (sa.astype(np.float64) @ sb_full.astype(np.float64).T)
    return qa, sa, qb, sb, want


@pytest.mark.parametrize("bn", [1, 128])
@pytest.mark.parametrize("M,N,K", [(5000, 5000, 384), (4300, 4404, 384), (8192, 8192, 2048)])
def test_layout_known_answer_persistent_tiles(dev, M, N, K, bn):
    """>= 128 tiles of 256 x 256 (the kernel bench.py times), with workgroups
    walking several tiles, ragged edges and both weight-scale layouts; the C3
    shape included.  Exact equality in f32, RNE of it in bf16."""
    qa, sa, qb, sb, want = _structured_operands(M, N, K, bn)
    c32 = _gemm(qa, sa, qb, sb, dev, bn=bn, out=torch.float32).cpu().numpy()
    np.testing.assert_array_equal(c32, want.astype(np.float32))
    c16 = _gemm(qa, sa, qb, sb, dev, bn=bn).view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(c16, ob.f32_to_bf16(want.astype(np.float32)))


@pytest.mark.parametrize("M,N,K,bn", [(5000, 5000, 384, 1), (4300, 4404, 384, 128), (8192, 2048, 8192, 1),
                                      (200, 136, 384, 1), (96, 4404, 256, 128), (2048, 3072, 768, 1)])
def test_gemm_km_same_bits(dev, M, N, K, bn):
    """tg_gemm_fp8_nt_km (scales K-block-major) = tg_gemm_fp8_nt on the
    transposed scales, bit for bit, in bf16 and f32, on the persistent 256-tile
    path (>= 128 tiles, ragged edges, both weight-scale layouts) and the
    128-tile path.  (The composites use this path internally; their parity
    tests cover it end to end.)"""
    import _tglib as L
    rng = np.random.default_rng(M + N + K + bn)
    qa, sa = fp8_ref.quantize_fp8(ob.bf16_to_f32(ob.randn_bf16(rng, (M, K))))
    if bn == 1:
        qb, sb = fp8_ref.quantize_fp8(ob.bf16_to_f32(ob.randn_bf16(rng, (N, K), std=0.02)))
    else:
        qb, sb = fp8_ref.quantize_weight_128x128(ob.bf16_to_f32(ob.randn_bf16(rng, (N, K), std=0.02)))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    for out in (torch.bfloat16, torch.float32):
        want = _gemm(qa, sa, qb, sb, dev, bn=bn, out=out)
        got = torch.empty_like(want)
        code = L.TG_DTYPE_F32 if out == torch.float32 else L.TG_DTYPE_BF16
        A, SA, B, SB = t(qa), t(sa.T), t(qb), t(sb.T)
        L.check(L.lib().tg_gemm_fp8_nt_km(L.ptr(A), L.ptr(SA), L.ptr(B), L.ptr(SB), bn, L.ptr(got), code,
                                          M, N, K, 128, L.stream_of(A)))
        assert torch.equal(got.view(torch.int32 if out == torch.float32 else torch.int16),
                           want.view(torch.int32 if out == torch.float32 else torch.int16))


@pytest.mark.parametrize("M,K,N", [(200, 256, 200), (64, 384, 100), (300, 128, 1000), (2048, 768, 3072),
                                   (8192, 2048, 8192)])
def test_composite_forward_same_bits_as_reference_layout(dev, M, K, N):
    """tg_block_scaled_matmul (K-block-major scales in its workspace: the row
    quantizer, the column quantizer's aligned, ragged and unaligned paths, and
    both GEMM tile paths) = quantize_fp8 + scaled_matmul in the reference's
    scale layout, bit for bit."""
    rng = np.random.default_rng(M + K + N)
    a = to_dev(ob.randn_bf16(rng, (M, K)), dev)
    b = to_dev(ob.randn_bf16(rng, (K, N), std=0.02), dev)
    y = fp8.block_scaled_matmul(a, b)
    qa, sa = fp8.quantize_fp8(a)
    qb, sb = fp8.quantize_fp8(b, transpose=True)
    want = fp8.scaled_matmul(qa.view(torch.uint8), sa, qb.view(torch.uint8), sb)
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))


def test_block_scaled_matmul_c1(dev):
    """Config 1: x [2048, 768] ~N(0,1), W [768, 3072] ~N(0, 0.02^2), seed 0."""
    rng = np.random.default_rng(0)
    x = ob.randn_bf16(rng, (2048, 768))
    w = ob.randn_bf16(rng, (768, 3072), std=0.02)
    y = fp8.block_scaled_matmul(to_dev(x, dev), to_dev(w, dev))
    assert y.dtype == torch.bfloat16 and y.shape == (2048, 3072)
    _, ref, (qa, sa), (qb, sb) = fp8_ref.fp8_forward(x, w)
    err = maxabs_rel(y, ref)
    assert err <= TOL
    # the operands the forward quantizes are bit-exact (fp8.py:66,68)
    qx, sx = fp8._quantize_to_fp8(to_dev(x, dev).float(), 128)
    np.testing.assert_array_equal(u8(qx), qa)
    assert same_scales(sx.cpu().numpy(), sa)
    qw, sw = fp8.quantize_fp8(to_dev(w, dev), transpose=True)
    np.testing.assert_array_equal(u8(qw), qb)
    assert same_scales(sw.cpu().numpy(), sb)
    bf = ob.bf16_to_f32(x).astype(np.float64) @ ob.bf16_to_f32(w).astype(np.float64)
    print(f"C1 rel err vs oracle {err:.3e}, vs bf16 matmul {maxabs_rel(y, bf):.3e}")


def test_c1_weight_tiles_128x128(dev):
    """Config 1 with its literal weight scales, one per 128x128 tile of W:
    x [2048, 768] ~N(0,1), W [768, 3072] ~N(0, 0.02^2), seed 0.  W's bytes and
    scales bit-exact against the oracle, the f32 GEMM output within F32_TOL of
    the float64 dequant product, the bf16 output its RNE."""
    rng = np.random.default_rng(0)
    x = ob.randn_bf16(rng, (2048, 768))
    w = ob.randn_bf16(rng, (768, 3072), std=0.02)
    qw, sw, bn = fp8.quantize_weight(to_dev(w, dev), "128x128")
    assert bn == 128 and sw.shape == (24, 6)
    qw_o, sw_o = fp8_ref.quantize_weight_128x128(np.ascontiguousarray(ob.bf16_to_f32(w).T))
    np.testing.assert_array_equal(u8(qw), qw_o)
    assert same_scales(sw.cpu().numpy(), sw_o)
    qx, sx = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    ref = fp8_ref.gemv_prequant(qx, sx, qw_o, sw_o, bn=128)
    c32 = _gemm(qx, sx, qw_o, sw_o, dev, bn=128, out=torch.float32).cpu().numpy()
    assert maxabs_rel(c32, ref) <= F32_TOL
    c16 = _gemm(qx, sx, qw_o, sw_o, dev, bn=128).view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(c16, ob.f32_to_bf16(c32))
    bf = ob.bf16_to_f32(x).astype(np.float64) @ ob.bf16_to_f32(w).astype(np.float64)
    print(f"C1 128x128 W scales: f32 err vs oracle {maxabs_rel(c32, ref):.3e}, "
          f"vs bf16 matmul {maxabs_rel(c32, bf):.3e}")


def test_block_scaled_matmul_leading_dims_and_errors(dev):
    rng = np.random.default_rng(1)
    x = ob.randn_bf16(rng, (2, 3, 256))
    w = ob.randn_bf16(rng, (256, 64), std=0.02)
    y = fp8.block_scaled_matmul(to_dev(x, dev), to_dev(w, dev))
    assert y.shape == (2, 3, 64)
    _, ref, _, _ = fp8_ref.fp8_forward(x, w)
    assert maxabs_rel(y.reshape(6, 64), ref) <= TOL
    with pytest.raises(ValueError, match="contracted-dim mismatch"):
        fp8.block_scaled_matmul(to_dev(x, dev), to_dev(w[:128], dev))
    with pytest.raises(ValueError, match="not divisible by block_k"):
        fp8.block_scaled_matmul(to_dev(x[..., :200], dev), to_dev(w[:200], dev))


def test_block_scaled_matmul_f32_inputs(dev):
    rng = np.random.default_rng(8)
    a = rng.standard_normal((64, 256)).astype(np.float32)
    b = (0.02 * rng.standard_normal((256, 96))).astype(np.float32)
    y = fp8.block_scaled_matmul(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev))
    qa, sa = fp8_ref.quantize_fp8(a)
    qb, sb = fp8_ref.quantize_fp8(np.ascontiguousarray(b.T))
    assert maxabs_rel(y, fp8_ref.dequant_gemm_nt(qa, sa, qb, sb)) <= TOL


@pytest.mark.parametrize("M,N,K", [(128, 128, 128), (256, 384, 512), (512, 256, 768)])
def test_fp8_backward(dev, M, N, K):
    rng = np.random.default_rng(M + N + K)
    a_u = ob.randn_bf16(rng, (M, K))
    b_u = ob.randn_bf16(rng, (K, N), std=0.02)
    g_u = ob.randn_bf16(rng, (M, N), std=1e-3)
    a = to_dev(a_u, dev).requires_grad_(True)
    b = to_dev(b_u, dev).requires_grad_(True)
    y = fp8.block_scaled_matmul(a, b)
    y.backward(to_dev(g_u, dev))
    dx_ref, dw_ref, ops = fp8_ref.fp8_backward_fp8(a_u, b_u, g_u)
    assert a.grad.dtype == torch.bfloat16 and b.grad.dtype == torch.bfloat16
    assert maxabs_rel(a.grad, dx_ref) <= TOL
    assert maxabs_rel(b.grad, dw_ref) <= TOL
    dx_bf, dw_bf = fp8_ref.fp8_backward_bf16(a_u, b_u, g_u)
    print(f"bwd ({M},{N},{K}): dX err vs bf16 rule {maxabs_rel(a.grad, dx_bf):.3e}, "
          f"dW {maxabs_rel(b.grad, dw_bf):.3e}")
    # the gradient operands are quantized bit-exactly
    qg, sg = fp8.quantize_fp8(to_dev(g_u, dev))
    np.testing.assert_array_equal(u8(qg), ops["g_rows"][0])
    qat, sat = fp8.quantize_fp8(to_dev(a_u, dev), transpose=True)
    np.testing.assert_array_equal(u8(qat), ops["a_cols"][0])
    assert same_scales(sat.cpu().numpy(), ops["a_cols"][1])


def test_prequant_backward_ragged_same_bits(dev):
    """block_scaled_matmul_prequant (left operand quantized by the caller, e.g.
    by rms_norm_fp8) shares block_scaled_matmul's backward, ragged M and N
    included: the same output and gradient bits."""
    rng = np.random.default_rng(77)
    a_u = ob.randn_bf16(rng, (200, 256))
    b_u = ob.randn_bf16(rng, (256, 200), std=0.02)
    g = to_dev(ob.randn_bf16(rng, (200, 200), std=1e-3), dev)
    a1, b1 = to_dev(a_u, dev).requires_grad_(True), to_dev(b_u, dev).requires_grad_(True)
    a2, b2 = to_dev(a_u, dev).requires_grad_(True), to_dev(b_u, dev).requires_grad_(True)
    y1 = fp8.block_scaled_matmul(a1, b1)
    aq, as_ = fp8.quantize_fp8(a2.detach())
    y2 = fp8.block_scaled_matmul_prequant(a2, aq, as_, b2)
    y1.backward(g)
    y2.backward(g)
    assert torch.equal(y1, y2)
    assert torch.equal(a1.grad, a2.grad) and torch.equal(b1.grad, b2.grad)


@pytest.mark.parametrize("lead,K,N", [((200,), 256, 200), ((256,), 384, 200), ((200,), 128, 384),
                                      ((3,), 128, 8), ((2, 100), 256, 128)])
def test_fp8_backward_ragged(dev, lead, K, N):
    """M or N not a multiple of 128 (fp8.py:85-98 accepts any shape): the FP8
    rule on zero-padded operands, i.e. the trailing partial block quantized
    over its valid elements (oracle: fp8_ref.fp8_backward_fp8)."""
    rng = np.random.default_rng(sum(lead) + 3 * N + K)
    a_u = ob.randn_bf16(rng, (*lead, K))
    b_u = ob.randn_bf16(rng, (K, N), std=0.02)
    g_u = ob.randn_bf16(rng, (*lead, N), std=1e-3)
    a = to_dev(a_u, dev).requires_grad_(True)
    b = to_dev(b_u, dev).requires_grad_(True)
    y = fp8.block_scaled_matmul(a, b)
    y.backward(to_dev(g_u, dev))
    dx_ref, dw_ref, _ = fp8_ref.fp8_backward_fp8(a_u, b_u, g_u)
    assert a.grad.shape == a.shape and b.grad.shape == b.shape
    assert maxabs_rel(a.grad.reshape(-1, K), dx_ref) <= TOL
    assert maxabs_rel(b.grad, dw_ref) <= TOL
    dx_bf, dw_bf = fp8_ref.fp8_backward_bf16(a_u, b_u, g_u)
    print(f"ragged bwd {tuple(a.shape)}x{tuple(b.shape)}: dX err vs bf16 rule "
          f"{maxabs_rel(a.grad.reshape(-1, K), dx_bf):.3e}, dW {maxabs_rel(b.grad, dw_bf):.3e}")


def test_gemm_c3_full_size_sampled(dev):
    """Config 3 forward+backward at full size; rows/columns sampled against the oracle."""
    rng = np.random.default_rng(2)
    M, K, N = 8192, 2048, 8192
    a_u = ob.randn_bf16(rng, (M, K))
    b_u = ob.randn_bf16(rng, (K, N), std=0.02)
    g_u = ob.randn_bf16(rng, (M, N), std=1e-3)
    a = to_dev(a_u, dev).requires_grad_(True)
    b = to_dev(b_u, dev).requires_grad_(True)
    y = fp8.block_scaled_matmul(a, b)
    y.backward(to_dev(g_u, dev))
    torch.cuda.synchronize()
    rows = np.sort(rng.choice(M, 256, replace=False))
    cols = np.sort(rng.choice(N, 256, replace=False))
    a32, b32, g32 = (ob.bf16_to_f32(v) for v in (a_u, b_u, g_u))
    qa, sa = fp8_ref.quantize_fp8(a32[rows])
    qbt, sbt = fp8_ref.quantize_fp8(np.ascontiguousarray(b32.T))
    assert maxabs_rel(y[torch.from_numpy(rows).to(dev)], fp8_ref.dequant_gemm_nt(qa, sa, qbt, sbt)) <= TOL
    qg, sg = fp8_ref.quantize_fp8(g32[rows])
    qb, sb = fp8_ref.quantize_fp8(b32)
    assert maxabs_rel(a.grad[torch.from_numpy(rows).to(dev)], fp8_ref.dequant_gemm_nt(qg, sg, qb, sb)) <= TOL
    qat, sat = fp8_ref.quantize_fp8(np.ascontiguousarray(a32.T))
    qgt, sgt = fp8_ref.quantize_fp8(np.ascontiguousarray(g32[:, cols].T))
    dw_ref = fp8_ref.dequant_gemm_nt(qat, sat, qgt, sgt)
    assert maxabs_rel(b.grad[:, torch.from_numpy(cols).to(dev)], dw_ref) <= TOL


@pytest.mark.parametrize("need", ["both", "a", "b"])
@pytest.mark.parametrize("shape", [(2, 128, 256, 384), (1, 1024, 640, 512)])
def test_fp8_backward_kept_residuals_same_bits(dev, need, shape):
    """The autograd path keeps FP8 forms of a.T and b from the forward; its
    output and gradients equal _fp8_forward / _fp8_backward on the bf16
    operands bit for bit, whichever operands need a gradient."""
    B, T, K, N = shape
    rng = np.random.default_rng(B + T + K + N)
    a_u = ob.randn_bf16(rng, (B, T, K))
    b_u = ob.randn_bf16(rng, (K, N), std=0.02)
    g = to_dev(ob.randn_bf16(rng, (B, T, N), std=1e-3), dev)
    a = to_dev(a_u, dev).requires_grad_(need in ("both", "a"))
    b = to_dev(b_u, dev).requires_grad_(need in ("both", "b"))
    y = fp8.block_scaled_matmul(a, b)
    y.backward(g)
    y_ref = fp8._fp8_forward(a.detach(), b.detach(), 128)
    da_ref, db_ref = fp8._fp8_backward(128, (a.detach(), b.detach()), g)
    assert torch.equal(y, y_ref)
    if need in ("both", "a"):
        assert a.grad.shape == a.shape and torch.equal(a.grad, da_ref)
    else:
        assert a.grad is None
    if need in ("both", "b"):
        assert torch.equal(b.grad, db_ref)
    else:
        assert b.grad is None


def test_fp8_backward_mode_switch_after_forward_raises(dev):
    a = torch.randn((128, 128), device=dev).to(torch.bfloat16).requires_grad_(True)
    b = torch.randn((128, 128), device=dev).to(torch.bfloat16).requires_grad_(True)
    y = fp8.block_scaled_matmul(a, b)
    old = fp8.BACKWARD_MODE
    try:
        fp8.BACKWARD_MODE = "bf16"
        with pytest.raises(RuntimeError, match="BACKWARD_MODE changed"):
            y.sum().backward()
    finally:
        fp8.BACKWARD_MODE = old


def test_composite_forward_non_finite_operands(dev):
    """NaN / +-inf in a and b through tg_block_scaled_matmul (fp8.py:50-78):
    a NaN element gives its block a NaN scale, an infinite one an infinite
    scale and a NaN byte (inf / inf), so exactly the rows of a and the columns
    of b that hold one come out NaN (the oracle's float64 product); every
    other output stays within the usual bar, and the operand bytes and scales
    the forward quantizes are bit-exact."""
    rng = np.random.default_rng(7)
    M, K, N = 256, 384, 320
    a = ob.randn_bf16(rng, (M, K))
    b = ob.randn_bf16(rng, (K, N), std=0.02)
    a[3, 10] = 0x7FC0                               # NaN in row 3, K block 0
    a[7, 200] = 0x7F80                              # +inf in row 7, K block 1
    b[5, 9] = 0xFF80                                # -inf in column 9, K block 0
    with np.errstate(invalid="ignore", over="ignore"):
        _, ref, (qa, sa), (qb, sb) = fp8_ref.fp8_forward(a, b)
    y = fp8.block_scaled_matmul(to_dev(a, dev), to_dev(b, dev)).float().cpu().numpy()
    nan_ref = np.isnan(ref)
    assert nan_ref.sum() == 2 * N + M - 2          # rows 3 and 7, column 9
    np.testing.assert_array_equal(np.isnan(y), nan_ref)
    assert maxabs_rel(y[~nan_ref], ref[~nan_ref]) <= TOL
    qx, sx = fp8.quantize_fp8(to_dev(a, dev))
    np.testing.assert_array_equal(u8(qx), qa)
    assert same_scales(sx.cpu().numpy(), sa)
    qw, sw = fp8.quantize_fp8(to_dev(b, dev), transpose=True)
    np.testing.assert_array_equal(u8(qw), qb)
    assert same_scales(sw.cpu().numpy(), sb)


def test_fp8_backward_non_finite_operands(dev):
    """NaN / +-inf through the FP8 backward (dX = fwd(g, b.T), dW = fwd(a.T, g)):
    a NaN in g poisons its row of dX and its column of dW, an inf in a its row
    of dW (the K index), an inf in b its column of dX; exactly where the float64
    oracle has NaN, the rest within the bar."""
    rng = np.random.default_rng(11)
    M, N, K = 256, 384, 256
    a_u = ob.randn_bf16(rng, (M, K))
    b_u = ob.randn_bf16(rng, (K, N), std=0.02)
    g_u = ob.randn_bf16(rng, (M, N), std=1e-3)
    g_u[3, 10] = 0x7FC0                             # NaN: dX row 3, dW column 10
    a_u[7, 200] = 0x7F80                            # +inf: dW row 200
    b_u[5, 9] = 0xFF80                              # -inf: dX column 5
    a = to_dev(a_u, dev).requires_grad_(True)
    b = to_dev(b_u, dev).requires_grad_(True)
    fp8.block_scaled_matmul(a, b).backward(to_dev(g_u, dev))
    with np.errstate(invalid="ignore", over="ignore"):
        dx_ref, dw_ref, _ = fp8_ref.fp8_backward_fp8(a_u, b_u, g_u)
    assert np.isnan(dx_ref).sum() == K + M - 1 and np.isnan(dw_ref).sum() == N + K - 1
    for got, ref in ((a.grad, dx_ref), (b.grad, dw_ref)):
        g = got.float().cpu().numpy()
        np.testing.assert_array_equal(np.isnan(g), np.isnan(ref))
        m = ~np.isnan(ref)
        assert maxabs_rel(g[m], ref[m]) <= TOL
