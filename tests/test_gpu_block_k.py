"""GPU parity of the general block-size path (block_k != 128) through the C ABI.

The reference's block_scaled_matmul takes any block_k that divides K
(/root/reference/fp8.py:30-36, 55-56).  block_k = 128 runs the tuned kernels;
every other block size runs the general kernels of csrc/block_generic.hip
behind the same entry points (tg_quantize_rows, tg_quantize_cols,
tg_gemm_fp8_nt, tg_block_scaled_matmul, tg_block_scaled_matmul_bwd_fp8).
Bars:
  * quantized bytes and scales bit-exact against the oracle's _quantize_to_fp8
    with the same block_k (fp8_ref.quantize_fp8), bf16 and f32 inputs, rows and
    transposed, with NaN / inf / zero / subnormal blocks;
  * the GEMM's f32 output within F32_TOL of the float64 dequantized GEMM of the
    same bytes (its block sums are f32 fma chains), exactly equal on
    power-of-two known answers with row-, column- and block-dependent scales,
    and its bf16 output the RNE of its f32 output;
  * the forward composite equal bit for bit to quantize_fp8 + scaled_matmul
    in the layout the composites give the tuned GEMM (block_k a multiple of
    128: each block's scale repeated per 128 columns; a divisor of 128: each
    block in a zero-filled 128-byte slot), and within the
    north star's 1e-2 of the float64 oracle; the FP8 backward within 1e-2 of
    fp8_ref.fp8_backward_fp8, ragged M / N included.
"""
import numpy as np
import pytest
import torch

import fp8
from helpers import maxabs_rel, same_scales, to_dev, u8
from oracle import bf16 as ob
from oracle import fp8_ref

pytestmark = pytest.mark.gpu

BLOCKS = [1, 16, 32, 64, 96, 256]
TOL = 1e-2
F32_TOL = 5e-5


def _specials_bf16(x_u16: np.ndarray) -> np.ndarray:
    x = x_u16.copy()
    x[0, :5] = [0x7FC0, 0x7F80, 0xFF80, 0x0000, 0x8000]   # NaN, +inf, -inf, +0, -0 in row 0
    x[1, :] = 0                                             # an all-zero row (scale floor)
    x[2, 3] = 0x0001                                        # a bf16 subnormal
    return x


@pytest.mark.parametrize("block_k", BLOCKS)
def test_quantize_rows_bf16_bit_exact(dev, block_k):
    rng = np.random.default_rng(block_k)
    x = _specials_bf16(ob.randn_bf16(rng, (5, 768)))
    q, s = fp8.quantize_fp8(to_dev(x, dev), block_k)
    qo, so = fp8_ref.quantize_fp8(ob.bf16_to_f32(x), block_k)
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


@pytest.mark.parametrize("block_k", [16, 64, 96, 768])
def test_quantize_rows_f32_bit_exact(dev, block_k):
    rng = np.random.default_rng(7 + block_k)
    x = (rng.standard_normal((6, 768)) * np.exp2(rng.integers(-20, 20, (6, 1)))).astype(np.float32)
    x[0, :4] = [np.nan, np.inf, -np.inf, 1e-42]                 # NaN, infs, an f32 subnormal
    x[3, :] = 0.0
    q, s = fp8.quantize_fp8(torch.from_numpy(x).to(dev), block_k)
    qo, so = fp8_ref.quantize_fp8(x, block_k)
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


@pytest.mark.parametrize("block_k", [16, 96, 128, 768])
def test_quantize_transposed_f32_bit_exact(dev, block_k):
    """f32 input to the transposed quantizer (fp8.py:68 quantizes b.T after
    astype(f32), whatever b's dtype): the general kernel at every block_k."""
    rng = np.random.default_rng(31 + block_k)
    x = (rng.standard_normal((768, 24)) * np.exp2(rng.integers(-20, 20, (1, 24)))).astype(np.float32)
    x[:4, 0] = [np.nan, np.inf, -np.inf, 1e-42]
    x[:, 3] = 0.0
    q, s = fp8.quantize_fp8(torch.from_numpy(x).to(dev), block_k, transpose=True)
    qo, so = fp8_ref.quantize_fp8(np.ascontiguousarray(x.T), block_k)
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


@pytest.mark.parametrize("block_k", BLOCKS)
def test_quantize_transposed_bit_exact(dev, block_k):
    rng = np.random.default_rng(100 + block_k)
    x = _specials_bf16(ob.randn_bf16(rng, (768, 40)))
    q, s = fp8.quantize_fp8(to_dev(x, dev), block_k, transpose=True)
    qo, so = fp8_ref.quantize_fp8(np.ascontiguousarray(ob.bf16_to_f32(x).T), block_k)
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


@pytest.mark.parametrize("block_k,R,C,transpose", [(512, 5, 1024, False), (64, 37, 1536, False), (16, 3, 2000, False),
                                                   (1024, 2048, 72, True), (512, 1024, 136, True),
                                                   (16, 96, 1000, True), (256, 512, 64, True)])
def test_quantize_wide_blocks_and_ragged_tiles_bit_exact(dev, block_k, R, C, transpose):
    """The wave-cooperative quantizers at their limits: rows with 64 lanes per
    block (512) and chunk counts that end mid-workgroup; columns with the
    largest LDS tile (1024 rows), a last tile of 8 / 40 columns, and one
    exactly 64 wide."""
    rng = np.random.default_rng(block_k * 7 + R + C)
    x = _specials_bf16(ob.randn_bf16(rng, (R, C)))
    if transpose:
        x[:, 5] = 0                                          # an all-zero column block
        x[7, 9] = 0x7F80                                     # +inf inside a column block
    q, s = fp8.quantize_fp8(to_dev(x, dev), block_k, transpose=transpose)
    xf = ob.bf16_to_f32(x)
    qo, so = fp8_ref.quantize_fp8(np.ascontiguousarray(xf.T) if transpose else xf, block_k)
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


def _gemm(qa, sa, qb, sb, dev, bn=1, out=torch.bfloat16):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return fp8.scaled_matmul(t(qa), t(sa), t(qb), t(sb), b_scale_bn=bn, out_dtype=out)


@pytest.mark.parametrize("block_k", BLOCKS)
@pytest.mark.parametrize("M,N,K", [(70, 90, 768), (130, 200, 1536)])
def test_scaled_gemm_random(dev, block_k, M, N, K):
    rng = np.random.default_rng(M + block_k)
    a = ob.bf16_to_f32(ob.randn_bf16(rng, (M, K)))
    b = ob.bf16_to_f32(ob.randn_bf16(rng, (N, K), std=0.02))
    qa, sa = fp8_ref.quantize_fp8(a, block_k)
    qb, sb = fp8_ref.quantize_fp8(b, block_k)
    ref = fp8_ref.dequant_gemm_nt(qa, sa, qb, sb, block_k)
    c32 = _gemm(qa, sa, qb, sb, dev, out=torch.float32).cpu().numpy()
    assert maxabs_rel(c32, ref) <= F32_TOL
    c16 = _gemm(qa, sa, qb, sb, dev).view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(c16, ob.f32_to_bf16(c32))


@pytest.mark.parametrize("bn", [1, 128])
@pytest.mark.parametrize("block_k", [8, 32, 96, 256])
def test_scaled_gemm_known_answer(dev, block_k, bn):
    """qa = 1.0 / 2.0 by k parity, qb = 1.0 / 2.0 by (k // 2) parity: a block of
    block_k (a multiple of 4) sums to block_k / 4 * 9 only if A and B pair the
    same k; power-of-two scales per row, column (or 128-column group) and
    block make every product and sum exact in f32."""
    M, N, K = 67, 300, 768
    k = np.arange(K)
    qa = np.broadcast_to(np.where(k % 2 == 0, 0x38, 0x40).astype(np.uint8), (M, K)).copy()
    qb = np.broadcast_to(np.where((k // 2) % 2 == 0, 0x38, 0x40).astype(np.uint8), (N, K)).copy()
    nkb = K // block_k
    kb = np.arange(nkb)
    sa = np.exp2(((np.arange(M)[:, None] * 7 + kb[None, :] * 3) % 5) - 2).astype(np.float32)
    rows_b = N if bn == 1 else (N + 127) // 128
    sb = np.exp2(((np.arange(rows_b)[:, None] * 5 + kb[None, :] * 11) % 7) - 3).astype(np.float32)
    sb_full = sb if bn == 1 else np.repeat(sb, 128, axis=0)[:N]
    want = (block_k // 4 * 9.0) * (sa.astype(np.float64) @ sb_full.astype(np.float64).T)
    c32 = _gemm(qa, sa, qb, sb, dev, bn=bn, out=torch.float32).cpu().numpy()
    np.testing.assert_array_equal(c32, want.astype(np.float32))


def _unaligned_bf16(x_u16: np.ndarray, dev) -> torch.Tensor:
    """x on the device at a 2-byte (not 16-byte) aligned address: a contiguous
    view one element into a larger buffer, so the scalar quantizer runs."""
    flat = torch.zeros(x_u16.size + 8, dtype=torch.bfloat16, device=dev)
    v = flat[1:1 + x_u16.size].view(x_u16.shape)
    v.copy_(to_dev(x_u16, dev))
    assert v.data_ptr() % 16 != 0 and v.is_contiguous()
    return v


COMPOSITE_CASES = [(bk, (96,), 512, 160) for bk in (16, 32, 64, 256)] + \
    [(bk, (3, 50), 768, 96) for bk in (16, 32, 64, 96, 256, 384)]


@pytest.mark.parametrize("unaligned", [False, True])
@pytest.mark.parametrize("block_k,lead,K,N", COMPOSITE_CASES)
def test_forward_composite(dev, block_k, lead, K, N, unaligned):
    """Random data through tg_block_scaled_matmul at every kind of block size:
    16 (eight zero slots per 128, one 16-byte vector per block), 32, 64, the
    untuned 96 (the general GEMM), 256 and 384 (scales repeated 2 and 3
    times); unaligned=True feeds a 2-byte aligned a (the scalar quantizer)."""
    if unaligned and block_k not in (16, 96, 384):
        pytest.skip("the unaligned input is exercised at one size of each kind")
    rng = np.random.default_rng(K + N + block_k)
    a = ob.randn_bf16(rng, (*lead, K))
    b = ob.randn_bf16(rng, (K, N), std=0.02)
    ad = _unaligned_bf16(a, dev) if unaligned else to_dev(a, dev)
    bd = to_dev(b, dev)
    y = fp8.block_scaled_matmul(ad, bd, block_k=block_k)
    _, ref, _, _ = fp8_ref.fp8_forward(a, b, block_k)
    assert y.shape == (*lead, N) and y.dtype == torch.bfloat16
    assert maxabs_rel(y.reshape(-1, N), ref) <= TOL
    # the composite (tg_block_scaled_matmul) = quantize_fp8 + scaled_matmul, bit for bit, in the
    # layout the composite feeds the tuned GEMM: a multiple of 128 repeats each block's scale per
    # 128 columns; a divisor of 128 puts each block at the start of a zero-filled 128-byte slot
    qa, sa = fp8.quantize_fp8(ad.reshape(-1, K), block_k)
    qb, sb = fp8.quantize_fp8(bd, block_k, transpose=True)
    qa, qb = qa.view(torch.uint8), qb.view(torch.uint8)
    if block_k % 128 != 0 and 128 % block_k != 0:
        pass                                  # untuned: the composite runs the general GEMM itself
    elif block_k % 128 == 0:
        sa, sb = sa.repeat_interleave(block_k // 128, dim=1), sb.repeat_interleave(block_k // 128, dim=1)
    else:
        def slots(q):
            r = q.shape[0]
            z = torch.zeros((r, K // block_k, 128), dtype=torch.uint8, device=dev)
            z[:, :, :block_k] = q.reshape(r, K // block_k, block_k)
            return z.reshape(r, -1)
        qa, qb = slots(qa), slots(qb)
    y2 = fp8.scaled_matmul(qa, sa, qb, sb)
    assert torch.equal(y.reshape(-1, N).view(torch.int16), y2.view(torch.int16))


BWD_CASES = [(bk, M, K, N) for bk in (16, 32, 64, 256)
             for (M, K, N) in ((128, 256, 192), (100, 256, 70), (512, 512, 768))] + \
    [(bk, M, K, N) for bk in (96, 384) for (M, K, N) in ((200, 768, 300), (768, 384, 96))]


@pytest.mark.parametrize("block_k,M,K,N", BWD_CASES)
def test_fp8_backward(dev, block_k, M, K, N):
    """BACKWARD_MODE "fp8" through autograd; ragged M / N (not multiples of
    block_k) take the zero-padded last block."""
    rng = np.random.default_rng(M * N + block_k)
    a = ob.randn_bf16(rng, (M, K))
    b = ob.randn_bf16(rng, (K, N), std=0.05)
    g = ob.randn_bf16(rng, (M, N))
    old = fp8.BACKWARD_MODE
    fp8.BACKWARD_MODE = "fp8"
    try:
        ad = to_dev(a, dev).requires_grad_(True)
        bd = to_dev(b, dev).requires_grad_(True)
        fp8.block_scaled_matmul(ad, bd, block_k=block_k).backward(to_dev(g, dev))
    finally:
        fp8.BACKWARD_MODE = old
    dx, dw, _ = fp8_ref.fp8_backward_fp8(a, b, g, block_k)
    assert maxabs_rel(ad.grad, dx) <= TOL
    assert maxabs_rel(bd.grad, dw) <= TOL


@pytest.mark.parametrize("block_k", [64, 256])
def test_c1_shape(dev, block_k):
    """Config 1's shape (x 2048 x 768, W 768 x 3072) through the general path:
    the quantized operands bit-exact, the f32 GEMM within F32_TOL and the bf16
    composite within the north star's 1e-2 of the float64 oracle."""
    rng = np.random.default_rng(block_k)
    x = ob.randn_bf16(rng, (2048, 768))
    w = ob.randn_bf16(rng, (768, 3072), std=0.02)
    xd, wd = to_dev(x, dev), to_dev(w, dev)
    y = fp8.block_scaled_matmul(xd, wd, block_k=block_k)
    _, ref, (qa, sa), (qb, sb) = fp8_ref.fp8_forward(x, w, block_k)
    assert maxabs_rel(y, ref) <= TOL
    q1, s1 = fp8.quantize_fp8(xd, block_k)
    q2, s2 = fp8.quantize_fp8(wd, block_k, transpose=True)
    np.testing.assert_array_equal(u8(q1), qa)
    np.testing.assert_array_equal(u8(q2), qb)
    assert same_scales(s1.cpu().numpy(), sa) and same_scales(s2.cpu().numpy(), sb)
    c32 = fp8.scaled_matmul(q1.view(torch.uint8), s1, q2.view(torch.uint8), s2, out_dtype=torch.float32)
    assert maxabs_rel(c32, ref) <= F32_TOL


def test_errors(dev):
    a = torch.zeros((4, 96), dtype=torch.bfloat16, device=dev)
    b = torch.zeros((96, 8), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="not divisible by block_k"):
        fp8.block_scaled_matmul(a, b, block_k=64)
    with pytest.raises(ValueError, match="positive"):
        fp8.quantize_fp8(a, block_k=0)
    y = fp8.block_scaled_matmul(a, b, block_k=48)          # 48 divides 96
    assert y.shape == (4, 8) and torch.all(y == 0)
    with pytest.raises(NotImplementedError):
        fp8.quantize_relu2(a, block_k=32)                   # a fused kernel of this library, 128 only
