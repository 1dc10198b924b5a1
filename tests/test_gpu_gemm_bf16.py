"""GPU parity of the straight-through bf16 backward (fp8.py:85-98).

The reference's dots take bf16 operands, accumulate in fp32 and round once to
bf16.  Bars:
  * small-integer operands (exact fp32 sums): the bf16 output equals the RNE
    of the exact result, bit for bit, which pins the fragment layout, the
    K-step order and the epilogue;
  * random operands: max-abs-normalised error <= 1e-2 against the float64
    oracle (fp8_ref.fp8_backward_bf16), and at least 99% of the outputs equal
    to the RNE of the float64 result (the rest differ by one bf16 ulp, where
    the fp32 sum lands on the other side of a rounding boundary);
  * the operand casts / transposes (tg_pack_bf16) are bit-exact.
"""
import ctypes

import numpy as np
import pytest
import torch

import _tglib as L
import fp8
from helpers import bf16_bits, maxabs_rel, to_dev
from oracle import bf16 as ob
from oracle import fp8_ref

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _gemm_bf16(a, b):
    """c = a . b.T through tg_gemm_bf16_nt (a (M, K), b (N, K) bf16 device tensors)."""
    M, K = a.shape
    N = b.shape[0]
    c = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    L.check(L.lib().tg_gemm_bf16_nt(L.ptr(a), L.ptr(b), L.ptr(c), M, N, K, L.stream_of(a)))
    return c


def _rne_equal(got_bits, ref_f64):
    """Fraction of bf16 outputs equal to the RNE of the float64 result."""
    return float(np.mean(got_bits == ob.f32_to_bf16(ref_f64.astype(np.float32))))


def _within_bound(got, ref, abs_sum, K):
    """Elementwise error bound of an fp32-accumulated dot rounded to bf16:
    |got - ref| <= 2^-8 |ref| (one bf16 rounding, with margin) + K 2^-23 sum|a_k b_k|
    (fp32 accumulation in any order).  Near-cancelling outputs may be many bf16
    ulps off, which this bound allows and a ulp count would not."""
    got = np.asarray(got, np.float64)
    return bool(np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + K * 2.0 ** -23 * abs_sum))


@pytest.mark.parametrize("M,N,K", [(40, 24, 64), (256, 256, 128), (300, 520, 192),
                                   (2100, 4000, 320), (4096, 2048, 64)])
def test_integer_operands_exact(dev, M, N, K):
    """Small integers: every partial sum is exact in fp32, so out = RNE(exact)."""
    m = np.arange(M)[:, None]
    n = np.arange(N)[:, None]
    k = np.arange(K)[None, :]
    a = ((m * 3 + k) % 5 - 2).astype(np.float32)
    b = ((n * 5 + 2 * k) % 7 - 3).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64).T
    got = _gemm_bf16(to_dev(ob.f32_to_bf16(a), dev), to_dev(ob.f32_to_bf16(b), dev))
    assert np.array_equal(bf16_bits(got), ob.f32_to_bf16(ref.astype(np.float32)))


@pytest.mark.parametrize("M,N,K", [(1, 8, 64), (17, 40, 128), (130, 200, 384), (512, 768, 64),
                                   (2100, 4000, 320), (3000, 2900, 640)])
def test_gemm_bf16_random(dev, M, N, K):
    rng = np.random.default_rng(M * 31 + N + K)
    a = ob.randn_bf16(rng, (M, K))
    b = ob.randn_bf16(rng, (N, K), std=0.02)
    a64 = ob.bf16_to_f32(a).astype(np.float64)
    b64 = ob.bf16_to_f32(b).astype(np.float64)
    ref = a64 @ b64.T
    got = _gemm_bf16(to_dev(a, dev), to_dev(b, dev))
    err = maxabs_rel(got, ref)
    eq = _rne_equal(bf16_bits(got), ref)
    print(f"bf16 gemm {M}x{N}x{K}: max-abs-rel {err:.2e}, RNE-equal {eq:.5f}")
    assert err <= TOL
    assert eq >= 0.99
    assert _within_bound(got.float().cpu().numpy(), ref, np.abs(a64) @ np.abs(b64).T, K)


def test_gemm_bf16_rejects_bad_k(dev):
    a = torch.zeros((16, 96), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="multiple of 64"):
        _gemm_bf16(a, a)


@pytest.mark.parametrize("transpose", [0, 1])
@pytest.mark.parametrize("src", ["bf16", "f32"])
@pytest.mark.parametrize("rows,cols,pad", [(1, 1, 63), (65, 130, 0), (100, 64, 28), (333, 77, 51),
                                           # 16-byte rows: the 128 x 128 tile kernel when transposing
                                           (200, 264, 56), (1000, 8, 0), (384, 1024, 0), (129, 136, 7)])
def test_pack_bf16(dev, transpose, src, rows, cols, pad):
    rng = np.random.default_rng(rows * 7 + cols)
    x32 = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    # include values that round differently under RNE vs truncation, and -0
    x32.reshape(-1)[::7] = np.float32(1.0 + 2.0 ** -8 + 2.0 ** -20)
    x32.reshape(-1)[::11] = np.float32(-0.0)
    if src == "bf16":
        xb = ob.f32_to_bf16(x32)
        x = to_dev(xb, dev)
        want = xb
    else:
        x = torch.from_numpy(x32).to(dev)
        want = ob.f32_to_bf16(x32)
    if transpose:
        want = want.T
    out_rows, width = want.shape
    pitch = width + pad
    y = torch.full((out_rows, pitch), 7.0, dtype=torch.bfloat16, device=dev)
    L.check(L.lib().tg_pack_bf16(L.ptr(x), L.dtype_code(x), rows, cols, transpose, L.ptr(y), pitch,
                                 L.stream_of(x)))
    got = bf16_bits(y)
    assert np.array_equal(got[:, :width], want)
    assert np.all(got[:, width:] == 0)


def test_pack_bf16_transpose_larger_than_infinity_cache(dev):
    """The transposing tile kernel's non-temporal-store variant (output > 256 MB),
    against torch's transpose, with row padding."""
    rows, cols, pad = 4096, 32832 + 8, 8
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn((rows, cols), generator=g, device=dev).to(torch.bfloat16)
    pitch = rows + pad
    y = torch.full((cols, pitch), 7.0, dtype=torch.bfloat16, device=dev)
    L.check(L.lib().tg_pack_bf16(L.ptr(x), L.TG_DTYPE_BF16, rows, cols, 1, L.ptr(y), pitch, L.stream_of(x)))
    assert torch.equal(y[:, :rows], x.t()) and torch.all(y[:, rows:] == 0)


def _bf16_bwd(a, b, g):
    old = fp8.BACKWARD_MODE
    fp8.BACKWARD_MODE = "bf16"
    try:
        a = a.detach().requires_grad_(True)
        b = b.detach().requires_grad_(True)
        y = fp8.block_scaled_matmul(a, b)
        y.backward(g)
        return a.grad, b.grad
    finally:
        fp8.BACKWARD_MODE = old


@pytest.mark.parametrize("lead,K,N", [((2048,), 768, 3072),     # C1 shapes
                                      ((100,), 256, 200),       # N, M not multiples of 64
                                      ((3, 50), 384, 136),      # 3-D activations
                                      ((1,), 128, 8)])
def test_bf16_backward_matches_oracle(dev, lead, K, N):
    rng = np.random.default_rng(K + N)
    a = ob.randn_bf16(rng, (*lead, K))
    b = ob.randn_bf16(rng, (K, N), std=0.02)
    g = ob.randn_bf16(rng, (*lead, N), std=1e-3)
    da, db = _bf16_bwd(to_dev(a, dev), to_dev(b, dev), to_dev(g, dev))
    assert da.dtype == torch.bfloat16 and db.dtype == torch.bfloat16
    assert da.shape == (*lead, K) and db.shape == (K, N)
    rda, rdb = fp8_ref.fp8_backward_bf16(a, b, g)
    # sums of |terms| for the error bound: the same products on |a|, |b|, |g|
    sda, sdb = fp8_ref.fp8_backward_bf16(a & 0x7FFF, b & 0x7FFF, g & 0x7FFF)
    M = rda.shape[0]
    for name, got, ref, s, k in (("da", da.reshape(-1, K), rda, sda, N), ("db", db, rdb, sdb, M)):
        err = maxabs_rel(got, ref)
        eq = _rne_equal(bf16_bits(got), ref)
        print(f"bf16 bwd {lead}x{K}x{N} {name}: max-abs-rel {err:.2e}, RNE-equal {eq:.5f}")
        assert err <= TOL
        assert eq >= 0.99
        assert _within_bound(got.float().cpu().numpy(), ref, s, k)


@pytest.mark.parametrize("M,K,N", [(100, 256, 200), (1, 128, 8), (515, 1152, 520), (2048, 768, 3072)])
def test_bf16_backward_tn_same_bits_as_packed(dev, M, K, N):
    """db = a.T . g from the contraction-major kernel (bf16 a and g, read in
    place through transposed LDS reads) equals, bit for bit, db from the NT
    kernel on the packed transposes (the same a passed as f32, which forces
    the packing): the same products in the same MFMA order.  Ragged output
    tiles (K, N not multiples of 256) and contraction (M not a multiple of 32)."""
    rng = np.random.default_rng(M + K + N)
    a = ob.randn_bf16(rng, (M, K))
    b = ob.randn_bf16(rng, (K, N), std=0.02)
    g = ob.randn_bf16(rng, (M, N), std=1e-3)
    _, db_tn = _bf16_bwd(to_dev(a, dev), to_dev(b, dev), to_dev(g, dev))
    a32 = torch.from_numpy(ob.bf16_to_f32(a)).to(dev)
    _, db_packed = _bf16_bwd(a32, to_dev(b, dev), to_dev(g, dev))
    assert db_tn.dtype == db_packed.dtype == torch.bfloat16
    np.testing.assert_array_equal(bf16_bits(db_tn), bf16_bits(db_packed))


def test_bf16_backward_f32_operands(dev):
    """f32 a / b: the operands are rounded to bf16 first (fp8.py:92-94) and the
    gradients come back as f32 holding bf16 values (fp8.py:95-96)."""
    rng = np.random.default_rng(5)
    M, K, N = 96, 256, 72
    a32 = rng.standard_normal((M, K)).astype(np.float32)
    b32 = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    g = ob.randn_bf16(rng, (M, N), std=1e-3)
    da, db = _bf16_bwd(torch.from_numpy(a32).to(dev), torch.from_numpy(b32).to(dev), to_dev(g, dev))
    assert da.dtype == torch.float32 and db.dtype == torch.float32
    rda, rdb = fp8_ref.fp8_backward_bf16(ob.f32_to_bf16(a32), ob.f32_to_bf16(b32), g)
    for got, ref in ((da, rda), (db, rdb)):
        v = got.cpu().numpy()
        assert np.all((v.view(np.uint32) & 0xFFFF) == 0)   # bf16-valued
        assert maxabs_rel(v, ref) <= TOL
        assert _rne_equal(ob.f32_to_bf16(v), ref) >= 0.99


def test_bf16_backward_empty_tokens(dev):
    """M = 0: da is empty and db is the zero matrix."""
    K, N = 128, 64
    a = torch.zeros((0, K), dtype=torch.bfloat16, device=dev)
    b = torch.ones((K, N), dtype=torch.bfloat16, device=dev)
    g = torch.zeros((0, N), dtype=torch.bfloat16, device=dev)
    da = torch.empty((0, K), dtype=torch.bfloat16, device=dev)
    db = torch.full((K, N), 3.0, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(256, dtype=torch.uint8, device=dev)
    L.check(L.lib().tg_block_scaled_matmul_bwd_bf16(
        L.ptr(a), L.TG_DTYPE_BF16, L.ptr(b), L.TG_DTYPE_BF16, L.ptr(g), L.TG_DTYPE_BF16,
        ctypes.c_void_p(0), L.ptr(db), 0, N, K, L.ptr(ws), 256, L.stream_of(b)))
    torch.cuda.synchronize()
    assert torch.all(db == 0)


def test_bf16_backward_c3_against_fp32_matmul(dev):
    """C3 shapes (x 8192x2048, W 2048x8192, dY 8192x8192): against a torch fp32
    matmul of the same bf16 values, rounded once to bf16."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    M, K, N = 8192, 2048, 8192
    x = torch.randn((M, K), device=dev, generator=gen).to(torch.bfloat16)
    w = (torch.randn((K, N), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
    dy = (torch.randn((M, N), device=dev, generator=gen) * 1e-3).to(torch.bfloat16)
    dx, dw = _bf16_bwd(x, w, dy)
    rdx = dy.float() @ w.float().t().contiguous()
    rdw = x.float().t().contiguous() @ dy.float()
    for name, got, ref in (("dX", dx, rdx), ("dW", dw, rdw)):
        err = float((got.float() - ref).abs().max() / ref.abs().max())
        eq = float((got == ref.to(torch.bfloat16)).float().mean())
        print(f"C3 bf16 bwd {name}: max-abs-rel {err:.2e}, RNE-equal {eq:.5f}")
        assert err <= TOL
        assert eq >= 0.99
