"""Pins the oracle's scaled GEMM (fp8.py:70-76), forward (fp8.py:50-78) and VJPs.

The scaled GEMM is checked against a brute-force exact sum (fractions) on
tiny shapes, the ones known answer (debug_fp8.py:104-109), bilinearity in
the scales and the transposition of operands; the forward against a plain
bf16 matmul (FP8 quantization error bound); both backward rules against
the analytic gradients of a bf16 matmul.
"""
from fractions import Fraction

import numpy as np

from oracle import bf16 as ob
from oracle import fp8_ref


def test_dequant_gemm_exact_tiny():
    rng = np.random.default_rng(0)
    M, N, K = 3, 2, 256
    qa = rng.integers(0, 256, size=(M, K), dtype=np.uint8)
    qb = rng.integers(0, 256, size=(N, K), dtype=np.uint8)
    qa[(qa & 0x7F) == 0x7F] = 0x10       # no NaN codes
    qb[(qb & 0x7F) == 0x7F] = 0x21
    sa = rng.random((M, 2)).astype(np.float32) + 0.5
    sb = rng.random((N, 2)).astype(np.float32) + 0.5
    got = fp8_ref.dequant_gemm_nt(qa, sa, qb, sb)
    da, db = fp8_ref.e4m3fn_decode(qa), fp8_ref.e4m3fn_decode(qb)
    for m in range(M):
        for n in range(N):
            exact = sum(Fraction(float(da[m, k])) * Fraction(float(db[n, k]))
                        * Fraction(float(sa[m, k // 128])) * Fraction(float(sb[n, k // 128]))
                        for k in range(K))
            assert abs(got[m, n] - float(exact)) <= 1e-12 * max(1.0, abs(float(exact)))


def test_ones_known_answer():
    y, out, _, _ = fp8_ref.fp8_forward(ob.f32_to_bf16(np.ones((4, 128), np.float32)),
                                       ob.f32_to_bf16(np.ones((128, 4), np.float32)))
    assert np.all(ob.bf16_to_f32(y) == 128.0)
    np.testing.assert_allclose(out, 128.0, rtol=1e-6)


def test_bilinear_in_scales_and_transpose():
    rng = np.random.default_rng(1)
    a = ob.bf16_to_f32(ob.randn_bf16(rng, (8, 256)))
    b = ob.bf16_to_f32(ob.randn_bf16(rng, (6, 256)))
    qa, sa = fp8_ref.quantize_fp8(a)
    qb, sb = fp8_ref.quantize_fp8(b)
    base = fp8_ref.dequant_gemm_nt(qa, sa, qb, sb)
    sa2 = sa.copy(); sa2[3, 1] *= 2
    bumped = fp8_ref.dequant_gemm_nt(qa, sa2, qb, sb)
    part = fp8_ref.dequant_gemm_nt(qa[:, 128:], sa[:, 1:], qb[:, 128:], sb[:, 1:])
    np.testing.assert_allclose(bumped[3] - base[3], part[3], rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(bumped[[0, 1, 2, 4, 5, 6, 7]], base[[0, 1, 2, 4, 5, 6, 7]])
    np.testing.assert_allclose(fp8_ref.dequant_gemm_nt(qb, sb, qa, sa), base.T, rtol=1e-12)


def test_forward_close_to_bf16_matmul():
    rng = np.random.default_rng(2)
    a = ob.randn_bf16(rng, (64, 768))
    b = ob.randn_bf16(rng, (768, 96), std=0.02)
    y, out, (qa, _), (qbt, _) = fp8_ref.fp8_forward(a, b)
    assert y.shape == (64, 96) and qa.shape == (64, 768) and qbt.shape == (96, 768)
    ref = ob.bf16_to_f32(a).astype(np.float64) @ ob.bf16_to_f32(b).astype(np.float64)
    err = np.max(np.abs(out - ref)) / np.max(np.abs(ref))
    assert 1e-3 < err < 0.1          # FP8 noise is present but bounded
    np.testing.assert_array_equal(y, ob.f32_to_bf16(out.astype(np.float32)))


def test_backward_rules():
    rng = np.random.default_rng(3)
    a = ob.randn_bf16(rng, (256, 128))
    b = ob.randn_bf16(rng, (128, 128), std=0.02)
    g = ob.randn_bf16(rng, (256, 128), std=1e-3)
    dx_bf, dw_bf = fp8_ref.fp8_backward_bf16(a, b, g)
    A, B, G = (ob.bf16_to_f32(v).astype(np.float64) for v in (a, b, g))
    np.testing.assert_allclose(dx_bf, G @ B.T, rtol=1e-12)
    np.testing.assert_allclose(dw_bf, A.T @ G, rtol=1e-12)
    dx, dw, ops = fp8_ref.fp8_backward_fp8(a, b, g)
    assert ops["a_cols"][0].shape == (128, 256) and ops["g_cols"][0].shape == (128, 256)
    for got, ref in ((dx, dx_bf), (dw, dw_bf)):
        err = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
        assert err < 0.1


def test_forward_errors():
    import pytest
    a = ob.f32_to_bf16(np.ones((4, 256), np.float32))
    with pytest.raises(ValueError, match="contracted-dim mismatch"):
        fp8_ref.fp8_forward(a, ob.f32_to_bf16(np.ones((128, 4), np.float32)))
    with pytest.raises(ValueError, match="not divisible by block_k"):
        fp8_ref.fp8_forward(a[:, :200], ob.f32_to_bf16(np.ones((200, 4), np.float32)))


def test_gemv_prequant_layouts():
    rng = np.random.default_rng(4)
    x = ob.bf16_to_f32(ob.randn_bf16(rng, (3, 256)))
    w_t = ob.bf16_to_f32(ob.randn_bf16(rng, (200, 256), std=0.02))
    qx, sx = fp8_ref.quantize_fp8(x)
    qw, sw = fp8_ref.quantize_weight_128x128(w_t)
    out = fp8_ref.gemv_prequant(qx, sx, qw, sw, bn=128)
    ref = x.astype(np.float64) @ w_t.T.astype(np.float64)
    assert np.max(np.abs(out - ref)) / np.max(np.abs(ref)) < 0.1
    full = np.repeat(sw, 128, axis=0)[:200]
    np.testing.assert_allclose(out, fp8_ref.dequant_gemm_nt(qx, sx, qw, full), rtol=1e-12)
