"""GPU parity of RMSNorm (kernels.py:30-33) and the fused norm -> FP8 quantize.

Bar: y bf16 bit-exact against the oracle's _rms_norm_pure (f64 sum of f32
squares, correctly rounded rsqrt, bf16 rounding after each op); q / scales
bit-exact against quantizing that y (fp8.py:39-47).
"""
import numpy as np
import pytest
import torch

import kernels
from helpers import as_dtype_values, bf16_bits, f32_bits, maxabs_rel, same_scales, to_dev, u8
from oracle import bf16 as ob
from oracle import cbind, norm_ref

pytestmark = pytest.mark.gpu


def _inputs(rng, shape, outliers=True):
    x = rng.standard_normal(shape)
    if outliers:
        mask = rng.random(shape) < 1e-3
        x = np.where(mask, x * 50.0, x)
    D = shape[-1]
    g = 1.0 + 0.1 * rng.standard_normal(D)        # non-uniform gamma (debug_bf16_norm.py:499-503)
    return ob.f32_to_bf16(x.astype(np.float32)), ob.f32_to_bf16(g.astype(np.float32))


@pytest.mark.parametrize("shape", [(1, 128), (5, 768), (64, 2048), (3, 7, 2304), (33, 9216), (2, 16384)])
def test_rms_norm_pure_bit_exact(dev, shape):
    rng = np.random.default_rng(sum(shape))
    x, g = _inputs(rng, shape)
    y = kernels._rms_norm_pure(to_dev(x, dev), to_dev(g, dev), 1e-6)
    assert y.shape == shape and y.dtype == torch.bfloat16
    yo = norm_ref.rms_norm_pure(x, g, 1e-6)
    np.testing.assert_array_equal(bf16_bits(y), yo)


@pytest.mark.parametrize("D", [8, 200, 1000])
def test_rms_norm_dims_not_multiple_of_128(dev, D):
    rng = np.random.default_rng(D)
    x, g = _inputs(rng, (6, D))
    y = kernels.rms_norm(to_dev(x, dev), to_dev(g, dev), 1e-5)
    np.testing.assert_array_equal(bf16_bits(y), norm_ref.rms_norm_pure(x, g, 1e-5))


@pytest.mark.parametrize("shape", [(4, 128), (64, 2048), (2, 5, 2304), (17, 4096)])
def test_rms_norm_fp8_bit_exact(dev, shape):
    rng = np.random.default_rng(sum(shape) + 1)
    x, g = _inputs(rng, shape)
    y, q, s = kernels.rms_norm_fp8(to_dev(x, dev), to_dev(g, dev), 1e-6)
    yo, qo, so = norm_ref.rms_norm_fp8(x, g, 1e-6)
    np.testing.assert_array_equal(bf16_bits(y), yo)
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


def test_rms_norm_fp8_c2_full_size(dev):
    """Config 2: x bf16 [8, 1024, 2048] with 0.1% x50 outliers, gamma 1+N(0,0.1^2), eps 1e-6, seed 1."""
    rng = np.random.default_rng(1)
    x, g = _inputs(rng, (8, 1024, 2048))
    y, q, s = kernels.rms_norm_fp8(to_dev(x, dev), to_dev(g, dev), 1e-6)
    yo, qo, so = cbind.rms_norm_quant_bf16(x, g, 1e-6)
    np.testing.assert_array_equal(bf16_bits(y).reshape(-1, 2048), yo)
    np.testing.assert_array_equal(u8(q).reshape(-1, 2048), qo)
    np.testing.assert_array_equal(f32_bits(s).reshape(-1, 16), so.view(np.uint32))
    # fp32 tolerance bar against the single-rounding arithmetic too (kernels.py:49-53)
    y1 = norm_ref.rms_norm_single_rounding(x[0, :64], g, 1e-6)
    assert maxabs_rel(ob.bf16_to_f32(bf16_bits(y)[0, :64]), ob.bf16_to_f32(y1)) <= 1e-2


def test_rms_norm_special_rows(dev):
    D = 256
    rows = np.stack([
        np.zeros(D), np.full(D, 3.0), -np.full(D, 1e-20), np.full(D, 1e30),
        np.where(np.arange(D) == 3, 1e4, 1e-4),
    ]).astype(np.float32)
    x = ob.f32_to_bf16(rows)
    g = ob.f32_to_bf16(np.linspace(0.5, 1.5, D).astype(np.float32))
    y, q, s = kernels.rms_norm_fp8(to_dev(x, dev), to_dev(g, dev), 1e-6)
    yo, qo, so = norm_ref.rms_norm_fp8(x, g, 1e-6)
    np.testing.assert_array_equal(bf16_bits(y), yo)
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


def test_rms_norm_errors(dev):
    x = torch.zeros((2, 100), dtype=torch.bfloat16, device=dev)
    g = torch.ones(100, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="not divisible by block_k"):
        kernels.rms_norm_fp8(torch.zeros((2, 200), dtype=torch.bfloat16, device=dev),
                             torch.ones(200, dtype=torch.bfloat16, device=dev), 1e-6)
    with pytest.raises(TypeError, match="bfloat16, float16 or float32"):
        kernels.rms_norm(x.double(), g, 1e-6)
    with pytest.raises(TypeError):
        kernels.rms_norm_fp8(x.half(), g, 1e-6)
    with pytest.raises(TypeError):
        kernels.rms_norm_fp8(x.float(), g, 1e-6)
    with pytest.raises(ValueError, match="scale must have shape"):
        kernels.rms_norm(x, g[:50], 1e-6)


@pytest.mark.parametrize("shape", [(1, 2304), (8, 2048), (5, 768), (3, 16384)])
@pytest.mark.parametrize("inplace", [False, True])
def test_add_rms_norm_fp8_bit_exact(dev, shape, inplace):
    """Residual add fused with norm -> FP8 (tg_add_rms_norm_fp8): x_out is the
    bf16 tensor sum (f32 add, one RNE rounding), y / q / scales are the oracle's
    rms_norm_fp8 of x_out, bit for bit."""
    rng = np.random.default_rng(sum(shape) + inplace)
    x, g = _inputs(rng, shape)
    d = ob.randn_bf16(rng, shape, std=0.5)
    xd = to_dev(x, dev)
    xo, q, s, y = kernels.add_rms_norm_fp8(xd, to_dev(d, dev), to_dev(g, dev), 1e-5,
                                            inplace=inplace, want_y=True)
    xs = ob.f32_to_bf16(ob.bf16_to_f32(x) + ob.bf16_to_f32(d))
    np.testing.assert_array_equal(bf16_bits(xo), xs)
    if inplace:
        assert xo.data_ptr() == xd.data_ptr()
    y_o, q_o, s_o = norm_ref.rms_norm_fp8(xs, g, 1e-5)
    np.testing.assert_array_equal(bf16_bits(y), y_o)
    np.testing.assert_array_equal(u8(q).reshape(q_o.shape), q_o)
    assert same_scales(s.cpu().numpy().reshape(s_o.shape), s_o)


def test_add_rms_norm_fp8_without_y(dev):
    rng = np.random.default_rng(11)
    x, g = _inputs(rng, (4, 2304))
    d = ob.randn_bf16(rng, (4, 2304))
    xo, q, s, y = kernels.add_rms_norm_fp8(to_dev(x, dev), to_dev(d, dev), to_dev(g, dev), 1e-5)
    assert y is None
    xs = ob.f32_to_bf16(ob.bf16_to_f32(x) + ob.bf16_to_f32(d))
    _, q_o, s_o = norm_ref.rms_norm_fp8(xs, g, 1e-5)
    np.testing.assert_array_equal(u8(q), q_o)
    assert same_scales(s.cpu().numpy(), s_o)


_ORACLE_DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


@pytest.mark.parametrize("x_dt,g_dt,D", [(torch.float32, torch.float32, 2048), (torch.float32, torch.bfloat16, 1000),
                                        (torch.bfloat16, torch.float32, 2304), (torch.bfloat16, torch.bfloat16, 20000),
                                        (torch.bfloat16, torch.bfloat16, 100), (torch.float16, torch.float16, 2048),
                                        (torch.float16, torch.float16, 100), (torch.float16, torch.bfloat16, 1000),
                                        (torch.bfloat16, torch.float16, 512), (torch.float16, torch.float32, 768)])
def test_rms_norm_any_dtype_and_width(dev, x_dt, g_dt, D):
    """_rms_norm_pure (kernels.py:30-33) keeps x's dtype for r and x * r and returns
    the promoted dtype (the common dtype, else f32: bf16 with f16 promotes to
    f32); bit-exact against norm_ref.rms_norm_pure_any, including widths the
    bf16 kernel does not take and f16 rows whose x * r is subnormal."""
    rng = np.random.default_rng(D)
    x = (rng.standard_normal((37, D)) * np.where(rng.random((37, D)) < 1e-3, 50, 1)).astype(np.float32)
    if x_dt == torch.float16:
        x[:4] *= 1e-3
        x[:4, 3] = 2000.0                      # x * r in f16's subnormal range for the rest of these rows
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    x, g = as_dtype_values(x, x_dt), as_dtype_values(g, g_dt)
    xt = torch.from_numpy(x).to(dev).to(x_dt)
    gt = torch.from_numpy(g).to(dev).to(g_dt)
    y = kernels._rms_norm_pure(xt, gt, 1e-6)
    want = norm_ref.rms_norm_pure_any(x, _ORACLE_DT[x_dt], g, 1e-6)
    out_dt = x_dt if x_dt == g_dt else torch.float32
    assert y.dtype == out_dt and y.shape == xt.shape
    if out_dt == torch.bfloat16:
        np.testing.assert_array_equal(bf16_bits(y), ob.f32_to_bf16(want))
    elif out_dt == torch.float16:
        np.testing.assert_array_equal(y.cpu().numpy().view(np.uint16), want.astype(np.float16).view(np.uint16))
    else:
        np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


def _non_finite_rows(D):
    """Rows of bf16 x that take the norm's special cases (kernels.py:30-33 op by op):
    one +inf / -inf (var = inf, r = 0: finite elements -> 0, the inf one -> NaN),
    one NaN (the whole row NaN), values whose f32 squares overflow (var = inf),
    values near the bf16 maximum, all zeros (r = rsqrt(eps)), bf16 subnormals,
    and an ordinary row between them."""
    rng = np.random.default_rng(D)
    x = rng.standard_normal((9, D)).astype(np.float32)
    x[1, 3] = np.inf
    x[2, D // 2] = np.nan
    x[3, D - 1] = -np.inf
    x[4] *= np.float32(1e30)
    x[5, :] = np.float32(3.0e38) * np.sign(x[5])
    x[6, :] = 0.0
    x[7] *= np.float32(1e-39)                          # bf16 subnormals (min normal ~1.18e-38)
    with np.errstate(over="ignore"):
        xb = ob.f32_to_bf16(x)
    g = ob.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    return xb, g


def _same_bf16(got_bits, ref_bits):
    """Bit equality, any NaN equal to any NaN (the NaN payload is the hardware's)."""
    gn = (got_bits & 0x7F80) == 0x7F80
    gn &= (got_bits & 0x7F) != 0
    rn = (ref_bits & 0x7F80) == 0x7F80
    rn &= (ref_bits & 0x7F) != 0
    assert np.array_equal(gn, rn)
    np.testing.assert_array_equal(got_bits[~gn], ref_bits[~rn])


@pytest.mark.parametrize("D", [256, 2048, 6000])
def test_rms_norm_non_finite_rows(dev, D):
    x, g = _non_finite_rows(D)
    y = kernels.rms_norm(to_dev(x, dev), to_dev(g, dev), 1e-6)
    yo = norm_ref.rms_norm_pure(x, g, 1e-6)
    assert np.isnan(ob.bf16_to_f32(yo[1])).sum() == 1 and np.all(np.isnan(ob.bf16_to_f32(yo[2])))
    _same_bf16(bf16_bits(y), yo)


@pytest.mark.parametrize("D", [256, 2048])
def test_rms_norm_fp8_non_finite_rows(dev, D):
    """The fused quantizer on those rows: a block holding a NaN has a NaN scale
    and NaN bytes (fp8.py:39-47 on the NaN y), the rest as the oracle."""
    x, g = _non_finite_rows(D)
    y, q, s = kernels.rms_norm_fp8(to_dev(x, dev), to_dev(g, dev), 1e-6)
    yo, qo, so = norm_ref.rms_norm_fp8(x, g, 1e-6)
    _same_bf16(bf16_bits(y), yo)
    qg = u8(q)
    nan_g, nan_o = (qg & 0x7F) == 0x7F, (qo & 0x7F) == 0x7F
    assert np.array_equal(nan_g, nan_o)
    np.testing.assert_array_equal(qg[~nan_g], qo[~nan_o])
    assert same_scales(s.cpu().numpy(), so)
