"""GPU parity of rms_norm's backward (the custom VJP of kernels.py:104-118).

Oracle: norm_ref.rms_norm_vjp in float64 (pinned in test_oracle_norm.py by
the closed form and by central finite differences of _rms_norm_pure's f64
restatement).  Bars:
  * max-abs-normalised error <= 1e-2 for dx and dscale (north star);
  * at least 99% of the bf16 outputs equal to the RNE of the float64 result
    (the kernel computes in f32; the rest sit next to a rounding boundary);
  * dscale identical across calls (fixed summation order).
"""
import numpy as np
import pytest
import torch

import kernels
from helpers import as_dtype_values, bf16_bits, maxabs_rel, to_dev
from oracle import bf16 as ob
from oracle import norm_ref

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _inputs(rng, shape):
    x = rng.standard_normal(shape)
    mask = rng.random(shape) < 1e-3
    x = np.where(mask, x * 50.0, x)                   # C2's outliers
    D = shape[-1]
    g = 1.0 + 0.1 * rng.standard_normal(D)
    dy = rng.standard_normal(shape) * 1e-2
    return (ob.f32_to_bf16(x.astype(np.float32)), ob.f32_to_bf16(g.astype(np.float32)),
            ob.f32_to_bf16(dy.astype(np.float32)))


def _bwd(x, g, dy, eps, dev):
    xt = to_dev(x, dev).requires_grad_(True)
    gt = to_dev(g, dev).requires_grad_(True)
    y = kernels.rms_norm(xt, gt, eps)
    y.backward(to_dev(dy, dev))
    return xt.grad, gt.grad


def _rne_equal(got_bits, ref):
    return float(np.mean(got_bits == ob.f32_to_bf16(np.asarray(ref, np.float32))))


@pytest.mark.parametrize("shape", [(1, 128), (5, 768), (64, 2048), (3, 7, 256), (8, 1024, 2048),
                                   (40, 520), (9, 1000), (33, 4096), (6, 3000)])
def test_rms_norm_bwd_matches_oracle(dev, shape):
    rng = np.random.default_rng(sum(shape) + 7)
    x, g, dy = _inputs(rng, shape)
    eps = 1e-6
    dx, dg = _bwd(x, g, dy, eps, dev)
    assert dx.shape == shape and dx.dtype == torch.bfloat16
    assert dg.shape == (shape[-1],) and dg.dtype == torch.bfloat16
    rdx, rdg = norm_ref.rms_norm_vjp(x, g, eps, dy)
    ex, eg = maxabs_rel(dx, rdx), maxabs_rel(dg, rdg)
    qx, qg = _rne_equal(bf16_bits(dx), rdx), _rne_equal(bf16_bits(dg), rdg)
    print(f"norm bwd {shape}: dx err {ex:.2e} RNE-equal {qx:.5f}; dscale err {eg:.2e} RNE-equal {qg:.5f}")
    assert ex <= TOL and eg <= TOL
    assert qx >= 0.99
    assert qg >= 0.99 if shape[-1] >= 128 else qg >= 0.9


def test_rms_norm_bwd_deterministic(dev):
    rng = np.random.default_rng(11)
    x, g, dy = _inputs(rng, (4096, 2048))
    a = _bwd(x, g, dy, 1e-6, dev)
    b = _bwd(x, g, dy, 1e-6, dev)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_rms_norm_bwd_constant_rows(dev):
    """Known answer: x = c * ones, scale = 1, dy = 1 gives normed = sign(c),
    mean(gs * normed) = sign(c), so dx = rnorm * (1 - 1) = 0 and dscale = rows * sign(c)."""
    D, R = 256, 48
    x = np.full((R, D), 3.0, np.float32)
    x[1::2] = -0.5
    xb, g, dy = ob.f32_to_bf16(x), ob.f32_to_bf16(np.ones(D, np.float32)), ob.f32_to_bf16(np.ones((R, D), np.float32))
    dx, dg = _bwd(xb, g, dy, 1e-6, dev)
    assert float(dx.float().abs().max()) < 1e-5
    # rows alternate +3 / -0.5: normed = +1 / -1 (to within eps), the sum over rows is ~0
    assert float(dg.float().abs().max()) < 1e-3


@pytest.mark.parametrize("x_dt,g_dt,D", [(torch.float32, torch.float32, 2048), (torch.float32, torch.bfloat16, 1000),
                                        (torch.bfloat16, torch.float32, 512), (torch.bfloat16, torch.bfloat16, 8192),
                                        (torch.bfloat16, torch.bfloat16, 100), (torch.float16, torch.float16, 2048),
                                        (torch.float16, torch.bfloat16, 1000), (torch.float32, torch.float16, 300)])
def test_rms_norm_bwd_any_dtype_and_width(dev, x_dt, g_dt, D):
    """kernels.py:104-118 for f32 / mixed operands and a width above the bf16
    kernel's 4096: dx in x's dtype, dscale in scale's, against the float64 VJP;
    dscale identical on a second call (fixed summation order)."""
    rng = np.random.default_rng(D + 1)
    x = rng.standard_normal((300, D)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    x, g = as_dtype_values(x, x_dt), as_dtype_values(g, g_dt)
    out_dt = x_dt if x_dt == g_dt else torch.float32
    dy = as_dtype_values((rng.standard_normal((300, D)) * 1e-2).astype(np.float32), out_dt)
    xt = torch.from_numpy(x).to(dev).to(x_dt).requires_grad_(True)
    gt = torch.from_numpy(g).to(dev).to(g_dt).requires_grad_(True)
    y = kernels.rms_norm(xt, gt, 1e-6)
    y.backward(torch.from_numpy(dy).to(dev).to(out_dt))
    gx, gg = norm_ref.rms_norm_vjp_vals(x, g, 1e-6, dy)
    assert xt.grad.dtype == x_dt and gt.grad.dtype == g_dt
    # the output's rounding: bf16 (TOL), f16 (11 significand bits), f32
    tol = {torch.bfloat16: TOL, torch.float16: 2e-3, torch.float32: 1e-5}
    assert maxabs_rel(xt.grad, gx) <= tol[x_dt]
    assert maxabs_rel(gt.grad, gg) <= max(tol[g_dt], 1e-4)
    first = gt.grad.clone()
    gt.grad = None
    kernels.rms_norm(xt, gt, 1e-6).backward(torch.from_numpy(dy).to(dev).to(out_dt))
    assert torch.equal(gt.grad, first)


def _nan_class_match(got, ref):
    g = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    np.testing.assert_array_equal(np.isnan(g), np.isnan(ref))
    m = ~np.isnan(ref)
    return g[m], ref[m]


@pytest.mark.parametrize("D", [256, 2048, 6000])
def test_rms_norm_bwd_infinite_rows(dev, D):
    """kernels.py:104-118 on rows holding +inf / -inf (rnorm = 0, normed NaN at the
    inf and 0 elsewhere, so the mean and the row's dx are NaN, and dscale is NaN
    in those columns only) and an all-zero row (rnorm = rsqrt(eps), dx = rnorm * gs);
    the other rows and columns as in the finite case."""
    rng = np.random.default_rng(D + 1)
    x, g, dy = _inputs(rng, (12, D))
    x[2, 5] = 0x7F80
    x[6, D - 3] = 0xFF80
    x[9, :] = 0
    with np.errstate(invalid="ignore", over="ignore"):
        rdx, rdg = norm_ref.rms_norm_vjp(x, g, 1e-6, dy)
    assert np.all(np.isnan(rdx[2])) and np.isnan(rdg).sum() == 2
    dx, dg = _bwd(x, g, dy, 1e-6, dev)
    a, b = _nan_class_match(dx, rdx)
    assert maxabs_rel(a, b) <= TOL
    a, b = _nan_class_match(dg, rdg)
    assert maxabs_rel(a, b) <= TOL


def test_rms_norm_bwd_nan_row(dev):
    """A NaN in x: that row's dx and every dscale entry are NaN (it enters every
    column's sum through normed); the other rows' dx unchanged."""
    rng = np.random.default_rng(3)
    x, g, dy = _inputs(rng, (8, 512))
    x[4, 100] = 0x7FC0
    with np.errstate(invalid="ignore"):
        rdx, rdg = norm_ref.rms_norm_vjp(x, g, 1e-6, dy)
    dx, dg = _bwd(x, g, dy, 1e-6, dev)
    a, b = _nan_class_match(dx, rdx)
    assert np.all(np.isnan(rdx[4])) and maxabs_rel(a, b) <= TOL
    assert torch.all(torch.isnan(dg))
