"""Pins the oracle's _rms_norm_pure (kernels.py:30-33), fused norm -> quant and VJP.

* the bf16 ops after the variance are checked against torch's own bf16
  arithmetic on the oracle's r (x * r and * scale are single roundings);
* the variance against an exact (fractions) mean of squares;
* the rsqrt against correctly rounded 1/sqrt (fractions, squared bracket);
* constant rows and scale invariance as closed forms;
* the VJP (kernels.py:104-118) against float64 finite differences.
"""
from fractions import Fraction

import numpy as np
import torch

from oracle import bf16 as ob
from oracle import cbind, norm_ref


def _inputs(rng, shape):
    x = rng.standard_normal(shape)
    x = np.where(rng.random(shape) < 1e-3, 50 * x, x)
    g = 1 + 0.1 * rng.standard_normal(shape[-1])
    return ob.f32_to_bf16(x.astype(np.float32)), ob.f32_to_bf16(g.astype(np.float32))


def _t(u16):
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).view(torch.bfloat16)


def test_bf16_ops_match_torch():
    rng = np.random.default_rng(0)
    x, g = _inputs(rng, (64, 2048))
    _, r = norm_ref.row_inv_rms(x, 1e-6)
    r_b = ob.f32_to_bf16(r)
    t = _t(x) * _t(r_b)[:, None]
    y = (t * _t(g)).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(y, norm_ref.rms_norm_pure(x, g, 1e-6))


def test_variance_and_rsqrt_exact():
    rng = np.random.default_rng(1)
    x, _ = _inputs(rng, (6, 2304))
    var, r = norm_ref.row_inv_rms(x, 1e-6)
    xf = ob.bf16_to_f32(x)
    for i in range(6):
        exact = sum(Fraction(float(np.float32(v) * np.float32(v))) for v in xf[i])
        ssum = np.float32(float(exact))           # sum rounded (double rounding negligible here)
        assert var[i] == np.float32(ssum / np.float32(2304))
        v = Fraction(float(np.float32(var[i] + np.float32(1e-6))))
        ri = Fraction(float(r[i]))
        ulp = Fraction(float(np.spacing(r[i])))
        # r is the f32 nearest to 1/sqrt(v): (r -+ ulp/2)^2 * v brackets 1
        assert (ri - ulp / 2) ** 2 * v <= 1 <= (ri + ulp / 2) ** 2 * v


def test_constant_rows_and_scale_invariance():
    D = 512
    x = ob.f32_to_bf16(np.stack([np.full(D, 3.0), np.full(D, -0.25)]).astype(np.float32))
    g = ob.f32_to_bf16(np.linspace(0.5, 2.0, D).astype(np.float32))
    y = ob.bf16_to_f32(norm_ref.rms_norm_pure(x, g, 0.0))
    gf = ob.bf16_to_f32(g)
    np.testing.assert_allclose(y[0], gf, rtol=2 ** -7)
    np.testing.assert_allclose(y[1], -gf, rtol=2 ** -7)
    rng = np.random.default_rng(2)
    x, g = _inputs(rng, (16, 1024))
    x2 = ob.f32_to_bf16(ob.bf16_to_f32(x) * 4)      # exact scaling by a power of two
    np.testing.assert_array_equal(norm_ref.rms_norm_pure(x, g, 0.0), norm_ref.rms_norm_pure(x2, g, 0.0))


def test_fused_is_quantize_of_norm_and_c_agrees():
    rng = np.random.default_rng(3)
    x, g = _inputs(rng, (40, 2048))
    y, q, s = norm_ref.rms_norm_fp8(x, g, 1e-6)
    y2, q2, s2 = cbind.rms_norm_quant_bf16(x, g, 1e-6)
    np.testing.assert_array_equal(y, y2)
    np.testing.assert_array_equal(q, q2)
    np.testing.assert_array_equal(s, s2)
    single = norm_ref.rms_norm_single_rounding(x, g, 1e-6)
    assert np.mean(single == y) > 0.5          # the two reference variants agree on most elements
    err = np.max(np.abs(ob.bf16_to_f32(single) - ob.bf16_to_f32(y))) / np.max(np.abs(ob.bf16_to_f32(y)))
    assert err < 1e-2


def test_vjp_finite_differences():
    rng = np.random.default_rng(4)
    x, g = _inputs(rng, (3, 256))
    dy = ob.randn_bf16(rng, (3, 256))
    gx, gg = norm_ref.rms_norm_vjp(x, g, 1e-6, dy)
    X = ob.bf16_to_f32(x).astype(np.float64)
    G = ob.bf16_to_f32(g).astype(np.float64)
    DY = ob.bf16_to_f32(dy).astype(np.float64)

    def loss(Xv, Gv):
        r = 1 / np.sqrt(np.mean(Xv * Xv, -1, keepdims=True) + 1e-6)
        return np.sum(Xv * r * Gv * DY)

    h = 1e-6
    for (i, j) in [(0, 0), (1, 17), (2, 255)]:
        Xp, Xm = X.copy(), X.copy()
        Xp[i, j] += h; Xm[i, j] -= h
        fd = (loss(Xp, G) - loss(Xm, G)) / (2 * h)
        assert abs(fd - gx[i, j]) <= 1e-5 * max(1, abs(fd))
    for j in (0, 100):
        Gp, Gm = G.copy(), G.copy()
        Gp[j] += h; Gm[j] -= h
        fd = (loss(X, Gp) - loss(X, Gm)) / (2 * h)
        assert abs(fd - gg[j]) <= 1e-5 * max(1, abs(fd))
