"""Pins the oracle's _quantize_to_fp8 (fp8.py:39-47).

Closed forms and invariants, each chosen so that a plausible mistake fails:
the scale is fl32(amax / 448) floored at fl32(1e-30) (computed here exactly
with fractions, not by retyping the oracle's numpy expression); the amax
element encodes to +-448 (a wrong divisor or a reciprocal-multiply off by an
ulp breaks it at the 0x7E/0x7F boundary); dequantized values are within half
an e4m3 step; NaN/inf propagate; the C and numpy restatements agree.
"""
from fractions import Fraction

import numpy as np
import torch

from oracle import bf16 as ob
from oracle import cbind, fp8_ref


def _round_f32(fr: Fraction) -> np.float32:
    """Correctly rounded (RNE) f32 of an exact rational (normal range)."""
    f = np.float32(float(fr))                       # within 1 ulp
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - fr),
                                     int(np.array(c, np.float32).view(np.uint32)) & 1))
    return np.float32(best)


def test_scale_closed_form():
    rng = np.random.default_rng(0)
    x = ob.bf16_to_f32(ob.randn_bf16(rng, (64, 512), std=3.0))
    x[0, :128] = 0.0
    x[1, :128] = 1e-35
    _, s = fp8_ref.quantize_fp8(x)
    for r in range(x.shape[0]):
        for b in range(4):
            amax = float(np.max(np.abs(x[r, 128 * b:128 * (b + 1)])))
            want = max(_round_f32(Fraction(amax) / 448), np.float32(1e-30))
            assert s[r, b] == want, (r, b, s[r, b], want)
    assert np.float32(1e-30).view(np.uint32) == 0x0DA24260


def test_ones_known_answer():
    """debug_fp8.py:104-109's operand: ones -> s = fl(1/448), x/s = 447.99997 -> 0x7E."""
    q, s = fp8_ref.quantize_fp8(np.ones((4, 128), np.float32))
    assert np.all(s == np.float32(1.0) / np.float32(448.0))
    assert np.all(q == 0x7E)


def test_amax_element_encodes_to_448():
    rng = np.random.default_rng(1)
    x = ob.bf16_to_f32(ob.randn_bf16(rng, (256, 1024)))
    q, s = fp8_ref.quantize_fp8(x)
    xb = x.reshape(256, 8, 128)
    qb = q.reshape(256, 8, 128)
    idx = np.argmax(np.abs(xb), axis=-1)
    top = np.take_along_axis(qb, idx[..., None], -1)[..., 0]
    assert np.all((top == 0x7E) | (top == 0xFE))


def test_dequant_error_bound():
    rng = np.random.default_rng(2)
    x = ob.bf16_to_f32(ob.randn_bf16(rng, (128, 512)))
    q, s = fp8_ref.quantize_fp8(x)
    deq = fp8_ref.e4m3fn_decode(q).reshape(128, 4, 128) * s[..., None]
    xb = x.reshape(128, 4, 128)
    # half an e4m3 step: 2^-4 relative for normals, 2^-10 * s absolute for subnormals
    bound = np.maximum(np.abs(xb) * 2.0 ** -4, s[..., None] * 2.0 ** -10) * (1 + 1e-6)
    assert np.all(np.abs(deq - xb) <= bound)


def test_special_blocks():
    x = np.zeros((5, 128), np.float32)
    x[1] = -0.0
    x[2, :] = 1.0; x[2, 3] = np.nan
    x[3, :] = 1.0; x[3, 4] = np.inf
    x[4, :] = -2.0; x[4, 0] = -np.inf
    q, s = fp8_ref.quantize_fp8(x)
    assert s[0, 0] == np.float32(1e-30) and np.all(q[0] == 0)
    assert np.all(q[1] == 0x80)
    assert np.isnan(s[2, 0]) and np.all(q[2] & 0x7F == 0x7F)
    assert s[3, 0] == np.inf and q[3, 4] in (0x7F, 0xFF) and np.all(q[3, :4] == 0)
    assert s[4, 0] == np.inf and np.all(q[4, 1:] == 0x80)


def test_c_and_numpy_restatements_agree():
    rng = np.random.default_rng(3)
    x = ob.randn_bf16(rng, (300, 768))
    x[0, 5] = 0x7FC0          # NaN
    x[1, 9] = 0x7F80          # inf
    x[2, :128] = 0x8000       # -0 block
    q1, s1 = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    q2, s2 = cbind.quantize_rows_bf16(x)
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(np.isnan(s1), np.isnan(s2))
    np.testing.assert_array_equal(s1[~np.isnan(s1)], s2[~np.isnan(s2)])
    w = ob.randn_bf16(rng, (256, 200), std=0.02)
    q3, s3 = cbind.quantize_cols_bf16(w)
    q4, s4 = fp8_ref.quantize_fp8(np.ascontiguousarray(ob.bf16_to_f32(w).T))
    np.testing.assert_array_equal(q3, q4)
    np.testing.assert_array_equal(s3, s4)


def test_weight_128x128_tiles():
    rng = np.random.default_rng(4)
    w_t = ob.bf16_to_f32(ob.randn_bf16(rng, (200, 256)))
    q, s = fp8_ref.quantize_weight_128x128(w_t)
    assert s.shape == (2, 2)
    assert s[1, 1] == np.float32(np.max(np.abs(w_t[128:, 128:]))) / np.float32(448)
    deq = fp8_ref.e4m3fn_decode(q) * np.repeat(np.repeat(s, 128, 0)[:200], 128, 1)
    assert np.max(np.abs(deq - w_t)) <= np.max(np.abs(w_t)) * 2.0 ** -4


def test_weight_128x128_every_tile_exact():
    """Every tile of a non-square, ragged grid: (300, 512) -> 3 x 4 tiles, the
    last row block 44 rows deep.  Each tile gets its own magnitude (a factor
    2^(row block) * 3^(col block)), so a transposed or shifted tile index picks
    a scale that is off by a factor >= 1.5 and fails.  Tile (1, 2) is all zero
    (scale floor 1e-30, bytes 0x00); one element of tile (2, 3) is -0.0.  The
    expected scale is the exact rational amax / 448 rounded once to f32 by
    _round_f32 (Fraction arithmetic, no numpy division), floored at
    fl32(1e-30); the expected bytes are torch's float8_e4m3fn cast of the IEEE
    f32 quotient, and the tile's amax element encodes to +-448."""
    rng = np.random.default_rng(11)
    N, K = 300, 512
    w = rng.standard_normal((N, K)).astype(np.float32)
    for tr in range(3):
        for tc in range(4):
            w[128 * tr:128 * (tr + 1), 128 * tc:128 * (tc + 1)] *= np.float32(2.0 ** tr * 3.0 ** tc)
    w[128:256, 256:384] = 0.0
    w[299, 511] = -0.0
    q, s = fp8_ref.quantize_weight_128x128(w)
    assert q.shape == (N, K) and s.shape == (3, 4)
    floor = np.float32(1e-30)
    for tr in range(3):
        rows = slice(128 * tr, min(128 * (tr + 1), N))
        for tc in range(4):
            cols = slice(128 * tc, 128 * (tc + 1))
            tile = w[rows, cols]
            amax = max(abs(float(v)) for v in tile.ravel())
            want = max(_round_f32(Fraction(amax) / 448), floor) if amax > 0 else floor
            assert s[tr, tc] == want, (tr, tc, s[tr, tc], want)
            quot = (tile / np.float32(want)).astype(np.float32)
            got = q[rows, cols]
            exp = torch.from_numpy(np.ascontiguousarray(quot)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            np.testing.assert_array_equal(got, exp, err_msg=f"tile ({tr}, {tc})")
            if amax > 0:
                r, c = np.unravel_index(np.argmax(np.abs(tile)), tile.shape)
                assert got[r, c] in (0x7E, 0xFE), (tr, tc, hex(int(got[r, c])))
    assert s[1, 2] == floor and np.all(q[128:256, 256:384] == 0)
    assert q[299, 511] == 0x80


def test_partial_trailing_block_is_its_valid_elements():
    """quantize_fp8_partial: the trailing block's scale is max(amax of its
    valid elements / 448, 1e-30) and its bytes e4m3(x / s), computed here
    directly (no padding), including an all-zero trailing block."""
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((5, 200)) * np.array([1, 3, 0.01, 100, 1])[:, None]).astype(np.float32)
    x[4, 128:] = 0.0
    q, s = fp8_ref.quantize_fp8_partial(x)
    assert q.shape == (5, 200) and s.shape == (5, 2)
    q_whole, s_whole = fp8_ref.quantize_fp8(x[:, :128])
    np.testing.assert_array_equal(q[:, :128], q_whole)
    np.testing.assert_array_equal(s[:, :1], s_whole)
    tail = x[:, 128:]
    with np.errstate(divide="ignore", invalid="ignore"):
        s_tail = np.maximum(np.max(np.abs(tail), axis=1) / np.float32(448.0), np.float32(1e-30)).astype(np.float32)
        q_tail = fp8_ref.e4m3fn_encode((tail / s_tail[:, None]).astype(np.float32))
    np.testing.assert_array_equal(s[:, 1], s_tail)
    np.testing.assert_array_equal(q[:, 128:], q_tail)
    assert s[4, 1] == np.float32(1e-30) and np.all(q[4, 128:] == 0)
