"""Pins the oracle's e4m3fn encoder (fp8.py:46's astype(float8_e4m3fn)).

Independent implementation: torch's CPU float8_e4m3fn cast (c10's own
conversion, OCP e4m3fn RNE non-saturating like ml_dtypes).  The C encoder is
compared on all 2**32 f32 bit patterns; the numpy encoder on a stratified
sweep that covers every rounding position; both on known answers from the
OCP FP8 spec.
"""
import numpy as np
import pytest
import torch

from oracle import cbind, fp8_ref

KNOWN = [
    (0.0, 0x00), (-0.0, 0x80), (1.0, 0x38), (-1.0, 0xB8), (0.5, 0x30), (448.0, 0x7E),
    (-448.0, 0xFE), (464.0, 0x7E),            # tie at the top rounds to even (0x7E)
    (464.0001, 0x7F), (480.0, 0x7F), (1e6, 0x7F), (-1e6, 0xFF),   # overflow -> NaN, no saturation
    (float("inf"), 0x7F), (float("-inf"), 0xFF), (float("nan"), 0x7F),
    (2.0 ** -6, 0x08),                        # smallest normal
    (2.0 ** -9, 0x01),                        # smallest subnormal
    (7 * 2.0 ** -9, 0x07),                    # largest subnormal
    (2.0 ** -10, 0x00),                       # tie between 0 and 2^-9 -> even (0)
    (1.5 * 2.0 ** -10, 0x01), (1.5 * 2.0 ** -9, 0x02),   # 1.5 * 2^-9 ties to even 2
    (2.5 * 2.0 ** -9, 0x02), (240.0, 0x77), (256.0, 0x78), (1.0625, 0x38), (1.0625 + 1e-6, 0x39),
    (1.1875, 0x3A),                           # tie between 1.125 (0x39) and 1.25 (0x3A) -> even
]


def _torch_cast(v: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()


@pytest.mark.parametrize("v,code", KNOWN)
def test_known_answers(v, code):
    x = np.array([v], dtype=np.float32)
    assert int(fp8_ref.e4m3fn_encode(x)[0]) == code
    assert int(cbind.encode_array(x)[0]) == code
    assert int(_torch_cast(x)[0]) == code


def test_decode_encode_roundtrip():
    codes = np.arange(256, dtype=np.uint8)
    vals = fp8_ref.e4m3fn_decode(codes)
    back = fp8_ref.e4m3fn_encode(vals)
    nan = np.isnan(vals)
    assert nan.sum() == 2 and set(codes[nan]) == {0x7F, 0xFF}
    np.testing.assert_array_equal(back[~nan], codes[~nan])
    # decode agrees with torch's float8 -> f32
    tv = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(tv), nan)
    np.testing.assert_array_equal(tv[~nan], vals[~nan])


def test_numpy_encoder_stratified_vs_torch():
    """Every (sign, exponent, top-7 mantissa bits) with low-bit patterns that
    hit each side of every rounding point."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF], dtype=np.uint32)
    mids = np.array([0, 0x7FFFF, 0x80000, 0x80001, 0xFFFFF], dtype=np.uint32)
    bits = (hi[:, None, None] | (mids[None, :, None] & 0xF0000) | lows[None, None, :]).ravel()
    bits = np.concatenate([bits, (hi[:, None] | mids[None, :]).ravel()])
    v = bits.view(np.float32)
    np.testing.assert_array_equal(fp8_ref.e4m3fn_encode(v), _torch_cast(v))


def test_c_encoder_exhaustive_vs_torch():
    """All 2**32 f32 bit patterns, 2**24 at a time."""
    n = 1 << 24
    base = torch.arange(0, n, dtype=torch.int64)
    for start in range(0, 1 << 32, n):
        c = cbind.encode_range(start, n)
        t = (base + start).to(torch.int32).view(torch.float32).to(torch.float8_e4m3fn)
        t = t.view(torch.uint8).numpy()
        if not np.array_equal(c, t):
            bad = np.nonzero(c != t)[0][:5] + start
            raise AssertionError(f"C encoder differs from torch at f32 bits {[hex(b) for b in bad]}")


def test_numpy_matches_c_random():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    np.testing.assert_array_equal(fp8_ref.e4m3fn_encode(v), cbind.encode_array(v))
