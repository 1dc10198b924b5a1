"""Device self-tests of two arithmetic building blocks of every quantizer.

* the gfx950 e4m3fn convert (v_cvt_pk_fp8_f32) against the integer RNE
  encoder over all 2**32 f32 bit patterns (the integer encoder is the same
  rule as oracle/tg_oracle.c, which tests/test_oracle_e4m3.py pins against
  torch's CPU float8_e4m3fn cast);
* the reciprocal-refinement divide against the device's IEEE divide for
  every bf16 (x, amax) pair.
"""
import ctypes

import pytest
import torch

import _tglib as L

pytestmark = pytest.mark.gpu


def _run(fn_name, dev, n=3):
    counts = torch.zeros(n, dtype=torch.int64, device=dev)
    L.check(getattr(L.lib(), fn_name)(L.ptr(counts), L.stream_of(counts)))
    torch.cuda.synchronize()
    return [int(v) for v in counts.cpu()]


def test_hw_fp8_convert_matches_integer_encoder(dev):
    in_range, finite_other, nonfinite = _run("tg_selftest_fp8_cvt", dev)
    print(f"hw cvt mismatches: |v|<=448.1: {in_range}, other finite: {finite_other}, "
          f"nan/inf: {nonfinite}")
    # Quantization only converts |v| <= 448*(1+2^-22) with a finite scale.
    assert in_range == 0


def test_divide_refinement_matches_ieee(dev):
    byte_mm, q_above, q_below, scale_mm, rcp_mm = _run("tg_selftest_divide", dev, 5)
    print(f"divide: byte mismatches {byte_mm}, quotient mismatches above 2^-10 {q_above}, "
          f"at/below 2^-10 {q_below}; scale mismatches {scale_mm}, reciprocal mismatches {rcp_mm}")
    assert scale_mm == 0
    assert rcp_mm == 0
    assert byte_mm == 0
    assert q_above == 0
