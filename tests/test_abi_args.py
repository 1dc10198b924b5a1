"""Argument checks of every compute entry point of include/tg_fp8.h, on the
CPU (no GPU work: each call below stops at a check before any launch).

For each entry point, one call per rule:
  * null buffers with a valid, non-empty shape -> TG_EINVAL, "... null pointer";
  * a negative extent -> TG_EINVAL, reported before the pointers are looked at;
  * an empty problem -> TG_OK with every pointer null (nothing to read or
    write), except where an empty extent is summed over: the backward's db
    (M == 0) and the norm backward's dscale (rows == 0) are zero arrays the
    call must write, so those still need their output pointers
    (test_gpu_empty_extents.py checks the zeros on the GPU).
"""
import pytest

import _tglib as L

N = None
BF = L.TG_DTYPE_BF16
BIG = 1 << 30   # a workspace size that passes the size check

# name -> (non-empty with null buffers, negative extent, empty)
CASES = {
    "tg_quantize_rows": ((N, BF, 4, 256, 128, N, N, N), (N, BF, -4, 256, 128, N, N, N),
                         (N, BF, 0, 256, 128, N, N, N)),
    "tg_quantize_rows_relu2": ((N, 4, 256, 128, N, N, N), (N, -4, 256, 128, N, N, N), (N, 0, 256, 128, N, N, N)),
    "tg_quantize_cols": ((N, BF, 256, 4, 128, N, N, N), (N, BF, 256, -4, 128, N, N, N),
                         (N, BF, 256, 0, 128, N, N, N)),
    "tg_quantize_dual": ((N, 256, 256, 128, N, N, N, N, N), (N, -256, 256, 128, N, N, N, N, N),
                         (N, 0, 256, 128, N, N, N, N, N)),
    "tg_quantize_dual_km": ((N, 256, 256, 128, N, N, N, N, N), (N, -256, 256, 128, N, N, N, N, N),
                            (N, 0, 256, 128, N, N, N, N, N)),
    "tg_quantize_dual_pair": ((N, 256, 256, N, N, N, N, N, 256, 256, N, N, N, N, 128, N),
                              (N, -256, 256, N, N, N, N, N, 256, 256, N, N, N, N, 128, N),
                              (N, 0, 256, N, N, N, N, N, 0, 256, N, N, N, N, 128, N)),
    "tg_quantize_dual_pair_km": ((N, 256, 256, N, N, N, N, N, 256, 256, N, N, N, N, 128, N),
                                 (N, -256, 256, N, N, N, N, N, 256, 256, N, N, N, N, 128, N),
                                 (N, 0, 256, N, N, N, N, N, 0, 256, N, N, N, N, 128, N)),
    "tg_gemm_fp8_nt": ((N, N, N, N, 1, N, BF, 4, 4, 256, 128, N), (N, N, N, N, 1, N, BF, -4, 4, 256, 128, N),
                       (N, N, N, N, 1, N, BF, 0, 4, 256, 128, N)),
    "tg_gemm_fp8_nt_km": ((N, N, N, N, 1, N, BF, 4, 4, 256, 128, N), (N, N, N, N, 1, N, BF, -4, 4, 256, 128, N),
                          (N, N, N, N, 1, N, BF, 0, 4, 256, 128, N)),
    "tg_block_scaled_matmul": ((N, N, N, 4, 4, 256, 128, N, BIG, N), (N, N, N, -4, 4, 256, 128, N, BIG, N),
                               (N, N, N, 0, 4, 256, 128, N, 0, N)),
    "tg_block_scaled_matmul_noalloc": ((N, N, N, 4, 4, 256, 128, N), (N, N, N, -4, 4, 256, 128, N),
                                       (N, N, N, 0, 4, 256, 128, N)),
    "tg_block_scaled_matmul_bwd_fp8": ((N, N, N, N, N, 256, 256, 256, 128, N, BIG, N),
                                       (N, N, N, N, N, -256, 256, 256, 128, N, BIG, N),
                                       (N, N, N, N, N, 0, 256, 256, 128, N, 0, N)),
    "tg_gemm_bf16_nt": ((N, N, N, 4, 4, 256, N), (N, N, N, -4, 4, 256, N), (N, N, N, 0, 4, 256, N)),
    "tg_pack_bf16": ((N, BF, 4, 256, 0, N, 256, N), (N, BF, -4, 256, 0, N, 256, N), (N, BF, 0, 256, 0, N, 256, N)),
    "tg_block_scaled_matmul_bwd_bf16": ((N, BF, N, BF, N, BF, N, N, 4, 4, 256, N, BIG, N),
                                        (N, BF, N, BF, N, BF, N, N, -4, 4, 256, N, BIG, N),
                                        (N, BF, N, BF, N, BF, N, N, 0, 4, 256, N, 0, N)),
    "tg_rms_norm": ((N, N, N, 4, 256, 1e-6, N), (N, N, N, -4, 256, 1e-6, N), (N, N, N, 0, 256, 1e-6, N)),
    "tg_rms_norm_ex": ((N, BF, N, BF, N, 4, 256, 1e-6, N), (N, BF, N, BF, N, -4, 256, 1e-6, N),
                       (N, BF, N, BF, N, 0, 256, 1e-6, N)),
    "tg_rms_norm_fp8": ((N, N, N, N, N, 4, 256, 1e-6, 128, N), (N, N, N, N, N, -4, 256, 1e-6, 128, N),
                        (N, N, N, N, N, 0, 256, 1e-6, 128, N)),
    "tg_add_rms_norm_fp8": ((N, N, N, N, N, N, N, 4, 256, 1e-6, 128, N), (N, N, N, N, N, N, N, -4, 256, 1e-6, 128, N),
                            (N, N, N, N, N, N, N, 0, 256, 1e-6, 128, N)),
    "tg_rms_norm_bwd": ((N, N, N, N, N, 4, 256, 1e-6, N, BIG, N), (N, N, N, N, N, -4, 256, 1e-6, N, BIG, N),
                        (N, N, N, N, N, 0, 256, 1e-6, N, 0, N)),
    "tg_rms_norm_bwd_ex": ((N, BF, N, BF, N, BF, N, N, 4, 256, 1e-6, N, BIG, N),
                           (N, BF, N, BF, N, BF, N, N, -4, 256, 1e-6, N, BIG, N),
                           (N, BF, N, BF, N, BF, N, N, 0, 256, 1e-6, N, 0, N)),
    "tg_gemv_fp8": ((N, N, N, N, 1, N, 4, 16, 256, 128, N), (N, N, N, N, 1, N, -4, 16, 256, 128, N),
                    (N, N, N, N, 1, N, 0, 16, 256, 128, N)),
    "tg_gemv_fp8_rowdot": ((N, N, N, N, 1, N, 1, 16, 256, 128, N), (N, N, N, N, 1, N, -1, 16, 256, 128, N),
                           (N, N, N, N, 1, N, 0, 16, 256, 128, N)),
    "tg_rms_norm_fp8_gemv": ((N, N, N, 1e-6, N, N, N, 1, N, 1, 16, 256, N),
                             (N, N, N, 1e-6, N, N, N, 1, N, -1, 16, 256, N),
                             (N, N, N, 1e-6, N, N, N, 1, N, 0, 16, 256, N)),
    "tg_relu2_fp8_gemv": ((N, N, N, 1, N, 1, 16, 256, N), (N, N, N, 1, N, -1, 16, 256, N),
                          (N, N, N, 1, N, 0, 16, 256, N)),
    "tg_gemv_fp8_rowdot_add": ((N, N, N, N, 1, N, N, 1, 16, 256, 128, N), (N, N, N, N, 1, N, N, -1, 16, 256, 128, N),
                               (N, N, N, N, 1, N, N, 0, 16, 256, 128, N)),
    "tg_relu2_fp8_gemv_add": ((N, N, N, 1, N, N, 1, 16, 256, N), (N, N, N, 1, N, N, -1, 16, 256, N),
                              (N, N, N, 1, N, N, 0, 16, 256, N)),
    "tg_quantize_weight_128x128": ((N, 256, 16, N, N, N), (N, 256, -16, N, N, N), (N, 256, 0, N, N, N)),
    "tg_decode_attention": ((N, N, N, N, N, N, N, 1, 2, 16, 128, 0.1, N), (N, N, N, N, N, N, N, -1, 2, 16, 128, 0.1, N),
                            (N, N, N, N, N, N, N, 0, 2, 16, 128, 0.1, N)),
    "tg_decode_embed": ((N, N, N, N, N, 1, 512, 64, 256, N), (N, N, N, N, N, -1, 512, 64, 256, N),
                        (N, N, N, N, N, 0, 512, 64, 256, N)),
    "tg_logit_cap": ((N, N, 50257, 15.0, N), (N, N, -1, 15.0, N), (N, N, 0, 15.0, N)),
    "tg_logit_cap_xent_fwd": ((N, N, 4, 256, 15.0, N, N, N), (N, N, -4, 256, 15.0, N, N, N),
                              (N, N, 0, 256, 15.0, N, N, N)),
    "tg_logit_cap_xent_bwd": ((N, N, N, N, 1.0, N, 4, 256, 15.0, N, N), (N, N, N, N, 1.0, N, -4, 256, 15.0, N, N),
                              (N, N, N, N, 1.0, N, 0, 256, 15.0, N, N)),
}

# empty problems whose result is a zero array the call must write
WRITES_ZEROS_WHEN_EMPTY = {"tg_block_scaled_matmul_bwd_fp8", "tg_block_scaled_matmul_bwd_bf16",
                           "tg_rms_norm_bwd", "tg_rms_norm_bwd_ex"}


def _call(name, args):
    rc = getattr(L.lib(), name)(*args)
    return rc, (L.lib().tg_last_error().decode() if rc else "")


def test_every_compute_entry_point_is_covered():
    support = {"tg_last_error", "tg_selftest_fp8_cvt", "tg_selftest_divide"}
    sizes = {n for n in L.SIGNATURES if n.endswith("_workspace")}
    assert set(CASES) == set(L.SIGNATURES) - support - sizes


@pytest.mark.parametrize("name", sorted(CASES))
def test_null_buffers_are_refused(name):
    rc, msg = _call(name, CASES[name][0])
    assert rc == L.TG_EINVAL and msg.startswith("invalid argument: ") and msg.endswith("null pointer"), msg


@pytest.mark.parametrize("name", sorted(CASES))
def test_negative_extent_is_refused_before_the_pointers(name):
    rc, msg = _call(name, CASES[name][1])
    assert rc == L.TG_EINVAL and not msg.endswith("null pointer"), msg


@pytest.mark.parametrize("name", sorted(CASES))
def test_empty_problem(name):
    rc, msg = _call(name, CASES[name][2])
    if name in WRITES_ZEROS_WHEN_EMPTY:
        assert rc == L.TG_EINVAL and msg.endswith("null pointer"), msg
    else:
        assert rc == L.TG_OK, msg
