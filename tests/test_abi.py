"""C-ABI checks that need no GPU: the library loads, exports every entry point
declared in include/tg_fp8.h, and rejects bad arguments before launching."""
import ctypes
import os
import re

import _tglib as L

HEADER = L.HEADER_PATH


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tg_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    names = _declared()
    assert len(names) >= 14
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes signature table covers the whole header
    assert sorted(L.SIGNATURES) == names


def test_invalid_arguments_return_einval_without_launch():
    lib = L.lib()
    nul = ctypes.c_void_p(0)
    assert lib.tg_quantize_rows(nul, 0, 4, 256, 0, nul, nul, nul) == L.TG_EINVAL
    assert b"block_k" in lib.tg_last_error()
    # any block_k dividing the extent is accepted (the general path); 96 does not divide 256
    assert lib.tg_quantize_rows(nul, 0, 4, 256, 64, nul, nul, nul) == L.TG_EINVAL
    assert b"null pointer" in lib.tg_last_error()
    assert lib.tg_quantize_rows(nul, 0, 4, 256, 96, nul, nul, nul) == L.TG_EINVAL
    assert b"not divisible" in lib.tg_last_error()
    assert lib.tg_gemm_fp8_nt(nul, nul, nul, nul, 1, nul, 0, 4, 4, 256, 0, nul) == L.TG_EINVAL
    assert b"block_k" in lib.tg_last_error()
    # the pre-quantized-weight GEMV and the K-block-major GEMM are block_k = 128 only
    assert lib.tg_gemv_fp8(nul, nul, nul, nul, 1, nul, 1, 4, 256, 64, nul) == L.TG_EINVAL
    assert b"block_k must be 128" in lib.tg_last_error()
    assert lib.tg_gemm_fp8_nt_km(nul, nul, nul, nul, 1, nul, 0, 4, 4, 256, 64, nul) == L.TG_EINVAL
    assert b"block_k must be 128" in lib.tg_last_error()
    assert lib.tg_quantize_rows(nul, 0, 4, 200, 128, nul, nul, nul) == L.TG_EINVAL
    assert b"not divisible" in lib.tg_last_error()
    assert lib.tg_quantize_rows(nul, 5, 4, 256, 128, nul, nul, nul) == L.TG_EINVAL
    assert lib.tg_quantize_cols(nul, 0, 100, 256, 128, nul, nul, nul) == L.TG_EINVAL
    assert lib.tg_gemm_fp8_nt(nul, nul, nul, nul, 1, nul, 0, 4, 4, 200, 128, nul) == L.TG_EINVAL
    assert lib.tg_gemm_fp8_nt(nul, nul, nul, nul, 7, nul, 0, 4, 4, 256, 128, nul) == L.TG_EINVAL
    assert lib.tg_rms_norm(nul, nul, nul, 2, 100, 1e-6, nul) == L.TG_EINVAL
    assert lib.tg_rms_norm_fp8(nul, nul, nul, nul, nul, 2, 200, 1e-6, 128, nul) == L.TG_EINVAL
    assert lib.tg_gemv_fp8(nul, nul, nul, nul, 1, nul, 65, 16, 256, 128, nul) == L.TG_EINVAL
    assert lib.tg_block_scaled_matmul_bwd_fp8(nul, nul, nul, nul, nul, 100, 128, 128, 128, nul, 0,
                                              nul) == L.TG_EINVAL
    # empty problems are no-ops
    assert lib.tg_quantize_rows(nul, 0, 0, 256, 128, nul, nul, nul) == L.TG_OK


def test_workspace_sizes():
    lib = L.lib()
    M, N, K = 8192, 8192, 2048
    ws = lib.tg_block_scaled_matmul_workspace(M, N, K, 128)
    assert ws >= M * K + N * K + (M + N) * (K // 128) * 4
    wb = lib.tg_block_scaled_matmul_bwd_workspace(M, N, K, 128)
    assert wb >= 2 * M * N + 2 * K * N * 0 + K * N + K * M


def test_check_maps_codes_to_exceptions():
    lib = L.lib()
    nul = ctypes.c_void_p(0)
    rc = lib.tg_quantize_rows(nul, 0, 4, 200, 128, nul, nul, nul)
    try:
        L.check(rc)
    except ValueError as e:
        assert "not divisible" in str(e)
    else:
        raise AssertionError("expected ValueError")


def test_product_does_not_import_oracle():
    pkg = os.path.dirname(L.LIB_PATH)
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(root, f)).read()
                assert "oracle" not in re.sub(r"#.*|//.*", "", text).lower() or f == "build.py", f
