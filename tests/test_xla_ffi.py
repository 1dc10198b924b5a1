"""The XLA FFI handlers (train-gpt_amd/csrc/ffi/tg_xla_ffi.cc) against the C ABI
and the registration table, checked on the CPU: jaxlib is not installed here,
so the XLA layer is not compiled (the build step says so and skips).  The
handlers' logic, tg_ffi_core.h, is compiled and run: test_ffi_core.py (CPU)
and test_gpu_ffi_core.py (GPU)."""
import os
import re

import _tglib as L
import build
import xla_ffi

SRC = build.FFI_SRC
CORE = build.FFI_CORE


def _code(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def _declared():
    return set(re.findall(r"\b(tg_[a-z0-9_]+)\s*\(", _code(L.HEADER_PATH)))


def _bodies(code, head):
    """name -> text of each function whose definition starts with `head` + name."""
    parts = re.split(rf"(?={re.escape(head)})", code)
    out = {}
    for p in parts:
        m = re.match(rf"{re.escape(head)}([A-Za-z0-9_]+)\(", p)
        if m:
            out[m.group(1)] = p
    return out


def test_handlers_call_only_declared_entry_points():
    called = set(re.findall(r"\b(tg_[a-z0-9_]+)\s*\(", _code(SRC) + _code(CORE))) - {"tg_last_error"}
    abi_calls = {n for n in called if not n.startswith("tg_ffi_")}
    assert abi_calls, "no C-ABI calls found"
    assert abi_calls <= _declared(), sorted(abi_calls - _declared())
    # the XLA layer itself calls no entry point: it converts and calls the core
    xla_calls = set(re.findall(r"\b(tg_[a-z0-9_]+)\s*\(", _code(SRC))) - {"tg_last_error"}
    assert {n for n in xla_calls if not n.startswith("tg_ffi_")} == set()


def test_handler_symbols_match_the_registration_table():
    defined = re.findall(r"XLA_FFI_DEFINE_HANDLER_SYMBOL\(\s*(tg_ffi_[a-z0-9_]+)\s*,", _code(SRC))
    assert len(defined) == len(set(defined))
    assert sorted(defined) == sorted(sym for sym, _ in xla_ffi.HANDLERS.values())
    # each handler symbol's function calls the core function of the same name,
    # and that calls every entry point the table lists for the target
    code = _code(SRC)
    fn_of = dict(re.findall(r"XLA_FFI_DEFINE_HANDLER_SYMBOL\(\s*(tg_ffi_[a-z0-9_]+)\s*,\s*([A-Za-z0-9_]+)", code))
    xla_fns = _bodies(code, "ffi::Error ")
    core_fns = _bodies(_code(CORE), "inline Status ")
    for target, (sym, abi) in xla_ffi.HANDLERS.items():
        core_name = sym[len("tg_ffi_"):]
        assert re.search(rf"tgffi::{core_name}\(", xla_fns[fn_of[sym]]), (sym, fn_of[sym])
        for name in abi:
            assert name in _declared(), (target, name)
            assert re.search(rf"\b{name}\s*\(", core_fns[core_name]), (target, name)


def test_every_compute_path_of_the_reference_has_a_handler():
    # fp8.py:39-47, 50-78 (+ the kept-weight GEMM), 85-98 (both rules);
    # kernels.py:30-33, fused norm -> quant, 104-118
    wrapped = {n for _, abi in xla_ffi.HANDLERS.values() for n in abi}
    for name in ("tg_quantize_rows", "tg_block_scaled_matmul", "tg_block_scaled_matmul_bwd_fp8",
                 "tg_block_scaled_matmul_bwd_bf16", "tg_rms_norm_ex", "tg_rms_norm_fp8",
                 "tg_rms_norm_bwd_ex", "tg_gemm_fp8_nt"):
        assert name in wrapped, name


def test_build_step_skips_without_jax(capsys):
    try:
        import jax  # noqa: F401
    except ImportError:
        assert build.build_xla_ffi() is None
        assert "skipping the XLA FFI handlers" in capsys.readouterr().out
    else:  # jaxlib present: the handlers must build
        assert os.path.exists(build.build_xla_ffi())


def test_handler_dtypes_are_accepted_by_their_c_abi():
    """Every handler that maps an operand's bf16 / f32 element type onto a
    dtype code forwards it to a C-ABI entry point, which must accept both
    codes: called with null pointers on a non-empty shape, each entry point
    gets past its dtype check and stops at the pointer check (no launch)."""
    import ctypes
    lib = L.lib()
    nul = ctypes.c_void_p(0)
    code = _code(CORE)
    # the handlers forwarding dtype codes, and the entry points they call with them
    assert re.search(r"tg_quantize_cols\(b\.data, b\.dtype,", code)
    assert re.search(r"tg_quantize_rows\(a\.data, a\.dtype,", code)
    calls = {
        "tg_quantize_rows": lambda d: lib.tg_quantize_rows(nul, d, 4, 256, 128, nul, nul, nul),
        "tg_quantize_cols": lambda d: lib.tg_quantize_cols(nul, d, 256, 4, 128, nul, nul, nul),
        "tg_quantize_cols (block_k 64)": lambda d: lib.tg_quantize_cols(nul, d, 256, 4, 64, nul, nul, nul),
        "tg_rms_norm_ex": lambda d: lib.tg_rms_norm_ex(nul, d, nul, d, nul, 4, 256, ctypes.c_float(1e-6), nul),
        "tg_rms_norm_bwd_ex": lambda d: lib.tg_rms_norm_bwd_ex(nul, d, nul, d, nul, d, nul, nul, 4, 256,
                                                               ctypes.c_float(1e-6), nul, 0, nul),
        "tg_block_scaled_matmul_bwd_bf16": lambda d: lib.tg_block_scaled_matmul_bwd_bf16(
            nul, d, nul, d, nul, d, nul, nul, 128, 128, 128, nul, 0, nul),
    }
    for name, call in calls.items():
        norm = name.startswith("tg_rms_norm")
        for d in (L.TG_DTYPE_BF16, L.TG_DTYPE_F32) + ((L.TG_DTYPE_F16,) if norm else ()):
            assert call(d) == L.TG_EINVAL, (name, d)
            msg = lib.tg_last_error().decode()
            assert "dtype" not in msg, (name, d, msg)
        # f16 is a norm-only code: the core forwards it (is_norm_float) to the norm entry points only
        if not norm:
            assert call(L.TG_DTYPE_F16) == L.TG_EINVAL and "dtype" in lib.tg_last_error().decode(), name
        assert call(9) == L.TG_EINVAL and "dtype" in lib.tg_last_error().decode(), name
    assert re.search(r"case ffi::DataType::F16: return tgffi::kF16;", _code(SRC))
    assert re.search(r"kF16 = TG_DTYPE_F16", code) and re.search(r"is_norm_float\(int d\).*d == kF16", code)
