"""The XLA FFI handlers' logic (train-gpt_amd/csrc/ffi/tg_ffi_core.h), run on
the CPU through libtg_ffi_core.so with no GPU work: dtype dispatch (which
element types each handler forwards to the C ABI and which it refuses with its
own message), the shapes it derives, and its scratch requests, including an
allocator that refuses.  Operand pointers are null, so every call that gets
past the handler stops at the C ABI's pointer check before any launch; the
GPU tests (test_gpu_ffi_core.py) run the same entry points on real buffers."""
import re

import ffi_core as C
import pytest

import build

FAKE = 1 << 44          # a scratch base address that is never dereferenced here
BIG = 1 << 40


def _code(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def test_every_core_function_is_exported_and_called_by_its_handler():
    core = set(re.findall(r"inline Status ([a-z0-9_]+)\(void\* stream", _code(build.FFI_CORE)))
    assert core == {n[len("tg_ffi_core_"):] for n in C.SIGNATURES}
    for name in C.SIGNATURES:
        assert getattr(C.lib(), name)
    xla = _code(build.FFI_SRC)
    for fn in core:
        assert re.search(rf"tgffi::{fn}\(", xla), fn
    # the XLA element types the layer maps, and nothing else mapped
    for xt, code in (("BF16", "kBF16"), ("F32", "kF32"), ("F16", "kF16"), ("F8E4M3FN", "kE4M3")):
        assert re.search(rf"case ffi::DataType::{xt}: return tgffi::{code};", xla), xt
    assert "default: return tgffi::kOther;" in xla


def _refused(rc, msg, who):
    """Refused by the handler itself, with its own message."""
    return rc == C.EINVAL and msg.startswith(who)


def _passed(rc, msg, text):
    """Forwarded to the C ABI, which stopped at its pointer check (tg_last_error)."""
    return rc == C.EINVAL and msg == "invalid argument: " + text


NULL = None
S = (4, 256)


@pytest.mark.parametrize("dt", [C.BF16, C.F32, C.F16, C.E4M3, C.OTHER])
def test_quantizers_forward_bf16_and_f32_only(dt):
    rc, msg = C.call("tg_ffi_core_quantize_rows", NULL, C.view(NULL, dt, (2, 4, 256)), NULL, NULL, 128)
    if dt in (C.BF16, C.F32):
        assert _passed(rc, msg, "quantize_rows: null pointer"), msg   # past the handler
    else:
        assert _refused(rc, msg, "tg_quantize_rows: x must be bf16 or f32"), msg
    rc, msg = C.call("tg_ffi_core_quantize_cols", NULL, C.view(NULL, dt, (256, 4)), NULL, NULL, 128)
    if dt in (C.BF16, C.F32):
        assert _passed(rc, msg, "quantize_cols: null pointer"), msg
    else:
        assert _refused(rc, msg, "tg_quantize_cols: x must be 2-D bf16 or f32"), msg


def test_quantize_cols_needs_two_dims():
    rc, msg = C.call("tg_ffi_core_quantize_cols", NULL, C.view(NULL, C.BF16, (2, 256, 4)), NULL, NULL, 128)
    assert _refused(rc, msg, "tg_quantize_cols: x must be 2-D"), msg


@pytest.mark.parametrize("da,db", [(C.BF16, C.BF16), (C.F32, C.BF16), (C.BF16, C.F32), (C.F32, C.F32),
                                   (C.F16, C.BF16), (C.BF16, C.E4M3)])
def test_forward_dispatch_and_scratch_request(da, db):
    M, N, K = 256, 384, 512
    sc = C.Scratch(FAKE, BIG, 0)
    rc, msg = C.call("tg_ffi_core_block_scaled_matmul", NULL, sc, C.view(NULL, da, (2, M // 2, K)),
                     C.view(NULL, db, (K, N)), NULL, 128)
    if C.F16 in (da, db) or C.E4M3 in (da, db):
        assert _refused(rc, msg, "block_scaled_matmul: a and b must be bf16 or f32"), msg
        assert sc.used == 0
        return
    lib = build_lib()
    assert sc.used == lib.tg_block_scaled_matmul_workspace(M, N, K, 128)   # M = rows of the 3-D a
    # bf16: the composite entry point; any f32 operand: the quantizers first
    want = "block_scaled_matmul: null pointer" if (da, db) == (C.BF16, C.BF16) else "quantize_rows: null pointer"
    assert _passed(rc, msg, want), msg


def build_lib():
    import _tglib
    return _tglib.lib()


@pytest.mark.parametrize("name,args", [
    ("tg_ffi_core_block_scaled_matmul", lambda: (C.view(NULL, C.BF16, (256, 512)), C.view(NULL, C.BF16, (512, 256)),
                                                 NULL, 128)),
    ("tg_ffi_core_block_scaled_matmul_bwd_fp8", lambda: (C.view(NULL, C.BF16, (256, 512)),
                                                         C.view(NULL, C.BF16, (512, 256)),
                                                         C.view(NULL, C.BF16, (256, 256)), NULL, NULL, 128)),
    ("tg_ffi_core_block_scaled_matmul_bwd_bf16", lambda: (C.view(NULL, C.F32, (256, 512)),
                                                          C.view(NULL, C.BF16, (512, 256)),
                                                          C.view(NULL, C.BF16, (256, 256)), NULL, NULL)),
    ("tg_ffi_core_rms_norm_bwd", lambda: (C.view(NULL, C.BF16, S), C.view(NULL, C.BF16, (256,)),
                                          C.view(NULL, C.BF16, S), C.view(NULL, C.BF16, S),
                                          C.view(NULL, C.BF16, (256,)), 1e-6)),
])
def test_refused_scratch_is_resource_exhausted(name, args):
    """XLA's allocator returning nothing: the handler reports it (kResourceExhausted)
    and calls nothing; a large enough one serves exactly the library's workspace."""
    a = args()
    rc, msg = C.call(name, NULL, C.Scratch(None, 0, 0), *a)
    assert rc == C.EXHAUSTED and msg == "tg_xla_ffi: scratch allocation failed", msg
    rc, msg = C.call(name, NULL, C.Scratch(FAKE, 1024, 0), *a)      # too small
    assert rc == C.EXHAUSTED, msg
    sc = C.Scratch(FAKE + 64, BIG, 0)                                  # misaligned base: rounded up
    rc, msg = C.call(name, NULL, sc, *a)
    assert rc == C.EINVAL and msg.startswith("invalid argument: ") and msg.endswith("null pointer"), msg
    L = build_lib()
    want = {"tg_ffi_core_block_scaled_matmul": L.tg_block_scaled_matmul_workspace(256, 256, 512, 128),
            "tg_ffi_core_block_scaled_matmul_bwd_fp8": L.tg_block_scaled_matmul_bwd_workspace(256, 256, 512, 128),
            "tg_ffi_core_block_scaled_matmul_bwd_bf16": L.tg_block_scaled_matmul_bwd_bf16_workspace(256, 256, 512),
            "tg_ffi_core_rms_norm_bwd": L.tg_rms_norm_bwd_workspace(4, 256)}[name]
    assert sc.used == want + 192          # the 256-byte alignment of FAKE + 64


def test_fp8_backward_takes_bf16_only():
    sc = C.Scratch(FAKE, BIG, 0)
    for bad in ((C.F32, C.BF16, C.BF16), (C.BF16, C.F32, C.BF16), (C.BF16, C.BF16, C.F16)):
        rc, msg = C.call("tg_ffi_core_block_scaled_matmul_bwd_fp8", NULL, sc,
                         *(C.view(NULL, d, s) for d, s in zip(bad, ((256, 512), (512, 256), (256, 256)))),
                         NULL, NULL, 128)
        assert _refused(rc, msg, "block_scaled_matmul FP8 backward: a, b, g must be bf16"), msg
    assert sc.used == 0


NORM = (C.BF16, C.F16, C.F32)


@pytest.mark.parametrize("dx", NORM + (C.E4M3,))
@pytest.mark.parametrize("ds", NORM + (C.OTHER,))
def test_norm_promotion_rule(dx, ds):
    """y must be the promoted dtype of x and scale (the common one, else f32)."""
    for dy in NORM:
        rc, msg = C.call("tg_ffi_core_rms_norm", NULL, C.view(NULL, dx, S), C.view(NULL, ds, (256,)),
                         C.view(NULL, dy, S), 1e-6)
        ok = dx in NORM and ds in NORM and dy == (dx if dx == ds else C.F32)
        if ok:
            assert _passed(rc, msg, "rms_norm_ex: null pointer"), msg
        else:
            assert _refused(rc, msg, "rms_norm: x, scale bf16, f16 or f32"), msg


def test_norm_backward_output_dtypes():
    sc = C.Scratch(FAKE, BIG, 0)
    for x, s, dy, dx, dsc, ok in ((C.F16, C.BF16, C.F32, C.F16, C.BF16, True),
                                  (C.F16, C.BF16, C.F32, C.F32, C.BF16, False),
                                  (C.F16, C.BF16, C.F32, C.F16, C.F32, False),
                                  (C.E4M3, C.BF16, C.BF16, C.E4M3, C.BF16, False)):
        rc, msg = C.call("tg_ffi_core_rms_norm_bwd", NULL, sc, C.view(NULL, x, S), C.view(NULL, s, (256,)),
                         C.view(NULL, dy, S), C.view(NULL, dx, S), C.view(NULL, dsc, (256,)), 1e-6)
        if ok:
            assert _passed(rc, msg, "rms_norm_bwd_ex: null pointer"), msg
        else:
            assert _refused(rc, msg, "rms_norm backward: bf16 / f16 / f32 operands"), msg


def test_fused_norm_and_gemm_operand_types():
    rc, msg = C.call("tg_ffi_core_rms_norm_fp8", NULL, C.view(NULL, C.F32, S), C.view(NULL, C.BF16, (256,)),
                     NULL, NULL, NULL, 1e-6, 128)
    assert _refused(rc, msg, "rms_norm_fp8: x and scale must be bf16"), msg
    rc, msg = C.call("tg_ffi_core_rms_norm_fp8", NULL, C.view(NULL, C.BF16, S), C.view(NULL, C.BF16, (256,)),
                     NULL, NULL, NULL, 1e-6, 128)
    assert _passed(rc, msg, "rms_norm_fp8: null pointer"), msg
    rc, msg = C.call("tg_ffi_core_gemm_fp8_nt", NULL, C.view(NULL, C.BF16, (128, 256)), NULL,
                     C.view(NULL, C.E4M3, (128, 256)), NULL, NULL, 1)
    assert _refused(rc, msg, "gemm_fp8_nt: a_q and b_q must be e4m3fn"), msg
    rc, msg = C.call("tg_ffi_core_gemm_fp8_nt", NULL, C.view(NULL, C.E4M3, (128, 256)), NULL,
                     C.view(NULL, C.E4M3, (128, 256)), NULL, NULL, 1)
    assert _passed(rc, msg, "gemm_fp8_nt: null pointer"), msg


def test_forward_f32_path_checks_block_k_before_laying_out_the_workspace():
    for bk in (0, -128, 96):   # 96 does not divide K = 512
        sc = C.Scratch(FAKE, BIG, 0)
        rc, msg = C.call("tg_ffi_core_block_scaled_matmul", NULL, sc, C.view(NULL, C.F32, (256, 512)),
                         C.view(NULL, C.BF16, (512, 256)), NULL, bk)
        assert rc == C.EINVAL, msg
        assert msg == "block_scaled_matmul: block_k must be positive and divide K", msg
