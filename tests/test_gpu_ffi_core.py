"""The XLA FFI handlers' logic (train-gpt_amd/csrc/ffi/tg_ffi_core.h) on the
GPU, through libtg_ffi_core.so: each handler, given its operands as the XLA
layer would pass them (pointer, element type, shape; 3-D activations where XLA
may hand them) and a scratch buffer for XLA's allocator, produces the same bits
as the C-ABI entry point it wraps called directly, and takes exactly that
entry point's workspace.  The f32 forward, which the handler assembles from
the quantizers and the GEMM itself, is checked against the float64 oracle and
against the bf16 composite on bf16-valued inputs."""
import ctypes

import ffi_core as C
import numpy as np
import pytest
import torch

import _tglib as L
from helpers import maxabs_rel
from oracle import fp8_ref

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


def _ok(res):
    rc, msg = res
    assert rc == C.OK, msg


def _same(a, b):
    torch.cuda.synchronize()
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


def _scratch(nbytes, dev):
    buf = torch.empty(max(nbytes, 1) + 512, dtype=torch.uint8, device=dev)
    return buf, C.Scratch(buf.data_ptr(), buf.numel(), 0)


def _vp(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bk", [128, 64])
def test_quantizers(dev, dt, bk):
    torch.manual_seed(1)
    x = torch.randn(3, 64, 512, device=dev).to(dt)
    q = torch.empty(3, 64, 512, dtype=torch.uint8, device=dev)
    s = torch.empty(3, 64, 512 // bk, dtype=torch.float32, device=dev)
    _ok(C.call("tg_ffi_core_quantize_rows", _st(), C.tview(x), q.data_ptr(), s.data_ptr(), bk))
    q2, s2 = torch.empty_like(q), torch.empty_like(s)
    L.check(L.lib().tg_quantize_rows(_vp(x), L.dtype_code(x), 192, 512, bk, _vp(q2), _vp(s2), None))
    assert _same(q, q2) and _same(s, s2)
    w = torch.randn(512, 192, device=dev).to(dt)
    qt = torch.empty(192, 512, dtype=torch.uint8, device=dev)
    stt = torch.empty(192, 512 // bk, dtype=torch.float32, device=dev)
    _ok(C.call("tg_ffi_core_quantize_cols", _st(), C.tview(w), qt.data_ptr(), stt.data_ptr(), bk))
    qt2, st2 = torch.empty_like(qt), torch.empty_like(stt)
    L.check(L.lib().tg_quantize_cols(_vp(w), L.dtype_code(w), 512, 192, bk, _vp(qt2), _vp(st2), None))
    assert _same(qt, qt2) and _same(stt, st2)


@pytest.mark.parametrize("bk", [128, 256, 64])
def test_forward_bf16_is_the_composite(dev, bk):
    torch.manual_seed(2)
    a = torch.randn(2, 128, 512, device=dev).bfloat16()
    b = (torch.randn(512, 384, device=dev) * 0.05).bfloat16()
    ws = L.lib().tg_block_scaled_matmul_workspace(256, 384, 512, bk)
    buf, sc = _scratch(ws, dev)
    out = torch.empty(2, 128, 384, dtype=torch.bfloat16, device=dev)
    _ok(C.call("tg_ffi_core_block_scaled_matmul", _st(), sc, C.tview(a), C.tview(b), out.data_ptr(), bk))
    assert sc.used - (-buf.data_ptr() % 256) == ws
    ref = torch.empty_like(out)
    wsb = torch.empty(ws, dtype=torch.uint8, device=dev)
    L.check(L.lib().tg_block_scaled_matmul(_vp(a), _vp(b), _vp(ref), 256, 384, 512, bk, _vp(wsb), ws, None))
    assert _same(out, ref)


@pytest.mark.parametrize("bk", [128, 64])
def test_forward_f32_operands(dev, bk):
    """f32 operands take the handler's own quantize + GEMM sequence.  Against the
    float64 oracle of fp8.py:50-78 on the f32 values (fp8.py:66,68 quantize
    a.astype(f32)), and, at block_k 128, on bf16-valued f32 inputs bit for bit
    against the bf16 composite, whose operands then quantize to the same bytes
    and scales and meet the same GEMM arithmetic."""
    torch.manual_seed(3)
    M, N, K = 192, 256, 512
    a = torch.randn(M, K, device=dev)
    b = torch.randn(K, N, device=dev) * 0.05
    ws = L.lib().tg_block_scaled_matmul_workspace(M, N, K, bk)
    buf, sc = _scratch(ws, dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    _ok(C.call("tg_ffi_core_block_scaled_matmul", _st(), sc, C.tview(a), C.tview(b), out.data_ptr(), bk))
    torch.cuda.synchronize()
    qa, sa = fp8_ref.quantize_fp8(a.cpu().numpy(), bk)
    qb, sb = fp8_ref.quantize_fp8(np.ascontiguousarray(b.cpu().numpy().T), bk)
    ref = fp8_ref.dequant_gemm_nt(qa, sa, qb, sb, bk)
    err = maxabs_rel(out, ref)
    assert err <= 1e-2, err
    if bk != 128:
        return   # below 128 the composite runs the padded tuned GEMM, the handler the general one
    # bf16-valued f32 operands (either or both): the bf16 composite's bits
    ab, bb = a.bfloat16(), b.bfloat16()
    ref_b = torch.empty_like(out)
    wsb = torch.empty(ws, dtype=torch.uint8, device=dev)
    L.check(L.lib().tg_block_scaled_matmul(_vp(ab), _vp(bb), _vp(ref_b), M, N, K, bk, _vp(wsb), ws, None))
    for x, y in ((ab.float(), bb.float()), (ab.float(), bb), (ab, bb.float())):
        buf, sc = _scratch(ws, dev)
        _ok(C.call("tg_ffi_core_block_scaled_matmul", _st(), sc, C.tview(x), C.tview(y), out.data_ptr(), bk))
        assert _same(out, ref_b), (x.dtype, y.dtype)


def test_backward_rules(dev):
    torch.manual_seed(4)
    M, N, K = 256, 384, 512
    a = torch.randn(M, K, device=dev).bfloat16()
    b = (torch.randn(K, N, device=dev) * 0.05).bfloat16()
    g = torch.randn(M, N, device=dev).bfloat16()
    lib = L.lib()
    # the FP8 rule
    ws = lib.tg_block_scaled_matmul_bwd_workspace(M, N, K, 128)
    buf, sc = _scratch(ws, dev)
    da, db = torch.empty_like(a), torch.empty_like(b)
    _ok(C.call("tg_ffi_core_block_scaled_matmul_bwd_fp8", _st(), sc, C.tview(a), C.tview(b), C.tview(g),
               da.data_ptr(), db.data_ptr(), 128))
    da2, db2 = torch.empty_like(a), torch.empty_like(b)
    wsb = torch.empty(ws, dtype=torch.uint8, device=dev)
    L.check(lib.tg_block_scaled_matmul_bwd_fp8(_vp(a), _vp(b), _vp(g), _vp(da2), _vp(db2), M, N, K, 128,
                                               _vp(wsb), ws, None))
    assert _same(da, da2) and _same(db, db2)
    # the straight-through bf16 rule, with an f32 operand
    af = a.float()
    ws = lib.tg_block_scaled_matmul_bwd_bf16_workspace(M, N, K)
    buf, sc = _scratch(ws, dev)
    _ok(C.call("tg_ffi_core_block_scaled_matmul_bwd_bf16", _st(), sc, C.tview(af), C.tview(b), C.tview(g),
               da.data_ptr(), db.data_ptr()))
    wsb = torch.empty(ws, dtype=torch.uint8, device=dev)
    L.check(lib.tg_block_scaled_matmul_bwd_bf16(_vp(af), L.TG_DTYPE_F32, _vp(b), L.TG_DTYPE_BF16, _vp(g),
                                                L.TG_DTYPE_BF16, _vp(da2), _vp(db2), M, N, K, _vp(wsb), ws,
                                                None))
    assert _same(da, da2) and _same(db, db2)


@pytest.mark.parametrize("xd,sd", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                   (torch.bfloat16, torch.float32), (torch.float32, torch.float16)])
def test_norm_forward_and_backward(dev, xd, sd):
    torch.manual_seed(5)
    x = torch.randn(2, 24, 768, device=dev).to(xd)
    s = (1 + 0.1 * torch.randn(768, device=dev)).to(sd)
    yd = xd if xd == sd else torch.float32
    y = torch.empty(2, 24, 768, dtype=yd, device=dev)
    _ok(C.call("tg_ffi_core_rms_norm", _st(), C.tview(x), C.tview(s), C.tview(y), 1e-6))
    y2 = torch.empty_like(y)
    lib = L.lib()
    L.check(lib.tg_rms_norm_ex(_vp(x), L.norm_dtype_code(x), _vp(s), L.norm_dtype_code(s), _vp(y2), 48, 768,
                               ctypes.c_float(1e-6), None))
    assert _same(y, y2)
    dy = torch.randn(2, 24, 768, device=dev).to(xd)
    ws = lib.tg_rms_norm_bwd_workspace(48, 768)
    buf, sc = _scratch(ws, dev)
    dx, ds = torch.empty_like(x), torch.empty_like(s)
    _ok(C.call("tg_ffi_core_rms_norm_bwd", _st(), sc, C.tview(x), C.tview(s), C.tview(dy), C.tview(dx),
               C.tview(ds), 1e-6))
    dx2, ds2 = torch.empty_like(x), torch.empty_like(s)
    wsb = torch.empty(ws, dtype=torch.uint8, device=dev)
    L.check(lib.tg_rms_norm_bwd_ex(_vp(x), L.norm_dtype_code(x), _vp(s), L.norm_dtype_code(s), _vp(dy),
                                   L.norm_dtype_code(dy), _vp(dx2), _vp(ds2), 48, 768, ctypes.c_float(1e-6),
                                   _vp(wsb), ws, None))
    assert _same(dx, dx2) and _same(ds, ds2)


def test_fused_norm_and_prequantized_gemm(dev):
    torch.manual_seed(6)
    lib = L.lib()
    x = torch.randn(2, 64, 1024, device=dev).bfloat16()
    s = (1 + 0.1 * torch.randn(1024, device=dev)).bfloat16()
    y, q = torch.empty_like(x), torch.empty(2, 64, 1024, dtype=torch.uint8, device=dev)
    sc = torch.empty(2, 64, 8, dtype=torch.float32, device=dev)
    _ok(C.call("tg_ffi_core_rms_norm_fp8", _st(), C.tview(x), C.tview(s), y.data_ptr(), q.data_ptr(),
               sc.data_ptr(), 1e-6, 128))
    y2, q2, sc2 = torch.empty_like(y), torch.empty_like(q), torch.empty_like(sc)
    L.check(lib.tg_rms_norm_fp8(_vp(x), _vp(s), _vp(y2), _vp(q2), _vp(sc2), 128, 1024, ctypes.c_float(1e-6),
                                128, None))
    assert _same(y, y2) and _same(q, q2) and _same(sc, sc2)
    # the GEMM on those FP8 rows against a kept weight (N = 384, per-row scales)
    w = (torch.randn(384, 1024, device=dev) * 0.05).bfloat16()
    wq = torch.empty(384, 1024, dtype=torch.uint8, device=dev)
    ws = torch.empty(384, 8, dtype=torch.float32, device=dev)
    L.check(lib.tg_quantize_rows(_vp(w), L.TG_DTYPE_BF16, 384, 1024, 128, _vp(wq), _vp(ws), None))
    c = torch.empty(2, 64, 384, dtype=torch.bfloat16, device=dev)
    _ok(C.call("tg_ffi_core_gemm_fp8_nt", _st(), C.tview(q, C.E4M3), sc.data_ptr(), C.tview(wq, C.E4M3),
               ws.data_ptr(), c.data_ptr(), 1))
    c2 = torch.empty_like(c)
    L.check(lib.tg_gemm_fp8_nt(_vp(q), _vp(sc), _vp(wq), _vp(ws), 1, _vp(c2), L.TG_DTYPE_BF16, 128, 384, 1024,
                               128, None))
    assert _same(c, c2)
