"""GPU parity of the decode-shape FP8 GEMM on a pre-quantized weight (config 5).

No reference function exists (generate.py never calls FP8); the oracle is the
float64 dequant GEMM of the same quantized operands.  Bar: 1e-2 max-abs-normalised.
The MFMA GEMV (tg_gemv_fp8, exact=True) serves every M <= 64; 1-2 rows take the
VALU one (tg_gemv_fp8_rowdot) by default, held additionally to the elementwise
bar of one bf16 rounding plus f32 accumulation (2^-8 |ref| + 1e-3 max|ref|).
"""
import numpy as np
import pytest
import torch

import _tglib as L
import fp8
from helpers import maxabs_rel, to_dev, u8
from oracle import bf16 as ob
from oracle import fp8_ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def weight(dev):
    rng = np.random.default_rng(4)
    w = ob.randn_bf16(rng, (4096, 14336), std=0.02)
    return w, to_dev(w, dev)


@pytest.mark.parametrize("layout", ["128x1", "128x128"])
@pytest.mark.parametrize("M", [1, 8, 32])
def test_gemv_c5(dev, weight, layout, M):
    w_u, w_d = weight
    rng = np.random.default_rng(100 + M)
    x = ob.randn_bf16(rng, (M, 4096))
    wq, ws, bn = fp8.quantize_weight(w_d, layout=layout)
    out = fp8.fp8_gemv(to_dev(x, dev), wq, ws, w_scale_bn=bn, exact=True)
    assert out.shape == (M, 14336) and out.dtype == torch.bfloat16
    qx, sx = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    ref = fp8_ref.gemv_prequant(qx, sx, u8(wq), ws.cpu().numpy(), bn)
    assert maxabs_rel(out, ref) <= 1e-2


# Ragged shapes: rows per workgroup not a multiple of 16, N not a multiple of 4
# (scalar output stores), K spanning several rounds of the 8 waves (K = 8192,
# 20480), waves without K blocks (K = 256), scale rows straddling a 128-row
# group, and every M bucket (<= 16, <= 32, <= 64).
RAGGED = [(3, 40, 256), (16, 100, 384), (64, 72, 512), (5, 16, 4096), (1, 14338, 4096),
          (20, 1001, 1280), (33, 130, 8192), (17, 515, 20480), (64, 3000, 2048), (2, 257, 128)]


@pytest.mark.parametrize("layout", ["128x1", "128x128"])
@pytest.mark.parametrize("M,N,K", RAGGED)
def test_gemv_ragged(dev, M, N, K, layout):
    rng = np.random.default_rng(M * N + K)
    x = ob.randn_bf16(rng, (M, K))
    w = ob.randn_bf16(rng, (K, N), std=0.02)
    wq, ws, bn = fp8.quantize_weight(to_dev(w, dev), layout=layout)
    out = fp8.fp8_gemv(to_dev(x, dev), wq, ws, w_scale_bn=bn, exact=True)
    qx, sx = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    ref = fp8_ref.gemv_prequant(qx, sx, u8(wq), ws.cpu().numpy(), bn)
    assert maxabs_rel(out, ref) <= 1e-2


def _rowdot_close(out, ref) -> bool:
    got = out.float().cpu().numpy().astype(np.float64)
    return bool(np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-3 * np.max(np.abs(ref))))


# N = 1 (one wave busy), N not a multiple of 4, K = 128 (one block, lanes past
# the row) up to K = 16384 (the LDS limit), rows beyond one sweep of the grid
# (N > 8 workgroups x 4 waves x CUs), both M.
ROWDOT = [(1, 1, 128), (2, 1, 128), (1, 3, 256), (2, 130, 1152), (1, 1001, 4096), (2, 14336, 4096),
          (1, 4096, 14336), (2, 2304, 9216), (1, 50257, 2304), (2, 77, 16384), (1, 9000, 640)]


@pytest.mark.parametrize("layout", ["128x1", "128x128"])
@pytest.mark.parametrize("M,N,K", ROWDOT)
def test_gemv_rowdot_vs_oracle(dev, M, N, K, layout):
    rng = np.random.default_rng(3 * M * N + K)
    x = ob.randn_bf16(rng, (M, K))
    w = ob.randn_bf16(rng, (K, N), std=0.02)
    wq, ws, bn = fp8.quantize_weight(to_dev(w, dev), layout=layout)
    out = fp8.fp8_gemv(to_dev(x, dev), wq, ws, w_scale_bn=bn)
    qx, sx = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    ref = fp8_ref.gemv_prequant(qx, sx, u8(wq), ws.cpu().numpy(), bn)
    assert out.shape == (M, N) and out.dtype == torch.bfloat16
    assert maxabs_rel(out, ref) <= 1e-2 and _rowdot_close(out, ref)
    exact = fp8.fp8_gemv(to_dev(x, dev), wq, ws, w_scale_bn=bn, exact=True)
    print(f"rowdot {M}x{N}x{K} {layout}: vs f64 {maxabs_rel(out, ref):.2e}, "
          f"vs MFMA GEMV {maxabs_rel(out, exact.float().cpu().numpy()):.2e}")
    assert maxabs_rel(out, exact.float().cpu().numpy()) <= 1e-2


def test_gemv_rowdot_deterministic_and_row_independent(dev):
    """Fixed reduction order: two calls give the same bits.  A weight with one
    non-zero row (in the grid's second sweep of rows) gives one non-zero output
    column per activation row."""
    K, N = 4096, 14336
    rng = np.random.default_rng(17)
    x = to_dev(ob.randn_bf16(rng, (2, K)), dev)
    w = np.zeros((K, N), dtype=np.uint16)
    col = 13001
    w[:, col] = ob.randn_bf16(rng, (K,), std=0.02)
    wq, ws, bn = fp8.quantize_weight(to_dev(w, dev), layout="128x128")
    a = fp8.fp8_gemv(x, wq, ws, w_scale_bn=bn)
    b = fp8.fp8_gemv(x, wq, ws, w_scale_bn=bn)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    out = a.float().cpu().numpy()
    for m in range(2):
        assert list(np.nonzero(out[m])[0]) == [col]


def test_gemv_rowdot_abi_limits(dev):
    """tg_gemv_fp8_rowdot takes at most 2 rows and K <= 16384 (x in LDS); past
    those fp8_gemv keeps the MFMA GEMV."""
    N, K = 16, 16512
    xq = torch.zeros((3, K), dtype=torch.uint8, device=dev)
    xs = torch.ones((3, K // 128), dtype=torch.float32, device=dev)
    wq = torch.zeros((N, K), dtype=torch.uint8, device=dev)
    ws = torch.ones((N, K // 128), dtype=torch.float32, device=dev)
    out = torch.empty((3, N), dtype=torch.bfloat16, device=dev)
    fn = L.lib().tg_gemv_fp8_rowdot
    with pytest.raises(ValueError, match="M must be <= 2"):
        L.check(fn(L.ptr(xq), L.ptr(xs), L.ptr(wq), L.ptr(ws), 1, L.ptr(out), 3, N, K, 128, L.stream_of(xq)))
    with pytest.raises(ValueError, match="K must be <= 16384"):
        L.check(fn(L.ptr(xq), L.ptr(xs), L.ptr(wq), L.ptr(ws), 1, L.ptr(out), 1, N, K, 128, L.stream_of(xq)))
    rng = np.random.default_rng(19)
    x = ob.randn_bf16(rng, (1, K))
    w = ob.randn_bf16(rng, (K, N), std=0.02)
    wq, ws, bn = fp8.quantize_weight(to_dev(w, dev), layout="128x1")
    got = fp8.fp8_gemv(to_dev(x, dev), wq, ws, w_scale_bn=bn)
    qx, sx = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    assert maxabs_rel(got, fp8_ref.gemv_prequant(qx, sx, u8(wq), ws.cpu().numpy(), bn)) <= 1e-2


def test_gemv_row_outputs_independent(dev):
    """Each output row depends only on its own weight row: a weight with a
    single non-zero row gives exactly one non-zero output column, equal to the
    dot product of that row's dequantized bytes with x's (checks the row
    ownership of the workgroups and the reduction of the K split)."""
    K, N, M = 4096, 14336, 8
    rng = np.random.default_rng(7)
    x = ob.randn_bf16(rng, (M, K))
    w = np.zeros((K, N), dtype=np.uint16)
    col = 8763                      # inside a workgroup's range, not 16-aligned
    w[:, col] = ob.randn_bf16(rng, (K,), std=0.02)
    wq, ws, bn = fp8.quantize_weight(to_dev(w, dev), layout="128x1")
    out = fp8.fp8_gemv(to_dev(x, dev), wq, ws, w_scale_bn=bn).float().cpu().numpy()
    nz = np.nonzero(np.any(out != 0, axis=0))[0]
    assert list(nz) == [col]
    qx, sx = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    ref = fp8_ref.gemv_prequant(qx, sx, u8(wq), ws.cpu().numpy(), bn)
    assert maxabs_rel(out, ref) <= 1e-2


def test_gemv_rejects_large_m(dev):
    x = torch.zeros((65, 256), dtype=torch.bfloat16, device=dev)
    wq = torch.zeros((16, 256), dtype=torch.uint8, device=dev)
    ws = torch.ones((16, 2), dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="M must be <= 64"):
        fp8.fp8_gemv(x, wq, ws)
