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


@pytest.mark.parametrize("layout", ["128x1", "128x128"])
def test_gemv_c5_rowdot_m1(dev, weight, layout):
    """Config 5 at M = 1 on the kernel the default fp8_gemv (and bench.py's
    C5 M = 1 line) runs, tg_gemv_fp8_rowdot, against the float64 oracle: the
    1e-2 bar and the elementwise one-bf16-rounding bar."""
    w_u, w_d = weight
    rng = np.random.default_rng(101)
    x = ob.randn_bf16(rng, (1, 4096))
    wq, ws, bn = fp8.quantize_weight(w_d, layout=layout)
    out = fp8.fp8_gemv(to_dev(x, dev), wq, ws, w_scale_bn=bn)
    assert out.shape == (1, 14336) and out.dtype == torch.bfloat16
    qx, sx = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    ref = fp8_ref.gemv_prequant(qx, sx, u8(wq), ws.cpu().numpy(), bn)
    assert maxabs_rel(out, ref) <= 1e-2 and _rowdot_close(out, ref)


# Ragged shapes: rows per workgroup not a multiple of 16, N not a multiple of 4
# (scalar output stores), K spanning several rounds of the 8 waves (K = 8192,
# 20480), waves without K blocks (K = 256), scale rows straddling a 128-row
# group, and every M bucket (<= 16, <= 32, <= 64).
RAGGED = [(3, 40, 256), (16, 100, 384), (64, 72, 512), (5, 16, 4096), (1, 14338, 4096),
          (20, 1001, 1280), (33, 130, 8192), (17, 515, 20480), (64, 3000, 2048), (2, 257, 128),
          # the direct kernel (<= 8 or 17-32 rows, <= 512 row blocks or N > 16384): 12 K blocks
          # per wave with the 16-chunk x copy, two x-row tiles, a grid walking many row
          # blocks per workgroup, 12 K blocks with the 4-chunk copy, more than 512 x scales
          (8, 2304, 9216), (32, 2304, 2304), (4, 50257, 2304), (1, 777, 12288), (24, 130, 4096)]


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
    # elementwise: one bf16 rounding of an f32 sum (a mis-placed scale or row fails this)
    assert _rowdot_close(out, ref)


def _rowdot_close(out, ref) -> bool:
    got = out.float().cpu().numpy().astype(np.float64)
    return bool(np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-3 * np.max(np.abs(ref))))


# N = 1 (one wave busy), N not a multiple of 4, K = 128 (one block, lanes past
# the row) up to K = 16384 (the LDS limit), rows beyond one sweep of the grid
# (N > 8 workgroups x 4 waves x CUs), both M.
ROWDOT = [(1, 1, 128), (2, 1, 128), (1, 3, 256), (2, 130, 1152), (1, 1001, 4096), (1, 14336, 4096),
          (2, 14336, 4096),
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


# ---------------------------------------------------------------- fused prologues
# tg_rms_norm_fp8_gemv / tg_relu2_fp8_gemv run the norm (or residual add + norm)
# and the relu^2 quantization inside the VALU GEMV; each must give the same
# bits as the stand-alone kernels followed by tg_gemv_fp8_rowdot, and the
# residual sum the same bits as tg_add_rms_norm_fp8's.
import kernels  # noqa: E402


def _bf16_rows(rng, M, K, outliers=True):
    x = ob.randn_bf16(rng, (M, K))
    if outliers:   # a few large values, as in the C2 inputs
        x = x.copy()
        idx = rng.choice(M * K, size=max(1, M * K // 500), replace=False)
        x.reshape(-1)[idx] = ob.randn_bf16(rng, (idx.size,), std=50.0)
    return x


NORM_FUSED = [(1, 1, 128), (2, 77, 640), (1, 6912, 2304), (2, 2304, 2304), (1, 3000, 4096), (2, 129, 1152),
              (1, 50257, 2304),
              # 3-16 rows: the MFMA GEMV with the norm prologue (rows w and w + 8 per wave,
              # K up to 2560, partial 8-row groups, one scale block, a grid past one wave)
              (3, 77, 640), (8, 6912, 2304), (16, 2304, 2304), (5, 129, 1152), (16, 1000, 2560),
              (9, 300, 128), (8, 50257, 2304), (12, 8, 256)]


@pytest.mark.parametrize("layout", ["128x1", "128x128"])
@pytest.mark.parametrize("add", [False, True])
@pytest.mark.parametrize("M,N,K", NORM_FUSED)
def test_rms_norm_fp8_gemv_same_bits(dev, M, N, K, add, layout):
    rng = np.random.default_rng(M * 7919 + N * 31 + K + int(add))
    x = to_dev(_bf16_rows(rng, M, K), dev)
    delta = to_dev(_bf16_rows(rng, M, K, outliers=False), dev)
    gamma = to_dev(ob.randn_bf16(rng, (K,), std=0.1, mean=1.0), dev)
    w = to_dev(ob.randn_bf16(rng, (K, N), std=0.02), dev)
    qw = fp8.QuantizedWeight.from_weight(w, layout)
    eps = 1e-6
    if add:
        xo_ref, q, s, _ = kernels.add_rms_norm_fp8(x, delta, gamma, eps)
        xout = torch.empty_like(x)
        got = qw.matmul_rms_norm(x, gamma, eps, delta=delta, xout=xout)
        assert torch.equal(xout.view(torch.int16), xo_ref.view(torch.int16))
    else:
        _, q, s = kernels.rms_norm_fp8(x, gamma, eps)
        got = qw.matmul_rms_norm(x, gamma, eps)
    ref = qw.matmul_prequant(q, s)          # tg_gemv_fp8_rowdot on the stand-alone bytes
    assert got.shape == (M, N) and got.dtype == torch.bfloat16
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_rms_norm_fp8_gemv_limits(dev):
    """3-16 rows take K <= 2560 (the FP8 rows and the norm's registers beside
    the MFMA GEMV's weight stages); more than 16 rows is an error."""
    rng = np.random.default_rng(5)
    for M, K, msg in ((4, 2688, "K=2688 too large"), (17, 256, "M must be <= 16")):
        x = to_dev(_bf16_rows(rng, M, K), dev)
        gamma = to_dev(ob.randn_bf16(rng, (K,), std=0.1, mean=1.0), dev)
        qw = fp8.QuantizedWeight.from_weight(to_dev(ob.randn_bf16(rng, (K, 64), std=0.02), dev), "128x128")
        with pytest.raises(ValueError, match=msg):
            qw.matmul_rms_norm(x, gamma, 1e-6)


def test_rms_norm_fp8_gemv_vs_oracle(dev):
    """One direct check of the fused path against the oracle's norm, quantizer
    and float64 GEMV (the same-bits tests above tie it to the stand-alone
    kernels, which are pinned there)."""
    from oracle import norm_ref
    rng = np.random.default_rng(12)
    M, N, K = 2, 1000, 2304
    x = _bf16_rows(rng, M, K)
    g = ob.randn_bf16(rng, (K,), std=0.1)
    w = ob.randn_bf16(rng, (K, N), std=0.02)
    qw = fp8.QuantizedWeight.from_weight(to_dev(w, dev), "128x128")
    got = qw.matmul_rms_norm(to_dev(x, dev), to_dev(g, dev), 1e-6)
    _, qx, sx = norm_ref.rms_norm_fp8(x, g, 1e-6)
    ref = fp8_ref.gemv_prequant(qx, sx, u8(qw.q), qw.scales.cpu().numpy(), qw.bn)
    assert maxabs_rel(got, ref) <= 1e-2 and _rowdot_close(got, ref)


RELU2_FUSED = [(1, 1, 128), (2, 129, 256), (1, 2304, 9216), (2, 2304, 9216), (1, 77, 16384), (2, 513, 16384),
               (1, 4096, 14336)]


@pytest.mark.parametrize("layout", ["128x1", "128x128"])
@pytest.mark.parametrize("M,N,K", RELU2_FUSED)
def test_relu2_fp8_gemv_same_bits(dev, M, N, K, layout):
    rng = np.random.default_rng(M * 131 + N * 7 + K)
    u = to_dev(_bf16_rows(rng, M, K), dev)
    w = to_dev(ob.randn_bf16(rng, (K, N), std=0.02), dev)
    qw = fp8.QuantizedWeight.from_weight(w, layout)
    got = qw.matmul_relu2(u)
    q, s = fp8.quantize_relu2(u)
    ref = qw.matmul_prequant(q, s)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_fused_gemv_errors(dev):
    w = to_dev(ob.randn_bf16(np.random.default_rng(3), (4224, 16), std=0.02), dev)
    qw = fp8.QuantizedWeight.from_weight(w, "128x1")
    x = torch.zeros((1, 4224), dtype=torch.bfloat16, device=dev)
    g = torch.ones(4224, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="K must be <= 4096"):
        qw.matmul_rms_norm(x, g, 1e-6)
    w2 = to_dev(ob.randn_bf16(np.random.default_rng(4), (256, 16), std=0.02), dev)
    qw2 = fp8.QuantizedWeight.from_weight(w2, "128x1")
    x3 = torch.zeros((3, 256), dtype=torch.bfloat16, device=dev)
    g2 = torch.ones(256, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="M must be <= 2"):
        qw2.matmul_relu2(x3)                  # the relu^2 fusion is the VALU GEMV's only
    for rows in (1, 3):                       # both the VALU and the MFMA path check the overlap
        xr = torch.zeros((rows, 256), dtype=torch.bfloat16, device=dev)
        with pytest.raises(ValueError, match="must not overlap"):
            qw2.matmul_rms_norm(xr, g2, 1e-6, delta=torch.zeros_like(xr), xout=xr)


@pytest.mark.parametrize("layout", ["128x1", "128x128"])
@pytest.mark.parametrize("M,exact,N", [(1, False, 12288), (1, True, 12288), (8, True, 12288), (8, True, 2048),
                                       (24, True, 12288), (32, True, 12288), (32, True, 2048)])
def test_gemv_non_finite_operands(dev, layout, M, exact, N):
    """NaN / inf through every GEMV kernel (VALU, x-copy MFMA, direct, 17-32
    rows from x_q): an inf in W makes its scale block's scale inf, so the
    outputs of its 128x1 column, or of its whole 128-row tile with 128x128
    scales (0 x inf), are NaN; a NaN in x makes its row NaN; exactly where the
    float64 oracle has them, the rest within the usual bar."""
    K = 1024
    rng = np.random.default_rng(M + N)
    w = ob.randn_bf16(rng, (K, N), std=0.02)
    w[5, 700] = 0x7F80                               # +inf: W.T row 700, K block 0
    x = ob.randn_bf16(rng, (M, K))
    nan_rows = 1 if M > 1 else 0                     # (with one row a NaN leaves nothing finite)
    if nan_rows:
        x[M - 1, 300] = 0x7FC0                       # NaN in the last row, K block 2
    wq, ws, bn = fp8.quantize_weight(to_dev(w, dev), layout=layout)
    out = fp8.fp8_gemv(to_dev(x, dev), wq, ws, w_scale_bn=bn, exact=exact).float().cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        qx, sx = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
        ref = fp8_ref.gemv_prequant(qx, sx, u8(wq), ws.cpu().numpy(), bn)
    nan_ref = np.isnan(ref)
    cols = 1 if layout == "128x1" else 128
    assert nan_ref.sum() == (M - nan_rows) * cols + nan_rows * N
    np.testing.assert_array_equal(np.isnan(out), nan_ref)
    assert maxabs_rel(out[~nan_ref], ref[~nan_ref]) <= 1e-2


# ------------------------------------------------- residual adds in the GEMV store
# tg_gemv_fp8_rowdot_add / tg_relu2_fp8_gemv_add: out = bf16(resid + the plain
# entry point's output), the bf16 tensor add (torch's bf16 + rounds the f32 sum
# once, as model.py:75-76's jax adds do); out may be resid itself.
RESID_ADD = [(1, 1, 128), (2, 77, 640), (1, 2304, 2304), (2, 2304, 2304), (1, 2304, 9216), (2, 513, 16384),
             (1, 14336, 4096)]


@pytest.mark.parametrize("layout", ["128x1", "128x128"])
@pytest.mark.parametrize("M,N,K", RESID_ADD)
def test_gemv_residual_add_same_bits(dev, M, N, K, layout):
    rng = np.random.default_rng(M * 131 + N + K)
    resid = to_dev(_bf16_rows(rng, M, N), dev)
    w = to_dev(ob.randn_bf16(rng, (K, N), std=0.02), dev)
    qw = fp8.QuantizedWeight.from_weight(w, layout)
    # projection of already-quantized rows (the o projection of a decode step)
    q, s = fp8.quantize_fp8(to_dev(_bf16_rows(rng, M, K), dev))
    want = resid + qw.matmul_prequant(q, s)
    got = qw.matmul_prequant_add(q, s, resid)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    inplace = resid.clone()
    qw.matmul_prequant_add(q, s, inplace, out=inplace)
    assert torch.equal(inplace.view(torch.int16), want.view(torch.int16))
    # relu^2 of u, then the projection (the down projection)
    u = to_dev(_bf16_rows(rng, M, K), dev)
    want = resid + qw.matmul_relu2(u)
    got = qw.matmul_relu2_add(u, resid)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    inplace = resid.clone()
    qw.matmul_relu2_add(u, inplace, out=inplace)
    assert torch.equal(inplace.view(torch.int16), want.view(torch.int16))


def test_gemv_residual_add_refuses_partial_overlap(dev):
    rng = np.random.default_rng(3)
    qw = fp8.QuantizedWeight.from_weight(to_dev(ob.randn_bf16(rng, (256, 64), std=0.02), dev), "128x128")
    q, s = fp8.quantize_fp8(to_dev(_bf16_rows(rng, 1, 256), dev))
    buf = torch.zeros(130, dtype=torch.bfloat16, device=dev)
    resid, out = buf[:64].view(1, 64), buf[2:66].view(1, 64)
    with pytest.raises(ValueError, match="out must be resid itself or not overlap it"):
        qw.matmul_prequant_add(q, s, resid, out=out)
