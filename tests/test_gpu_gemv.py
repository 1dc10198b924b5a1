"""GPU parity of the decode-shape FP8 GEMM on a pre-quantized weight (config 5).

No reference function exists (generate.py never calls FP8); the oracle is the
float64 dequant GEMM of the same quantized operands.  Bar: 1e-2 max-abs-normalised.
"""
import numpy as np
import pytest
import torch

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
    out = fp8.fp8_gemv(to_dev(x, dev), wq, ws, w_scale_bn=bn)
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
    out = fp8.fp8_gemv(to_dev(x, dev), wq, ws, w_scale_bn=bn)
    qx, sx = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    ref = fp8_ref.gemv_prequant(qx, sx, u8(wq), ws.cpu().numpy(), bn)
    assert maxabs_rel(out, ref) <= 1e-2


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
