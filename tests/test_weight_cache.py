"""Pre-quantized weight format (fp8.QuantizedWeight): safetensors round trip
on the CPU, and on the GPU the kept weight gives the same products as
re-quantizing W on every call (fp8.py:68)."""
import os

import numpy as np
import pytest
import torch

import fp8
from helpers import f32_bits, maxabs_rel, to_dev, u8
from oracle import bf16 as ob
from oracle import fp8_ref


def test_round_trip_cpu(tmp_path):
    g = torch.Generator().manual_seed(0)
    q = torch.randint(0, 256, (384, 512), dtype=torch.uint8, generator=g)
    for bn, srows in ((1, 384), (128, 3)):
        s = torch.rand((srows, 4), generator=g)
        w = fp8.QuantizedWeight(q, s, bn)
        path = os.path.join(tmp_path, f"w{bn}.safetensors")
        w.save(path)
        w2 = fp8.QuantizedWeight.load(path)
        assert w2.shape == (512, 384) and w2.bn == bn and w2.block_k == 128
        assert w2.q.dtype == torch.float8_e4m3fn
        assert torch.equal(w2.q.view(torch.uint8), q) and torch.equal(w2.scales, s)


def test_rejects_inconsistent_shapes(tmp_path):
    q = torch.zeros((300, 256), dtype=torch.uint8)
    with pytest.raises(ValueError):
        fp8.QuantizedWeight(q, torch.zeros((300, 3)), 1)          # K/128 = 2 scale columns
    with pytest.raises(ValueError):
        fp8.QuantizedWeight(q, torch.zeros((2, 2)), 128)          # ceil(300/128) = 3 rows
    from safetensors.torch import save_file
    path = os.path.join(tmp_path, "other.safetensors")
    save_file({"q": q, "scales": torch.zeros((300, 2))}, path, metadata={"format": "something-else"})
    with pytest.raises(ValueError, match="not a"):
        fp8.QuantizedWeight.load(path)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 8, 48, 300, 2048])
def test_kept_weight_matches_requantizing(dev, M):
    """layout 128x1 keeps exactly fp8.py:68's bytes and scales, so the kept
    weight's product equals block_scaled_matmul's bit for bit at M > 64 (same
    GEMM) and matches the oracle at the GEMV sizes."""
    rng = np.random.default_rng(M)
    K, N = 768, 1024
    x = ob.randn_bf16(rng, (M, K))
    w = ob.randn_bf16(rng, (K, N), std=0.02)
    xd, wd = to_dev(x, dev), to_dev(w, dev)
    qw = fp8.QuantizedWeight.from_weight(wd, "128x1")
    qo, so = fp8_ref.quantize_fp8(np.ascontiguousarray(ob.bf16_to_f32(w).T))
    np.testing.assert_array_equal(u8(qw.q), qo)
    np.testing.assert_array_equal(f32_bits(qw.scales), so.view(np.uint32))
    y = qw.matmul(xd)
    ref = fp8.block_scaled_matmul(xd, wd)
    if M > 64:
        assert torch.equal(y, ref)
    yo, _, _, _ = fp8_ref.fp8_forward(x, w)
    assert maxabs_rel(y, ob.bf16_to_f32(yo)) <= 1e-2


@pytest.mark.gpu
def test_kept_weight_128x128_save_load_gpu(dev, tmp_path):
    rng = np.random.default_rng(7)
    K, N = 1024, 640
    w = ob.randn_bf16(rng, (K, N), std=0.02)
    x = ob.randn_bf16(rng, (96, K))
    qw = fp8.QuantizedWeight.from_weight(to_dev(w, dev), "128x128")
    path = os.path.join(tmp_path, "w.safetensors")
    qw.save(path)
    qw2 = fp8.QuantizedWeight.load(path, device=dev)
    assert torch.equal(qw2.q.view(torch.uint8), qw.q.view(torch.uint8))
    assert torch.equal(qw2.scales, qw.scales)
    y = qw2.matmul(to_dev(x, dev))
    qo, so = fp8_ref.quantize_weight_128x128(np.ascontiguousarray(ob.bf16_to_f32(w).T))
    np.testing.assert_array_equal(u8(qw2.q), qo)
    np.testing.assert_array_equal(f32_bits(qw2.scales), so.view(np.uint32))
    qa, sa = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    ref = fp8_ref.gemv_prequant(qa, sa, qo, so, 128)     # float64 dequant product, 128x128 scales
    assert maxabs_rel(y, ref) <= 1e-2
