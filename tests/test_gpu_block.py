"""Config 4: one decoder block training step through the FP8 hot path
(train-gpt_amd/block.py) against the same step in float32 torch ops.

FP8 is a lossy format (3 mantissa bits), so the bar is on agreement, not
bits: the loss within 2e-2 relative and every parameter gradient within
0.15 max-abs-normalised error (cosine similarity >= 0.99).  The bf16 variant
of the block (same wiring, bf16 GEMMs) checks the wiring itself more
tightly.  Every number is printed.
"""
import pytest
import torch

import block

pytestmark = pytest.mark.gpu

SMALL = block.BlockConfig(d_model=256, n_heads=2, head_dim=128, d_ff=1024, vocab=1024, seq_len=256,
                          batch=2)


def _compare(cfg, dev, impl, loss_tol, grad_tol, cos_min):
    params = block.init_params(cfg, dev)
    ids, tgt = block.random_batch(cfg, dev)
    l, g = block.step_grads(params, ids, tgt, cfg, impl)
    lr, gr = block.step_grads(params, ids, tgt, cfg, "ref")
    rel = abs(float(l) - float(lr)) / abs(float(lr))
    print(f"{impl} loss {float(l):.6f} ref {float(lr):.6f} rel {rel:.2e}")
    assert torch.isfinite(l) and rel <= loss_tol
    for name in block.PARAM_NAMES:
        a, b = g[name].float(), gr[name].float()
        assert a.shape == b.shape and torch.isfinite(a).all()
        err = float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))
        cos = float((a * b).sum() / (a.norm() * b.norm()).clamp_min(1e-30))
        print(f"  {name:10s} max-abs-rel {err:.3e} cos {cos:.5f}")
        assert err <= grad_tol and cos >= cos_min, name


def test_block_small_fp8(dev):
    _compare(SMALL, dev, "fp8", 2e-2, 0.15, 0.99)


def test_block_small_bf16_wiring(dev):
    _compare(SMALL, dev, "bf16", 5e-3, 0.05, 0.999)


def test_block_c4_fp8(dev):
    _compare(block.C4, dev, "fp8", 2e-2, 0.15, 0.99)


def test_block_prequant_matches_block_scaled_matmul(dev):
    """The fused norm -> quant feeding q/k/v gives the same product as quantizing h inside the matmul."""
    import fp8
    import kernels
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((512, 1024), generator=g, device=dev).to(torch.bfloat16)
    s = (1 + 0.1 * torch.randn((1024,), generator=g, device=dev)).to(torch.bfloat16)
    w = (torch.randn((1024, 768), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    h, hq, hs = kernels.rms_norm_fp8(x, s, 1e-5)
    assert torch.equal(fp8.block_scaled_matmul_prequant(h, hq, hs, w), fp8.block_scaled_matmul(h, w))
