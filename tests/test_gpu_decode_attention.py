"""GPU parity of the HIP decode attention (tg_decode_attention) through the C ABI.

Reference: float64 numpy softmax(q . K^T / sqrt(Dh)) V over positions 0 .. t of
the same bf16 values (the cached keys plus the appended one).  Bars:
  * o (bf16) within 1e-2 max-abs-normalised and 2 bf16 ulps elementwise of
    the float64 result (f32 online softmax, then one rounding to bf16);
  * o_q / o_s bit-exact against the oracle's _quantize_to_fp8 of the returned
    bf16 o (fp8.py:39-47);
  * the cache holds k, v at position t exactly and is unchanged elsewhere;
  * a position outside the cache touches no memory and returns NaN scales.
"""
import math

import numpy as np
import pytest
import torch

import decode
from helpers import bf16_bits, f32_bits, u8
from oracle import bf16 as ob
from oracle import fp8_ref

pytestmark = pytest.mark.gpu


def _inputs(dev, B, H, S, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    qkv = torch.randn((B, 3 * H * 128), generator=g, device=dev).to(torch.bfloat16)
    kc = torch.randn((B, H, S, 128), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((B, H, S, 128), generator=g, device=dev).to(torch.bfloat16)
    return qkv, kc, vc


def _reference(qkv, kc, vc, t, H):
    B = qkv.shape[0]
    x = qkv.float().cpu().numpy().astype(np.float64).reshape(B, 3, H, 128)
    K = kc.float().cpu().numpy().astype(np.float64)[:, :, :t + 1].copy()
    V = vc.float().cpu().numpy().astype(np.float64)[:, :, :t + 1].copy()
    K[:, :, t], V[:, :, t] = x[:, 1], x[:, 2]
    s = np.einsum("bhd,bhjd->bhj", x[:, 0], K) / math.sqrt(128)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhj,bhjd->bhd", p, V).reshape(B, H * 128)


@pytest.mark.parametrize("B,H,S,t", [(1, 18, 2048, 0), (1, 18, 2048, 160), (3, 4, 256, 17),
                                     (2, 2, 64, 63), (5, 3, 1000, 999), (1, 1, 4096, 3000)])
def test_decode_attention_matches_float64(dev, B, H, S, t):
    qkv, kc, vc = _inputs(dev, B, H, S, seed=B * 1000 + t)
    k0, v0 = kc.clone(), vc.clone()
    ref = _reference(qkv, kc, vc, t, H)
    tt = torch.tensor([t], dtype=torch.long, device=dev)
    o_q, o_s, o = decode.decode_attention(qkv, kc, vc, tt, H, want_bf16=True)
    torch.cuda.synchronize()
    got = o.float().cpu().numpy().astype(np.float64)
    err = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
    tol = np.abs(ref) * 2.0 ** -6 + 1e-4 * np.max(np.abs(ref))   # >= 2 bf16 ulps, plus f32 cancellation
    print(f"B={B} H={H} S={S} t={t}: max-abs-rel {err:.2e}")
    assert err <= 1e-2 and np.all(np.abs(got - ref) <= tol)
    # quantized output: bit-exact vs the oracle on the returned bf16 o
    q_ref, s_ref = fp8_ref.quantize_fp8(ob.bf16_to_f32(bf16_bits(o)))
    assert np.array_equal(u8(o_q), q_ref)
    assert np.array_equal(f32_bits(o_s), s_ref.view(np.uint32))
    # cache: appended at t, unchanged elsewhere
    x = qkv.reshape(B, 3, H, 128)
    assert torch.equal(kc[:, :, t], x[:, 1]) and torch.equal(vc[:, :, t], x[:, 2])
    mask = torch.ones(S, dtype=torch.bool, device=dev)
    mask[t] = False
    assert torch.equal(kc[:, :, mask], k0[:, :, mask]) and torch.equal(vc[:, :, mask], v0[:, :, mask])


def test_decode_attention_position_outside_cache(dev):
    B, H, S = 2, 3, 64
    qkv, kc, vc = _inputs(dev, B, H, S, seed=7)
    k0, v0 = kc.clone(), vc.clone()
    tt = torch.tensor([S], dtype=torch.long, device=dev)
    _, o_s, _ = decode.decode_attention(qkv, kc, vc, tt, H)
    torch.cuda.synchronize()
    assert torch.isnan(o_s).all()
    assert torch.equal(kc, k0) and torch.equal(vc, v0)


def test_decode_attention_rejects_bad_arguments(dev):
    qkv, kc, vc = _inputs(dev, 1, 2, 32, seed=8)
    tt = torch.zeros(1, dtype=torch.long, device=dev)
    with pytest.raises(ValueError, match="disagree"):
        decode.decode_attention(qkv, kc, vc, tt, 3)
    with pytest.raises(ValueError, match="one-element int64"):
        decode.decode_attention(qkv, kc, vc, tt.int(), 2)
