"""GPU parity of tg_logit_cap (model.py:97 on the decode step's bf16 logits)
through the C ABI.

Bar: the same f32 bits as torch's `cap * torch.tanh(logits.float() / cap)`
on the same device.  The special values are zeros of both signs, the largest
finite bf16 values, infinities and NaN.  The decode step tests hold the step
that uses it against the steps that keep torch's epilogue (test_decode.py).
"""
import pytest
import torch

import decode

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,cap", [(50257, 15.0), (1, 15.0), (4097, 30.0), (256, 1.0)])
def test_logit_cap_same_bits_as_torch(dev, n, cap):
    g = torch.Generator(device=dev).manual_seed(n)
    x = (torch.randn((n,), generator=g, device=dev) * 20).to(torch.bfloat16)
    got = decode.logit_cap(x, cap)
    want = cap * torch.tanh(x.float() / cap)
    torch.cuda.synchronize()
    assert got.dtype == torch.float32 and got.shape == x.shape
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_logit_cap_special_values(dev):
    vals = [0.0, -0.0, 3.3895e38, -3.3895e38, float("inf"), float("-inf"), float("nan"), 1e-30, -7.5]
    x = torch.tensor(vals, device=dev).to(torch.bfloat16).reshape(3, 3)
    got = decode.logit_cap(x, 15.0)
    want = 15.0 * torch.tanh(x.float() / 15.0)
    torch.cuda.synchronize()
    assert got.shape == (3, 3)
    assert torch.equal(got.isnan(), want.isnan())
    fin = ~want.isnan()
    assert torch.equal(got[fin].view(torch.int32), want[fin].view(torch.int32))


def test_logit_cap_rejects_bad_arguments(dev):
    with pytest.raises(ValueError, match="bf16"):
        decode.logit_cap(torch.zeros(4, device=dev), 15.0)
    with pytest.raises(ValueError, match="cap must be finite"):
        decode.logit_cap(torch.zeros(4, device=dev, dtype=torch.bfloat16), 0.0)
