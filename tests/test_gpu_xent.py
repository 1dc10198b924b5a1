"""GPU parity of the fused logit cap + cross entropy (tg_logit_cap_xent_fwd /
tg_logit_cap_xent_bwd, through losses.py) against float64 torch.  cap 15 (the
reference's) takes the table kernels, cap 40 the direct ones.

Reference: z = cap * tanh(l / cap) on the same bf16 logits in float64, nll =
logsumexp(z) - z[t] (losses.py:8-12 after model.py:96-97), the mean or masked
mean (losses.py:15-34), and its autograd gradient.  Bars:
  * nll and loss within 5e-5 + 1e-5 |ref| (f32 arithmetic on the hardware
    exp / reciprocal: z is within ~6e-6 of the exact cap * tanh);
  * dlogits (bf16) within 2^-8 |ref| + 3e-5 max |ref| elementwise (one bf16
    rounding of an f32 value, plus the cancellation of p_t - 1 at the target);
  * two calls give the same bits; V = 1 gives a zero loss and gradient (to
    1e-6); a NaN logit makes its row's loss and gradient NaN and no other.
"""
import pytest
import torch

import losses

pytestmark = pytest.mark.gpu

CAP = 15.0


def _inputs(dev, R, V, seed, scale=4.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    logits = (torch.randn((R, V), generator=g, device=dev) * scale).to(torch.bfloat16)
    tgt = torch.randint(0, V, (R,), generator=g, device=dev)
    return logits, tgt


def _reference(logits, tgt, cap, mask=None):
    l = logits.double().requires_grad_(True)
    z = cap * torch.tanh(l / cap)
    nll = torch.logsumexp(z, -1) - z.gather(-1, tgt[..., None]).squeeze(-1)
    if mask is None:
        loss = nll.mean()
    else:
        m = mask.double()
        loss = (nll * m).sum() / m.sum().clamp_min(1.0)
    loss.backward()
    return nll.detach(), loss.detach(), l.grad


def _close(got, ref, atol, rtol):
    got, ref = got.double(), ref.double()
    return bool(((got - ref).abs() <= atol + rtol * ref.abs()).all())


def _grad_ok(dl, gref):
    tol = gref.abs() * 2.0 ** -8 + 3e-5 * gref.abs().max()
    return bool(((dl.double() - gref).abs() <= tol).all())


SHAPES = [(8, 50304), (3, 1000), (5, 1001), (1, 7), (64, 50257), (130, 4096), (2, 8), (4, 50304 + 8)]


@pytest.mark.parametrize("cap", [CAP, 40.0])
@pytest.mark.parametrize("R,V", SHAPES)
def test_xent_matches_float64(dev, R, V, cap):
    logits, tgt = _inputs(dev, R, V, seed=R * 7 + V)
    logits.requires_grad_(True)
    loss = losses.capped_cross_entropy(logits, tgt, cap)
    loss.backward()
    nll, _ = losses.capped_cross_entropy_rows(logits.detach(), tgt, cap)
    nll_ref, loss_ref, g_ref = _reference(logits.detach(), tgt, cap)
    print(f"cap={cap} R={R} V={V}: loss {float(loss):.7f} ref {float(loss_ref):.7f} "
          f"nll max err {float((nll.double() - nll_ref).abs().max()):.2e}")
    assert _close(nll, nll_ref, 5e-5, 1e-5)
    assert _close(loss.detach(), loss_ref, 5e-5, 1e-5)
    assert logits.grad.dtype == torch.bfloat16
    assert _grad_ok(logits.grad, g_ref)


def test_xent_saturated_logits(dev):
    """Logits far past the cap: tanh saturates, the gradient's sech^2 factor
    stays relatively accurate instead of cancelling to 0 or NaN."""
    logits, tgt = _inputs(dev, 16, 4096, seed=3, scale=60.0)
    logits.requires_grad_(True)
    loss = losses.capped_cross_entropy(logits, tgt, CAP)
    loss.backward()
    nll_ref, loss_ref, g_ref = _reference(logits.detach(), tgt, CAP)
    assert torch.isfinite(logits.grad.float()).all()
    assert _close(loss.detach(), loss_ref, 5e-5, 1e-5)
    assert _grad_ok(logits.grad, g_ref)


@pytest.mark.parametrize("cap", [24.0, 25.0])
def test_xent_table_range_edges(dev, cap):
    """Logits up to ~400 (past the table's 256) and down to 2^-30 (below its
    2^-24) at the largest cap the table serves (24) and just past it."""
    logits, tgt = _inputs(dev, 8, 4096, seed=31, scale=100.0)
    logits[:, :64] = (torch.randn((8, 64), device=dev) * 2.0 ** -30).to(torch.bfloat16)
    logits[:, 64:72] = torch.tensor([0.0, -0.0, 256.0, -256.0, 400.0, -400.0, 2.0 ** -24, -(2.0 ** -25)],
                                    device=dev).to(torch.bfloat16)
    logits.requires_grad_(True)
    loss = losses.capped_cross_entropy(logits, tgt, cap)
    loss.backward()
    nll, _ = losses.capped_cross_entropy_rows(logits.detach(), tgt, cap)
    nll_ref, loss_ref, g_ref = _reference(logits.detach(), tgt, cap)
    assert _close(nll, nll_ref, 5e-5, 1e-5) and _close(loss.detach(), loss_ref, 5e-5, 1e-5)
    assert _grad_ok(logits.grad, g_ref)


@pytest.mark.parametrize("cap", [CAP, 40.0])
def test_xent_nan_logit_poisons_its_row(dev, cap):
    logits, tgt = _inputs(dev, 3, 1024, seed=41)
    logits[1, 77] = float("nan")
    logits.requires_grad_(True)
    nll, lse = losses.capped_cross_entropy_rows(logits.detach(), tgt, cap)
    assert torch.isnan(nll[1]) and torch.isnan(lse[1])
    assert torch.isfinite(nll[[0, 2]]).all() and torch.isfinite(lse[[0, 2]]).all()
    loss = losses.capped_cross_entropy(logits, tgt, cap, loss_mask=torch.tensor([1.0, 0.0, 1.0], device=dev))
    loss.backward()
    assert torch.isnan(logits.grad[1].float()).all()
    assert torch.isfinite(logits.grad[[0, 2]].float()).all()


def test_xent_masked_mean(dev):
    logits, tgt = _inputs(dev, 96, 2048, seed=11)
    g = torch.Generator(device=dev).manual_seed(12)
    mask = (torch.rand((96,), generator=g, device=dev) < 0.4).to(torch.float32)
    logits.requires_grad_(True)
    loss = losses.capped_cross_entropy(logits, tgt, CAP, loss_mask=mask)
    loss.backward()
    _, loss_ref, g_ref = _reference(logits.detach(), tgt, CAP, mask)
    assert _close(loss.detach(), loss_ref, 5e-5, 1e-5)
    assert _grad_ok(logits.grad, g_ref)
    assert torch.all(logits.grad[mask == 0] == 0)


def test_xent_all_masked_is_zero(dev):
    logits, tgt = _inputs(dev, 4, 512, seed=13)
    logits.requires_grad_(True)
    loss = losses.capped_cross_entropy(logits, tgt, CAP, loss_mask=torch.zeros(4, device=dev))
    loss.backward()
    assert float(loss) == 0.0 and torch.all(logits.grad == 0)


def test_xent_batched_shape_and_upstream_gradient(dev):
    """(B, T, V) logits as the model emits them, and a non-unit upstream gradient."""
    logits, tgt = _inputs(dev, 2 * 33, 1024, seed=21)
    logits = logits.reshape(2, 33, 1024).requires_grad_(True)
    tgt = tgt.reshape(2, 33)
    (3.5 * losses.capped_cross_entropy(logits, tgt, CAP)).backward()
    _, _, g_ref = _reference(logits.detach().reshape(66, 1024), tgt.reshape(66), CAP)
    assert logits.grad.shape == (2, 33, 1024)
    assert _grad_ok(logits.grad.reshape(66, 1024), 3.5 * g_ref)


def test_xent_deterministic(dev):
    logits, tgt = _inputs(dev, 32, 50304, seed=5)
    outs = []
    for _ in range(2):
        l = logits.clone().requires_grad_(True)
        loss = losses.capped_cross_entropy(l, tgt, CAP)
        loss.backward()
        outs.append((loss.detach().clone(), l.grad.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("cap", [CAP, 40.0])
def test_xent_single_class_is_zero(dev, cap):
    """V = 1: the loss and gradient are 0 (the direct kernel exactly; the table
    kernel up to log(exp(y)) != y in the last bit)."""
    logits, tgt = _inputs(dev, 5, 1, seed=6)
    logits.requires_grad_(True)
    loss = losses.capped_cross_entropy(logits, tgt, cap)
    loss.backward()
    assert abs(float(loss)) <= 1e-6 and float(logits.grad.float().abs().max()) <= 1e-6


def test_xent_target_outside_vocab_gives_nan(dev):
    logits, tgt = _inputs(dev, 3, 64, seed=9)
    tgt[1] = 64
    nll, lse = losses.capped_cross_entropy_rows(logits, tgt, CAP)
    assert torch.isnan(nll[1]) and torch.isfinite(nll[[0, 2]]).all() and torch.isfinite(lse).all()


def test_xent_rejects_bad_arguments(dev):
    logits, tgt = _inputs(dev, 2, 64, seed=10)
    with pytest.raises(TypeError, match="bfloat16"):
        losses.capped_cross_entropy(logits.float(), tgt, CAP)
    with pytest.raises(ValueError, match="int64"):
        losses.capped_cross_entropy(logits, tgt.int(), CAP)
    with pytest.raises(ValueError, match="logit_cap"):
        losses.capped_cross_entropy(logits, tgt, 0.0)
    with pytest.raises(ValueError, match="loss_mask"):
        losses.capped_cross_entropy(logits, tgt, CAP, loss_mask=torch.ones(3, device=dev))
