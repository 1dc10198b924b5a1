"""Cross entropy of the capped logits on MI355X -- the loss of the reference's
losses.py fused with the logit cap at the end of model.forward.

/root/reference/losses.py:8-12 (cross_entropy_loss) and :15-34
(masked_cross_entropy_loss) take the model's logits, which model.py:96-97 has
capped as cap * tanh(logits / cap), cast them to f32 and take the mean (or
masked mean) of -log_softmax at the targets.  Here the cap, the log-sum-exp
and the target pick are one read of the bf16 pre-cap logits
(tg_logit_cap_xent_fwd), and the backward -- softmax minus one-hot times the
cap's derivative 1 - (z / cap)^2 -- is one more read and one bf16 write
(tg_logit_cap_xent_bwd).  The cap is computed in f32 from the bf16 logits.

The entry point takes the pre-cap logits, not params: the model forward that
produces them is the caller's (block.py's step, or a full model).
"""
import torch

import _tglib as _L


class _CappedXent(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, targets, cap, loss_mask):
        V = logits.shape[-1]
        l2 = logits.reshape(-1, V).contiguous()
        t2 = targets.reshape(-1).contiguous()
        R = l2.shape[0]
        row_loss = torch.empty(R, dtype=torch.float32, device=logits.device)
        row_lse = torch.empty(R, dtype=torch.float32, device=logits.device)
        _L.check(_L.lib().tg_logit_cap_xent_fwd(_L.ptr(l2), _L.ptr(t2), R, V, float(cap),
                                                _L.ptr(row_loss), _L.ptr(row_lse),
                                                _L.stream_of(l2)))
        if loss_mask is None:
            loss, w = row_loss.mean(), None                                 # losses.py:12
        else:
            m = loss_mask.reshape(-1).to(torch.float32)
            denom = torch.clamp_min(m.sum(), 1.0)                           # losses.py:34
            loss, w = (row_loss * m).sum() / denom, (m / denom).contiguous()
        ctx.save_for_backward(l2, t2, row_lse, w)
        ctx.cap, ctx.shape = float(cap), logits.shape
        return loss

    @staticmethod
    def backward(ctx, g):
        l2, t2, row_lse, w = ctx.saved_tensors
        R, V = l2.shape
        g1 = g.reshape(1).to(torch.float32).contiguous()
        dl = torch.empty_like(l2)
        g_scale = 1.0 if w is not None else 1.0 / max(R, 1)
        _L.check(_L.lib().tg_logit_cap_xent_bwd(_L.ptr(l2), _L.ptr(t2), _L.ptr(row_lse), _L.ptr(g1),
                                                g_scale, _L.ptr(w) if w is not None else None,
                                                R, V, ctx.cap, _L.ptr(dl), _L.stream_of(l2)))
        return dl.reshape(ctx.shape), None, None, None


def _check(logits, targets, cap, loss_mask):
    _L.require_gpu(logits, targets, *([loss_mask] if loss_mask is not None else []))
    if logits.dtype != torch.bfloat16:
        raise TypeError("capped_cross_entropy: logits must be bfloat16 (the model's output dtype)")
    if targets.dtype != torch.int64 or targets.shape != logits.shape[:-1]:
        raise ValueError("capped_cross_entropy: targets must be int64 with logits.shape[:-1]")
    if not cap > 0 or cap == float("inf"):
        raise ValueError("capped_cross_entropy: logit_cap must be finite and > 0")
    if loss_mask is not None and loss_mask.shape != targets.shape:
        raise ValueError("capped_cross_entropy: loss_mask must have targets' shape")


def capped_cross_entropy(logits: torch.Tensor, target_ids: torch.Tensor, logit_cap: float,
                         loss_mask: torch.Tensor = None) -> torch.Tensor:
    """mean(-log_softmax(cap * tanh(logits / cap))[target]) in f32.

    logits: (..., vocab) bf16 before the cap (model.py:95's x @ w_out);
    target_ids: (...) int64.  Without loss_mask this is losses.py:8-12's
    cross_entropy_loss; with it (0/1 per target) losses.py:15-34's
    masked_cross_entropy_loss, sum(nll * mask) / max(sum(mask), 1).
    Differentiable in logits (the gradient is bf16).
    """
    _check(logits, target_ids, logit_cap, loss_mask)
    return _CappedXent.apply(logits, target_ids, logit_cap, loss_mask)


def capped_cross_entropy_rows(logits: torch.Tensor, target_ids: torch.Tensor, logit_cap: float):
    """Per-position (nll, log-sum-exp), both f32 with target_ids' shape: the
    nll of losses.py:10-11 before its mean.  No autograd."""
    _check(logits, target_ids, logit_cap, None)
    V = logits.shape[-1]
    l2 = logits.reshape(-1, V).contiguous()
    t2 = target_ids.reshape(-1).contiguous()
    R = l2.shape[0]
    nll = torch.empty(R, dtype=torch.float32, device=logits.device)
    lse = torch.empty(R, dtype=torch.float32, device=logits.device)
    _L.check(_L.lib().tg_logit_cap_xent_fwd(_L.ptr(l2), _L.ptr(t2), R, V, float(logit_cap),
                                            _L.ptr(nll), _L.ptr(lse), _L.stream_of(l2)))
    return nll.reshape(target_ids.shape), lse.reshape(target_ids.shape)
