"""One pre-norm decoder block training step wired through the FP8 hot path.

The block of /root/reference/model.py:57-78 as bench_fp8_norm.py:81-128
builds it with `mm = block_scaled_matmul`: every linear (q, k, v, o, up,
down) is fp8.block_scaled_matmul (FP8 forward and FP8 backward) and both
norms are kernels.rms_norm (HIP forward and backward).  One difference is on
purpose: the three q/k/v projections share one fused norm -> FP8 quantize of
their input (kernels.rms_norm_fp8), instead of quantizing it three times.

Configuration (the baseline's config 4): d_model 2048, 16 heads of 128,
MLP 8192, batch 4 x 2048 tokens, vocab 50304, weights ~N(0, 0.02^2) bf16,
seed 3.  The MLP activation follows the baseline's wording (GELU, tanh form)
rather than model.py:71-72's squared ReLU, a one-line swap (MLP_ACT).  The
rest follows model.py: learned positional embedding (model.py:83), logit cap
15 tanh (model.py:97, config.py:24), rms eps 1e-5 (config.py:17), untied
unembedding kept in bf16 as bench_fp8_norm.py:117-118 does -- here on the
bf16 MFMA GEMM (fp8.bf16_matmul) -- and the cap fused with the loss
(losses.capped_cross_entropy: f32 cap of the bf16 logits, one HIP kernel
forward and one backward).

Attention is not on the hot path (it stays bf16 in the reference too): it is
torch's scaled_dot_product_attention restricted to its flash / memory-
efficient kernels.  The math backend is excluded: its bf16 batched products
are a known fault risk on this platform.

impl = "fp8": the hot path as described.  impl = "bf16": the same block with
every linear on the bf16 GEMM (fp8.bf16_matmul) and the same HIP norms -- the
reference's numerics without FP8.  reference_loss() is the float32 torch
restatement used as the parity baseline in tests and in bench.py.
"""
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

import fp8
import kernels
import losses


@dataclass(frozen=True)
class BlockConfig:
    d_model: int = 2048
    n_heads: int = 16
    head_dim: int = 128
    d_ff: int = 8192
    vocab: int = 50304
    seq_len: int = 2048
    batch: int = 4
    rms_eps: float = 1e-5
    logit_cap: float = 15.0
    init_std: float = 0.02


C4 = BlockConfig()

MLP_ACT = "gelu_tanh"     # the baseline's config 4; model.py:71-72 uses relu(x)**2


def _act(x):
    if MLP_ACT == "gelu_tanh":
        return F.gelu(x, approximate="tanh")
    return F.relu(x) ** 2


PARAM_NAMES = ("embed", "pos", "norm1", "wq", "wk", "wv", "wo", "norm2", "w_up", "w_down",
               "final_norm", "unembed")


def init_params(cfg: BlockConfig, device, seed: int = 3):
    """bf16 parameters (requires_grad) drawn from one seeded torch generator."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    d, h, f, V = cfg.d_model, cfg.n_heads * cfg.head_dim, cfg.d_ff, cfg.vocab

    def normal(*shape):
        return (torch.randn(shape, generator=g, device=device) * cfg.init_std).to(torch.bfloat16)

    p = {
        "embed": normal(V, d), "pos": normal(cfg.seq_len, d),
        "norm1": torch.ones(d, dtype=torch.bfloat16, device=device),
        "wq": normal(d, h), "wk": normal(d, h), "wv": normal(d, h), "wo": normal(h, d),
        "norm2": torch.ones(d, dtype=torch.bfloat16, device=device),
        "w_up": normal(d, f), "w_down": normal(f, d),
        "final_norm": torch.ones(d, dtype=torch.bfloat16, device=device),
        "unembed": normal(d, V),
    }
    for t in p.values():
        t.requires_grad_(True)
    return p


def random_batch(cfg: BlockConfig, device, seed: int = 3):
    g = torch.Generator(device=device)
    g.manual_seed(seed + 1)
    ids = torch.randint(0, cfg.vocab, (cfg.batch, cfg.seq_len), generator=g, device=device)
    tgt = torch.randint(0, cfg.vocab, (cfg.batch, cfg.seq_len), generator=g, device=device)
    return ids, tgt


def _attention(q, k, v):
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return F.scaled_dot_product_attention(q, k, v, is_causal=True)


def loss(params, ids, tgt, cfg: BlockConfig, impl: str = "fp8"):
    """Mean next-token cross entropy of embed -> block -> final norm -> logits."""
    if impl not in ("fp8", "bf16"):
        raise ValueError("impl must be 'fp8' or 'bf16'")
    B, T = ids.shape
    H, Dh = cfg.n_heads, cfg.head_dim
    p = params
    mm = fp8.block_scaled_matmul if impl == "fp8" else fp8.bf16_matmul
    x = p["embed"][ids] + p["pos"][:T]                                   # model.py:83
    # attention half (model.py:59-68, 75)
    if impl == "fp8":
        h, h_q, h_s = kernels.rms_norm_fp8(x, p["norm1"], cfg.rms_eps)
        proj = lambda w: fp8.block_scaled_matmul_prequant(h, h_q, h_s, w)
    else:
        h = kernels.rms_norm(x, p["norm1"], cfg.rms_eps)
        proj = lambda w: mm(h, w)
    q = proj(p["wq"]).reshape(B, T, H, Dh).transpose(1, 2)
    k = proj(p["wk"]).reshape(B, T, H, Dh).transpose(1, 2)
    v = proj(p["wv"]).reshape(B, T, H, Dh).transpose(1, 2)
    o = _attention(q, k, v).transpose(1, 2).reshape(B, T, H * Dh)
    x = x + mm(o, p["wo"])
    # MLP half (model.py:71-72, 76)
    h2 = kernels.rms_norm(x, p["norm2"], cfg.rms_eps)
    x = x + mm(_act(mm(h2, p["w_up"])), p["w_down"])
    # head (model.py:93-97), logits in bf16 on the bf16 GEMM; the cap and the
    # loss (losses.py:8-12) are one fused HIP pass each way
    xf = kernels.rms_norm(x, p["final_norm"], cfg.rms_eps)
    return losses.capped_cross_entropy(fp8.bf16_matmul(xf, p["unembed"]), tgt, cfg.logit_cap)


def _norm_f32(x, w, eps):
    return x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + eps) * w


def reference_loss(params, ids, tgt, cfg: BlockConfig):
    """The same step in float32 torch ops (no FP8, no bf16 roundings inside):
    the parity baseline.  Attention uses float32 math, which is safe here."""
    p = {k: v.float() for k, v in params.items()}
    B, T = ids.shape
    H, Dh = cfg.n_heads, cfg.head_dim
    x = p["embed"][ids] + p["pos"][:T]
    h = _norm_f32(x, p["norm1"], cfg.rms_eps)
    q = (h @ p["wq"]).reshape(B, T, H, Dh).transpose(1, 2).contiguous()
    k = (h @ p["wk"]).reshape(B, T, H, Dh).transpose(1, 2).contiguous()
    v = (h @ p["wv"]).reshape(B, T, H, Dh).transpose(1, 2).contiguous()
    o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    x = x + o.transpose(1, 2).reshape(B, T, H * Dh) @ p["wo"]
    h2 = _norm_f32(x, p["norm2"], cfg.rms_eps)
    x = x + _act(h2 @ p["w_up"]) @ p["w_down"]
    xf = _norm_f32(x, p["final_norm"], cfg.rms_eps)
    logits = xf @ p["unembed"]
    logits = cfg.logit_cap * torch.tanh(logits / cfg.logit_cap)
    return F.cross_entropy(logits.reshape(B * T, -1), tgt.reshape(-1))


def step_grads(params, ids, tgt, cfg: BlockConfig, impl: str = "fp8"):
    """(loss, {name: grad}) of one training step (forward + backward)."""
    for t in params.values():
        t.grad = None
    if impl == "ref":
        l = reference_loss(params, ids, tgt, cfg)
    else:
        l = loss(params, ids, tgt, cfg, impl)
    l.backward()
    return l.detach(), {k: params[k].grad.detach().clone() for k in PARAM_NAMES}


def flops_per_step(cfg: BlockConfig) -> float:
    """Matmul FLOPs of one step (forward + backward = 3 x forward):
    the six FP8 linears, the bf16 logits and causal attention (half of 4 T^2 Dh H per sequence)."""
    tok = cfg.batch * cfg.seq_len
    d, h, f, V = cfg.d_model, cfg.n_heads * cfg.head_dim, cfg.d_ff, cfg.vocab
    lin = 2.0 * tok * (3 * d * h + h * d + 2 * d * f)
    logits = 2.0 * tok * d * V
    attn = 2.0 * cfg.batch * cfg.n_heads * cfg.seq_len * cfg.seq_len * cfg.head_dim
    return 3.0 * (lin + logits + attn)
