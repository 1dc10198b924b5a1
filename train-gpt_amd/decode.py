"""KV-cached autoregressive decoding on the FP8 hot path.

The reference's generate.py:134-187 re-runs model.forward over the whole
(padded) context for every new token (generate.py:166-171).  Here one prefill
pass over the prompt fills a KV cache and every further token is one decode
step over one row per sequence:

    x   = embed[tok] + pos[t]                                 model.py:83
    per layer (model.py:74-77):
      h_q, h_s    = rms_norm_fp8(x, norm1) (for layers > 0 fused with the
                    residual add of the previous layer's MLP)
      q | k | v   = one decode GEMV on the kept [wq|wk|wv]    model.py:59-65
      K[:, t], V[:, t] = k, v ; o = attention(q, K[:t+1], V[:t+1]) -> FP8 rows
                    (one HIP kernel, tg_decode_attention)     model.py:67
      x = x + GEMV(o, wo); h2_q, h2_s = rms_norm_fp8(x, norm2)    (one kernel)  model.py:68, 75
      u_q, u_s = quantize(relu(GEMV(h2, w_up))^2)                (one kernel)  model.py:71-72
      x = x + GEMV(u, w_down)                                                 model.py:76
    logits = cap * tanh(GEMV(rms_norm_fp8(x, final_norm), unembed) / cap)   model.py:93-97

Every linear runs on a weight quantized once (fp8.QuantizedWeight): the decode
GEMV for at most 64 rows, the scaled GEMM for the prefill.  The unembedding is
kept in FP8 as well (the reference keeps logits in bf16; the FP8 unembedding
halves the largest weight read of a decode step).  The prefill's causal
attention is torch's scaled_dot_product_attention (flash / memory-efficient
kernels; attention is not on the FP8 hot path in the reference either); a
decode step's attention is the HIP kernel above, which reads the position
from device memory so that one captured HIP graph serves every token.

Sliding window (generate.py:160-164): the learned positional embedding covers
seq_len positions, and the reference re-runs the last seq_len tokens at
positions 0 .. seq_len-1 once the context is longer.  Every cached key would
change position, so past that point each token is a fresh prefill of the
window -- exactly the reference's computation.

sample_next restates generate.py:93-131 (float64 numpy on the host).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

import _tglib as _L
import fp8
import kernels


@dataclass(frozen=True)
class Config:
    """config.py:6-27 (the model dtype is bf16; remat / Pallas flags do not apply)."""
    vocab_size: int = 50257
    seq_len: int = 2048
    d_model: int = 2304
    n_layers: int = 24
    n_heads: int = 18
    head_dim: int = 128
    d_ff: int = 9216
    init_std: float = 0.02
    rms_eps: float = 1e-5
    tie_embeddings: bool = False
    logit_cap: float = 15.0


SMALL = Config(vocab_size=256, seq_len=128, d_model=128, n_layers=2, n_heads=4, head_dim=32,
               d_ff=512)                                                 # config.py:30-38


def init_params(cfg: Config, device, seed: int = 0):
    """bf16 parameters with model.py:19-54's names and scales (layers as a list)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    std = cfg.init_std
    proj_std = cfg.init_std / math.sqrt(2.0 * cfg.n_layers)
    d, h, f = cfg.d_model, cfg.n_heads * cfg.head_dim, cfg.d_ff

    def normal(shape, s=std):
        return (torch.randn(shape, generator=g, device=device) * s).to(torch.bfloat16)

    def ones(n):
        return torch.ones(n, dtype=torch.bfloat16, device=device)

    layers = [{"norm1": ones(d), "wq": normal((d, h)), "wk": normal((d, h)), "wv": normal((d, h)),
               "wo": normal((h, d), proj_std), "norm2": ones(d), "w_up": normal((d, f)),
               "w_down": normal((f, d), proj_std)} for _ in range(cfg.n_layers)]
    p = {"embed": normal((cfg.vocab_size, d)), "pos": normal((cfg.seq_len, d)), "layers": layers,
         "final_norm": ones(d)}
    if not cfg.tie_embeddings:
        p["unembed"] = normal((d, cfg.vocab_size))
    return p


_LAYER_KEYS = ("norm1", "wq", "wk", "wv", "wo", "norm2", "w_up", "w_down")


def config_from_reference(c) -> Config:
    """Config from the reference's config object or a dict of its fields
    (config.py:6-27, as stored under "config" in a checkpoint payload,
    train_modal.py:402-407); dtype, use_remat and use_pallas_norm do not apply."""
    get = (lambda k: c[k]) if isinstance(c, dict) else (lambda k: getattr(c, k))
    kw = {}
    for f in Config.__dataclass_fields__:
        try:
            kw[f] = get(f)
        except (KeyError, AttributeError):
            pass
    return Config(**kw)


def _to_bf16(a, device) -> torch.Tensor:
    """One parameter leaf as a bf16 tensor on device: a torch tensor, or a numpy
    array in any float dtype, bfloat16 (2-byte, e.g. ml_dtypes' bfloat16 from a
    checkpoint of jax arrays) taken bit for bit, f16 / f32 / f64 rounded to bf16."""
    if isinstance(a, torch.Tensor):
        return a.detach().to(device=device, dtype=torch.bfloat16)
    a = np.asarray(a)
    if a.dtype.name == "bfloat16" and a.dtype.itemsize == 2:
        t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
        return t.to(device)
    if a.dtype.kind != "f":
        raise TypeError(f"parameter of dtype {a.dtype} is not a float array")
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device).to(torch.bfloat16)


def params_from_reference(tree, device) -> dict:
    """The reference's parameter tree (model.py:19-54, e.g. the "params" of a
    checkpoint payload, train_modal.py:402-407, after the caller has loaded it)
    as this module's parameters: bf16 tensors on device, "layers" a list of
    per-layer dicts.  The reference stacks the layers' leaves along a leading
    n_layers axis (jax.vmap of init_layer, model.py:44); a list of per-layer
    dicts is taken as it is."""
    layers = tree["layers"]
    if isinstance(layers, dict):
        missing = [k for k in _LAYER_KEYS if k not in layers]
        if missing:
            raise KeyError(f"layers is missing {missing}")
        n = len(layers["norm1"])
        for k in _LAYER_KEYS:
            if len(layers[k]) != n:
                raise ValueError(f"layers[{k!r}] stacks {len(layers[k])} layers, norm1 stacks {n}")
        layers = [{k: layers[k][i] for k in _LAYER_KEYS} for i in range(n)]
    out = {k: _to_bf16(tree[k], device) for k in ("embed", "pos", "final_norm")}
    if "unembed" in tree:
        out["unembed"] = _to_bf16(tree["unembed"], device)
    out["layers"] = [{k: _to_bf16(lp[k], device) for k in _LAYER_KEYS} for lp in layers]
    return out


def _check_fp8_dims(cfg: Config):
    h = cfg.n_heads * cfg.head_dim
    for name, k in (("d_model", cfg.d_model), ("n_heads*head_dim", h), ("d_ff", cfg.d_ff)):
        if k % fp8.DEFAULT_BLOCK_K:
            raise ValueError(f"{name}={k} must be a multiple of {fp8.DEFAULT_BLOCK_K} "
                             "(every linear contracts over it in 128-wide scale blocks)")


def _attention(q, k, v, causal: bool):
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return F.scaled_dot_product_attention(q, k, v, is_causal=causal)


# the decode steps of decode_attn "hip" form their input rows and apply the
# logit cap in one HIP kernel each (tg_decode_embed, tg_logit_cap: the same
# bits as torch's three and four kernels)
HIP_LOGIT_CAP = True


def decode_embed(embed: torch.Tensor, pos: torch.Tensor, tok: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
    """The step's input rows embed[tok] + pos[t] (model.py:89-90), bf16, in one
    HIP kernel (tg_decode_embed, the bits of torch's index, index_select and
    add).  A token or position outside its table reads a zero row."""
    if embed.dtype != torch.bfloat16 or pos.dtype != torch.bfloat16 or embed.shape[1] != pos.shape[1]:
        raise ValueError("decode_embed: embed (V, d) and pos (P, d) must be bf16 with one d")
    if tok.dim() != 1 or t.dtype != torch.int64 or t.numel() != 1:
        raise ValueError("decode_embed: tok must be (B,) and t a one-element int64 tensor")
    _L.require_gpu(embed, pos, t)
    # an int64 device tok (the captured step's) is used as it is: no copy, no launch
    tk = tok.to(device=embed.device, dtype=torch.int64).contiguous()
    e, p = embed.contiguous(), pos.contiguous()
    out = torch.empty((tk.shape[0], e.shape[1]), dtype=torch.bfloat16, device=e.device)
    _L.check(_L.lib().tg_decode_embed(_L.ptr(e), _L.ptr(p), _L.ptr(tk), _L.ptr(t), _L.ptr(out), tk.shape[0],
                                      e.shape[0], p.shape[0], e.shape[1], _L.stream_of(e)))
    return out


def logit_cap(logits: torch.Tensor, cap: float) -> torch.Tensor:
    """model.py:97 on bf16 logits: f32 cap * tanh(logits / cap), one HIP kernel
    (tg_logit_cap) with the bits of `cap * torch.tanh(logits.float() / cap)`."""
    if logits.dtype != torch.bfloat16:
        raise ValueError("logit_cap: logits must be bf16")
    _L.require_gpu(logits)
    x = logits.contiguous()
    out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    _L.check(_L.lib().tg_logit_cap(_L.ptr(x), _L.ptr(out), x.numel(), float(cap), _L.stream_of(x)))
    return out


def decode_attention(qkv: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     t: torch.Tensor, n_heads: int, want_bf16: bool = False):
    """The HIP decode attention (tg_decode_attention): appends k, v of qkv
    (B, 3 H Dh) at position t (int64 device tensor of one element) to the
    caches (B, H, S, Dh) and attends the new queries over positions 0 .. t.
    Returns (o_q e4m3fn (B, H Dh), o_s f32 (B, H), o bf16 (B, H Dh) or None)."""
    _L.require_gpu(qkv, k_cache, v_cache, t)
    B, S, Dh = qkv.shape[0], k_cache.shape[2], k_cache.shape[3]
    if qkv.shape[1] != 3 * n_heads * Dh or tuple(k_cache.shape) != (B, n_heads, S, Dh):
        raise ValueError("decode_attention: qkv (B, 3 H Dh) and caches (B, H, S, Dh) disagree")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous() and qkv.is_contiguous()):
        raise ValueError("decode_attention: qkv and caches must be contiguous")
    if t.dtype != torch.int64 or t.numel() != 1:
        raise ValueError("decode_attention: t must be a one-element int64 tensor")
    o_q = torch.empty((B, n_heads * Dh), dtype=torch.uint8, device=qkv.device)
    o_s = torch.empty((B, n_heads), dtype=torch.float32, device=qkv.device)
    o = torch.empty((B, n_heads * Dh), dtype=torch.bfloat16, device=qkv.device) if want_bf16 else None
    _L.check(_L.lib().tg_decode_attention(
        _L.ptr(qkv), _L.ptr(k_cache), _L.ptr(v_cache), _L.ptr(t), _L.ptr(o_q), _L.ptr(o_s),
        _L.ptr(o) if o is not None else None, B, n_heads, S, Dh, 1.0 / math.sqrt(Dh),
        _L.stream_of(qkv)))
    return o_q.view(torch.float8_e4m3fn), o_s, o


class FP8Decoder:
    """The reference model (model.py) with kept FP8 weights and a KV cache.

    params: this module's layout (init_params) or the reference's tree with
    the layers stacked (model.py:19-54, e.g. a checkpoint's "params"), whose
    numpy leaves go to the current GPU (params_from_reference).
    layout: scale layout of the kept weights, "128x128" (one scale per
    128x128 tile, the baseline's decode config) or "128x1" (per column, the
    bytes and scales fp8.py:68 computes on every call).
    decode_attn: "hip" (tg_decode_attention: cache append, attention and the
    FP8 quantization of its output in one kernel; graph-capturable) or "sdpa"
    (torch's attention over the cached keys, the arithmetic of the prefill;
    eager only -- with it a decode step reproduces the full forward bit for bit).
    exact_gemv: for 1-2 rows use the MFMA GEMV (the GEMM's block arithmetic)
    rather than the faster VALU one (tg_gemv_fp8_rowdot); default: on with
    decode_attn "sdpa" (the bit-exact mode), off with "hip".
    fused: a decode step runs each norm (or residual add + norm) inside the
    GEMV that consumes it (tg_rms_norm_fp8_gemv), and for 1-2 rows also the
    relu^2 quantization (tg_relu2_fp8_gemv): 5 kernels per layer instead of 8
    (1-2 rows, VALU GEMV) or 6 (3-16 rows, MFMA GEMV, d_model <= 2560), the
    same bits.  Default: on for up to 8 rows (measured at the reference
    config: batch 4 and 8 steps 14% and 11% faster); at 9-16 rows each wave
    normalises two rows in the GEMV's prologue and the fused step measured 2%
    slower at 16, so it is off unless asked for.
    """

    def __init__(self, params, cfg: Config, layout: str = "128x128", max_batch: int = 1,
                 decode_attn: str = "hip", exact_gemv: bool = None, fused: bool = None):
        _check_fp8_dims(cfg)
        if isinstance(params["layers"], dict) or not isinstance(params["embed"], torch.Tensor):
            dev = (params["embed"].device if isinstance(params["embed"], torch.Tensor)
                   else torch.device("cuda", torch.cuda.current_device()))
            params = params_from_reference(params, dev)
        if decode_attn not in ("hip", "sdpa"):
            raise ValueError("decode_attn must be 'hip' or 'sdpa'")
        self.decode_attn = decode_attn
        self.exact_gemv = decode_attn == "sdpa" if exact_gemv is None else bool(exact_gemv)
        can_fuse = ((max_batch <= 2 and not self.exact_gemv and cfg.d_model <= 4096)
                    or (3 <= max_batch <= 16 and cfg.d_model <= 2560))
        if fused and not can_fuse:
            raise ValueError("fused decode steps need max_batch <= 2 with exact_gemv=False and d_model <= 4096, "
                             "or 3 <= max_batch <= 16 and d_model <= 2560")
        self.fused = (can_fuse and max_batch <= 8) if fused is None else bool(fused)
        if not 1 <= max_batch <= 64:
            raise ValueError("max_batch must be in [1, 64] (decode rows per GEMV)")
        self.cfg = cfg
        dev = params["embed"].device
        self.device = dev
        self.embed = params["embed"].to(torch.bfloat16)
        self.pos = params["pos"].to(torch.bfloat16)
        qw = lambda w: fp8.QuantizedWeight.from_weight(w.detach().to(torch.bfloat16).contiguous(), layout)
        self.layers = []
        for lp in params["layers"]:
            # q, k and v share their input: one kept weight W_qkv = [wq | wk | wv]
            # (d, 3h), one GEMV.  Its scale blocks are the blocks of the three
            # weights (h is a multiple of 128), so the product is theirs.
            wqkv = torch.cat([lp["wq"], lp["wk"], lp["wv"]], dim=1)
            self.layers.append({
                "norm1": lp["norm1"].to(torch.bfloat16), "norm2": lp["norm2"].to(torch.bfloat16),
                "wqkv": qw(wqkv), "wo": qw(lp["wo"]),
                "w_up": qw(lp["w_up"]), "w_down": qw(lp["w_down"])})
        self.final_norm = params["final_norm"].to(torch.bfloat16)
        w_out = params["embed"].t() if cfg.tie_embeddings else params["unembed"]   # model.py:95
        self.unembed = qw(w_out)
        H, Dh, L = cfg.n_heads, cfg.head_dim, cfg.n_layers
        self.max_batch = max_batch
        self.k_cache = torch.zeros((L, max_batch, H, cfg.seq_len, Dh), dtype=torch.bfloat16, device=dev)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.length = 0
        self._graph = None

    # -- one transformer block over the prompt rows x (B, T, d), positions 0 .. T-1 --
    def _block(self, li: int, x: torch.Tensor) -> torch.Tensor:
        cfg, lp = self.cfg, self.layers[li]
        B, T, d = x.shape
        H, Dh = cfg.n_heads, cfg.head_dim
        h, h_q, h_s = kernels.rms_norm_fp8(x, lp["norm1"], cfg.rms_eps)
        qkv = lp["wqkv"].matmul_prequant(h_q.reshape(B * T, d), h_s.reshape(B * T, -1),
                                       exact=self.exact_gemv)
        q, k, v = qkv.reshape(B, T, 3, H, Dh).permute(2, 0, 3, 1, 4).unbind(0)   # each (B, H, T, Dh)
        self.k_cache[li, :B, :, :T] = k
        self.v_cache[li, :B, :, :T] = v
        o = _attention(q, k, v, causal=True)                           # model.py:67
        o = o.transpose(1, 2).reshape(B * T, H * Dh)
        x = x + lp["wo"].matmul(o, exact=self.exact_gemv).reshape(B, T, d)   # model.py:68, 75
        h2, h2_q, h2_s = kernels.rms_norm_fp8(x, lp["norm2"], cfg.rms_eps)
        u = lp["w_up"].matmul_prequant(h2_q.reshape(B * T, d), h2_s.reshape(B * T, -1),
                                        exact=self.exact_gemv)
        u = F.relu(u).square()                                         # model.py:72 (bf16)
        return x + lp["w_down"].matmul(u, exact=self.exact_gemv).reshape(B, T, d)   # model.py:76

    def _head(self, x: torch.Tensor) -> torch.Tensor:
        """Final norm -> FP8 unembedding -> logit cap (model.py:93-97); f32 (rows, V)."""
        cfg = self.cfg
        d = x.shape[-1]
        _, xq, xs = kernels.rms_norm_fp8(x.reshape(-1, d), self.final_norm, cfg.rms_eps)
        logits = self.unembed.matmul_prequant(xq, xs, exact=self.exact_gemv).float()
        return cfg.logit_cap * torch.tanh(logits / cfg.logit_cap)

    @torch.no_grad()
    def prefill(self, ids: torch.Tensor, all_logits: bool = False) -> torch.Tensor:
        """Run ids (B, T) at positions 0 .. T-1 and fill the cache.  Returns the
        f32 logits of the last position (B, V), or of every position (B, T, V)."""
        B, T = ids.shape
        if not 1 <= B <= self.max_batch:
            raise ValueError(f"batch {B} exceeds max_batch={self.max_batch}")
        if not 1 <= T <= self.cfg.seq_len:
            raise ValueError(f"prompt length {T} must be in [1, seq_len={self.cfg.seq_len}]")
        x = self.embed[ids] + self.pos[:T]                              # model.py:83
        for li in range(self.cfg.n_layers):
            x = self._block(li, x)
        self.length = T
        if all_logits:
            return self._head(x).reshape(B, T, -1)
        return self._head(x[:, -1])

    @torch.no_grad()
    def step(self, tok: torch.Tensor) -> torch.Tensor:
        """Append one token per sequence (tok (B,)) at position `length`; returns
        the f32 logits of that position (B, V).  The attention is the HIP decode
        attention over positions 0 .. t (tg_decode_attention); the step replays
        the captured HIP graph once capture_step() has been called."""
        t = self.length
        if t == 0:
            raise RuntimeError("step() before prefill()")
        if t >= self.cfg.seq_len:
            raise RuntimeError("the cache is full (seq_len positions); prefill the window again")
        B = tok.shape[0]
        if self._graph is not None and B == self._gB:
            self._g_tok.copy_(tok)
            self._g_t.fill_(t)
            self._graph.replay()
            self.length = t + 1
            return self._g_logits.clone()
        if B != self.max_batch:
            raise ValueError(f"step: batch {B} must equal max_batch={self.max_batch} (the cache rows)")
        logits = self._step_dev(tok, torch.full((1,), t, dtype=torch.long, device=self.device), B)
        self.length = t + 1
        return logits

    # -- graph-capturable decode step: the position lives in device memory --
    def _step_dev(self, tok: torch.Tensor, t: torch.Tensor, B: int) -> torch.Tensor:
        if self.fused:
            return self._step_dev_fused(tok, t, B)
        cfg = self.cfg
        H = cfg.n_heads
        if HIP_LOGIT_CAP and self.decode_attn == "hip":
            x = decode_embed(self.embed, self.pos, tok, t)                 # (B, d), model.py:89-90
        else:
            x = self.embed[tok] + self.pos.index_select(0, t)
        _, h_q, h_s = kernels.rms_norm_fp8(x, self.layers[0]["norm1"], cfg.rms_eps)
        for li, lp in enumerate(self.layers):
            qkv = lp["wqkv"].matmul_prequant(h_q, h_s, self.exact_gemv)                      # (B, 3 H Dh)
            if self.decode_attn == "hip":
                o_q, o_s, _ = decode_attention(qkv, self.k_cache[li], self.v_cache[li], t, H)
                a = lp["wo"].matmul_prequant(o_q, o_s, self.exact_gemv)                      # model.py:68
            else:
                a = lp["wo"].matmul(self._sdpa_step(li, qkv, int(t.item())), exact=self.exact_gemv)
            # x = x + a (model.py:75) fused with norm2 -> FP8 rows
            x, h2_q, h2_s, _ = kernels.add_rms_norm_fp8(x, a, lp["norm2"], cfg.rms_eps, inplace=True)
            u_q, u_s = fp8.quantize_relu2(lp["w_up"].matmul_prequant(h2_q, h2_s, self.exact_gemv))   # model.py:72
            m = lp["w_down"].matmul_prequant(u_q, u_s, self.exact_gemv)
            # x = x + m (model.py:76) fused with the next norm (norm1 or final_norm)
            nxt = self.layers[li + 1]["norm1"] if li + 1 < len(self.layers) else self.final_norm
            x, h_q, h_s, _ = kernels.add_rms_norm_fp8(x, m, nxt, cfg.rms_eps, inplace=True)
        logits = self.unembed.matmul_prequant(h_q, h_s, self.exact_gemv)                    # model.py:96
        if HIP_LOGIT_CAP and self.decode_attn == "hip":
            return logit_cap(logits, cfg.logit_cap)                                          # model.py:97
        return cfg.logit_cap * torch.tanh(logits.float() / cfg.logit_cap)  # model.py:97

    def _step_dev_fused(self, tok: torch.Tensor, t: torch.Tensor, B: int) -> torch.Tensor:
        """_step_dev with each norm / relu^2 quantization inside the GEMV that
        consumes it.  At 1-2 rows the residual adds (model.py:75-76) run in the
        stores of the o and down projections, on the residual stream in place,
        so the norms after them have no add of their own; at 3-16 rows the
        norm GEMV adds, and the residual stream alternates between two
        buffers (a fused kernel reads one while its workgroup 0 writes the
        other).  The same bits either way."""
        cfg = self.cfg
        H, eps = cfg.n_heads, cfg.rms_eps
        if HIP_LOGIT_CAP and self.decode_attn == "hip":
            xa = decode_embed(self.embed, self.pos, tok, t)                 # (B, d), model.py:89-90
        else:
            xa = self.embed[tok] + self.pos.index_select(0, t)
        qkv = self.layers[0]["wqkv"].matmul_rms_norm(xa, self.layers[0]["norm1"], eps)   # model.py:61-64
        if B <= 2:
            for li, lp in enumerate(self.layers):
                if self.decode_attn == "hip":
                    o_q, o_s, _ = decode_attention(qkv, self.k_cache[li], self.v_cache[li], t, H)
                else:
                    o_q, o_s = fp8.quantize_fp8(self._sdpa_step(li, qkv, int(t.item())))
                lp["wo"].matmul_prequant_add(o_q, o_s, xa, out=xa)          # x += o wo (model.py:68, 75)
                u = lp["w_up"].matmul_rms_norm(xa, lp["norm2"], eps)        # model.py:71, 75
                lp["w_down"].matmul_relu2_add(u, xa, out=xa)                # x += relu(u)^2 w_down (72, 76)
                last = li + 1 == len(self.layers)
                nxt = self.final_norm if last else self.layers[li + 1]["norm1"]
                w = self.unembed if last else self.layers[li + 1]["wqkv"]
                qkv = w.matmul_rms_norm(xa, nxt, eps)
            if HIP_LOGIT_CAP and self.decode_attn == "hip":
                return logit_cap(qkv, cfg.logit_cap)                          # model.py:97
            return cfg.logit_cap * torch.tanh(qkv.float() / cfg.logit_cap)  # model.py:97
        xb = torch.empty_like(xa)
        for li, lp in enumerate(self.layers):
            if self.decode_attn == "hip":
                o_q, o_s, _ = decode_attention(qkv, self.k_cache[li], self.v_cache[li], t, H)
                a = lp["wo"].matmul_prequant(o_q, o_s)                     # model.py:68
            else:
                a = lp["wo"].matmul(self._sdpa_step(li, qkv, int(t.item())))
            # x = x + a (model.py:75), norm2, w_up (model.py:71-72)
            u = lp["w_up"].matmul_rms_norm(xa, lp["norm2"], eps, delta=a, xout=xb)
            m = lp["w_down"].matmul_prequant(*fp8.quantize_relu2(u))        # model.py:72-73
            # x = x + m (model.py:76), then the next layer's norm1 and q|k|v, or
            # the final norm and the unembedding (model.py:93-96)
            last = li + 1 == len(self.layers)
            nxt = self.final_norm if last else self.layers[li + 1]["norm1"]
            w = self.unembed if last else self.layers[li + 1]["wqkv"]
            qkv = w.matmul_rms_norm(xb, nxt, eps, delta=m, xout=xa)
        if HIP_LOGIT_CAP and self.decode_attn == "hip":
            return logit_cap(qkv, cfg.logit_cap)                              # model.py:97
        return cfg.logit_cap * torch.tanh(qkv.float() / cfg.logit_cap)      # model.py:97

    def _sdpa_step(self, li: int, qkv: torch.Tensor, t: int) -> torch.Tensor:
        """decode_attn="sdpa": append k, v at t, torch attention over 0 .. t."""
        cfg = self.cfg
        B, H, Dh = qkv.shape[0], cfg.n_heads, cfg.head_dim
        q, k, v = qkv.reshape(B, 3, H, 1, Dh).unbind(1)
        self.k_cache[li, :, :, t:t + 1] = k
        self.v_cache[li, :, :, t:t + 1] = v
        o = _attention(q, self.k_cache[li, :, :, :t + 1], self.v_cache[li, :, :, :t + 1], causal=False)
        return o.reshape(B, H * Dh)

    @torch.no_grad()
    def capture_step(self, batch: int) -> None:
        """Capture one decode step for `batch` sequences as a HIP graph (the
        kernels of every layer replay without host launch overhead).  The graph
        reads the token ids and the position from device buffers."""
        if batch != self.max_batch:
            raise ValueError("capture_step: batch must equal max_batch (the cache rows the graph reads)")
        if self.decode_attn != "hip":
            raise ValueError("capture_step: needs decode_attn='hip' (the position is read on the device)")
        self._graph = None
        self._gB = batch
        self._g_tok = torch.zeros(batch, dtype=torch.long, device=self.device)
        self._g_t = torch.zeros(1, dtype=torch.long, device=self.device)
        k_save, v_save = self.k_cache.clone(), self.v_cache.clone()
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(2):                                             # warm-up (allocator, kernels)
                self._step_dev(self._g_tok, self._g_t, batch)
        torch.cuda.current_stream(self.device).wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._g_logits = self._step_dev(self._g_tok, self._g_t, batch)
        self.k_cache.copy_(k_save)                                         # capture ran nothing, warm-up wrote row 0
        self.v_cache.copy_(v_save)
        self._graph = g

    @torch.no_grad()
    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        """model.forward (model.py:81-98) over the whole context: f32 logits (B, T, V).
        The cache is refilled as a side effect."""
        return self.prefill(ids, all_logits=True)


def sample_next(logits, temperature: float, top_k: int, top_p: float,
                rng: np.random.Generator) -> int:
    """generate.py:93-131: one token id from a (vocab,) logit vector.

    temperature == 0 is greedy; top_k <= 0 disables top-k; top_p >= 1
    disables nucleus filtering; top-k applies first, then top-p.
    """
    logits = np.asarray(logits, dtype=np.float64)
    if temperature == 0.0:
        return int(logits.argmax())
    logits = logits / temperature
    if top_k and top_k > 0:
        k = min(top_k, logits.shape[-1])
        kth = np.partition(logits, -k)[-k]
        logits = np.where(logits < kth, -np.inf, logits)
    logits = logits - logits.max()
    probs = np.exp(logits)
    probs /= probs.sum()
    if top_p < 1.0:
        order = np.argsort(probs)[::-1]
        cum = np.cumsum(probs[order])
        keep = cum - probs[order] < top_p          # the mass before a token is under top_p
        probs[order[~keep]] = 0.0
        probs /= probs.sum()
    return int(rng.choice(probs.shape[-1], p=probs))


def generate(model: FP8Decoder, prompt_ids: list[int], max_new_tokens: int, *,
             temperature: float = 0.8, top_k: int = 50, top_p: float = 1.0, seed: int = 0,
             eot_token: int | None = None, stop_on_eot: bool = True,
             use_cache: bool = True) -> list[int]:
    """generate.py:134-187 on the FP8 decoder: the newly sampled ids (not the prompt).

    use_cache=False re-runs the full context for every token, as the
    reference does; use_cache=True prefills once and then decodes one row per
    token while the context fits in seq_len positions.
    """
    if max_new_tokens <= 0:
        raise ValueError(f"max_new_tokens must be > 0, got {max_new_tokens}")
    if temperature < 0.0:
        raise ValueError(f"temperature must be >= 0, got {temperature}")
    if not (0.0 < top_p <= 1.0):
        raise ValueError(f"top_p must be in (0, 1], got {top_p}")
    if not prompt_ids:
        raise ValueError("prompt_ids is empty; pass at least one token")
    rng = np.random.default_rng(seed)
    seq_len = model.cfg.seq_len
    dev = model.device
    ids = list(prompt_ids)
    new: list[int] = []
    cached = False
    for _ in range(max_new_tokens):
        if use_cache and cached and len(ids) <= seq_len:
            logits = model.step(torch.tensor([ids[-1]], device=dev))[0]
        else:
            context = ids[-seq_len:]                                  # generate.py:162
            logits = model.prefill(torch.tensor([context], device=dev))[0]
            cached = len(ids) < seq_len
        tok = sample_next(logits.cpu().numpy(), temperature, top_k, top_p, rng)
        ids.append(tok)
        new.append(tok)
        if stop_on_eot and eot_token is not None and tok == eot_token:
            break
    return new
