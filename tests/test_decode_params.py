"""The reference's parameter tree as the decoder's parameters.

model.py:19-54 builds the layers with jax.vmap, so a checkpoint's "params"
(train_modal.py:402-407) holds each layer leaf stacked along a leading
n_layers axis; decode.params_from_reference unstacks it into the decoder's
list of per-layer dicts (bf16 tensors), and FP8Decoder takes either layout.
The caller loads the checkpoint; nothing here unpickles anything.  Leaves
that are 2-byte bfloat16 numpy arrays (ml_dtypes, which jax brings) are
viewed bit for bit; ml_dtypes is not installed in this image, so that branch
is exercised only through the float32 and torch leaves below.
"""
import numpy as np
import pytest
import torch

import decode

CFG = decode.Config(vocab_size=256, seq_len=64, d_model=128, n_layers=3, n_heads=2, head_dim=128, d_ff=256)


def _stacked_numpy_tree(cfg, seed=0):
    """The reference's layout (model.py:19-54) with float32 numpy leaves."""
    rng = np.random.default_rng(seed)
    L, d, h, f = cfg.n_layers, cfg.d_model, cfg.n_heads * cfg.head_dim, cfg.d_ff
    n = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)
    layers = {"norm1": np.ones((L, d), np.float32) + n(L, d), "wq": n(L, d, h), "wk": n(L, d, h),
              "wv": n(L, d, h), "wo": n(L, h, d), "norm2": np.ones((L, d), np.float32) + n(L, d),
              "w_up": n(L, d, f), "w_down": n(L, f, d)}
    return {"embed": n(cfg.vocab_size, d), "pos": n(cfg.seq_len, d), "layers": layers,
            "final_norm": np.ones(d, np.float32), "unembed": n(d, cfg.vocab_size)}


def _bf16(a):
    return torch.from_numpy(a).to(torch.bfloat16)


def test_stacked_numpy_tree_unstacks_and_rounds_to_bf16():
    tree = _stacked_numpy_tree(CFG)
    p = decode.params_from_reference(tree, "cpu")
    assert len(p["layers"]) == CFG.n_layers
    for i, lp in enumerate(p["layers"]):
        for k in decode._LAYER_KEYS:
            assert lp[k].dtype == torch.bfloat16
            assert torch.equal(lp[k], _bf16(tree["layers"][k][i])), (i, k)
    for k in ("embed", "pos", "final_norm", "unembed"):
        assert torch.equal(p[k], _bf16(tree[k]))


def test_stacked_torch_tree_and_list_layout_give_the_same_params():
    tree = _stacked_numpy_tree(CFG, seed=1)
    as_torch = {k: (_bf16(v) if k != "layers" else {n: _bf16(a) for n, a in v.items()}) for k, v in tree.items()}
    a = decode.params_from_reference(as_torch, "cpu")
    b = decode.params_from_reference(tree, "cpu")
    listed = dict(b, layers=[dict(lp) for lp in b["layers"]])
    c = decode.params_from_reference(listed, "cpu")                 # a list is taken as it is
    for x, y in ((a, b), (b, c)):
        for lx, ly in zip(x["layers"], y["layers"]):
            assert all(torch.equal(lx[k], ly[k]) for k in decode._LAYER_KEYS)


def test_tied_embeddings_tree_has_no_unembed():
    tree = _stacked_numpy_tree(CFG)
    del tree["unembed"]
    assert "unembed" not in decode.params_from_reference(tree, "cpu")


def test_bad_trees_are_refused():
    tree = _stacked_numpy_tree(CFG)
    broken = dict(tree, layers={k: v for k, v in tree["layers"].items() if k != "wo"})
    with pytest.raises(KeyError, match="wo"):
        decode.params_from_reference(broken, "cpu")
    ragged = dict(tree, layers=dict(tree["layers"], w_up=tree["layers"]["w_up"][:2]))
    with pytest.raises(ValueError, match="w_up"):
        decode.params_from_reference(ragged, "cpu")
    ints = dict(tree, pos=np.zeros((CFG.seq_len, CFG.d_model), np.int32))
    with pytest.raises(TypeError, match="int32"):
        decode.params_from_reference(ints, "cpu")


def test_config_from_reference_fields():
    """config.py:6-27's fields; dtype / use_remat / use_pallas_norm are dropped."""
    ref = {"vocab_size": 256, "seq_len": 64, "d_model": 128, "n_layers": 3, "n_heads": 2, "head_dim": 128,
           "d_ff": 256, "dtype": "bfloat16", "init_std": 0.02, "rms_eps": 1e-5, "tie_embeddings": False,
           "logit_cap": 15.0, "use_remat": True, "use_pallas_norm": True}
    assert decode.config_from_reference(ref) == CFG

    class Obj:
        pass
    o = Obj()
    for k, v in ref.items():
        setattr(o, k, v)
    assert decode.config_from_reference(o) == CFG


@pytest.mark.gpu
def test_decoder_from_stacked_tree_matches_list_params(dev):
    """FP8Decoder on the reference's stacked numpy tree = on the unstacked bf16
    tensors: same kept weights, same logits bit for bit (prefill and steps)."""
    tree = _stacked_numpy_tree(CFG, seed=2)
    a = decode.FP8Decoder(tree, CFG)
    b = decode.FP8Decoder(decode.params_from_reference(tree, dev), CFG)
    ids = torch.randint(0, CFG.vocab_size, (1, 16), device=dev, generator=torch.Generator(device=dev).manual_seed(0))
    la, lb = a.prefill(ids), b.prefill(ids)
    assert torch.equal(la, lb)
    tok = la[:, -1].argmax(-1) if la.dim() == 3 else la.argmax(-1)
    for _ in range(4):
        sa, sb = a.step(tok), b.step(tok)
        assert torch.equal(sa, sb)
        tok = sa.argmax(-1)
