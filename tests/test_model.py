"""The backbone mirror (model_amd/model.py, model.py:15-145 of the
reference) on the CPU with the pool switched off (use_memory=False): the
KV-cache decode path reproduces the full causal forward (tests:486-502 for
the backbone part), and the parameter tree has the Flax names and shapes."""

import numpy as np
import torch

from model_amd.model import MemoryPoolLM, ModelConfig


def _cfg(**kw):
    base = dict(vocab_size=50, max_len=16, d_model=32, n_heads=2, n_layers=2, ffn_mult=2, use_memory=False)
    base.update(kw)
    return ModelConfig(**base)


def test_decode_matches_full_forward_without_pool():
    cfg = _cfg()
    full_m = MemoryPoolLM(cfg)
    params = full_m.init(1, device="cpu")
    toks = torch.tensor(np.random.default_rng(0).integers(0, 50, (2, 12)))
    full, _ = full_m.apply(params, toks)
    dec = MemoryPoolLM(cfg, decode=True)
    cache = dec.init_cache(2, device="cpu")
    steps = []
    for t in range(12):
        lg, _ = dec.apply(params, toks[:, t:t + 1], positions=torch.tensor([t]), cache=cache)
        steps.append(lg[:, 0])
    np.testing.assert_allclose(torch.stack(steps, 1).numpy(), full.numpy(), atol=1e-5)


def test_parameter_tree_has_flax_names():
    cfg = _cfg(use_memory=False, n_layers=1)
    p = MemoryPoolLM(cfg).init(0, device="cpu")["params"]
    assert p["attn_0"]["query"]["kernel"].shape == (32, 2, 16)
    assert p["attn_0"]["out"]["kernel"].shape == (2, 16, 32)
    assert p["ffn_in_0"]["kernel"].shape == (32, 64) and p["ffn_out_0"]["bias"].shape == (32,)
    assert set(p) == {"embed", "pos_embed", "ln_attn_0", "attn_0", "ln_ffn_0", "ffn_in_0", "ffn_out_0", "ln_final"}


def test_dropout_only_in_training():
    """model.py:91 (attention weights) and :122 (residual branch) with
    train=True; no effect with train=False; reproducible from rngs."""
    cfg = _cfg(dropout=0.3)
    m = MemoryPoolLM(cfg)
    params = m.init(2, device="cpu")
    toks = torch.tensor(np.random.default_rng(5).integers(0, 50, (2, 10)))
    ref, _ = MemoryPoolLM(_cfg(dropout=0.0)).apply(params, toks)
    ev, _ = m.apply(params, toks)
    assert torch.equal(ev, ref)
    a, _ = m.apply(params, toks, train=True, rngs={"dropout": 7})
    b, _ = m.apply(params, toks, train=True, rngs={"dropout": 7})
    c, _ = m.apply(params, toks, train=True, rngs={"dropout": 8})
    assert torch.equal(a, b) and not torch.equal(a, c) and not torch.equal(a, ref)


def test_dropout_mask_statistics():
    from model_amd.model import _make_dropout

    drop = _make_dropout(0.25, {"dropout": 3}, torch.device("cpu"))
    y = drop(torch.ones(200000))
    kept = y != 0
    assert abs(kept.float().mean().item() - 0.75) < 0.005
    assert torch.allclose(y[kept], torch.full_like(y[kept], 1 / 0.75))
    import pytest

    with pytest.raises(ValueError):
        _make_dropout(1.0, None, torch.device("cpu"))
