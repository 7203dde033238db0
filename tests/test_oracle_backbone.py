"""Pins of oracle/backbone.py (model.py:29-127 restated in numpy) on the
CPU, then the torch backbone mirror (model_amd/model.py) against it with the
pool switched off.

Pinned by: torch's own layer_norm, tanh-gelu and causal
scaled_dot_product_attention (library routines) for the pieces; a tiny
model whose logits are worked out by hand in closed form; the causality
invariant with memory layers on (logits at position t do not depend on
later tokens); and Flax's DenseGeneral layouts through a one-head case
where the kernels are identities."""

import math

import numpy as np
import torch
import torch.nn.functional as F

from model_amd.model import MemoryPoolLM, ModelConfig
from oracle import backbone as ob


def _np_tree(t):
    if isinstance(t, dict):
        return {k: _np_tree(v) for k, v in t.items()}
    return t.detach().float().cpu().numpy() if isinstance(t, torch.Tensor) else t


def test_pieces_match_torch_routines():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 5, 16))
    p = {"scale": rng.standard_normal(16), "bias": rng.standard_normal(16)}
    want = F.layer_norm(torch.tensor(x), (16,), torch.tensor(p["scale"]), torch.tensor(p["bias"]), eps=1e-6)
    np.testing.assert_allclose(ob.layer_norm(x, p), want.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ob.gelu_tanh(x), F.gelu(torch.tensor(x), approximate="tanh").numpy(), rtol=1e-12,
                               atol=1e-14)
    assert abs(ob.gelu_tanh(np.array(1.0)) - 0.8411919906082768) < 1e-15
    np.testing.assert_allclose(ob.silu(x), F.silu(torch.tensor(x)).numpy(), rtol=1e-12)
    # attention: projections by a reshaped matmul, then torch's causal SDPA
    B, T, d, n = 2, 7, 12, 3
    hd = d // n
    h = rng.standard_normal((B, T, d))
    att = {nm: {"kernel": rng.standard_normal((d, n, hd)), "bias": rng.standard_normal((n, hd))}
           for nm in ("query", "key", "value")}
    att["out"] = {"kernel": rng.standard_normal((n, hd, d)), "bias": rng.standard_normal(d)}
    ht = torch.tensor(h)

    def proj(nm):
        w = torch.tensor(att[nm]["kernel"]).reshape(d, n * hd)
        return (ht @ w + torch.tensor(att[nm]["bias"]).reshape(-1)).reshape(B, T, n, hd).transpose(1, 2)

    o = F.scaled_dot_product_attention(proj("query"), proj("key"), proj("value"), is_causal=True)
    o = o.transpose(1, 2).reshape(B, T, n * hd) @ torch.tensor(att["out"]["kernel"]).reshape(n * hd, d)
    o = o + torch.tensor(att["out"]["bias"])
    np.testing.assert_allclose(ob.attention(att, h), o.numpy(), rtol=1e-10, atol=1e-10)


def test_hand_computed_tiny_model():
    """vocab 2, d_model 2, one head, one layer, no pool; tokens [0, 1].
    Embedding = identity, positions 0, LayerNorms unit/zero, q/k/v/out
    kernels identity, FFN kernels zero with ffn_out bias (0.5, 0).  Then
    LN([1, 0]) = (c, -c) with c = 0.5 / sqrt(0.25 + 1e-6); position 0
    attends to itself; position 1 weighs positions 0 and 1 by a softmax of
    (-2c^2, 2c^2) / sqrt(2), so its output is tanh(sqrt(2) c^2) (-c, c)."""
    eye = np.eye(2)
    unit = {"scale": np.ones(2), "bias": np.zeros(2)}
    params = {
        "embed": {"embedding": eye}, "pos_embed": np.zeros((2, 2)),
        "ln_attn_0": unit, "ln_ffn_0": unit, "ln_final": unit,
        "attn_0": {nm: {"kernel": eye.reshape(2, 1, 2), "bias": np.zeros((1, 2))} for nm in ("query", "key", "value")},
        "ffn_in_0": {"kernel": np.zeros((2, 2)), "bias": np.zeros(2)},
        "ffn_out_0": {"kernel": np.zeros((2, 2)), "bias": np.array([0.5, 0.0])},
    }
    params["attn_0"]["out"] = {"kernel": eye.reshape(1, 2, 2), "bias": np.zeros(2)}
    cfg = ModelConfig(vocab_size=2, max_len=2, d_model=2, n_layers=1, n_heads=1, ffn_mult=1, use_memory=False)
    logits, _ = ob.forward(params, np.array([[0, 1]]), cfg)
    c = 0.5 / math.sqrt(0.25 + 1e-6)
    t = math.tanh(math.sqrt(2.0) * c * c)
    x = [np.array([1.0 + c + 0.5, 0.0 - c]), np.array([0.0 - t * c + 0.5, 1.0 + t * c])]
    want = []
    for v in x:
        half = (v[0] - v[1]) / 2.0
        s = half / math.sqrt(half * half + 1e-6)
        want.append([s, -s])
    np.testing.assert_allclose(logits[0], np.array(want), rtol=1e-12)


def _pool_cfg(**kw):
    base = dict(vocab_size=40, max_len=12, d_model=32, n_heads=2, n_layers=3, ffn_mult=2, memory_layers=(1, 2),
                n_sub_keys=8, pool_heads=2, d_key=16, d_value=24, top_k=4, values_dtype=torch.float32)
    base.update(kw)
    return ModelConfig(**base)


def test_causality_with_memory_layers():
    cfg = _pool_cfg()
    rng = np.random.default_rng(1)
    params = _np_tree(_cpu_params(cfg, 2))
    a = rng.integers(0, 40, (2, 10))
    b = a.copy()
    b[:, 6:] = rng.integers(0, 40, (2, 4))
    la, _ = ob.forward(params, a, cfg)
    lb, _ = ob.forward(params, b, cfg)
    np.testing.assert_array_equal(la[:, :6], lb[:, :6])
    assert not np.allclose(la[:, 6:], lb[:, 6:])


def _cpu_params(cfg, seed):
    """A parameter tree of the mirror's layout drawn on the CPU (the pool's
    init needs no GPU), values in fp32."""
    m = MemoryPoolLM(ModelConfig(**{**cfg.__dict__, "use_memory": False}))
    p = m.init(seed, device="cpu")["params"]
    g = torch.Generator().manual_seed(seed + 7)
    d = cfg.d_model
    for i in cfg.memory_layers:
        p[f"router_{i}"] = {"kernel": torch.randn((d, cfg.pool_heads * cfg.d_key), generator=g) * d ** -0.5,
                            "bias": torch.zeros(cfg.pool_heads * cfg.d_key)}
        p[f"mem_gate_{i}"] = {"kernel": torch.randn((d, cfg.d_value), generator=g) * d ** -0.5,
                              "bias": torch.zeros(cfg.d_value)}
        p[f"mem_out_{i}"] = {"kernel": torch.randn((cfg.d_value, d), generator=g) * cfg.d_value ** -0.5,
                             "bias": torch.zeros(d)}
        if not cfg.memory_ffn:
            p.pop(f"ffn_in_{i}", None)
            p.pop(f"ffn_out_{i}", None)
    keys = torch.randn((cfg.pool_heads, 2, cfg.n_sub_keys, cfg.d_key // 2), generator=g)
    p["pool"] = {"sub_keys": keys / keys.norm(dim=-1, keepdim=True),
                 "values": torch.randn((cfg.n_sub_keys ** 2, cfg.d_value), generator=g) * cfg.d_value ** -0.5,
                 "log_temperature": torch.tensor(math.log(cfg.init_temperature))}
    return p


def test_mirror_without_pool_matches_oracle():
    """The torch backbone (product code) and the numpy oracle, pool off."""
    cfg = ModelConfig(vocab_size=50, max_len=16, d_model=32, n_heads=4, n_layers=2, ffn_mult=2, use_memory=False)
    m = MemoryPoolLM(cfg)
    params = m.init(3, device="cpu")
    toks = torch.tensor(np.random.default_rng(4).integers(0, 50, (3, 11)))
    got, _ = m.apply(params, toks)
    want, _ = ob.forward(_np_tree(params["params"]), toks.numpy(), cfg)
    np.testing.assert_allclose(got.double().numpy(), want, rtol=1e-4, atol=2e-5)
