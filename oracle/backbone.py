"""Backbone of the memory-pool LM restated in numpy.  TEST INFRASTRUCTURE ONLY.

Follows KumarDev7/model ``memory_pool_model/model.py:29-127`` with
``train=False`` (no dropout, no routing noise):
  * token + position embedding                        model.py:52-64
  * per layer: LayerNorm, causal multi-head attention  model.py:87-95
    (Flax MultiHeadDotProductAttention: DenseGeneral q/k/v kernels
    [d, heads, hd], queries divided by sqrt(hd), softmax over the keys,
    DenseGeneral out kernel [heads, hd, d])
  * LayerNorm, FFN (tanh-approximate gelu) unless the layer is a memory
    layer without memory_ffn                            model.py:97-102
  * memory layers: router Dense -> [B, T, H, d_key] queries, the pool read
    (oracle.lookup.lookup_forward, memory.py:132-193), silu gate, mem_out
    Dense                                               model.py:104-120
  * final LayerNorm and the tied output embedding      model.py:124-126
Flax LayerNorm's epsilon is 1e-6.  Parameters are the Flax tree with numpy
leaves (``params["attn_0"]["query"]["kernel"]`` ...).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
use this module, and only to check results.
"""

from __future__ import annotations

import numpy as np

from . import lookup as ol

LN_EPS = 1e-6


def layer_norm(x, p, eps: float = LN_EPS):
    """flax.linen.LayerNorm: (x - mean) / sqrt(var + eps) * scale + bias."""
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * p["scale"] + p["bias"]


def gelu_tanh(x):
    """flax.linen.gelu (approximate=True)."""
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def silu(x):
    return x / (1.0 + np.exp(-x))


def dense(x, p):
    return x @ p["kernel"] + p["bias"]


def attention(p, h):
    """Causal self-attention of nn.MultiHeadDotProductAttention(h, h,
    mask=make_causal_mask) (model.py:88-94)."""
    q = np.einsum("btd,dnh->btnh", h, p["query"]["kernel"]) + p["query"]["bias"]
    k = np.einsum("btd,dnh->btnh", h, p["key"]["kernel"]) + p["key"]["bias"]
    v = np.einsum("btd,dnh->btnh", h, p["value"]["kernel"]) + p["value"]["bias"]
    q = q / np.sqrt(q.shape[-1])
    logits = np.einsum("bqnh,bknh->bnqk", q, k)
    T = h.shape[1]
    causal = np.tril(np.ones((T, T), dtype=bool))
    logits = np.where(causal, logits, np.finfo(logits.dtype).min)
    w = ol.softmax(logits, axis=-1)
    o = np.einsum("bnqk,bknh->bqnh", w, v)
    return np.einsum("bqnh,nhd->bqd", o, p["out"]["kernel"]) + p["out"]["bias"]


def forward(params, tokens, cfg, *, dtype=np.float64, pool_off: bool = False, shuffle_pool: bool = False):
    """model.py:29-127 (train=False).  ``cfg`` needs the ModelConfig fields
    n_layers, memory_layers, memory_ffn, use_memory, pool_heads, d_key,
    top_k, min_temperature, max_temperature, router_query_scale.  Returns
    (logits [B, T, vocab], the router queries of each memory layer
    [B*T, H, d_key] in read order)."""
    p = {k: v for k, v in params.items()}
    cast = lambda t: np.asarray(t, dtype=dtype)  # noqa: E731
    tokens = np.asarray(tokens)
    B, T = tokens.shape
    emb = cast(p["embed"]["embedding"])
    x = emb[tokens] + cast(p["pos_embed"])[None, :T]
    pool = p.get("pool")
    queries = []
    tree = lambda d: {k: (tree(v) if isinstance(v, dict) else cast(v)) for k, v in d.items()}  # noqa: E731
    for i in range(cfg.n_layers):
        h = layer_norm(x, tree(p[f"ln_attn_{i}"]))
        x = x + attention(tree(p[f"attn_{i}"]), h)
        h = layer_norm(x, tree(p[f"ln_ffn_{i}"]))
        mem_layer = cfg.use_memory and i in cfg.memory_layers
        y = np.zeros_like(x)
        if not mem_layer or cfg.memory_ffn:
            y = dense(gelu_tanh(dense(h, tree(p[f"ffn_in_{i}"]))), tree(p[f"ffn_out_{i}"]))
        if mem_layer and not pool_off:
            q = dense(h, tree(p[f"router_{i}"])).reshape(B * T, cfg.pool_heads, cfg.d_key)
            queries.append(q)
            r = ol.lookup_forward(q, cast(pool["sub_keys"]), np.asarray(pool["values"]),
                                  float(np.asarray(pool["log_temperature"])), top_k_=cfg.top_k,
                                  min_temperature=cfg.min_temperature, max_temperature=cfg.max_temperature,
                                  query_scale=cfg.router_query_scale, shuffle_reads=shuffle_pool, dtype=dtype,
                                  with_dense=False)
            mem = r["out"].reshape(B, T, -1)
            gate = silu(dense(h, tree(p[f"mem_gate_{i}"])))
            y = y + dense(mem * gate, tree(p[f"mem_out_{i}"]))
        x = x + y
    x = layer_norm(x, tree(p["ln_final"]))
    return x @ emb.T, queries
