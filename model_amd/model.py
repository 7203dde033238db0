"""Host mirror of the reference backbone (memory_pool_model/model.py:15-145,
config.py:9-61) around this library's MemoryPool.

The backbone (embedding, attention, layer norms, feed-forward blocks, router
and gated memory write-back) is small dense work and runs as plain torch ops
in fp32; every memory read is MemoryPool (libmpl.so).  Parameter names and
shapes follow the Flax modules, so a checkpoint of the reference
(model_amd/checkpoint.py) loads into it:

  embed/embedding [vocab, d]            nn.Embed (logits use embed.attend)
  pos_embed [max_len, d]
  ln_attn_i, ln_ffn_i, ln_final         nn.LayerNorm {scale, bias}, eps 1e-6
  attn_i/{query,key,value}              DenseGeneral {kernel [d, heads, hd], bias [heads, hd]}
  attn_i/out                            DenseGeneral {kernel [heads, hd, d], bias [d]}
  ffn_in_i, ffn_out_i, router_i,        nn.Dense {kernel [in, out], bias [out]}
  mem_gate_i, mem_out_i
  pool/{sub_keys, values, log_temperature}

With ``decode=True`` the attention keeps a key/value cache of max_len
positions per layer (Flax's decode mode): one token per call at a position
given as a device tensor, so a decode step has static shapes and can be
captured in a HIP graph (model_amd/generate.py).  On the GPU a decode step
is libmpl.so launches: the attention of the new token (cache write, scores,
softmax, weighted values; mpl_decode_attention) and every dense layer with
the layer norm before it and its activation and residual add after it
(mpl_rows_linear), on a fused query/key/value projection whose weights are
concatenated once per parameter version, not on every step.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Any, Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from .memory import MemoryPool

LN_EPS = 1e-6  # flax.linen.LayerNorm default


@dataclasses.dataclass(frozen=True)
class ModelConfig:
    """config.py:9-61 (the fields the forward pass reads)."""

    vocab_size: int = 256
    max_len: int = 128
    d_model: int = 128
    n_layers: int = 2
    n_heads: int = 4
    ffn_mult: int = 1
    dropout: float = 0.0
    use_memory: bool = True
    memory_layers: Tuple[int, ...] = (1,)
    memory_ffn: bool = False
    n_sub_keys: int = 64
    pool_heads: int = 4
    d_key: int = 64
    d_value: int = 128
    top_k: int = 16
    routing_noise: float = 1.0
    init_temperature: float = 10.0
    min_temperature: float = 10.0
    balance_temperature_grad: bool = False
    max_temperature: float = 100.0
    router_query_scale: bool = False
    host_pool: str = ""  # config.py:33: name of a HostPool (model_amd/host_pool.py) holding the table
    values_dtype: torch.dtype = torch.float16  # the pool table in HBM (fp32 in the reference)

    @property
    def pool_size(self) -> int:
        return self.n_sub_keys ** 2


def _dense(x, p):
    return torch.matmul(x, p["kernel"]) + p["bias"]


_ACT = {None: 0, "gelu_tanh": 1, "silu": 2}


def decode_embed(emb: torch.Tensor, pos_emb: torch.Tensor, tokens: torch.Tensor,
                 position: torch.Tensor) -> torch.Tensor:
    """mpl_decode_embed: emb[tokens] + pos_emb[position] for one token per
    stream (tokens int64 [B], position a device int64 tensor [1]), in one
    launch; the same bits as the two indexings and the add.  An id outside
    its table gives a NaN row."""
    from . import _lib

    for t in (emb, pos_emb):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.dim() != 2 or t.device != tokens.device:
            raise ValueError("decode_embed: tables must be contiguous 2-d fp32 on the tokens' device")
    tok = tokens.reshape(-1)
    if tok.dtype != torch.int64 or not tok.is_contiguous() or position.dtype != torch.int64:
        raise ValueError("decode_embed: tokens and position must be contiguous int64")
    if tokens.device.type != "cuda":
        raise ValueError("decode_embed runs on the GPU only (libmpl.so)")
    B, d = tok.numel(), emb.shape[1]
    if pos_emb.shape[1] != d:
        raise ValueError(f"decode_embed: widths {d} and {pos_emb.shape[1]} differ")
    out = torch.empty((B, d), dtype=torch.float32, device=tokens.device)
    P = _lib.ptr
    _lib.check(_lib.lib().mpl_decode_embed(P(emb), emb.shape[0], P(pos_emb), pos_emb.shape[0], d, P(tok),
                                           P(position), B, P(out), _lib.stream_ptr(tokens.device)),
               "mpl_decode_embed")
    return out


def rows_linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None, *,
                out_in: bool = False, ln: Optional[Dict[str, torch.Tensor]] = None, eps: float = LN_EPS,
                x_mul: Optional[torch.Tensor] = None, act: Optional[str] = None,
                residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """mpl_rows_linear: act((LayerNorm(x) if ln else x) * x_mul . W + bias)
    + residual for x [rows, K] fp32 on the GPU.  W is a Dense kernel [K, N]
    (any [K, ...] shape, flattened) or, with out_in, a table [N, K] (the
    embedding of embed.attend)."""
    from . import _lib

    rows, K = x.shape
    W = weight.reshape(-1, K) if out_in else weight.reshape(K, -1)
    N = W.shape[0] if out_in else W.shape[1]
    ts = [x, W] + [t for t in (bias, x_mul, residual) if t is not None]
    if ln is not None:
        ts += [ln["scale"], ln["bias"]]
    for t in ts:
        if t.dtype != torch.float32 or not t.is_contiguous() or t.device != x.device:
            raise ValueError("rows_linear: operands must be contiguous fp32 on one device")
    if x.device.type != "cuda":
        raise ValueError("rows_linear runs on the GPU only (libmpl.so)")
    if ((bias is not None and bias.numel() != N) or (x_mul is not None and x_mul.shape != x.shape)
            or (residual is not None and residual.shape != (rows, N))
            or (ln is not None and (ln["scale"].numel() != K or ln["bias"].numel() != K))):
        raise ValueError(f"rows_linear: operand shapes do not fit x {tuple(x.shape)} and W {tuple(W.shape)}")
    out = torch.empty((rows, N), dtype=torch.float32, device=x.device)
    P = _lib.ptr
    _lib.check(_lib.lib().mpl_rows_linear(
        P(x), P(x_mul), P(None if ln is None else ln["scale"]), P(None if ln is None else ln["bias"]), float(eps),
        P(W), _lib.MPL_W_OUT_IN if out_in else _lib.MPL_W_IN_OUT, P(bias), _ACT[act], P(residual), rows, K, N,
        P(out), _lib.stream_ptr(x.device)), "mpl_rows_linear")
    return out


def rows_linear_pair(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], n1: int, *,
                     ln: Optional[Dict[str, torch.Tensor]] = None, eps: float = LN_EPS, act1: Optional[str] = None,
                     act2: Optional[str] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """mpl_rows_linear_pair: two Dense layers of the same (LayerNorm(x) if
    ln else x) rows as one launch, weight [K, n1 + n2] their kernels side by
    side and bias [n1 + n2]; returns (act1(. W[:, :n1] + b[:n1]),
    act2(. W[:, n1:] + b[n1:])), each equal to rows_linear of its layer."""
    from . import _lib

    rows, K = x.shape
    W = weight.reshape(K, -1)
    N = W.shape[1]
    n2 = N - n1
    ts = [x, W] + ([bias] if bias is not None else [])
    if ln is not None:
        ts += [ln["scale"], ln["bias"]]
    for t in ts:
        if t.dtype != torch.float32 or not t.is_contiguous() or t.device != x.device:
            raise ValueError("rows_linear_pair: operands must be contiguous fp32 on one device")
    if x.device.type != "cuda":
        raise ValueError("rows_linear_pair runs on the GPU only (libmpl.so)")
    if (not 0 < n1 < N or (bias is not None and bias.numel() != N)
            or (ln is not None and (ln["scale"].numel() != K or ln["bias"].numel() != K))):
        raise ValueError(f"rows_linear_pair: operand shapes do not fit x {tuple(x.shape)}, W {tuple(W.shape)}, "
                         f"n1 {n1}")
    out1 = torch.empty((rows, n1), dtype=torch.float32, device=x.device)
    out2 = torch.empty((rows, n2), dtype=torch.float32, device=x.device)
    P = _lib.ptr
    _lib.check(_lib.lib().mpl_rows_linear_pair(
        P(x), P(None if ln is None else ln["scale"]), P(None if ln is None else ln["bias"]), float(eps), P(W),
        P(bias), _ACT[act1], _ACT[act2], rows, K, n1, n2, P(out1), P(out2), _lib.stream_ptr(x.device)),
        "mpl_rows_linear_pair")
    return out1, out2


def decode_attention(qkv: torch.Tensor, positions: torch.Tensor, layer_cache: Dict[str, torch.Tensor], heads: int,
                     scale: float) -> torch.Tensor:
    """mpl_decode_attention: qkv [B, 3 * heads * hd] fp32 (query, key and
    value of the new token, biases added) -> [B, heads * hd]; writes the key
    and value into layer_cache ("kt" [B, heads, hd, max_len], "v" [B, heads,
    max_len, hd]) at positions[0] first."""
    from . import _lib

    kt, v = layer_cache["kt"], layer_cache["v"]
    B, H, hd, L = kt.shape
    if (H != heads or qkv.shape != (B, 3 * H * hd) or v.shape != (B, H, L, hd) or positions.numel() != 1
            or positions.dtype != torch.int64):
        raise ValueError(f"decode_attention: qkv {tuple(qkv.shape)}, kt {tuple(kt.shape)}, v {tuple(v.shape)}, "
                         f"positions {tuple(positions.shape)} {positions.dtype} do not fit together")
    for t in (qkv, kt, v):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.device != qkv.device:
            raise ValueError("decode_attention: qkv and caches must be contiguous fp32 on one device")
    if qkv.device.type != "cuda" or positions.device != qkv.device:
        raise ValueError("decode_attention: qkv, caches and positions must be on the same GPU")
    out = torch.empty((B, H * hd), dtype=torch.float32, device=qkv.device)
    _lib.check(_lib.lib().mpl_decode_attention(qkv.data_ptr(), B, H, hd, L, positions.data_ptr(), kt.data_ptr(),
                                               v.data_ptr(), out.data_ptr(), float(scale),
                                               _lib.stream_ptr(qkv.device)), "mpl_decode_attention")
    return out


def vocab_logits(x: torch.Tensor, ln_scale: torch.Tensor, ln_bias: torch.Tensor, emb: torch.Tensor) -> torch.Tensor:
    """mpl_vocab_logits: LayerNorm(x) . emb^T (model.py:125-126, ln_final then
    embed.attend) for at most 64 rows of d <= 256 (d % 4 == 0), one launch."""
    from . import _lib

    rows, d = x.shape
    V = emb.shape[0]
    out = torch.empty((rows, V), dtype=torch.float32, device=x.device)
    P = lambda t: t.data_ptr()
    _lib.check(_lib.lib().mpl_vocab_logits(P(x), P(ln_scale.contiguous()), P(ln_bias.contiguous()), LN_EPS, P(emb),
                                           rows, d, V, P(out), _lib.stream_ptr(x.device)), "mpl_vocab_logits")
    return out


def _ln(x, p):
    return F.layer_norm(x, (x.shape[-1],), p["scale"], p["bias"], LN_EPS)


def merge_layer_aux(layer_aux: List[Dict[str, Any]]) -> Dict[str, Any]:
    """model.py:130-145."""
    if not layer_aux:
        return {}
    return {
        "balance_loss": torch.stack([a["balance_loss"] for a in layer_aux]).mean(),
        "subkey_counts": sum(a["subkey_counts"] for a in layer_aux),
        "slot_counts": sum(a["slot_counts"] for a in layer_aux),
        "queries": [a["queries"] for a in layer_aux],
        "slots": [a["slots"] for a in layer_aux],
        "weights": [a["weights"] for a in layer_aux],
        "temperature": layer_aux[0]["temperature"],
        "top1_weight": torch.stack([a["top1_weight"] for a in layer_aux]).mean(),
    }


class _LazyMerged(dict):
    """merge_layer_aux computed on first access (decode never reads it)."""

    def __init__(self, layer_aux):
        super().__init__()
        self._layer_aux = layer_aux

    def _fill(self):
        if self._layer_aux is not None:
            self.update(merge_layer_aux(self._layer_aux))
            self._layer_aux = None

    def __getitem__(self, key):
        self._fill()
        return dict.__getitem__(self, key)

    def __contains__(self, key):
        self._fill()
        return dict.__contains__(self, key)

    def keys(self):
        self._fill()
        return dict.keys(self)


def _make_dropout(rate: float, rngs, device):
    """Inverted dropout at ``rate`` (model.py:91, 122 with train=True): keeps
    each element with probability 1 - rate and scales the kept ones by
    1 / (1 - rate).  ``rngs["dropout"]`` (an int seed or a torch.Generator
    on the device) draws the masks; otherwise torch's default generator.
    The mask stream differs from Flax's."""
    if not 0.0 <= rate < 1.0:
        raise ValueError(f"dropout rate must be in [0, 1), got {rate}")
    r = None if rngs is None else rngs.get("dropout")
    gen = None
    if isinstance(r, torch.Generator):
        gen = r
    elif r is not None:
        gen = torch.Generator(device=device).manual_seed(int(r))
    keep = 1.0 - rate

    def drop(t: torch.Tensor) -> torch.Tensor:
        mask = torch.rand(t.shape, generator=gen, device=t.device, dtype=t.dtype) < keep
        return t * mask * (1.0 / keep)

    return drop


class MemoryPoolLM:
    """model.py:15-127."""

    def __init__(self, cfg: ModelConfig, decode: bool = False):
        self.cfg, self.decode = cfg, decode
        self._qkv_cache: Dict[int, Tuple[tuple, torch.Tensor, torch.Tensor]] = {}
        self._rg_cache: Dict[int, Tuple[tuple, torch.Tensor, torch.Tensor]] = {}
        self.pool = None
        if cfg.use_memory:
            self.pool = MemoryPool(cfg.n_sub_keys, cfg.pool_heads, cfg.d_key, cfg.d_value, cfg.top_k,
                                   routing_noise=cfg.routing_noise, init_temperature=cfg.init_temperature,
                                   min_temperature=cfg.min_temperature,
                                   balance_temperature_grad=cfg.balance_temperature_grad,
                                   max_temperature=cfg.max_temperature, query_scale=cfg.router_query_scale,
                                   host_pool=cfg.host_pool, values_dtype=cfg.values_dtype)

    # ------------------------------------------------------------ params
    def init(self, seed: int = 0, device="cuda", pool_values: Optional[torch.Tensor] = None) -> Dict[str, Any]:
        """Random parameters with Flax's default initialisers in spirit
        (lecun-normal kernels, zero biases, unit layer-norm scales);
        ``pool_values`` supplies the value table instead of a fresh draw."""
        cfg = self.cfg
        g = torch.Generator(device=device).manual_seed(int(seed))
        d, hd = cfg.d_model, cfg.d_model // cfg.n_heads

        def normal(shape, std):
            return torch.randn(shape, generator=g, device=device) * std

        def dense(i, o):
            return {"kernel": normal((i, o), i ** -0.5), "bias": torch.zeros(o, device=device)}

        def ln():
            return {"scale": torch.ones(d, device=device), "bias": torch.zeros(d, device=device)}

        p: Dict[str, Any] = {"embed": {"embedding": normal((cfg.vocab_size, d), d ** -0.5)},
                             "pos_embed": normal((cfg.max_len, d), 0.02)}
        for i in range(cfg.n_layers):
            p[f"ln_attn_{i}"] = ln()
            att = {nm: {"kernel": normal((d, cfg.n_heads, hd), d ** -0.5),
                        "bias": torch.zeros((cfg.n_heads, hd), device=device)} for nm in ("query", "key", "value")}
            att["out"] = {"kernel": normal((cfg.n_heads, hd, d), d ** -0.5), "bias": torch.zeros(d, device=device)}
            p[f"attn_{i}"] = att
            p[f"ln_ffn_{i}"] = ln()
            mem = self.pool is not None and i in cfg.memory_layers
            if not mem or cfg.memory_ffn:
                p[f"ffn_in_{i}"] = dense(d, d * cfg.ffn_mult)
                p[f"ffn_out_{i}"] = dense(d * cfg.ffn_mult, d)
            if mem:
                p[f"router_{i}"] = dense(d, cfg.pool_heads * cfg.d_key)
                p[f"mem_gate_{i}"] = dense(d, cfg.d_value)
                p[f"mem_out_{i}"] = dense(cfg.d_value, d)
        p["ln_final"] = ln()
        if self.pool is not None:
            p["pool"] = self.pool.init(int(seed) + 1, device=device, values=pool_values)["params"]
        return {"params": p}

    def init_cache(self, batch_size: int, device="cuda") -> List[Dict[str, torch.Tensor]]:
        """Per layer the keys transposed, "kt" [B, heads, hd, max_len], and the
        values, "v" [B, heads, max_len, hd]: both products of a decode step
        then read their cache operand as stored, without a transposed copy of
        the whole cache."""
        cfg = self.cfg
        hd = cfg.d_model // cfg.n_heads
        return [{"kt": torch.zeros((batch_size, cfg.n_heads, hd, cfg.max_len), device=device),
                 "v": torch.zeros((batch_size, cfg.n_heads, cfg.max_len, hd), device=device)}
                for _ in range(cfg.n_layers)]

    # ----------------------------------------------------------- forward
    @staticmethod
    def _qkv_sources(pa) -> List[torch.Tensor]:
        return [pa[nm][part] for nm in ("query", "key", "value") for part in ("kernel", "bias")]

    def copied_parameters(self, p) -> List[torch.Tensor]:
        """The parameters a GPU decode step reads through copies made before
        a HIP-graph capture (the fused query/key/value weights, and the
        router and gate weights of the memory layers) rather than from their
        own storage: a captured step is stale once any of them changes in
        place."""
        if not self.decode:
            return []
        out = [t for i in range(self.cfg.n_layers) for t in self._qkv_sources(p[f"attn_{i}"])]
        if self.pool is not None:
            out += [t for i in self.cfg.memory_layers if i < self.cfg.n_layers
                    for t in self._router_gate_sources(p, i)]
        return out

    @staticmethod
    def _router_gate_sources(p, i: int) -> List[torch.Tensor]:
        return [p[nm][part] for nm in (f"router_{i}", f"mem_gate_{i}") for part in ("kernel", "bias")]

    def _fused_router_gate(self, p, i: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """[d, pool_heads * d_key + d_value] kernel and bias of memory layer
        i's router and gate side by side, rebuilt when one of them was
        replaced or changed in place (storage and version key)."""
        src = self._router_gate_sources(p, i)
        key = tuple((t.data_ptr(), t._version) for t in src)
        hit = self._rg_cache.get(i)
        if hit is not None and hit[0] == key:
            return hit[1], hit[2]
        d = self.cfg.d_model
        with torch.no_grad():
            w = torch.cat([src[0].reshape(d, -1), src[2].reshape(d, -1)], 1)
            b = torch.cat([src[1].reshape(-1), src[3].reshape(-1)])
        self._rg_cache[i] = (key, w, b)
        return w, b

    def _fused_qkv(self, i: int, pa) -> Tuple[torch.Tensor, torch.Tensor]:
        """[d, 3 * heads * hd] kernel and [3 * heads * hd] bias of layer i's
        three projections, rebuilt when one of them was replaced or changed
        in place (storage and version key)."""
        src = self._qkv_sources(pa)
        key = tuple((t.data_ptr(), t._version) for t in src)
        hit = self._qkv_cache.get(i)
        if hit is not None and hit[0] == key:
            return hit[1], hit[2]
        d = self.cfg.d_model
        with torch.no_grad():
            w = torch.cat([src[j].reshape(d, -1) for j in (0, 2, 4)], 1)
            b = torch.cat([src[j].reshape(-1) for j in (1, 3, 5)])
        self._qkv_cache[i] = (key, w, b)
        return w, b

    def _decode_step_gpu(self, p, tokens, positions, cache, noise_scale, rngs, input_rows=None):
        """One decode step on the GPU (inference: no autograd, no dropout):
        the computation of the general path of apply() for T = 1, with every
        dense layer of a block one mpl_rows_linear launch that also applies
        the layer norm before it, its activation and the residual add after
        it, and the attention one mpl_decode_attention launch per layer.  With
        memory_ffn the residual branch's two terms are added to x one after
        the other (x + ffn, then + mem_out)."""
        cfg = self.cfg
        B = tokens.shape[0]
        d, H = cfg.d_model, cfg.n_heads
        hd = d // H
        emb = p["embed"]["embedding"]
        layer_aux = []
        with torch.no_grad():
            pe = p["pos_embed"]
            if input_rows is not None:
                x = input_rows
            elif (emb.shape[1] % 4 == 0 and tokens.dtype == torch.int64 and positions.dtype == torch.int64
                    and all(t.dtype == torch.float32 and t.is_contiguous() and t.data_ptr() % 16 == 0
                            for t in (emb, pe))):
                x = decode_embed(emb, pe, tokens[:, 0].contiguous(), positions)  # [B, d], one launch
            else:
                x = emb[tokens[:, 0]] + pe[positions]
            for i in range(cfg.n_layers):
                pa = p[f"attn_{i}"]
                w, b = self._fused_qkv(i, pa)
                qkv = rows_linear(x, w, b, ln=p[f"ln_attn_{i}"])
                a = decode_attention(qkv, positions, cache[i], H, hd ** -0.5)
                x = rows_linear(a, pa["out"]["kernel"], pa["out"]["bias"], residual=x)
                ln = p[f"ln_ffn_{i}"]
                mem_layer = self.pool is not None and i in cfg.memory_layers
                x_in = x
                if not mem_layer or cfg.memory_ffn:
                    fi, fo = p[f"ffn_in_{i}"], p[f"ffn_out_{i}"]
                    hid = rows_linear(x_in, fi["kernel"], fi["bias"], ln=ln, act="gelu_tanh")
                    x = rows_linear(hid, fo["kernel"], fo["bias"], residual=x)
                if mem_layer:
                    # the router and the gate read the same LayerNorm(x): one launch
                    mo = p[f"mem_out_{i}"]
                    wrg, brg = self._fused_router_gate(p, i)
                    q, gate = rows_linear_pair(x_in, wrg, brg, cfg.pool_heads * cfg.d_key, ln=ln, act2="silu")
                    q = q.reshape(B, cfg.pool_heads, cfg.d_key)
                    mem, aux = self.pool.apply({"params": p["pool"]}, q, noise_scale=noise_scale, rngs=rngs)
                    x = rows_linear(mem.float().contiguous(), mo["kernel"], mo["bias"], x_mul=gate, residual=x)
                    layer_aux.append(aux)
            lf = p["ln_final"]
            if (B <= 64 and d % 4 == 0 and d <= 256 and emb.dtype == torch.float32 and emb.is_contiguous()
                    and x.is_contiguous()
                    and all(t.dtype == torch.float32 and t.is_contiguous() and t.data_ptr() % 16 == 0
                            for t in (emb, x, lf["scale"], lf["bias"]))):
                logits = vocab_logits(x, lf["scale"], lf["bias"], emb)[:, None]  # one launch
            else:
                logits = F.linear(_ln(x, lf), emb)[:, None]
        return logits, _LazyMerged(layer_aux)

    def _attention(self, p, h, layer_cache, positions, drop=None):
        cfg = self.cfg
        B, T, d = h.shape
        hd = d // cfg.n_heads

        # the three DenseGeneral projections to (heads, hd) as one product
        names = ("query", "key", "value")
        w = torch.cat([p[nm]["kernel"].reshape(d, cfg.n_heads * hd) for nm in names], 1)
        b = torch.cat([p[nm]["bias"].reshape(cfg.n_heads * hd) for nm in names])
        qkv = (torch.matmul(h, w) + b).reshape(B, T, 3, cfg.n_heads, hd)
        q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))  # [B, heads, T, hd]
        q = q * (hd ** -0.5)
        if layer_cache is not None:  # decode: write position `positions`, attend to <= it
            layer_cache["kt"].index_copy_(3, positions, k.transpose(-1, -2))
            layer_cache["v"].index_copy_(2, positions, v)
            kt, v = layer_cache["kt"], layer_cache["v"]
            mask = (torch.arange(cfg.max_len, device=h.device) <= positions[:, None])[None, None]
        else:
            kt = k.transpose(-1, -2).contiguous()
            mask = torch.ones((T, T), dtype=torch.bool, device=h.device).tril()[None, None]
        s = torch.matmul(q, kt)
        s = s.masked_fill(~mask, torch.finfo(s.dtype).min)
        w = torch.softmax(s, dim=-1)
        if drop is not None:  # dropout on the attention weights (Flax MultiHeadDotProductAttention dropout_rate)
            w = drop(w)
        a = torch.matmul(w, v)  # [B, heads, T, hd]
        a = a.permute(0, 2, 1, 3).reshape(B, T, cfg.n_heads * hd)
        return torch.matmul(a, p["out"]["kernel"].reshape(cfg.n_heads * hd, d)) + p["out"]["bias"]

    def apply(self, variables: Dict[str, Any], tokens: torch.Tensor, *, train: bool = False, pool_off: bool = False,
              route_through_pool: bool = False, sparse_grad: bool = False,
              probes: Optional[Dict[int, torch.Tensor]] = None, positions: Optional[torch.Tensor] = None,
              noise_scale: float = 1.0, shuffle_pool: bool = False, cache=None, rngs=None,
              input_rows: Optional[torch.Tensor] = None):
        """model.py:27-127: (logits [B, T, vocab], aux).  In decode mode pass
        ``cache`` (init_cache) and ``positions`` (int64 device tensor [1]).
        ``input_rows`` (GPU decode step only): the step's input rows
        emb[tokens] + pos_embed[positions], [B, d_model] fp32, already formed
        (the greedy token step writes them, mpl_decode_next_token_embed); the
        tokens are then not read."""
        cfg = self.cfg
        p = variables["params"] if "params" in variables else variables
        B, T = tokens.shape
        if (self.decode and tokens.is_cuda and cache is not None and positions is not None and T == 1 and not train
                and not pool_off and not route_through_pool and probes is None and not shuffle_pool):
            return self._decode_step_gpu(p, tokens, positions, cache, noise_scale, rngs, input_rows)
        emb = p["embed"]["embedding"]
        if positions is None:
            x = emb[tokens] + p["pos_embed"][None, :T]
        else:
            x = emb[tokens] + p["pos_embed"][positions][None]
        if self.decode and (cache is None or positions is None):
            raise ValueError("decode mode needs cache and positions")
        drop = _make_dropout(cfg.dropout, rngs, x.device) if (train and cfg.dropout > 0) else None
        layer_aux = []
        for i in range(cfg.n_layers):
            h = _ln(x, p[f"ln_attn_{i}"])
            x = x + self._attention(p[f"attn_{i}"], h, cache[i] if self.decode else None, positions, drop)
            h = _ln(x, p[f"ln_ffn_{i}"])
            mem_layer = self.pool is not None and i in cfg.memory_layers
            y = torch.zeros_like(x)
            if not mem_layer or cfg.memory_ffn:
                y = _dense(F.gelu(_dense(h, p[f"ffn_in_{i}"]), approximate="tanh"), p[f"ffn_out_{i}"])
            if mem_layer:
                if route_through_pool:
                    x, y = x.detach(), y.detach()
                if not pool_off:
                    q = _dense(h, p[f"router_{i}"]).reshape(B, T, cfg.pool_heads, cfg.d_key)
                    mem, aux = self.pool.apply({"params": p["pool"]}, q, train=train, sparse_grad=sparse_grad,
                                               noise_scale=noise_scale, shuffle_reads=shuffle_pool, rngs=rngs)
                    if probes is not None:
                        mem = mem + probes[i]
                    h_gate = h.detach() if route_through_pool else h
                    gate = F.silu(_dense(h_gate, p[f"mem_gate_{i}"]))
                    y = y + _dense(mem * gate, p[f"mem_out_{i}"])
                    layer_aux.append(aux)
            if drop is not None:  # model.py:122: dropout on the layer's residual branch
                y = drop(y)
            x = x + y
        x = _ln(x, p["ln_final"])
        logits = F.linear(x, emb)  # x . emb^T as one product, no transposed copy of the table
        return logits, _LazyMerged(layer_aux)

    __call__ = apply
