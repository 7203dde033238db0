"""Host mirror of the reference's Flax ``MemoryPool`` (memory_pool_model/memory.py:64-227).

Same attributes, parameter names and layout (``sub_keys`` [H, 2, n, d_key/2],
``values`` [n*n, d_value], ``log_temperature`` []), same call keywords
(``train``, ``sparse_grad``, ``noise_scale``, ``shuffle_reads``) and the same
``aux`` keys.  Parameters are torch tensors on the GPU; every step of the
lookup runs in libmpl.so (include/mpl.h) on torch's current HIP stream:

  mpl_pack_keys      keys (cached per version)  memory.py:139
  mpl_score_select   query normalisation,       memory.py:136-138,
                     scores + 2-stage top-k     memory.py:149-178
                     + routing softmax
  mpl_gather_wsum    value read                 memory.py:179-193
  mpl_lookup         both of the above in one call (one kernel for
                     stage 2 and the value read at H = 4, k = 16)
  mpl_route_counts,  routing statistics, and    memory.py:196-215
  mpl_balance_fwd    the balance loss
  mpl_key_diversity  key_diversity_loss         memory.py:230-240
  mpl_revive_keys    revive_dead_keys           memory.py:243-281

The routing statistics of ``aux`` (memory.py:196-215) are derived from the
returned ids on first access, so a decode loop that never reads them never
pays for the N-sized ``slot_counts`` (the reference relies on XLA dead-code
elimination for the same effect, memory.py:215).
"""

from __future__ import annotations

import math
from typing import Any, Dict, Optional, Tuple

import torch

from . import _lib
from ._lib import MPL_F16, MPL_F32, check, ptr

NORM_EPS = 1e-6
# The routed query gradient inside the dense balance pass where it applies
# (mpl_lookup_bwd_dense_queries); False keeps the separate query pass.
FUSED_QUERY_BWD = True
# In that pass, fp16 operand packs made from the raw queries (normalised in
# the pack, the same bits as the fp32 q_hat pass); False packs q_hat.
RAW_QUERY_PACK = True


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float16:
        return MPL_F16
    if dt == torch.float32:
        return MPL_F32
    raise TypeError(f"unsupported dtype {dt} (float16 or float32)")


def _capturing() -> bool:
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


class _KeyCache:
    """Normalised + MFMA-packed sub-keys, rebuilt when the parameter changes
    (tracked by tensor identity, storage pointer and torch's in-place
    version counter: a new tensor at a freed tensor's address, whose version
    counter starts again at 0, is a change).

    Under HIP graph capture the pack is recorded into the graph (so every
    replay packs the keys as they are then) unless ``frozen``: a caller that
    keeps the keys fixed across replays (the generator's decode step) sets it
    and re-captures when the keys change."""

    def __init__(self):
        self.key = None
        self.src = None  # the keys tensor the cache was built from (held, so its identity stays unique)
        self.k_hat = None
        self.packed = None
        self.frozen = False

    def get(self, sub_keys: torch.Tensor, score_code: int):
        key = (sub_keys.data_ptr(), sub_keys._version, tuple(sub_keys.shape), score_code)
        if _capturing() and not self.frozen:
            return self._pack(sub_keys, score_code)
        if key != self.key or sub_keys is not self.src:
            self.k_hat, self.packed = self._pack(sub_keys, score_code)
            self.key, self.src = key, sub_keys
        return self.k_hat, self.packed

    @staticmethod
    def _pack(sub_keys: torch.Tensor, score_code: int):
        H, _, n, half = sub_keys.shape
        L = _lib.lib()
        nbytes = L.mpl_packed_keys_bytes(H, n, half, score_code)
        if nbytes == 0:
            raise _lib.MplError(f"unsupported key shape {tuple(sub_keys.shape)}")
        src = sub_keys.detach().float().contiguous()
        k_hat = torch.empty_like(src)
        packed = torch.empty(nbytes, dtype=torch.uint8, device=src.device)
        check(L.mpl_pack_keys(ptr(src), H, n, half, score_code, ptr(k_hat), ptr(packed),
                              _lib.stream_ptr(src.device)), "mpl_pack_keys")
        return k_hat, packed


class LazyAux(dict):
    """The ``aux`` dict of memory.py:217-226.  ``slots``, ``weights`` and
    ``temperature`` are stored; ``balance_loss`` and ``subkey_counts`` are
    computed together, and ``slot_counts``, ``queries`` and ``top1_weight``
    each on their own, the first time they are read (a training step that
    merges the fetched rows takes ``slot_counts`` from the merge instead:
    SparseRowUpdate(count_slots=True))."""

    _LAZY = ("balance_loss", "subkey_counts")
    _INTERNAL = ("_counts", "_state")

    def __init__(self, eager: Dict[str, Any], compute, **lazy):
        super().__init__(eager)
        self._compute = compute
        self._lazy = lazy  # further keys computed on first access (e.g. queries)

    def __missing__(self, key):
        if key in self._lazy:
            v = self._lazy[key]()
            self[key] = v
            return v
        if key in self._LAZY:
            stats = self._compute()
            self.internal = {k: stats.pop(k) for k in self._INTERNAL if k in stats}
            self.update(stats)
            return dict.__getitem__(self, key)
        raise KeyError(key)

    def __contains__(self, key):
        return key in self._LAZY or key in self._lazy or dict.__contains__(self, key)

    def keys(self):
        pending = [k for k in (*self._lazy, *self._LAZY) if not dict.__contains__(self, k)]
        return list(dict.keys(self)) + pending

    def materialize(self) -> "LazyAux":
        for k in (*self._lazy, *self._LAZY):
            self[k]
        return self


class _Result(dict):
    """The lookup's result; "q_hat" (fp32 normalised queries, which the
    scoring kernel does not need) is computed on first access."""

    def __missing__(self, key):
        if key != "q_hat":
            raise KeyError(key)
        q = self["q"]
        M, H, _, half = q.shape
        q_hat = torch.empty_like(q)
        check(_lib.lib().mpl_l2_normalize(ptr(q), M * H * 2, half, NORM_EPS, ptr(q_hat), None, None,
                                          _lib.stream_ptr(q.device)), "mpl_l2_normalize")
        self["q_hat"] = q_hat
        return q_hat


def routing_seed(rngs: Optional[Dict[str, Any]]) -> int:
    """64-bit seed of the routing noise (the reference's make_rng("routing")):
    ``rngs["routing"]`` as an int seed (the same noise on every call, like a
    fixed JAX key), one draw from a torch.Generator given there, or one draw
    from torch's default CPU generator (so torch.manual_seed reproduces runs).
    A CPU draw needs no device synchronisation; a CUDA generator's does."""
    r = None if rngs is None else rngs.get("routing")
    top = (1 << 63) - 1
    if r is None:
        return int(torch.randint(0, top, (1,)).item())
    if isinstance(r, torch.Generator):
        return int(torch.randint(0, top, (1,), generator=r, device=r.device).item())
    return int(r) & ((1 << 64) - 1)


class MemoryPool:
    """memory.py:64-113 attributes, memory.py:119-227 call."""

    def __init__(self, n_sub_keys: int, heads: int, d_key: int, d_value: int, top_k: int,
                 routing_noise: float = 1.0, init_temperature: float = 10.0,
                 min_temperature: float = 10.0, balance_temperature_grad: bool = False,
                 max_temperature: float = 100.0, query_scale: bool = False, host_pool: str = "",
                 name: str = "pool", *, values_dtype: torch.dtype = torch.float16,
                 score_dtype: Optional[torch.dtype] = None):
        assert d_key % 2 == 0, "d_key must be even (split into two halves)"  # memory.py:95
        assert top_k <= n_sub_keys  # memory.py:96
        self.n_sub_keys, self.heads, self.d_key, self.d_value, self.top_k = n_sub_keys, heads, d_key, d_value, top_k
        self.routing_noise = routing_noise
        self.init_temperature = init_temperature
        self.min_temperature, self.max_temperature = min_temperature, max_temperature
        self.balance_temperature_grad = balance_temperature_grad
        self.query_scale = query_scale
        self.host_pool = host_pool
        self.name = name
        self.values_dtype = values_dtype
        # fp16 MFMA scoring for fp16 tables, fp32 MFMA scoring for fp32 tables; fp16 scoring
        # reads 8-dim query vectors, so key halves of other widths score in fp32
        if score_dtype is None:
            fp16_ok = values_dtype == torch.float16 and (d_key // 2) % 8 == 0
            score_dtype = torch.float16 if fp16_ok else torch.float32
        elif score_dtype == torch.float16 and (d_key // 2) % 8 != 0:
            raise ValueError(f"fp16 scoring needs d_key/2 to be a multiple of 8, got d_key={d_key}")
        self.score_dtype = score_dtype
        self._keys = _KeyCache()
        self._temp_key = None
        self._temp_src = None
        self._temp_tensor = None
        self._constants = {}
        self._side = None  # the second stream of early_clean

    def _constant(self, value: float, dev) -> torch.Tensor:
        """A device fp32 scalar [1] holding ``value``, made once per (value,
        device) and reused (read-only), so a step does not launch a fill for
        it every call."""
        key = (float(value), str(dev))
        t = self._constants.get(key)
        if t is None:
            if _capturing():  # not cached from inside a capture: the graph keeps its own
                return torch.full((1,), float(value), dtype=torch.float32, device=dev)
            t = self._constants[key] = torch.full((1,), float(value), dtype=torch.float32, device=dev)
        return t

    @property
    def frozen_under_capture(self) -> bool:
        """When True, a HIP graph captured around a lookup reuses the packed
        keys and temperature computed before the capture instead of
        recomputing them in the graph (for callers that keep the sub-keys and
        log_temperature fixed while the graph is replayed)."""
        return self._keys.frozen

    @frozen_under_capture.setter
    def frozen_under_capture(self, value: bool) -> None:
        self._keys.frozen = bool(value)

    @property
    def pool_size(self) -> int:
        return self.n_sub_keys ** 2

    # ------------------------------------------------------------ params
    def init(self, rng: int | torch.Generator = 0, queries=None, *, device="cuda",
             values: Optional[torch.Tensor] = None) -> Dict[str, Any]:
        """memory.py:94-113: sub_keys on the unit sphere, values ~ N(0, d^-1/2),
        log_temperature = log(init_temperature).  ``rng`` is a seed or a
        torch.Generator on ``device``.  ``values`` [n*n, d_value] may be given
        (e.g. a table filled in place) instead of a fresh draw.  With a host
        pool there is no values parameter (memory.py:103-109): the table is
        the named HostPool (model_amd/host_pool.py)."""
        g = rng if isinstance(rng, torch.Generator) else torch.Generator(device=device).manual_seed(int(rng))
        H, n, half = self.heads, self.n_sub_keys, self.d_key // 2
        keys = torch.randn((H, 2, n, half), generator=g, device=device, dtype=torch.float32)
        keys = keys * torch.rsqrt((keys * keys).sum(-1, keepdim=True) + NORM_EPS)
        log_t = torch.tensor(math.log(self.init_temperature), dtype=torch.float32, device=device)
        if self.host_pool:
            return {"params": {"sub_keys": keys, "log_temperature": log_t}}
        if values is None:
            values = torch.randn((self.pool_size, self.d_value), generator=g, device=device, dtype=self.values_dtype)
            values.mul_(self.d_value ** -0.5)
        elif tuple(values.shape) != (self.pool_size, self.d_value):
            raise ValueError(f"values must be [{self.pool_size}, {self.d_value}], got {tuple(values.shape)}")
        return {"params": {"sub_keys": keys, "values": values, "log_temperature": log_t}}

    def temperature(self, log_temperature: torch.Tensor) -> torch.Tensor:
        """memory.py:143-146: the clamped temperature exp(clip(log_t, ln
        min_temperature, ln max_temperature)) as a device fp32 scalar [1],
        computed on the device (no host read), cached per parameter version
        outside graph capture."""
        key = (log_temperature.data_ptr(), log_temperature._version)
        if ((_capturing() and not self._keys.frozen) or key != self._temp_key
                or log_temperature is not self._temp_src):
            lt = log_temperature.detach().reshape(1).to(torch.float32).contiguous()
            t = torch.empty(1, dtype=torch.float32, device=lt.device)
            check(_lib.lib().mpl_temperature(ptr(lt), math.log(self.min_temperature), math.log(self.max_temperature),
                                             ptr(t), _lib.stream_ptr(lt.device)), "mpl_temperature")
            if _capturing() and not self._keys.frozen:
                return t
            self._temp_tensor, self._temp_key, self._temp_src = t, key, log_temperature
        return self._temp_tensor

    # -------------------------------------------------------------- call
    def apply(self, variables: Dict[str, Any], queries: torch.Tensor, *, train: bool = False,
              sparse_grad: bool = False, noise_scale: float | torch.Tensor = 1.0,
              shuffle_reads: bool = False, rngs: Optional[Dict[str, Any]] = None
              ) -> Tuple[torch.Tensor, LazyAux]:
        """memory.py:119-227.  ``variables`` = {"params": {...}} as from init();
        ``rngs["routing"]`` (seed or torch.Generator) drives the Gumbel noise."""
        params = variables["params"] if "params" in variables else variables
        if _needs_grad(params, queries, sparse_grad):
            return _lookup_with_grad(self, params, queries, train=train, sparse_grad=sparse_grad,
                                     noise_scale=noise_scale, shuffle_reads=shuffle_reads, rngs=rngs)
        res = self.lookup(params, queries, train=train, noise_scale=noise_scale,
                          shuffle_reads=shuffle_reads, rngs=rngs)
        return res["out"], res["aux"]

    __call__ = apply

    def forward_backward(self, variables: Dict[str, Any], queries: torch.Tensor, g_out: torch.Tensor,
                         g_balance: Optional[torch.Tensor] = None, *, train: bool = True,
                         noise_scale: float | torch.Tensor = 1.0, shuffle_reads: bool = False,
                         rngs: Optional[Dict[str, Any]] = None, g_diversity: Optional[torch.Tensor] = None,
                         on_forward=None, on_dq=None):
        """The forward of memory.py:119-227 and its backward for a given
        upstream gradient, without torch autograd: returns
        (out, aux, (d queries, d sub_keys, d log_temperature)).  The values
        get no dense gradient (the trainer's sparse_grad=True path: the rows
        come from aux["slots"], aux["weights"] and g_out).  ``g_balance`` is
        the gradient of aux["balance_loss"] (None: no balance term).  Only
        library kernels and tensor allocations, and no host read, so a whole
        training step built on it can be captured in one HIP graph; the
        results equal apply() followed by torch.autograd.grad bit for bit.
        ``g_diversity`` (a device scalar: the coefficient of
        key_diversity_loss in the training loss, memory.py:230-240) adds that
        term's gradient to d sub_keys and puts the loss in
        aux["key_diversity_loss"]; where the fused dense pass applies, its
        Gram tiles reuse this call's key packs and both sub-key terms share
        one normalisation backward (within fp32 rounding of the sum of the
        separate gradients).  ``on_forward(aux)``, when given, is called once
        the selection and the value read are enqueued (before the balance
        statistics and the backward), so a caller can start work that needs
        only aux["slots"] and aux["weights"] (the sparse row merge,
        SparseRowUpdate.merge) on another stream beside the rest.
        ``on_dq(d_queries)``, when given, is called once d queries (fp32,
        shaped like the queries) is enqueued and before the sub-key
        gradient's passes, so the caller can start what needs only d queries
        (the projection's weight gradient) on another stream beside them;
        such work must not write d_queries."""
        params = variables["params"] if "params" in variables else variables
        res = self.lookup(params, queries, train=train, noise_scale=noise_scale, shuffle_reads=shuffle_reads,
                          rngs=rngs, early_clean=g_balance is not None)
        aux = res["aux"]
        if on_forward is not None:  # the selection and the read are enqueued
            on_forward(aux)
        internal = {}
        if g_balance is not None:
            aux["balance_loss"]  # computes f and p (memory.py:196-213)
            internal = aux.internal
        sub_keys = params["sub_keys"]
        shapes = (tuple(queries.shape), queries.dtype, sub_keys.dtype, params["log_temperature"].dtype)
        values = params["values"] if "values" in params else sub_keys.new_empty(0)
        extra = {}
        dq, dk, dlt, _ = _lookup_backward(self, res, internal, sub_keys.detach(), values.detach(), shapes, g_out,
                                          g_balance, bool(shuffle_reads), False, g_diversity, extra, on_dq)
        if "key_diversity_loss" in extra:
            dict.__setitem__(aux, "key_diversity_loss", extra["key_diversity_loss"])
        out = res["out"].reshape(*tuple(queries.shape[:-2]), self.d_value)
        return out, aux, (dq, dk, dlt)

    def lookup(self, params, queries: torch.Tensor, *, train: bool = False,
               noise_scale: float | torch.Tensor = 1.0, shuffle_reads: bool = False,
               rngs: Optional[Dict[str, Any]] = None, gumbel: Optional[torch.Tensor] = None,
               early_clean: bool = False) -> Dict[str, Any]:
        """Forward lookup; returns out, aux and the tensors a backward needs.
        ``gumbel`` [M, H, 2, n] may be given explicitly (parity tests).
        ``early_clean`` (a training step that will read the balance loss):
        with routing noise, the clean stage-1 selection behind the balance
        statistics (memory.py:207) starts at once on a second stream, beside
        the noise draw and the noisy selection."""
        H, n, k, d = self.heads, self.n_sub_keys, self.top_k, self.d_value
        half = self.d_key // 2
        lead = tuple(queries.shape[:-2])
        if tuple(queries.shape[-2:]) != (H, self.d_key):
            raise ValueError(f"queries must be [..., {H}, {self.d_key}], got {tuple(queries.shape)}")
        dev = queries.device
        if dev.type != "cuda":
            raise RuntimeError("MemoryPool runs on the GPU only (libmpl.so); got a tensor on " + str(dev))
        L = _lib.lib()
        stream = _lib.stream_ptr(dev)
        q = queries.detach().reshape(-1, H, 2, half).float().contiguous()
        M = q.shape[0]
        score_code = _dtype_code(self.score_dtype)
        # the scoring kernel normalises the raw queries itself (and computes
        # q_len with query_scale); the fp32 q_hat is produced only on demand
        q_mode = _lib.MPL_Q_RAW_SCALED if self.query_scale else _lib.MPL_Q_RAW
        q_len = torch.empty((M, H, 2), dtype=torch.float32, device=dev) if self.query_scale else None
        k_hat, packed = self._keys.get(params["sub_keys"], score_code)
        T = self.temperature(params["log_temperature"])
        early = None
        if early_clean and train and self.routing_noise > 0 and gumbel is None and M > 0:
            early = self._clean_early(q, packed, score_code, T, M)

        noise_coef = None  # device scalar routing_noise * noise_scale (memory.py:157)
        if gumbel is None and train and self.routing_noise > 0:
            # memory.py:156: Gumbel(0,1) over the score shape, one fill pass
            gumbel = torch.empty((M, H, 2, n), dtype=torch.float32, device=dev)
            check(L.mpl_gumbel_noise(routing_seed(rngs), M * H * 2, n, ptr(gumbel), stream), "mpl_gumbel_noise")
        if gumbel is not None:
            if isinstance(noise_scale, torch.Tensor):  # an annealed, traced noise_scale stays on the device
                noise_coef = noise_scale.detach().to(device=dev, dtype=torch.float32).reshape(1) * float(
                    self.routing_noise)
            else:
                noise_coef = self._constant(float(self.routing_noise) * float(noise_scale), dev)
            gumbel = gumbel.reshape(M, H, 2, n).float().contiguous()

        ws_bytes = L.mpl_score_select_workspace_bytes(M, H, n, half, k)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        sub_idx = torch.empty((M, H, 2, k), dtype=torch.int32, device=dev)
        sub_scores = torch.empty((M, H, 2, k), dtype=torch.float32, device=dev)
        flat_idx = torch.empty((M, H, k), dtype=torch.int32, device=dev)
        slots = torch.empty((M, H, k), dtype=torch.int32, device=dev)
        weights = torch.empty((M, H, k), dtype=torch.float32, device=dev)
        out = torch.empty((M, d), dtype=torch.float32, device=dev)
        staged = None
        if not self.host_pool:
            # selection and value read in one call (memory.py:132-193): with
            # H = 4 and k = 16 the pair stage and the read share one kernel
            values = params["values"]
            if values.dtype not in (torch.float16, torch.float32) or not values.is_contiguous():
                raise TypeError("values must be a contiguous float16/float32 [n*n, d_value] tensor")
            if tuple(values.shape) != (self.pool_size, d):
                raise ValueError(f"values must be [{self.pool_size}, {d}], got {tuple(values.shape)}")
            check(L.mpl_lookup(ptr(q), q_mode, ptr(q_len), ptr(packed), M, H, n, half, k, score_code,
                               ptr(T), ptr(gumbel), ptr(noise_coef), ptr(ws), ws_bytes, ptr(sub_idx),
                               ptr(sub_scores), ptr(flat_idx), ptr(slots), ptr(weights),
                               ptr(values), _dtype_code(values.dtype), d, int(bool(shuffle_reads)), ptr(out),
                               stream), "mpl_lookup")
        else:
            check(L.mpl_score_select(ptr(q), q_mode, ptr(q_len), ptr(packed), M, H, n, half, k, score_code,
                                     ptr(T), ptr(gumbel), ptr(noise_coef), ptr(ws), ws_bytes, ptr(sub_idx),
                                     ptr(sub_scores), ptr(flat_idx), ptr(slots), ptr(weights), stream),
                  "mpl_score_select")
            # memory.py:182-183 (hp.fetch): the unique rows cross the host
            # link once into device memory; the weighted sum reads them there
            from . import host_pool as hp
            read = slots
            if shuffle_reads:  # memory.py:179
                N = self.pool_size
                read = ((slots.long() + N // 2 + 1) % N).to(torch.int32)
            rows, inverse, _ = hp.get(self.host_pool).stage(read)
            staged = (rows, inverse.reshape(M, H, k))
            check(L.mpl_gather_wsum(ptr(rows), _dtype_code(rows.dtype), max(rows.shape[0], 1), d, ptr(staged[1]),
                                    ptr(weights), M, H * k, 0, ptr(out), stream), "mpl_gather_wsum")

        noisy = gumbel is not None
        res = _Result()

        def stats():
            return self._routing_stats(params, res, k_hat, T, q_len, sub_idx, slots, weights,
                                       noisy, packed, score_code, M, early)

        aux = LazyAux({
            "slots": slots.reshape(*lead, H, k),
            "weights": weights.reshape(*lead, H, k),
            "temperature": T.reshape(()),
        }, stats, queries=lambda: res["q_hat"], top1_weight=lambda: weights.max(-1).values.mean(),
            slot_counts=lambda: self._slot_counts(slots, M))
        res.update({
            "out": out.reshape(*lead, d), "aux": aux, "q": q, "q_len": q_len,
            "k_hat": k_hat, "packed": packed, "score_code": score_code, "temperature": T, "sub_idx": sub_idx, "sub_scores": sub_scores,
            "flat_idx": flat_idx, "slots": slots, "weights": weights, "gumbel": gumbel, "staged": staged,
            "noise_coef": noise_coef,
        })
        return res

    # ------------------------------------------------------------- stats
    def _routing_stats(self, params, res, k_hat, T, q_len, sub_idx, slots, weights, noisy,
                       packed, score_code, M, early=None):
        """memory.py:196-215 from the selected ids: the counts on the GPU
        (mpl_route_counts) and the balance loss fused over the MFMA score
        tiles of the scoring precision (mpl_balance_fwd)."""
        H, n, k = self.heads, self.n_sub_keys, self.top_k
        half = self.d_key // 2
        dev = sub_idx.device
        L = _lib.lib()
        stream = _lib.stream_ptr(dev)
        if noisy and early is not None:  # started on the side stream by lookup()
            cur = torch.cuda.current_stream(dev)
            cur.wait_stream(early[1])
            clean = early[0]
            clean.record_stream(cur)
        elif noisy:  # memory.py:207: an extra clean selection
            clean = self._clean_sub_idx(res["q"], packed, score_code, T, M)
        else:
            clean = sub_idx
        subkey_counts = torch.empty((H, 2, n), dtype=torch.float32, device=dev)
        clean_counts = torch.empty((H, 2, n), dtype=torch.float32, device=dev)
        check(L.mpl_route_counts(ptr(slots), ptr(clean), M, H, n, k, ptr(subkey_counts), ptr(clean_counts),
                                 None, stream), "mpl_route_counts")
        stats = {"subkey_counts": subkey_counts}
        scaled = int(bool(self.balance_temperature_grad and self.query_scale))
        state = torch.empty(max(L.mpl_balance_state_bytes(M, H), 16), dtype=torch.uint8, device=dev)
        loss = torch.empty(1, dtype=torch.float32, device=dev)
        check(L.mpl_balance_fwd(ptr(res["q"]) if M > 0 else None, scaled, ptr(packed), ptr(clean_counts), M, H, n,
                                half, k, score_code, ptr(T), ptr(state), ptr(loss), stream), "mpl_balance_fwd")
        stats.update(balance_loss=loss.reshape(()), _counts=clean_counts, _state=state)
        return stats

    def _slot_counts(self, slots, M):
        """memory.py:215: zeros(pool_size).at[slots].add(1), fp32."""
        H, n, k = self.heads, self.n_sub_keys, self.top_k
        dev = slots.device
        out = torch.empty(self.pool_size, dtype=torch.float32, device=dev)
        check(_lib.lib().mpl_route_counts(ptr(slots), None, M, H, n, k, None, None, ptr(out), _lib.stream_ptr(dev)),
              "mpl_route_counts(slots)")
        return out

    def _clean_early(self, q, packed, score_code, T, M):
        """The clean stage-1 lists on the pool's side stream (default
        priority), after everything the current stream has enqueued: returns
        (sub_idx, stream); the reader waits for that stream first."""
        dev = q.device
        if self._side is None or self._side.device != dev:
            self._side = torch.cuda.Stream(device=dev)
        side = self._side
        cur = torch.cuda.current_stream(dev)
        side.wait_stream(cur)
        for t in (q, packed, T):
            t.record_stream(side)
        with torch.cuda.stream(side):
            clean = self._clean_sub_idx(q, packed, score_code, T, M)
        return clean, side

    def _clean_sub_idx(self, q, packed, score_code, T, M):
        """memory.py:207: the stage-1 top-k of the clean scores (no stage 2)."""
        H, n, k, half = self.heads, self.n_sub_keys, self.top_k, self.d_key // 2
        dev = q.device
        q_mode = _lib.MPL_Q_RAW_SCALED if self.query_scale else _lib.MPL_Q_RAW
        L = _lib.lib()
        ws_bytes = L.mpl_score_topk_workspace_bytes(M, H, n, half, k)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        sub_idx = torch.empty((M, H, 2, k), dtype=torch.int32, device=dev)
        sub_scores = torch.empty((M, H, 2, k), dtype=torch.float32, device=dev)
        check(L.mpl_score_topk(ptr(q), q_mode, None, ptr(packed), M, H, n, half, k, score_code, ptr(T),
                               None, None, ptr(ws), ws_bytes, ptr(sub_idx), ptr(sub_scores), _lib.stream_ptr(dev)),
              "mpl_score_topk(clean)")
        return sub_idx


# ------------------------------------------------------------ regularisers
def _fp16_gram_ok(half: int) -> bool:
    return half % 8 == 0 and half <= 128


def _key_diversity_fwd(sub_keys: torch.Tensor, code: int, need_grad: bool):
    """memory.py:230-240 on MFMA Gram tiles (mpl_key_diversity): the loss
    [1], the fp32 keys and, with need_grad, d loss / d k_hat (formed in the
    same pass over the Gram tiles)."""
    H, C, n, half = sub_keys.shape
    dev = sub_keys.device
    L = _lib.lib()
    stream = _lib.stream_ptr(dev)
    src = sub_keys.detach().float().contiguous()
    k_hat = torch.empty_like(src)
    packed = torch.empty(L.mpl_packed_keys_bytes(H, n, half, code), dtype=torch.uint8, device=dev)
    check(L.mpl_pack_keys(ptr(src), H, n, half, code, ptr(k_hat), ptr(packed), stream), "mpl_pack_keys")
    wsb = L.mpl_key_diversity_workspace_bytes(H, n, half, code)
    ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev)
    loss = torch.empty(1, dtype=torch.float32, device=dev)
    dk = torch.empty_like(src) if need_grad else None
    check(L.mpl_key_diversity(ptr(k_hat), ptr(packed), H, n, half, code, ptr(ws), wsb, ptr(loss), ptr(dk), stream),
          "mpl_key_diversity")
    return loss, src, dk


def _key_diversity_bwd(src: torch.Tensor, dk: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """The l2-normalisation backward (mpl_l2_normalize_bwd) of d k_hat scaled
    by the upstream gradient g (a device scalar): d loss / d sub_keys, fp32."""
    H, C, n, half = src.shape
    dx = torch.empty_like(src)
    gs = g.reshape(1).float().contiguous()
    check(_lib.lib().mpl_l2_normalize_bwd(ptr(src), ptr(dk), H * C * n, half, NORM_EPS, ptr(gs), ptr(dx),
                                          _lib.stream_ptr(src.device)), "mpl_l2_normalize_bwd")
    return dx


class _KeyDiversity(torch.autograd.Function):
    """memory.py:230-240 on MFMA Gram tiles (mpl_key_diversity) in fp16 or
    fp32; the gradient with respect to the normalised keys is formed in the
    forward (one pass over the Gram tiles) and taken through the
    l2-normalisation backward (mpl_l2_normalize_bwd) with the upstream
    gradient."""

    @staticmethod
    def forward(ctx, sub_keys, code):
        loss, src, dk = _key_diversity_fwd(sub_keys, code, ctx.needs_input_grad[0])
        ctx.save_for_backward(src, dk)
        ctx.dtype = sub_keys.dtype
        return loss.reshape(())

    @staticmethod
    def backward(ctx, g):
        src, dk = ctx.saved_tensors
        return _key_diversity_bwd(src, dk, g).to(ctx.dtype), None


def _key_diversity_code(sub_keys: torch.Tensor, score_dtype: Optional[torch.dtype]) -> int:
    if sub_keys.device.type != "cuda":
        raise RuntimeError("key_diversity_loss runs on the GPU only (libmpl.so)")
    H, C, n, half = sub_keys.shape
    if score_dtype is None:
        score_dtype = torch.float16 if _fp16_gram_ok(half) else torch.float32
    if half > 128 or (score_dtype == torch.float16 and not _fp16_gram_ok(half)):
        raise ValueError(f"key_diversity_loss: no {score_dtype} Gram kernel for sub-key width {half} "
                         "(fp16: multiples of 8 up to 128; fp32: up to 128)")
    return _dtype_code(score_dtype)


def key_diversity_loss(sub_keys: torch.Tensor, score_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """memory.py:230-240: mean squared off-diagonal cosine inside each
    sub-key codebook, differentiable with respect to ``sub_keys``.  The Gram
    tiles run on MFMA in ``score_dtype``: fp16 (sub-key widths d_key/2 that
    are multiples of 8, up to 128) or fp32 (any width up to 128, the
    reference's precision).  By default fp16 where it applies, else fp32; a
    pool passes its own scoring precision (``MemoryPool.score_dtype``)."""
    return _KeyDiversity.apply(sub_keys, _key_diversity_code(sub_keys, score_dtype))


def key_diversity_value_and_grad(sub_keys: torch.Tensor, g: torch.Tensor,
                                 score_dtype: Optional[torch.dtype] = None):
    """key_diversity_loss and its gradient with respect to ``sub_keys`` for
    the upstream gradient ``g`` (a device scalar), without torch autograd:
    (loss [], d sub_keys).  The same kernels as key_diversity_loss + autograd,
    for training steps captured in a HIP graph."""
    loss, src, dk = _key_diversity_fwd(sub_keys, _key_diversity_code(sub_keys, score_dtype), True)
    return loss.reshape(()), _key_diversity_bwd(src, dk, g).to(sub_keys.dtype)


def revive_dead_keys(sub_keys: torch.Tensor, subkey_usage: torch.Tensor, queries: torch.Tensor, rng,
                     threshold: float, noise: float = 0.05, *, pick: Optional[torch.Tensor] = None,
                     normal: Optional[torch.Tensor] = None):
    """memory.py:243-281 (mpl_revive_keys): returns (new_sub_keys,
    new_subkey_usage, dead_mask).  ``rng`` (seed or torch.Generator) draws
    the picked query per key and the normal noise; ``pick`` [H,2,n] and
    ``normal`` [H,2,n,d] may be given instead."""
    H, C, n, d = sub_keys.shape
    dev = sub_keys.device
    q = queries.detach().reshape(-1, H, C, d).float().contiguous()
    M = q.shape[0]
    if M < 1:
        raise ValueError("revive_dead_keys needs at least one query")
    if pick is None or normal is None:
        gen = rng if isinstance(rng, torch.Generator) else torch.Generator(device=dev).manual_seed(int(rng))
        pick = torch.randint(0, M, (H, C, n), generator=gen, device=dev)
        normal = torch.randn((H, C, n, d), generator=gen, device=dev)
    pick = pick.to(device=dev, dtype=torch.int32).contiguous()
    normal = normal.to(device=dev, dtype=torch.float32).contiguous()
    new_keys = sub_keys.detach().float().clone()
    new_usage = subkey_usage.detach().float().clone()
    dead = torch.empty((H, C, n), dtype=torch.uint8, device=dev)
    check(_lib.lib().mpl_revive_keys(ptr(new_keys), ptr(new_usage), ptr(q), M, ptr(pick), ptr(normal), H, n, d,
                                     float(threshold), float(noise), ptr(dead), _lib.stream_ptr(dev)),
          "mpl_revive_keys")
    return new_keys.to(sub_keys.dtype), new_usage, dead.bool()


# ------------------------------------------------------------------ autograd
def _needs_grad(params, queries, sparse_grad) -> bool:
    if not torch.is_grad_enabled():
        return False
    ts = [queries, params["sub_keys"], params["log_temperature"]]
    if not sparse_grad and "values" in params:
        ts.append(params["values"])
    return any(isinstance(t, torch.Tensor) and t.requires_grad for t in ts)


class _LookupFunction(torch.autograd.Function):
    """(queries, sub_keys, log_temperature, values) -> (out, balance_loss) with
    the backward of memory.py:136-213 on the GPU (include/mpl.h
    mpl_lookup_bwd_*): the selection is piecewise constant, so gradients flow
    through the selected clean scores, the routing softmax, the value read and
    (dense over n) the balance loss."""

    @staticmethod
    def forward(ctx, queries, sub_keys, log_temperature, values, pool, opts):
        _refuse_capture()
        params = {"sub_keys": sub_keys, "values": values, "log_temperature": log_temperature}
        res = pool.lookup(params, queries.detach(), train=opts["train"], noise_scale=opts["noise_scale"],
                          shuffle_reads=opts["shuffle_reads"], rngs=opts["rngs"])
        aux = res["aux"]
        balance = aux["balance_loss"]  # also computes f and p (memory.py:196-213)
        ctx.pool, ctx.opts, ctx.res = pool, opts, res
        ctx.internal = aux.internal
        opts["_aux"] = aux  # handed back to the caller with the differentiable balance loss
        ctx.shapes = (tuple(queries.shape), queries.dtype, sub_keys.dtype, log_temperature.dtype)
        ctx.save_for_backward(sub_keys, values)
        return res["out"], balance.detach()

    @staticmethod
    def backward(ctx, g_out, g_balance):
        _refuse_capture()  # a forward run eagerly and a backward captured: refused too
        sub_keys, values = ctx.saved_tensors
        need_dv = ctx.needs_input_grad[3] and not ctx.opts["sparse_grad"]
        dq, dk, dlt, dv = _lookup_backward(ctx.pool, ctx.res, ctx.internal, sub_keys, values, ctx.shapes, g_out,
                                           g_balance, bool(ctx.opts["shuffle_reads"]), need_dv)
        return dq, dk, dlt, dv, None, None


def _lookup_backward(pool, res, internal, sub_keys, values, shapes, g_out, g_balance, shuffle_reads: bool,
                     need_dv: bool, g_diversity: Optional[torch.Tensor] = None, extra: Optional[Dict] = None,
                     on_dq=None):
    """The backward of memory.py:136-213 on the GPU for one forward result
    ``res`` of MemoryPool.lookup: (d queries, d sub_keys, d log_temperature,
    d values or None).  ``g_balance`` is the gradient of the balance loss
    (None: no balance term); ``internal`` holds the balance statistics of the
    forward.  Only library kernels and tensor allocations: no host read."""
    q_shape, q_dtype, k_dtype, t_dtype = shapes
    H, n, k, d = pool.heads, pool.n_sub_keys, pool.top_k, pool.d_value
    half = pool.d_key // 2
    q = res["q"]
    M = q.shape[0]
    dev = q.device
    L = _lib.lib()
    stream = _lib.stream_ptr(dev)
    T = res["temperature"]
    q_len, k_hat = res["q_len"], res["k_hat"]
    if g_out is None:
        g_out = torch.zeros((M, d), dtype=torch.float32, device=dev)
    g_out = g_out.reshape(M, d).float().contiguous()

    # route: dw, softmax backward, scatter to the stage-1 ranks
    d_sub = torch.empty((M, H, 2, k), dtype=torch.float32, device=dev)
    dlogt_part = torch.empty(max(M, 1), dtype=torch.float32, device=dev)
    if res["staged"] is not None:  # host pool: the staged unique rows, indexed by inverse
        vals, vslots = res["staged"]
        vN, vshuffle = max(vals.shape[0], 1), 0
    else:
        vals, vslots = values.detach(), res["slots"]
        vN, vshuffle = pool.pool_size, int(shuffle_reads)
    check(L.mpl_lookup_bwd_route(ptr(g_out), ptr(vals), _dtype_code(vals.dtype), vN, d,
                                 ptr(vslots), ptr(res["weights"]), ptr(res["flat_idx"]),
                                 ptr(res["sub_scores"]), M, H, k, vshuffle, None,
                                 ptr(d_sub), ptr(dlogt_part), stream), "mpl_lookup_bwd_route")

    # dense over n on MFMA tiles of the scoring precision: the balance
    # loss (memory.py:208-213) together with the routed sub-key term.
    # Without the balance term, fp32 scoring takes the routed term alone
    # from a sort-by-key segmented sum (O(M k) instead of O(M n)).
    dq_extra = dlen_extra = dlogt_extra = None
    btg = pool.balance_temperature_grad
    raw_keys = sub_keys.detach().float().contiguous()
    dk = torch.empty((H, 2, n, half), dtype=torch.float32, device=dev)
    bal = g_balance is not None and "_state" in internal
    code = res["score_code"]
    dense = M > 0 and (code == MPL_F16 or bal)
    # the routed query gradient inside the balance pass (one launch fewer)
    fused_q = (FUSED_QUERY_BWD and dense and bal and not btg and not pool.query_scale and k <= 16
               and half % 4 == 0 and half <= 128 and q.data_ptr() % 16 == 0)
    dq = torch.empty((M, H, 2, half), dtype=torch.float32, device=dev)
    if fused_q:
        dk_hat = torch.empty((H, 2, n, half), dtype=torch.float32, device=dev)
        gb = g_balance.reshape(1).float().contiguous()
        wsb = L.mpl_lookup_bwd_dense_workspace_bytes(M, H, n, half, code)
        ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev)
        # fp16 operands at half 64 / 128 are packed from the raw queries
        # (normalised in the pack): no fp32 q_hat pass
        raw_pack = RAW_QUERY_PACK and code == MPL_F16 and half in (64, 128)
        q_hat = None if raw_pack else res["q_hat"]
        gd = dws = div_loss = None
        dwsb = 0
        if g_diversity is not None and n > 1:  # the diversity Gram pass on this call's key packs
            gd = g_diversity.reshape(1).float().contiguous()
            dwsb = L.mpl_key_diversity_workspace_bytes(H, n, half, code)
            dws = torch.empty(max(dwsb, 256), dtype=torch.uint8, device=dev)
            div_loss = torch.empty(1, dtype=torch.float32, device=dev)
        def dense(phase):
            check(L.mpl_lookup_bwd_dense_queries(ptr(q_hat), ptr(q), ptr(k_hat), ptr(res["packed"]),
                                                 ptr(res["sub_idx"]), ptr(d_sub), ptr(internal["_counts"]),
                                                 ptr(internal["_state"]), ptr(gb), M, H, n, half, k, code, ptr(T),
                                                 ptr(ws), wsb, NORM_EPS, ptr(dq), ptr(raw_keys), ptr(gd), ptr(dws),
                                                 dwsb, ptr(div_loss), ptr(dk), phase, stream),
                  "mpl_lookup_bwd_dense_queries")

        if on_dq is None:
            dense(0)
        else:  # the query side, the caller's hook (d queries is enqueued), then the sub-key side
            dense(1)
            on_dq(dq.reshape(q_shape))
            dense(2)
        if div_loss is not None:
            g_diversity = None  # taken in the fused pass
            if extra is not None:
                extra["key_diversity_loss"] = div_loss.reshape(())
    elif dense:
        q_hat = res["q_hat"]
        dk_hat = torch.empty((H, 2, n, half), dtype=torch.float32, device=dev)
        gb = None
        if bal:
            dq_extra = torch.empty((M, H, 2, half), dtype=torch.float32, device=dev)
            dlen_extra = torch.empty((M, H, 2), dtype=torch.float32, device=dev) if (btg and q_len is not None) else None
            dlogt_extra = torch.empty(1, dtype=torch.float32, device=dev) if btg else None
            gb = g_balance.reshape(1).float().contiguous()
        wsb = L.mpl_lookup_bwd_dense_workspace_bytes(M, H, n, half, code)
        ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev)
        check(L.mpl_lookup_bwd_dense(ptr(q_hat), ptr(q_len), ptr(k_hat), ptr(res["packed"]), ptr(res["sub_idx"]),
                                     ptr(d_sub), ptr(internal["_counts"]) if bal else None,
                                     ptr(internal["_state"]) if bal else None, ptr(gb), int(btg),
                                     int(bool(pool.query_scale)), M, H, n, half, k, code, ptr(T), ptr(ws), wsb,
                                     ptr(dq_extra), ptr(dk_hat), ptr(dlen_extra), ptr(dlogt_extra), stream),
              "mpl_lookup_bwd_dense")
        check(L.mpl_l2_normalize_bwd(ptr(raw_keys), ptr(dk_hat), H * 2 * n, half, NORM_EPS, None, ptr(dk),
                                     stream), "mpl_l2_normalize_bwd")

    # queries
    if not fused_q:
        check(L.mpl_lookup_bwd_queries(ptr(q), ptr(q_len), ptr(k_hat), ptr(res["sub_idx"]), ptr(d_sub),
                                       ptr(res["sub_scores"]), ptr(dq_extra), ptr(dlen_extra), M, H, n, half, k,
                                       ptr(T), ptr(dq), stream), "mpl_lookup_bwd_queries")
        if on_dq is not None:
            on_dq(dq.reshape(q_shape))
    # sub-keys (fp32 scoring without the balance term, or no tokens):
    # sort-by-key segmented sum
    if not dense:
        wsb = max(L.mpl_lookup_bwd_keys_workspace_bytes(M, H, n, half, k), 256)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        check(L.mpl_lookup_bwd_keys(ptr(raw_keys), ptr(res["q_hat"]), ptr(q_len), ptr(res["sub_idx"]), ptr(d_sub),
                                    None, M, H, n, half, k, ptr(T), ptr(ws), wsb, ptr(dk), stream),
              "mpl_lookup_bwd_keys")
    if g_diversity is not None:  # the key diversity term on its own (memory.py:230-240)
        dloss, ddk = key_diversity_value_and_grad(sub_keys, g_diversity, pool.score_dtype)
        dk = dk + ddk
        if extra is not None:
            extra["key_diversity_loss"] = dloss
    # log_temperature: straight-through clamp, dT/dlog_t = T (memory.py:143-146)
    dlt = torch.empty(1, dtype=torch.float32, device=dev)
    check(L.mpl_sum(ptr(dlogt_part), M, ptr(dlogt_extra), ptr(dlt), stream), "mpl_sum")

    # values: dense gradient only when the table is differentiated (sparse_grad=False)
    dv = None
    if need_dv:
        N = pool.pool_size
        sl = res["slots"].long()
        if shuffle_reads:
            sl = (sl + N // 2 + 1) % N
        from .rows import merge_fetches
        m = merge_fetches(sl.to(torch.int32), res["weights"], g_out, N)
        dv_ext = torch.zeros((N + 1, d), dtype=torch.float32, device=dev)
        dv_ext.index_copy_(0, m.uniq.long(), m.rows)  # padding rows (all zero) land on row N
        dv = dv_ext[:N].to(values.dtype)

    return dq.reshape(q_shape).to(q_dtype), dk.to(k_dtype), dlt.reshape(()).to(t_dtype), dv


_CAPTURE_MSG = ("MemoryPool: torch autograd through the lookup is not supported under HIP graph capture (a "
                "captured autograd training step crashed torch's graph instantiation on this stack); capture "
                "MemoryPool.forward_backward instead, which runs the same forward and backward kernels without "
                "autograd, or run the autograd step eagerly")


def _refuse_capture() -> None:
    if _capturing():
        raise RuntimeError(_CAPTURE_MSG)


def _lookup_with_grad(pool, params, queries, *, train, sparse_grad, noise_scale, shuffle_reads, rngs):
    _refuse_capture()  # before any library call or allocation
    opts = {"train": train, "sparse_grad": sparse_grad, "noise_scale": noise_scale,
            "shuffle_reads": shuffle_reads, "rngs": rngs}
    if pool.host_pool and not sparse_grad:
        raise ValueError("a host pool is updated sparsely: call with sparse_grad=True (train.py:214-215)")
    values = params["values"] if "values" in params else params["sub_keys"].new_empty(0)
    out, balance = _LookupFunction.apply(queries, params["sub_keys"], params["log_temperature"],
                                         values, pool, opts)
    aux = opts.pop("_aux")
    dict.__setitem__(aux, "balance_loss", balance)  # the autograd-tracked copy
    return out.reshape(*tuple(queries.shape[:-2]), pool.d_value), aux
