"""Sparse pool-row gradients and row-wise optimizers on the GPU (libmpl.so).

Host mirror of the sparse half of the reference training step
(memory_pool_model/train.py):

  * ``fetched_row_grads(aux, probe_grads, layers, pool_size)``  train.py:146-163
  * ``merge_rows(slots, contribs, pool_size)``                 train.py:166-172
  * ``clip_scale(row_sq, rest_sq, grad_clip)``                 train.py:395-399
  * ``sum_squares(tensors, add)`` (the dense gradients' norm)   train.py:395-397
  * ``rowwise_adagrad(...)``                                   train.py:412-416
  * ``lazy_adam(...)``                                         train.py:417-426
  * ``warmup_cosine(step, lr, warmup_steps, steps)``           train.py:100-103
  * ``SparseRowUpdate``: the whole sparse step of train.py:378-429 on one GPU

Every tensor stays on the device: the number of distinct rows and the clip
scale are device scalars, so a step never synchronises with the host.
"""

from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass
from typing import Dict, Optional, Sequence

import torch

from . import _lib
from ._lib import check, ptr

MPL_F16, MPL_F32 = _lib.MPL_F16, _lib.MPL_F32


def _vcode(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return MPL_F16
    if t.dtype == torch.float32:
        return MPL_F32
    raise TypeError(f"pool values must be float16 or float32, got {t.dtype}")


@dataclass
class MergedRows:
    """Result of a row merge: ``uniq`` [cap] int32 (ascending, padded with
    pool_size), ``rows`` [cap, d] fp32, ``row_sq`` [cap] fp32 squared row
    norms and ``num_unique`` [1] int32, all on the device."""

    uniq: torch.Tensor
    rows: torch.Tensor
    row_sq: torch.Tensor
    num_unique: torch.Tensor


def merge_fetches(slots: torch.Tensor, weights: Optional[torch.Tensor], g: torch.Tensor,
                  pool_size: int, zero_padding: bool = True,
                  slot_counts: Optional[torch.Tensor] = None) -> MergedRows:
    """Sum weights[p] * g[p // fpt] per distinct slot, fpt = P / g.shape[0]
    (the fetches of one token are consecutive).  zero_padding=False leaves
    the padding rows [num_unique, cap) unwritten (the row optimizers skip
    them).  ``slot_counts`` (a contiguous fp32 [pool_size] tensor, or None)
    receives the number of fetches of every slot (memory.py:215), taken from
    the segments of the same sort."""
    dev = g.device
    slots = slots.reshape(-1).to(torch.int32).contiguous()
    P = slots.shape[0]
    g = g.reshape(-1, g.shape[-1]).float().contiguous()
    tokens, d = g.shape
    if tokens == 0 or P % tokens:
        if P == 0 and tokens == 0:
            fpt = 1
        else:
            raise ValueError(f"{P} fetches do not divide evenly over {tokens} gradient rows")
    else:
        fpt = P // tokens
    if weights is not None:
        weights = weights.reshape(-1).float().contiguous()
        if weights.shape[0] != P:
            raise ValueError("weights must have one entry per fetch")
    cap = min(P, pool_size)
    L = _lib.lib()
    uniq = torch.empty(cap, dtype=torch.int32, device=dev)
    rows = torch.empty((cap, d), dtype=torch.float32, device=dev)
    row_sq = torch.empty(cap, dtype=torch.float32, device=dev)
    num_unique = torch.empty(1, dtype=torch.int32, device=dev)
    wsb = L.mpl_merge_rows_workspace_bytes(P, d, pool_size)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    if slot_counts is not None:
        if (slot_counts.dtype != torch.float32 or not slot_counts.is_contiguous()
                or slot_counts.numel() != pool_size or slot_counts.device != dev):
            raise ValueError(f"slot_counts must be a contiguous fp32 [{pool_size}] tensor on {dev}")
        check(L.mpl_merge_rows_counts(ptr(slots), ptr(weights), P, fpt, ptr(g), d, pool_size, ptr(ws), wsb,
                                      ptr(uniq), ptr(rows), ptr(row_sq), ptr(num_unique), int(bool(zero_padding)),
                                      ptr(slot_counts), _lib.stream_ptr(dev)), "mpl_merge_rows_counts")
    else:
        check(L.mpl_merge_rows(ptr(slots), ptr(weights), P, fpt, ptr(g), d, pool_size, ptr(ws), wsb, ptr(uniq),
                               ptr(rows), ptr(row_sq), ptr(num_unique), int(bool(zero_padding)),
                               _lib.stream_ptr(dev)), "mpl_merge_rows")
    return MergedRows(uniq, rows, row_sq, num_unique)


def merge_rows(slots: torch.Tensor, contribs: torch.Tensor, pool_size: int):
    """train.py:166-172: (uniq [cap], rows [cap, d]) for materialised
    per-fetch contribution rows."""
    m = merge_fetches(slots, None, contribs.reshape(-1, contribs.shape[-1]), pool_size)
    return m.uniq, m.rows


def fetched_row_grads_full(aux: Dict, probe_grads, layers: Sequence[int], pool_size: int,
                           zero_padding: bool = True, slot_counts: Optional[torch.Tensor] = None) -> MergedRows:
    """train.py:146-163 with the extra outputs (row norms, distinct count,
    and with ``slot_counts`` the fetch count of every slot over the layers)."""
    slots, weights, grads = [], [], []
    for layer, sl, w in zip(layers, aux["slots"], aux["weights"]):
        g = probe_grads[layer]
        d = g.shape[-1]
        hk = sl.shape[-2] * sl.shape[-1]
        slots.append(sl.reshape(-1, hk).reshape(-1))
        weights.append(w.detach().reshape(-1))
        grads.append(g.reshape(-1, d))
    if len(slots) == 1:  # one layer: its own tensors (views), no concatenated copies
        return merge_fetches(slots[0], weights[0], grads[0], pool_size, zero_padding, slot_counts)
    return merge_fetches(torch.cat(slots), torch.cat(weights), torch.cat(grads), pool_size, zero_padding,
                         slot_counts)


def fetched_row_grads(aux: Dict, probe_grads, layers: Sequence[int], pool_size: int):
    """train.py:146-163: (unique_slots [cap], row_grads [cap, d])."""
    m = fetched_row_grads_full(aux, probe_grads, layers, pool_size)
    return m.uniq, m.rows


def clip_scale(row_sq: torch.Tensor, rest_sq: Optional[torch.Tensor], grad_clip: float,
               dense: Optional[Sequence[torch.Tensor]] = None) -> torch.Tensor:
    """train.py:395-397: device tensor [scale, gnorm].  ``dense`` (at most
    7 tensors, instead of rest_sq) adds the squares of the dense gradients
    in the same pass (mpl_clip_scale_dense)."""
    dev = row_sq.device
    out = torch.empty(2, dtype=torch.float32, device=dev)
    if dense is not None:
        if rest_sq is not None:
            raise ValueError("give the dense gradients either as rest_sq or as dense, not both")
        if len(dense) > 7:
            raise ValueError("clip_scale takes at most 7 dense gradient tensors")
        xs = [t.detach().reshape(-1).float().contiguous() for t in dense]
        L = _lib.lib()
        wsb = L.mpl_clip_scale_workspace_bytes()
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        ptrs = (C.c_void_p * max(len(xs), 1))(*[x.data_ptr() for x in xs])
        ns = (C.c_int64 * max(len(xs), 1))(*[x.numel() for x in xs])
        rs = row_sq.contiguous()
        check(L.mpl_clip_scale_dense(ptr(rs), rs.shape[0], C.cast(ptrs, C.c_void_p), C.cast(ns, C.c_void_p),
                                     len(xs), float(grad_clip), ptr(out), ptr(ws), wsb, _lib.stream_ptr(dev)),
              "mpl_clip_scale_dense")
        return out
    if rest_sq is not None:
        rest_sq = rest_sq.reshape(1).float().contiguous()
    L = _lib.lib()
    wsb = L.mpl_clip_scale_workspace_bytes()
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    check(L.mpl_clip_scale(ptr(row_sq.contiguous()), row_sq.shape[0], ptr(rest_sq), float(grad_clip), ptr(out),
                           ptr(ws), wsb, _lib.stream_ptr(dev)), "mpl_clip_scale")
    return out


def sum_squares(tensors: Sequence[torch.Tensor], add: Optional[torch.Tensor] = None) -> torch.Tensor:
    """train.py:395-397: the squared global norm of the dense gradients,
    sum of x^2 over ``tensors`` (fp32, at most 8; each made contiguous) plus
    ``add`` (a device scalar or None), as a device fp32 tensor [1].  Fixed
    order with fp64 accumulation, no memset: it captures in a HIP graph, where
    torch's multi-block sum records a memset of its semaphores."""
    if len(tensors) > 8:
        head = sum_squares(tensors[:8], add)
        return sum_squares(tensors[8:], head)
    dev = tensors[0].device if tensors else add.device
    xs = [t.detach().reshape(-1).float().contiguous() for t in tensors]
    out = torch.empty(1, dtype=torch.float32, device=dev)
    if add is not None:
        add = add.reshape(1).float().contiguous()
    L = _lib.lib()
    wsb = L.mpl_sum_squares_workspace_bytes()
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ptrs = (C.c_void_p * max(len(xs), 1))(*[x.data_ptr() for x in xs])
    ns = (C.c_int64 * max(len(xs), 1))(*[x.numel() for x in xs])
    check(L.mpl_sum_squares(C.cast(ptrs, C.c_void_p), C.cast(ns, C.c_void_p), len(xs), ptr(add), ptr(out), ptr(ws),
                            wsb, _lib.stream_ptr(dev)), "mpl_sum_squares")
    return out


def rowwise_adagrad(values: torch.Tensor, acc: torch.Tensor, uniq: torch.Tensor, rows: torch.Tensor, lr: float,
                    master: Optional[torch.Tensor] = None, grad_scale: Optional[torch.Tensor] = None) -> None:
    """train.py:412-416, in place on values / master / acc."""
    _check_table(values, master)
    cap, d = rows.shape
    check(_lib.lib().mpl_row_adagrad(ptr(values), _vcode(values), ptr(master), ptr(acc), ptr(uniq.contiguous()),
                                     ptr(rows.contiguous()), cap, d, values.shape[0], float(lr), ptr(grad_scale),
                                     _lib.stream_ptr(values.device)), "mpl_row_adagrad")


def lazy_adam(values: torch.Tensor, m: torch.Tensor, v: torch.Tensor, uniq: torch.Tensor, rows: torch.Tensor,
              lr: float, step: int, master: Optional[torch.Tensor] = None,
              grad_scale: Optional[torch.Tensor] = None) -> None:
    """train.py:417-426, in place; ``step`` is the 0-based TrainState.step."""
    _check_table(values, master)
    cap, d = rows.shape
    check(_lib.lib().mpl_row_adam(ptr(values), _vcode(values), ptr(master), ptr(m), ptr(v), ptr(uniq.contiguous()),
                                  ptr(rows.contiguous()), cap, d, values.shape[0], float(lr), int(step),
                                  ptr(grad_scale), _lib.stream_ptr(values.device)), "mpl_row_adam")


def _check_table(values, master):
    if not values.is_contiguous() or values.dim() != 2:
        raise ValueError("pool values must be a contiguous [N, d] tensor")
    if master is not None and (master.shape != values.shape or master.dtype != torch.float32
                               or not master.is_contiguous()):
        raise ValueError("master must be a contiguous fp32 tensor shaped like values")


def warmup_cosine(step: int, lr: float, warmup_steps: int, steps: int) -> float:
    """train.py:100-103: optax.warmup_cosine_decay_schedule(0, lr, warmup,
    max(steps, warmup + 1), 0.1 * lr) evaluated at ``step``."""
    decay_steps = max(steps, warmup_steps + 1)
    if step < warmup_steps:
        return lr * step / warmup_steps
    d = decay_steps - warmup_steps
    t = min(step - warmup_steps, d)
    return lr * (0.9 * 0.5 * (1.0 + math.cos(math.pi * t / d)) + 0.1)


class SparseRowUpdate:
    """The sparse pool update of train.py:378-429 on one GPU.

    Holds the pool optimizer state: ``acc`` [N] (row-wise Adagrad, the
    default ``pool_optimizer``) or ``m``, ``v`` [N, d] (lazy Adam), and an
    optional fp32 ``master`` copy of an fp16 table.  ``values`` may instead
    be a HostPool (model_amd/host_pool.py; train.py:210-221, 250-258): the
    pool then keeps its own optimizer state and receives the merged, clipped
    rows with the 1-based step."""

    def __init__(self, values, *, optimizer: str = "rowwise_adagrad", lr: float = 3e-4,
                 pool_lr_mult: float = 3.0, warmup_steps: int = 0, steps: int = 1, grad_clip: float = 1.0,
                 master: bool = True):
        if optimizer not in ("rowwise_adagrad", "adam"):
            raise ValueError(f"unknown pool optimizer {optimizer!r}")
        self.optimizer = optimizer
        self.lr, self.pool_lr_mult = lr, pool_lr_mult
        self.warmup_steps, self.steps, self.grad_clip = warmup_steps, steps, grad_clip
        self.step = 0
        self.host = None
        if not isinstance(values, torch.Tensor):  # a HostPool
            if values.optimizer != optimizer:
                raise ValueError(f"host pool optimizer {values.optimizer!r} != {optimizer!r}")
            self.host, self.values = values, None
            self.master = self.acc = self.m = self.v = None
            return
        self.values = values
        N, d = values.shape
        dev = values.device
        self.master = values.float().clone() if (master and values.dtype != torch.float32) else None
        if optimizer == "rowwise_adagrad":
            self.acc = torch.zeros(N, dtype=torch.float32, device=dev)
            self.m = self.v = None
        else:
            self.acc = None
            self.m = torch.zeros((N, d), dtype=torch.float32, device=dev)
            self.v = torch.zeros((N, d), dtype=torch.float32, device=dev)
        self.step = 0

    def resume(self, state: Dict) -> None:
        """Continues from a TrainState checkpoint (checkpoint.load_train_state,
        train.py:36-44, 559-583): the step count (state.step, the 0-based
        step of the next update), and the pool optimizer state: row-wise
        Adagrad's accumulator is TrainState.pool_v [N] (pool_m is empty,
        train.py:284-285); lazy Adam's moments are pool_m, pool_v [N, d].
        With an fp32 master the master takes the checkpoint's fp32 table
        (params/pool/values) and the table its cast."""
        if self.host is not None:
            raise ValueError("a host pool keeps its own state: load it with HostPool.load (train.py:576)")
        N, d = self.values.shape
        self.step = int(state["step"])
        pm, pv = state["pool_m"], state["pool_v"]
        if self.optimizer == "rowwise_adagrad":
            if tuple(pv.shape) != (N,):
                raise ValueError(f"pool_v must be [{N}] for rowwise_adagrad, got {tuple(pv.shape)}")
            self.acc.copy_(pv)
        else:
            if tuple(pm.shape) != (N, d) or tuple(pv.shape) != (N, d):
                raise ValueError(f"pool_m / pool_v must be [{N}, {d}] for adam, got {tuple(pm.shape)}, {tuple(pv.shape)}")
            self.m.copy_(pm)
            self.v.copy_(pv)
        table = state["params"]["pool"]["values"] if "values" in state["params"].get("pool", {}) else None
        if table is not None:
            if tuple(table.shape) != (N, d):
                raise ValueError(f"params/pool/values must be [{N}, {d}], got {tuple(table.shape)}")
            if self.master is not None:
                self.master.copy_(table)
            self.values.copy_(table)

    def train_state_pool(self) -> Dict[str, torch.Tensor]:
        """The pool fields of a TrainState for checkpoint.save_train_state:
        step, pool_m, pool_v (and the fp32 table to store as
        params/pool/values: the master when kept)."""
        dev = self.values.device
        empty = torch.zeros(0, dtype=torch.float32, device=dev)
        if self.optimizer == "rowwise_adagrad":
            pm, pv = empty, self.acc
        else:
            pm, pv = self.m, self.v
        table = self.master if self.master is not None else self.values.float()
        return {"step": self.step, "pool_m": pm, "pool_v": pv, "values": table}

    def merge(self, aux: Dict, probe_grads, layers: Sequence[int], count_slots: bool = False) -> Dict:
        """The first half of an update (train.py:146-172): the fetched rows'
        gradients merged per slot, on the current stream, as a handle for
        apply().  It depends only on the forward's slots and weights and the
        probe gradients, so a training step may run it on a second stream
        beside the dense backward (the handle's tensors are marked for the
        stream apply() runs on).  With count_slots the handle also carries
        the per-slot fetch counts (memory.py:215)."""
        N = self.host.n_slots if self.host is not None else self.values.shape[0]
        dev = self.values.device if self.values is not None else aux["slots"][0].device
        stream = torch.cuda.current_stream(dev)
        for layer, sl, w in zip(layers, aux["slots"], aux["weights"]):
            for t in (sl, w, probe_grads[layer]):  # read here, perhaps made on another stream
                if t.is_cuda:
                    t.record_stream(stream)
        counts = torch.empty(N, dtype=torch.float32, device=dev) if count_slots else None
        merged = fetched_row_grads_full(aux, probe_grads, layers, N, zero_padding=False,  # optimizers skip padding
                                        slot_counts=counts)
        return {"merged": merged, "slot_counts": counts}

    def apply(self, handle: Dict, rest_sq: Optional[torch.Tensor] = None,
              dense_grads: Optional[Sequence[torch.Tensor]] = None) -> Dict[str, torch.Tensor]:
        """The second half (train.py:395-429): the global-norm clip over the
        merged rows and the dense gradients (rest_sq, their squared norm as
        a device scalar, or dense_grads, the tensors, summed in the clip's
        own pass), then the row optimizer step.  Call it on a stream that
        has waited for the merge's."""
        merged, counts = handle["merged"], handle["slot_counts"]
        stream = torch.cuda.current_stream(merged.rows.device)
        for t in (merged.uniq, merged.rows, merged.row_sq, merged.num_unique, counts):
            if t is not None:
                t.record_stream(stream)
        sg = clip_scale(merged.row_sq, rest_sq, self.grad_clip, dense_grads)
        lr = warmup_cosine(self.step, self.lr, self.warmup_steps, self.steps) * self.pool_lr_mult
        scale = sg[0:1]
        if self.host is not None:
            self.host.update(merged.uniq, merged.rows, self.step + 1, lr, grad_scale=scale)
        elif self.optimizer == "rowwise_adagrad":
            rowwise_adagrad(self.values, self.acc, merged.uniq, merged.rows, lr, self.master, scale)
        else:
            lazy_adam(self.values, self.m, self.v, merged.uniq, merged.rows, lr, self.step, self.master, scale)
        self.step += 1
        out = {"grad_scale": sg[0], "grad_norm": sg[1], "rows_updated": merged.num_unique[0],
               "uniq": merged.uniq, "row_grads": merged.rows}
        if counts is not None:
            out["slot_counts"] = counts
        return out

    def __call__(self, aux: Dict, probe_grads, layers: Sequence[int],
                 rest_sq: Optional[torch.Tensor] = None, count_slots: bool = False,
                 dense_grads: Optional[Sequence[torch.Tensor]] = None) -> Dict[str, torch.Tensor]:
        """One update from the fetches of ``layers`` (aux["slots"][i],
        aux["weights"][i], probe_grads[layer]): merge() then apply().  With
        count_slots the result also holds "slot_counts" [N] fp32, the fetches
        of every slot summed over the layers (the aux slot_counts of
        memory.py:215 / model.py:136 that train.py:456 folds into the usage
        average), from the merge's own sort instead of a separate histogram.
        The global norm takes the dense gradients as rest_sq (their squared
        norm, a device scalar) or as dense_grads (the tensors, summed in the
        clip's own pass)."""
        return self.apply(self.merge(aux, probe_grads, layers, count_slots), rest_sq, dense_grads)
