"""Sparse row gradients and row-wise optimizers restated in numpy.
TEST INFRASTRUCTURE ONLY.

Follows KumarDev7/model ``memory_pool_model/train.py``:
  * ``fetched_row_grads``  train.py:146-163
  * ``merge_rows``         train.py:166-172 (jnp.unique(size=cap,
                           fill_value=pool_size, return_inverse) +
                           jax.ops.segment_sum)
  * ``clip_scale``         train.py:395-399
  * ``rowwise_adagrad``    train.py:412-416 (host twin host_pool.py:145-152)
  * ``lazy_adam``          train.py:417-426 (host twin host_pool.py:154-163)
  * ``warmup_cosine``      train.py:100-103, i.e. optax>=0.2.3
                           ``warmup_cosine_decay_schedule`` (optax is not
                           installed; its published definition is restated)
"""

from __future__ import annotations

import math

import numpy as np

ADAM_B1, ADAM_B2, ADAM_EPS = 0.9, 0.999, 1e-8  # train.py:32
ADAGRAD_EPS = 1e-8                              # train.py:415, host_pool.py:28


def fetched_row_grads(slots_per_layer, weights_per_layer, g_per_layer, pool_size: int,
                      dtype=np.float32):
    """train.py:146-163: contributions w_f * dL/dout per fetch, concatenated
    over memory layers, then merged per distinct slot."""
    slots, contribs = [], []
    for sl, w, g in zip(slots_per_layer, weights_per_layer, g_per_layer):
        g = np.asarray(g, dtype=dtype)
        d = g.shape[-1]
        sl = np.asarray(sl).reshape(-1, sl.shape[-2] * sl.shape[-1])
        w = np.asarray(w, dtype=dtype).reshape(sl.shape)
        contribs.append((w[..., None] * g.reshape(-1, 1, d)).reshape(-1, d))
        slots.append(sl.reshape(-1))
    return merge_rows(np.concatenate(slots), np.concatenate(contribs), pool_size)


def merge_rows(slots, contribs, pool_size: int):
    """train.py:166-172.  cap = min(#fetches, pool_size); uniq ascending,
    padded with pool_size; rows[i] = sum of contribs whose slot == uniq[i]."""
    slots = np.asarray(slots).reshape(-1).astype(np.int64)
    contribs = np.asarray(contribs)
    cap = min(slots.shape[0], pool_size)
    u, inv = np.unique(slots, return_inverse=True)
    uniq = np.full(cap, pool_size, dtype=np.int64)
    uniq[: u.shape[0]] = u
    rows = np.zeros((cap, contribs.shape[-1]), dtype=contribs.dtype)
    np.add.at(rows, inv.reshape(-1), contribs)
    return uniq, rows


def clip_scale(rest_sq_norm: float, g_rows: np.ndarray, grad_clip: float) -> float:
    """train.py:395-399: one global norm over the dense grads and the rows."""
    gnorm = math.sqrt(float(rest_sq_norm) + float(np.sum(np.asarray(g_rows, np.float64) ** 2)))
    return min(1.0, grad_clip / (gnorm + 1e-6)), gnorm


def rowwise_adagrad(values, acc, uniq, g_rows, lr: float, master=None):
    """train.py:412-416, in place.  Padding entries (uniq >= N) are dropped
    (take mode="fill" fill 0; scatter mode="drop").  For a half-precision
    table the update is done in float32 and cast back (host_pool.py:152); with
    an fp32 ``master`` the master takes the update and the table is its cast."""
    N = values.shape[0]
    uniq = np.asarray(uniq).astype(np.int64)
    g = np.asarray(g_rows, dtype=np.float32)
    keep = uniq < N
    r = uniq[keep]
    gk = g[keep]
    a = acc[r] + np.mean(gk * gk, axis=-1, dtype=np.float32)
    step = -(np.float32(lr) / (np.sqrt(a) + np.float32(ADAGRAD_EPS)))[:, None] * gk
    _apply(values, master, r, step)
    acc[r] = a


def lazy_adam(values, m, v, uniq, g_rows, lr: float, step: int, master=None):
    """train.py:417-426, in place; ``step`` is the 0-based state.step, so the
    bias corrections use n = step + 1."""
    N = values.shape[0]
    uniq = np.asarray(uniq).astype(np.int64)
    g = np.asarray(g_rows, dtype=np.float32)
    keep = uniq < N
    r = uniq[keep]
    gk = g[keep]
    n = np.float32(step + 1)
    b1, b2 = np.float32(ADAM_B1), np.float32(ADAM_B2)
    # (1 - ADAM_B*) are Python-float expressions in train.py:421-422, rounded
    # once to fp32 by JAX's weak typing (not 1 - float32(b), which cancels)
    m_rows = b1 * m[r] + np.float32(1 - ADAM_B1) * gk
    v_rows = b2 * v[r] + np.float32(1 - ADAM_B2) * gk * gk
    c1 = np.float32(1) - b1 ** n
    c2 = np.float32(1) - b2 ** n
    upd = -np.float32(lr) * (m_rows / c1) / (np.sqrt(v_rows / c2) + np.float32(ADAM_EPS))
    _apply(values, master, r, upd)
    m[r] = m_rows
    v[r] = v_rows


def _apply(values, master, r, step):
    if master is not None:
        master[r] = master[r] + step
        values[r] = master[r].astype(values.dtype)
    elif values.dtype == np.float32:
        values[r] = values[r] + step
    else:
        values[r] = (values[r].astype(np.float32) + step).astype(values.dtype)


def warmup_cosine(step: int, lr: float, warmup_steps: int, steps: int) -> float:
    """train.py:100-103: optax.warmup_cosine_decay_schedule(0, lr, warmup,
    max(steps, warmup + 1), 0.1 * lr): linear 0 -> lr over ``warmup`` steps,
    then a half-cosine from lr down to 0.1 * lr, constant afterwards."""
    decay_steps = max(steps, warmup_steps + 1)
    if step < warmup_steps:
        return lr * step / warmup_steps
    d = decay_steps - warmup_steps
    t = min(step - warmup_steps, d)
    alpha = 0.1
    return lr * ((1.0 - alpha) * 0.5 * (1.0 + math.cos(math.pi * t / d)) + alpha)
