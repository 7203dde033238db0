"""Forward memory-layer lookup restated in numpy.  TEST INFRASTRUCTURE ONLY.

Follows KumarDev7/model ``memory_pool_model/memory.py``:
  * ``l2_normalize``   memory.py:30-31
  * ``top_k``          memory.py:34-57 (lax.top_k semantics: descending,
                       ties broken by lowest index, as the argmax loop of
                       memory.py:34-45 documents and tests:55-63 pins)
  * ``lookup_forward`` memory.py:132-193
  * ``aux_stats``      memory.py:196-226
  * ``key_diversity_loss`` memory.py:230-240
  * ``revive_dead_keys``   memory.py:243-281 (the random draws are inputs)

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only to check results.
"""

from __future__ import annotations

import numpy as np

NORM_EPS = 1e-6  # memory.py:30 default eps, also the q_len eps of memory.py:137


def l2_normalize(x: np.ndarray, eps: float = NORM_EPS) -> np.ndarray:
    """memory.py:30-31: ``x * rsqrt(sum(x*x, -1) + eps)`` in x's own dtype."""
    x = np.asarray(x)
    dt = x.dtype.type
    s = np.sum(x * x, axis=-1, keepdims=True, dtype=x.dtype)
    return x * (dt(1.0) / np.sqrt(s + dt(eps))).astype(x.dtype)


def _top_k_partition(flat: np.ndarray, k: int) -> np.ndarray:
    """Exact top-k indices for long rows: partition to the k-th largest value,
    then order every candidate >= it by (value desc, index asc)."""
    rows_n, n = flat.shape
    kth = np.partition(flat, n - k, axis=1)[:, n - k]
    rows, cols = np.nonzero(flat >= kth[:, None])
    vals = flat[rows, cols]
    order = np.lexsort((cols, -vals, rows))
    rows, cols = rows[order], cols[order]
    starts = np.searchsorted(rows, np.arange(rows_n))
    return cols[starts[:, None] + np.arange(k)[None, :]]


def top_k(x: np.ndarray, k: int):
    """Values and indices of the k largest entries along the last axis.

    memory.py:48-57 dispatches to ``lax.top_k`` (CPU) or an argmax loop (GPU,
    memory.py:34-45); both return descending values with ties resolved to the
    lowest index first.  Restated as a stable sort of the negated values.
    """
    x = np.asarray(x)
    lead, n = x.shape[:-1], x.shape[-1]
    if not 0 < k <= n:
        raise ValueError(f"top_k: need 0 < k <= {n}, got {k}")
    flat = x.reshape(-1, n)
    if n <= 4096 or flat.shape[0] * n <= (1 << 22):
        idx = np.argsort(-flat, axis=1, kind="stable")[:, :k]
    else:
        idx = _top_k_partition(flat, k)
    vals = np.take_along_axis(flat, idx, axis=1)
    return vals.reshape(*lead, k), idx.reshape(*lead, k)


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """jax.nn.softmax as used at memory.py:178 and memory.py:211."""
    x = np.asarray(x)
    e = np.exp(x - np.max(x, axis=axis, keepdims=True))
    return e / np.sum(e, axis=axis, keepdims=True)


def clamp_temperature(log_temperature, min_temperature: float, max_temperature: float,
                      dtype=np.float32):
    """memory.py:143-146: the value is exp(clip(log_t, log min, log max)); the
    gradient passes straight through (d T / d log_t = T)."""
    dt = np.dtype(dtype).type
    log_t = dt(log_temperature)
    log_t = np.clip(log_t, np.log(dt(min_temperature)), np.log(dt(max_temperature)))
    return dt(np.exp(log_t))


def cosine_scores(q_hat: np.ndarray, k_hat: np.ndarray) -> np.ndarray:
    """memory.py:149: einsum("mhcd,hcnd->mhcn") as one BLAS product per (h, c)."""
    M, H, C, _ = q_hat.shape
    n = k_hat.shape[2]
    cos = np.empty((M, H, C, n), dtype=np.result_type(q_hat, k_hat))
    for h in range(H):
        for c in range(C):
            cos[:, h, c, :] = q_hat[:, h, c, :] @ k_hat[h, c].T
    return cos


def lookup_forward(queries, sub_keys, values, log_temperature, *, top_k_: int,
                   min_temperature: float = 10.0, max_temperature: float = 100.0,
                   query_scale: bool = False, gumbel=None, noise_coef: float = 0.0,
                   shuffle_reads: bool = False, dtype=np.float32,
                   with_dense: bool = True) -> dict:
    """memory.py:132-193 for queries [..., H, d_key] and sub_keys [H, 2, n, d_key/2].

    ``values`` may be None (selection only) or [n*n, d_value] in any float
    dtype; rows are read as float (host_pool.py:117-127 returns float32 rows
    for an fp16 table).  ``gumbel`` [M, H, 2, n] replaces jax.random.gumbel of
    memory.py:156 (the noise is an input so both sides see the same draw);
    the select scores are ``scores + noise_coef * gumbel`` (memory.py:157).
    ``dtype`` is the arithmetic dtype (float32 = the reference's; float64 for
    near-tie analysis).
    """
    dt = np.dtype(dtype).type
    H, C, n, half = sub_keys.shape
    if C != 2:
        raise ValueError("sub_keys must be [H, 2, n, d_key/2]")
    k = int(top_k_)
    lead = queries.shape[:-2]
    q = np.asarray(queries, dtype=dtype).reshape(-1, H, 2, half)
    M = q.shape[0]
    q_len = np.sqrt(np.sum(q * q, axis=-1, keepdims=True, dtype=dtype) + dt(NORM_EPS)) / dt(np.sqrt(half))
    q_hat = l2_normalize(q)
    k_hat = l2_normalize(np.asarray(sub_keys, dtype=dtype))
    T = clamp_temperature(log_temperature, min_temperature, max_temperature, dtype)

    cos = cosine_scores(q_hat, k_hat)
    scores = cos * T
    if query_scale:
        scores = scores * q_len
    if gumbel is not None:
        select = scores + dt(noise_coef) * np.asarray(gumbel, dtype=dtype).reshape(scores.shape)
    else:
        select = scores

    # stage 1 (memory.py:162-164)
    _, sub_idx = top_k(select, k)
    sub_scores = np.take_along_axis(scores, sub_idx, axis=-1)
    sub_select = np.take_along_axis(select, sub_idx, axis=-1)
    # stage 2 (memory.py:167-175)
    cand = (sub_scores[..., 0, :, None] + sub_scores[..., 1, None, :]).reshape(M, H, k * k)
    cand_sel = (sub_select[..., 0, :, None] + sub_select[..., 1, None, :]).reshape(M, H, k * k)
    _, flat_idx = top_k(cand_sel, k)
    slot_scores = np.take_along_axis(cand, flat_idx, axis=-1)
    idx_a = np.take_along_axis(sub_idx[:, :, 0, :], flat_idx // k, axis=-1)
    idx_b = np.take_along_axis(sub_idx[:, :, 1, :], flat_idx % k, axis=-1)
    slots = (idx_a.astype(np.int64) * n + idx_b).astype(np.int64)
    # softmax + read (memory.py:178-193)
    weights = softmax(slot_scores, axis=-1)
    N = n * n
    read = (slots + N // 2 + 1) % N if shuffle_reads else slots
    res = dict(
        q=q, q_len=q_len, q_hat=q_hat, k_hat=k_hat, temperature=T,
        raw_keys=np.asarray(sub_keys, dtype=dtype),
        sub_idx=sub_idx, sub_scores=sub_scores, sub_select=sub_select,
        flat_idx=flat_idx, slot_scores=slot_scores, idx_a=idx_a, idx_b=idx_b,
        slots=slots, weights=weights, read_slots=read, lead_shape=lead,
    )
    if with_dense:
        res.update(cos=cos, scores=scores, select=select)
    if values is not None:
        res["out"] = gather_wsum(values, read, weights, dtype=dtype).reshape(*lead, -1)
    return res


def gather_wsum(values, read_slots, weights, dtype=np.float32) -> np.ndarray:
    """memory.py:186 + 192: out[m] = sum_{h,j} w[m,h,j] * values[read[m,h,j]]."""
    M = read_slots.shape[0]
    rows = np.asarray(values)[read_slots.reshape(-1)].astype(dtype)
    rows = rows.reshape(M, -1, rows.shape[-1])
    w = np.asarray(weights, dtype=dtype).reshape(M, -1)
    return np.einsum("mr,mrd->md", w, rows)


def aux_stats(res: dict, *, n: int, noisy: bool, balance_temperature_grad: bool = False) -> dict:
    """memory.py:196-226: usage counts, balance loss and the aux dict keys."""
    sub_idx, idx_a, idx_b = res["sub_idx"], res["idx_a"], res["idx_b"]
    M, H, _, k = sub_idx.shape
    codebook = (np.arange(H)[:, None, None] * 2 + np.arange(2)[None, :, None]) * n

    def count_subkeys(ids):  # memory.py:199-201
        flat = (ids + codebook[None]).reshape(-1)
        return np.bincount(flat, minlength=H * 2 * n).astype(np.float32).reshape(H, 2, n)

    subkey_counts = count_subkeys(np.stack([idx_a, idx_b], axis=2))
    clean_idx = top_k(res["scores"], k)[1] if noisy else sub_idx  # memory.py:207
    f = count_subkeys(clean_idx) / (M * k)
    T = res["temperature"]
    p_scores = res["scores"] if balance_temperature_grad else res["cos"] * T
    P = softmax(p_scores, axis=-1).mean(axis=0)
    balance_loss = n * np.mean(np.sum(f * P, axis=-1))
    slot_counts = np.bincount(res["slots"].reshape(-1), minlength=n * n).astype(np.float32)
    lead = res["lead_shape"]
    w = res["weights"]
    return {
        "balance_loss": np.float32(balance_loss),
        "subkey_counts": subkey_counts,
        "slot_counts": slot_counts,
        "queries": res["q_hat"],
        "slots": res["slots"].reshape(*lead, H, k),
        "weights": w.reshape(*lead, H, k),
        "temperature": T,
        "top1_weight": np.float32(w.max(-1).mean()),
        "_f": f,
    }


def near_tie_free_rows(queries, sub_keys, log_temperature, *, top_k_: int,
                       min_temperature: float = 10.0, max_temperature: float = 100.0,
                       query_scale: bool = False, gumbel=None, noise_coef: float = 0.0,
                       rel: float = 1e-3):
    """Rows (token, head) whose k-th and (k+1)-th select scores, computed in
    fp64 from the same inputs, differ by more than ``rel * |s_k|``.  Slot ids
    must match the reference exactly on these rows.

    Returns (mask [M, H] bool, fp64 forward result at k, fp64 k+1-th scores).
    The product-key search of memory.py:161-175 is exact for any k <= n, so
    running it at k+1 yields the true (k+1)-th best slot score.
    """
    kw = dict(min_temperature=min_temperature, max_temperature=max_temperature,
              query_scale=query_scale, gumbel=gumbel, noise_coef=noise_coef, dtype=np.float64,
              with_dense=False)
    n = sub_keys.shape[2]
    k1 = min(top_k_ + 1, n)
    r1 = lookup_forward(queries, sub_keys, None, log_temperature, top_k_=k1, **kw)
    sel = _slot_select_scores(r1)
    sk, sk1 = sel[..., top_k_ - 1], sel[..., k1 - 1]
    if k1 == top_k_:  # k == n: no (k+1)-th candidate, every row is tie free
        mask = np.ones(sk.shape, bool)
    else:
        mask = np.abs(sk - sk1) > rel * np.abs(sk)
    r = lookup_forward(queries, sub_keys, None, log_temperature, top_k_=top_k_, **kw)
    return mask, r


def _slot_select_scores(r: dict) -> np.ndarray:
    k = r["sub_idx"].shape[-1]
    ss = r["sub_select"]
    cand_sel = (ss[..., 0, :, None] + ss[..., 1, None, :]).reshape(ss.shape[0], ss.shape[1], k * k)
    return np.take_along_axis(cand_sel, r["flat_idx"], axis=-1)


def brute_force_slots(queries, sub_keys, log_temperature, *, top_k_: int, dtype=np.float64,
                      min_temperature: float = 10.0, max_temperature: float = 100.0,
                      query_scale: bool = False):
    """tests:40-52: top-k over all n*n slot sums, no product-key shortcut."""
    H, _, n, half = sub_keys.shape
    q = np.asarray(queries, dtype=dtype).reshape(-1, H, 2, half)
    T = clamp_temperature(log_temperature, min_temperature, max_temperature, dtype)
    s = cosine_scores(l2_normalize(q), l2_normalize(np.asarray(sub_keys, dtype=dtype))) * T
    if query_scale:
        s = s * (np.sqrt(np.sum(q * q, -1, keepdims=True) + NORM_EPS) / np.sqrt(half))
    full = (s[:, :, 0, :, None] + s[:, :, 1, None, :]).reshape(q.shape[0], H, n * n)
    return top_k(full, top_k_)[1]


def key_diversity_loss(sub_keys, dtype=np.float64) -> float:
    """memory.py:230-240: mean squared off-diagonal cosine inside each
    codebook, sum(offdiag(G)^2) / (H * 2 * n * (n - 1))."""
    keys = l2_normalize(np.asarray(sub_keys, dtype=dtype))
    H, C, n, _ = keys.shape
    gram = np.einsum("hcnd,hcmd->hcnm", keys, keys)
    off = gram * (1.0 - np.eye(n, dtype=dtype))
    return float(np.sum(off ** 2) / (H * C * n * (n - 1)))


def revive_dead_keys(sub_keys, subkey_usage, queries, pick, normal, threshold: float, noise: float = 0.05,
                     dtype=np.float64):
    """memory.py:243-281 with the two random draws given: ``pick`` [H,2,n]
    int (the jax.random.randint of :270) and ``normal`` [H,2,n,d] (the
    jax.random.normal of :274).  Returns (new_keys, new_usage, dead)."""
    keys = np.asarray(sub_keys, dtype=dtype)
    usage = np.asarray(subkey_usage, dtype=dtype)
    q = np.asarray(queries, dtype=dtype)
    H, C, n, d = keys.shape
    dead = usage < threshold / n                                     # :268
    h_idx = np.arange(H)[:, None, None]
    c_idx = np.arange(C)[None, :, None]
    replacement = q[np.asarray(pick), h_idx, c_idx]                  # :271-273
    replacement = l2_normalize(replacement + noise * np.asarray(normal, dtype=dtype))  # :274-275
    new_keys = np.where(dead[..., None], replacement, keys)          # :276
    new_usage = np.where(dead, 1.0 / n, usage)                       # :278
    new_usage = new_usage / new_usage.sum(axis=-1, keepdims=True)    # :280
    return new_keys, new_usage, dead
