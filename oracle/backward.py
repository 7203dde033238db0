"""Backward of the memory-layer lookup restated in numpy.  TEST INFRASTRUCTURE ONLY.

The reference has no hand-written backward: XLA differentiates
memory.py:136-213.  This module writes that derivative out so a HIP backward
can be checked against it.  It is itself pinned by torch-CPU autograd of an
independent torch restatement of the forward (tests/test_oracle.py).

Given the forward result of ``oracle.lookup.lookup_forward`` (its selection is
piecewise constant, so gradients flow only through the selected scores, the
softmax, the gather and the balance loss), returns gradients w.r.t. the raw
queries, raw sub_keys, log_temperature and (dense mode, sparse_grad=False,
memory.py:185) the value table.
"""

from __future__ import annotations

import numpy as np


def _l2_normalize_bwd(x: np.ndarray, dy: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """d/dx of x * (sum x^2 + eps)^-1/2  (memory.py:30-31)."""
    s = np.sum(x * x, axis=-1, keepdims=True) + eps
    r = 1.0 / np.sqrt(s)
    return r * dy - (r ** 3) * np.sum(x * dy, axis=-1, keepdims=True) * x


def lookup_backward(res: dict, values, g_out, *, n: int, query_scale: bool = False,
                    g_balance: float = 0.0, f=None, balance_temperature_grad: bool = False,
                    dense_values: bool = False, dtype=np.float64) -> dict:
    """Gradients of  <g_out, out> + g_balance * balance_loss  (memory.py:136-213).

    ``f`` is the stop-gradient usage fraction [H, 2, n] of memory.py:208
    (``aux_stats(...)["_f"]``); needed only when g_balance != 0.
    """
    q = res["q"].astype(dtype)
    M, H, _, half = q.shape
    k = res["sub_idx"].shape[-1]
    T = dtype(res["temperature"])
    q_hat = res["q_hat"].astype(dtype)
    k_hat = res["k_hat"].astype(dtype)
    q_len = res["q_len"].astype(dtype)
    w = res["weights"].astype(dtype)
    read = res["read_slots"]
    g = np.asarray(g_out, dtype=dtype).reshape(M, -1)

    rows = np.asarray(values)[read.reshape(-1)].astype(dtype).reshape(M, H, k, -1)
    dw = np.matmul(rows.reshape(M, H * k, -1), g[:, :, None]).reshape(M, H, k)  # memory.py:192
    ds = w * (dw - np.sum(w * dw, axis=-1, keepdims=True))         # softmax, memory.py:178
    fa, fb = res["flat_idx"] // k, res["flat_idx"] % k             # memory.py:167-175
    dsub = np.zeros((M, H, 2, k), dtype)
    mi, hi = np.meshgrid(np.arange(M), np.arange(H), indexing="ij")
    for j in range(k):
        np.add.at(dsub, (mi, hi, 0, fa[:, :, j]), ds[:, :, j])
        np.add.at(dsub, (mi, hi, 1, fb[:, :, j]), ds[:, :, j])
    # sub_scores = take(scores, sub_idx)   (memory.py:163)
    dscores = np.zeros((M, H, 2, n), dtype)
    np.put_along_axis(dscores, res["sub_idx"], dsub, axis=-1)

    dcos = np.zeros_like(dscores)
    dT = 0.0
    dq_len = np.zeros((M, H, 2, 1), dtype)
    cos = res["cos"].astype(dtype)
    scale = T * q_len if query_scale else T
    dcos += dscores * scale                                        # scores = cos*T(*q_len), memory.py:150-152
    dT += np.sum(dscores * cos * (q_len if query_scale else 1.0))
    if query_scale:
        dq_len += np.sum(dscores * cos * T, axis=-1, keepdims=True)

    if g_balance != 0.0:                                           # memory.py:208-213
        if f is None:
            raise ValueError("f (memory.py:208) is required when g_balance != 0")
        scores = res["scores"].astype(dtype)
        p_scores = scores if balance_temperature_grad else cos * T
        p = np.exp(p_scores - p_scores.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        dP = g_balance * n / (H * 2) * np.asarray(f, dtype)       # d(n*mean(sum f*P))/dP
        dp = np.broadcast_to(dP[None] / M, p.shape)                # P = mean_m p
        dps = p * (dp - np.sum(p * dp, axis=-1, keepdims=True))   # softmax over n
        if balance_temperature_grad:
            dcos += dps * scale
            dT += np.sum(dps * cos * (q_len if query_scale else 1.0))
            if query_scale:
                dq_len += np.sum(dps * cos * T, axis=-1, keepdims=True)
        else:
            dcos += dps * T

    # per codebook (h, c): dq_hat = dcos k_hat, dk_hat = dcos^T q_hat
    dq_hat = np.empty_like(q_hat)
    dk_hat = np.empty_like(k_hat)
    for h in range(H):
        for c in range(2):
            dq_hat[:, h, c] = dcos[:, h, c] @ k_hat[h, c]
            dk_hat[h, c] = dcos[:, h, c].T @ q_hat[:, h, c]
    dq = _l2_normalize_bwd(q, dq_hat)
    if query_scale:  # q_len = sqrt(sum q^2 + eps) / sqrt(half)   (memory.py:137)
        nrm = np.sqrt(np.sum(q * q, -1, keepdims=True) + 1e-6)
        dq += dq_len * q / (nrm * np.sqrt(half))
    raw_keys = res["raw_keys"].astype(dtype) if "raw_keys" in res else None
    if raw_keys is None:
        raise ValueError("res must carry 'raw_keys' (the un-normalised sub_keys)")
    dkeys = _l2_normalize_bwd(raw_keys, dk_hat)
    out = {
        "d_queries": dq.reshape(*res["lead_shape"], H, 2 * half),
        "d_sub_keys": dkeys,
        "d_log_temperature": dtype(dT * T),                        # straight-through clamp, memory.py:143-146
        "d_weights": dw, "d_slot_scores": ds, "d_sub_scores": dsub, "d_cos": dcos,
    }
    if dense_values:
        N = np.asarray(values).shape[0]
        dv = np.zeros((N, g.shape[1]), dtype)
        np.add.at(dv, read.reshape(-1), (w[..., None] * g[:, None, None, :]).reshape(-1, g.shape[1]))
        out["d_values"] = dv
    return out


def key_diversity_backward(sub_keys, dtype=np.float64) -> np.ndarray:
    """d key_diversity_loss / d sub_keys (memory.py:230-240 under autodiff):
    d k_hat = 4 / (H * 2 * n * (n - 1)) * (G - diag G) k_hat, then the
    l2-normalisation backward."""
    raw = np.asarray(sub_keys, dtype=dtype)
    s = np.sum(raw * raw, axis=-1, keepdims=True) + 1e-6
    k_hat = raw / np.sqrt(s)
    H, C, n, _ = raw.shape
    gram = np.einsum("hcnd,hcmd->hcnm", k_hat, k_hat)
    off = gram * (1.0 - np.eye(n, dtype=dtype))
    dk_hat = 4.0 / (H * C * n * (n - 1)) * np.einsum("hcnm,hcmd->hcnd", off, k_hat)
    return _l2_normalize_bwd(raw, dk_hat)
