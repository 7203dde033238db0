"""Shared helpers of the GPU parity tests: run the HIP lookup and compare it
with the oracle under the parity rule (exact slot sets wherever the k-th and
(k+1)-th fp64 select scores differ by more than 1e-3 relative)."""

from __future__ import annotations

import numpy as np
import torch

from model_amd.memory import MemoryPool
from oracle import lookup as ol

TOL = {torch.float16: 1e-2, torch.float32: 1e-5}  # parity tolerance: fp16 / fp32 paths, relative


def make_params(pool: MemoryPool, seed: int, *, key_std=None, value_std=None, device="cuda"):
    """Seeded synthetic parameters: sub_keys ~ N(0, key_std) (unit-sphere when
    None), values ~ N(0, value_std) (d^-1/2 when None) in the pool's dtype."""
    g = torch.Generator(device=device).manual_seed(seed)
    H, n, half = pool.heads, pool.n_sub_keys, pool.d_key // 2
    keys = torch.randn((H, 2, n, half), generator=g, device=device)
    if key_std is None:
        keys = keys * torch.rsqrt((keys * keys).sum(-1, keepdim=True) + 1e-6)
    else:
        keys = keys * key_std
    vstd = pool.d_value ** -0.5 if value_std is None else value_std
    values = torch.randn((pool.pool_size, pool.d_value), generator=g, device=device, dtype=pool.values_dtype)
    values.mul_(vstd)
    log_t = torch.tensor(np.log(pool.init_temperature), dtype=torch.float32, device=device)
    return {"sub_keys": keys, "values": values, "log_temperature": log_t}


def oracle_check(pool: MemoryPool, params, queries: torch.Tensor, res, *, gumbel=None, noise_coef=0.0,
                 shuffle_reads=False, min_tie_free=0.5, tol=None):
    """Asserts parity of one GPU lookup result `res` against the oracle
    (``tol``: the relative tolerance, by default the parity rule's for the
    pool's scoring precision)."""
    H, n, k, d = pool.heads, pool.n_sub_keys, pool.top_k, pool.d_value
    tol = TOL[pool.score_dtype] if tol is None else tol
    q = queries.detach().float().cpu().numpy()
    keys = params["sub_keys"].detach().float().cpu().numpy()
    log_t = float(params["log_temperature"].cpu())
    g = None if gumbel is None else gumbel.detach().float().cpu().numpy()
    mask, r = ol.near_tie_free_rows(q, keys, log_t, top_k_=k, min_temperature=pool.min_temperature,
                                    max_temperature=pool.max_temperature, query_scale=pool.query_scale,
                                    gumbel=g, noise_coef=noise_coef)
    M = mask.shape[0]
    assert mask.mean() >= min_tie_free, f"only {mask.mean():.2%} of rows are tie free"
    got = res["slots"].cpu().numpy().reshape(M, H, k).astype(np.int64)
    want = r["slots"]
    assert got.min() >= 0 and got.max() < n * n, "slot id out of range"
    diff = mask & np.any(np.sort(got, -1) != np.sort(want, -1), -1)
    assert not diff.any(), f"slot sets differ on {diff.sum()} tie-free rows, first at {np.argwhere(diff)[:3].tolist()}"
    # weights per slot on tie-free rows (softmax of the fp64 clean slot scores)
    gw = res["weights"].cpu().numpy().reshape(M, H, k).astype(np.float64)
    og = np.argsort(got, -1)
    ow = np.argsort(want, -1)
    gws = np.take_along_axis(gw, og, -1)[mask]
    wws = np.take_along_axis(r["weights"], ow, -1)[mask]
    np.testing.assert_allclose(gws, wws, rtol=tol, atol=tol * 1e-2)
    # sums to one
    np.testing.assert_allclose(gw.sum(-1), 1.0, rtol=1e-5)
    # value read: tokens whose heads are all tie free, against the pure oracle
    N = n * n
    read_want = (want + N // 2 + 1) % N if shuffle_reads else want
    vals = params["values"]
    rows_w = vals[torch.as_tensor(read_want.reshape(-1), device=vals.device)].float().cpu().numpy().astype(np.float64)
    out_want = np.einsum("mr,mrd->md", r["weights"].reshape(M, -1), rows_w.reshape(M, H * k, d))
    out_got = res["out"].detach().cpu().numpy().reshape(M, d).astype(np.float64)
    tok = mask.all(-1)
    scale = np.abs(out_want[tok]).max(-1, keepdims=True) + 1e-30
    err = np.abs(out_got[tok] - out_want[tok]) / scale
    assert err.size == 0 or err.max() <= tol, f"out relative error {err.max():.3g} > {tol}"
    # the gather alone: GPU slots and weights read back through fp64 arithmetic
    read_got = (got + N // 2 + 1) % N if shuffle_reads else got
    rows_g = vals[torch.as_tensor(read_got.reshape(-1), device=vals.device)].float().cpu().numpy().astype(np.float64)
    out_g64 = np.einsum("mr,mrd->md", gw.reshape(M, -1), rows_g.reshape(M, H * k, d))
    np.testing.assert_allclose(out_got, out_g64, rtol=2e-5, atol=2e-6 * (np.abs(out_g64).max() + 1e-30))
    return mask


def zipf_slots(M: int, H: int, k: int, N: int, *, s: float = 1.1, seed: int = 5) -> np.ndarray:
    """[M, H, k] int32 slots drawn by rank with p(r) ~ r^-s over 1..N, mapped
    through a fixed random permutation, distinct within each (token, head)."""
    rng = np.random.default_rng(seed)
    w = np.arange(1, N + 1, dtype=np.float64) ** -s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    perm = rng.permutation(N)
    G = M * H
    out = np.empty((G, k), dtype=np.int64)
    draws = np.minimum(np.searchsorted(cdf, rng.random((G, 8 * k))), N - 1)
    order = np.argsort(draws, axis=1, kind="stable")
    sd = np.take_along_axis(draws, order, 1)
    dup_sorted = np.zeros_like(sd, dtype=bool)
    dup_sorted[:, 1:] = sd[:, 1:] == sd[:, :-1]
    dup = np.empty_like(dup_sorted)
    np.put_along_axis(dup, order, dup_sorted, 1)
    nd = ~dup
    c = np.cumsum(nd, axis=1)
    full = c[:, -1] >= k
    out[full] = draws[full][(nd & (c <= k))[full]].reshape(-1, k)
    for g in np.flatnonzero(~full):  # extremely rare: top up with unused ranks
        first = draws[g][nd[g]]
        extra = np.setdiff1d(np.arange(N), first)[: k - first.shape[0]]
        out[g] = np.concatenate([first, extra])
    return perm[out].reshape(M, H, k).astype(np.int32)
