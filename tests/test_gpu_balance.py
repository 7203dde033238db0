"""Routing counts and the fused load-balance loss on the GPU (include/mpl.h
mpl_route_counts, mpl_balance_fwd, mpl_lookup_bwd_dense) against the oracle
(oracle/lookup.py aux_stats and oracle/backward.py lookup_backward, fp64).

Counts are integers and must match exactly.  The balance loss and its
gradients come from MFMA score tiles of the scoring precision.  fp16: the
loss is checked to 1e-3 relative, the gradients to 1e-2 of their largest
magnitude (the fp16-path tolerance); fp32: 1e-5 for both.  d
log_temperature is measured against the sum of the magnitudes of its
terms."""

import numpy as np
import pytest
import torch

from model_amd import _lib
from model_amd._lib import check, ptr
from model_amd.memory import MemoryPool
from oracle import backward as ob
from oracle import lookup as ol
from tests.test_gpu_backward import _check, _setup, _with_selection

pytestmark = pytest.mark.gpu


def _bincount_in_range(ids, size):
    ids = ids[(ids >= 0) & (ids < size)]
    return np.bincount(ids, minlength=size).astype(np.float32)


@pytest.mark.parametrize("M,H,n,k", [
    (3000, 4, 512, 16),   # LDS histograms
    (777, 2, 5000, 8),    # n > 4096: direct atomics
    (5, 1, 7, 3),         # tiny
    (0, 2, 16, 4),        # no tokens: all counts zero
])
def test_route_counts_exact(gpu_lib, M, H, n, k):
    """memory.py:199-204, 206-208, 215 as numpy bincounts; ids out of range
    are not counted."""
    rng = np.random.default_rng(M + n)
    slots = rng.integers(0, n * n, (M, H, k)).astype(np.int32)
    clean = rng.integers(0, n, (M, H, 2, k)).astype(np.int32)
    if M > 1:
        slots[0, 0, 0] = -1
        slots[-1, -1, -1] = n * n
        clean[1, 0, 1, 0] = n
    dev = "cuda"
    ts, tc = torch.tensor(slots, device=dev), torch.tensor(clean, device=dev)
    sub = torch.full((H, 2, n), 7.0, device=dev)  # outputs are overwritten
    cln = torch.full((H, 2, n), 7.0, device=dev)
    sc = torch.full((n * n,), 7.0, device=dev)
    check(_lib.lib().mpl_route_counts(ptr(ts), ptr(tc), M, H, n, k, ptr(sub), ptr(cln), ptr(sc),
                                      _lib.stream_ptr(torch.device(dev))), "mpl_route_counts")
    want_sub = np.zeros((H, 2, n), np.float32)
    want_cln = np.zeros((H, 2, n), np.float32)
    for h in range(H):
        s = slots[:, h].reshape(-1)
        s = s[(s >= 0) & (s < n * n)]
        want_sub[h, 0] = np.bincount(s // n, minlength=n)
        want_sub[h, 1] = np.bincount(s % n, minlength=n)
        for c in range(2):
            want_cln[h, c] = _bincount_in_range(clean[:, h, c].reshape(-1), n)
    np.testing.assert_array_equal(sub.cpu().numpy(), want_sub)
    np.testing.assert_array_equal(cln.cpu().numpy(), want_cln)
    np.testing.assert_array_equal(sc.cpu().numpy(), _bincount_in_range(slots.reshape(-1), n * n))


def test_aux_counts_under_noise(gpu_lib):
    """A noisy training lookup: subkey_counts / slot_counts come from the
    final slots, and their sums are M*H*k per codebook (tests:30-37)."""
    n, H, k, M = 128, 2, 8, 500
    pool = MemoryPool(n, H, 64, 32, k, values_dtype=torch.float16)
    g = torch.Generator(device="cuda").manual_seed(3)
    params = {"sub_keys": torch.randn((H, 2, n, 32), generator=g, device="cuda"),
              "values": torch.randn((n * n, 32), generator=g, device="cuda").half(),
              "log_temperature": torch.tensor(np.log(10.0), device="cuda")}
    q = torch.randn((M, H, 64), generator=g, device="cuda")
    res = pool.lookup(params, q, train=True, rngs={"routing": 5})
    aux = res["aux"]
    slots = res["slots"].cpu().numpy()
    sc = aux["slot_counts"].cpu().numpy()
    np.testing.assert_array_equal(sc, np.bincount(slots.reshape(-1), minlength=n * n))
    skc = aux["subkey_counts"].cpu().numpy()
    for h in range(H):
        np.testing.assert_array_equal(skc[h, 0], np.bincount(slots[:, h].reshape(-1) // n, minlength=n))
        np.testing.assert_array_equal(skc[h, 1], np.bincount(slots[:, h].reshape(-1) % n, minlength=n))
    assert np.all(skc.sum(-1) == M * k)


@pytest.mark.parametrize("n,H,d_key,M,k,qs,btg,seed", [
    (512, 4, 256, 300, 16, False, False, 31),  # the text-study layer's widths
    (100, 2, 64, 77, 8, True, True, 32),       # n not a multiple of 32, ragged M, q_len in the logits
    (64, 2, 16, 40, 4, False, True, 33),       # half = 8, temperature gradient
    (256, 1, 128, 50, 16, True, False, 34),    # query_scale without balance_temperature_grad
])
def test_balance_loss_and_gradients(gpu_lib, n, H, d_key, M, k, qs, btg, seed):
    """loss = balance_loss alone (g_out = 0): the dense-over-n gradient of
    memory.py:208-213 through the raw queries, raw sub-keys and
    log_temperature, for the GPU's selection."""
    pool, params, tq, q, keys, vals, _, log_t = _setup(
        seed, n=n, H=H, d_key=d_key, d=16, k=k, M=M, values_dtype=torch.float16, score_dtype=torch.float16,
        query_scale=qs, btg=btg)
    res_gpu = pool.lookup(params, tq.detach())
    out, aux = pool.apply({"params": params}, tq, sparse_grad=True)
    assert "_state" in aux.internal, "the fused balance path must run for fp16 scoring"
    gq, gk, gt = torch.autograd.grad(aux["balance_loss"], [tq, params["sub_keys"], params["log_temperature"]])

    res = ol.lookup_forward(q, keys, vals, float(log_t), top_k_=k, query_scale=qs, dtype=np.float64)
    sel = _with_selection(res, res_gpu["sub_idx"].cpu().numpy(), res_gpu["flat_idx"].cpu().numpy(),
                          res_gpu["slots"].cpu().numpy())
    ao = ol.aux_stats(sel, n=n, noisy=False, balance_temperature_grad=btg)
    np.testing.assert_allclose(float(aux["balance_loss"]), ao["balance_loss"], rtol=1e-3)
    ref = ob.lookup_backward(sel, vals, np.zeros((M, 16)), n=n, query_scale=qs, g_balance=1.0, f=ao["_f"],
                             balance_temperature_grad=btg)
    _check(gq.cpu().numpy(), ref["d_queries"], 1e-2, "d_queries")
    _check(gk.cpu().numpy(), ref["d_sub_keys"], 1e-2, "d_sub_keys")
    if btg:
        lt_scale = float(np.abs(ref["d_cos"] * sel["cos"]).sum())
        _check(float(gt), ref["d_log_temperature"], 1e-2, "d_log_temperature", lt_scale)
    else:
        assert float(gt) == 0.0  # T is stop-gradient in the balance logits (memory.py:210)


@pytest.mark.parametrize("n,H,d_key,M,k,qs,btg,seed", [
    (128, 4, 256, 1024, 16, False, False, 51),  # the fact-task layer: fp32, 16,384 slots, 1,024 tokens
    (100, 2, 20, 77, 8, True, True, 52),        # half = 10 (not a multiple of 8), ragged n and M
    (300, 1, 64, 513, 4, False, True, 53),      # query range split over workgroups, temperature gradient
    (40, 2, 6, 33, 5, True, False, 54),         # half = 3: the narrowest padded width (8)
])
def test_balance_loss_and_gradients_fp32(gpu_lib, n, H, d_key, M, k, qs, btg, seed):
    """memory.py:208-213 with fp32 scoring on v_mfma_f32_32x32x2_f32 tiles
    (mpl_balance_fwd / mpl_lookup_bwd_dense with MPL_F32): loss and the
    gradients through the raw queries, raw sub-keys and log_temperature,
    against the fp64 oracle for the GPU's selection, to 1e-5."""
    pool, params, tq, q, keys, vals, _, log_t = _setup(
        seed, n=n, H=H, d_key=d_key, d=16, k=k, M=M, values_dtype=torch.float32, score_dtype=torch.float32,
        query_scale=qs, btg=btg)
    res_gpu = pool.lookup(params, tq.detach())
    out, aux = pool.apply({"params": params}, tq, sparse_grad=True)
    assert "_state" in aux.internal
    gq, gk, gt = torch.autograd.grad(aux["balance_loss"], [tq, params["sub_keys"], params["log_temperature"]])
    res = ol.lookup_forward(q, keys, vals, float(log_t), top_k_=k, query_scale=qs, dtype=np.float64)
    sel = _with_selection(res, res_gpu["sub_idx"].cpu().numpy(), res_gpu["flat_idx"].cpu().numpy(),
                          res_gpu["slots"].cpu().numpy())
    ao = ol.aux_stats(sel, n=n, noisy=False, balance_temperature_grad=btg)
    np.testing.assert_allclose(float(aux["balance_loss"]), ao["balance_loss"], rtol=1e-5)
    ref = ob.lookup_backward(sel, vals, np.zeros((M, 16)), n=n, query_scale=qs, g_balance=1.0, f=ao["_f"],
                             balance_temperature_grad=btg)
    _check(gq.cpu().numpy(), ref["d_queries"], 1e-5, "d_queries")
    _check(gk.cpu().numpy(), ref["d_sub_keys"], 1e-5, "d_sub_keys")
    if btg:
        lt_scale = float(np.abs(ref["d_cos"] * sel["cos"]).sum())
        _check(float(gt), ref["d_log_temperature"], 1e-5, "d_log_temperature", lt_scale)
    else:
        assert float(gt) == 0.0


def test_balance_loss_of_no_tokens_is_nan(gpu_lib):
    """memory.py:208-213 with M = 0: f = counts / (M k) and the mean over
    tokens are both 0/0."""
    for sd in (torch.float16, torch.float32):
        pool, params, tq, *_ = _setup(55, n=64, H=2, d_key=32, d=16, k=4, M=3, values_dtype=torch.float16,
                                      score_dtype=sd, query_scale=False, btg=False)
        out, aux = pool.apply({"params": params}, tq[:0])
        assert out.shape == (0, 16) and torch.isnan(aux["balance_loss"])


@pytest.mark.parametrize("fused", [False, True])
def test_balance_scales_with_upstream_gradient_and_matches_dense_path(gpu_lib, monkeypatch, fused):
    """The fp16 path against the fp32 path of the same module on one input:
    the losses agree to the fp16 scoring error and the gradients scale
    linearly with the balance coefficient: to fp32 rounding with the
    separate query pass (the fp16 operand there does not depend on the
    coefficient), to the fp16 operand's rounding (2^-11 relative) when the
    routed term shares the query pass (mpl_lookup_bwd_dense_queries, whose
    operand scale follows the coefficient)."""
    from model_amd import memory as mem
    monkeypatch.setattr(mem, "FUSED_QUERY_BWD", fused)
    n, H, d_key, M, k = 128, 2, 64, 200, 8
    pool16, params, tq, *_ = _setup(41, n=n, H=H, d_key=d_key, d=16, k=k, M=M, values_dtype=torch.float16,
                                    score_dtype=torch.float16, query_scale=False, btg=False)
    pool32 = MemoryPool(n, H, d_key, 16, k, values_dtype=torch.float16, score_dtype=torch.float32)
    _, a16 = pool16.apply({"params": params}, tq, sparse_grad=True)
    _, a32 = pool32.apply({"params": params}, tq, sparse_grad=True)
    np.testing.assert_allclose(float(a16["balance_loss"]), float(a32["balance_loss"]), rtol=1e-3)
    g1 = torch.autograd.grad(0.01 * a16["balance_loss"], [tq], retain_graph=True)[0]
    g2 = torch.autograd.grad(0.03 * a16["balance_loss"], [tq])[0]
    if fused:
        torch.testing.assert_close(g2, 3.0 * g1, rtol=0, atol=1e-3 * float(g2.abs().max()))
    else:
        torch.testing.assert_close(g2, 3.0 * g1, rtol=1e-5, atol=1e-12)
