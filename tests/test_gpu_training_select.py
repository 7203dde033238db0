"""GPU parity of the training-time selection and its backward at the
training layer's widths (n_sub_keys = 512, H = 4, d_key = 256, k = 16 or 32,
d_value = 256) against the oracle, with routing noise on as the reference
trains (memory.py:155-164, train.py:378-416).

fp16 scoring with noise at a sub-key half of 128 runs the stage-1 kernel
that stages key blocks in LDS (k = 16 and k = 32 instantiations).  The
Gumbel draw is the library's own fill (mpl_gumbel_noise, seeded through
rngs["routing"]); the same tensor is handed to the oracle, so both sides
select on identical noisy scores.  Slot sets must match on near-tie-free
rows; weights (softmax of the clean scores) and gradients within the fp16
tolerance of 1e-2 relative."""

import numpy as np
import pytest
import torch

from model_amd.memory import MemoryPool
from oracle import backward as ob
from oracle import lookup as ol
from tests.gpu_helpers import make_params, oracle_check
from tests.test_gpu_backward import _check, _setup, _with_selection

pytestmark = pytest.mark.gpu

N_SUB, H, D_KEY, D = 512, 4, 256, 256


@pytest.mark.parametrize("k,M,noise_scale", [(16, 8192, 1.0), (16, 2048, 0.3), (32, 2048, 1.0)])
def test_noisy_selection_training_widths(gpu_lib, k, M, noise_scale):
    pool = MemoryPool(N_SUB, H, D_KEY, D, k, routing_noise=1.0, values_dtype=torch.float16)
    params = make_params(pool, 41 + k, key_std=(D_KEY // 2) ** -0.5, value_std=0.02)
    g = torch.Generator(device="cuda").manual_seed(42 + M)
    q = torch.randn((M, H, D_KEY), generator=g, device="cuda")
    print(f"noisy selection k={k} M={M} noise_scale={noise_scale}", flush=True)
    res = pool.lookup(params, q, train=True, noise_scale=noise_scale, rngs={"routing": 1234 + k})
    torch.cuda.synchronize()
    gumbel = res["gumbel"]
    assert gumbel is not None and tuple(gumbel.shape) == (M, H, 2, N_SUB)
    oracle_check(pool, params, q, res, gumbel=gumbel, noise_coef=noise_scale)
    # the noise moved picks: the clean lookup differs on some rows
    clean = pool.lookup(params, q)
    assert not torch.equal(clean["slots"], res["slots"])


def _stage1_tie_free(scores: np.ndarray, k: int) -> np.ndarray:
    """Rows of a stage-1 top-k whose k-th and (k+1)-th scores differ by more
    than 1e-3 relative (the clean top-k of memory.py:207)."""
    v, _ = ol.top_k(scores, k + 1)
    return np.abs(v[..., k - 1] - v[..., k]) > 1e-3 * np.abs(v[..., k - 1])


def test_training_backward_c4_with_noise(gpu_lib):
    """The training layer at its full token count (8,192) with noise on and
    balance coefficient 0.01: gradients of the queries, sub-keys and
    log-temperature for the GPU's selection against oracle/backward.py.  The
    balance loss's usage f comes from the clean stage-1 top-k (memory.py:207),
    which is also checked against the oracle's on its tie-free rows."""
    k, M, g_bal = 16, 8192, 0.01
    pool, params, tq, q, keys, vals, g, log_t = _setup(
        71, n=N_SUB, H=H, d_key=D_KEY, d=D, k=k, M=M, values_dtype=torch.float16, score_dtype=torch.float16,
        query_scale=False, btg=False)
    pool.routing_noise = 1.0
    rngs = {"routing": 77}
    res_gpu = pool.lookup(params, tq.detach(), train=True, rngs=rngs)
    out, aux = pool.apply({"params": params}, tq, train=True, sparse_grad=True, rngs=rngs)
    assert torch.equal(aux["slots"].reshape(M, H, k), res_gpu["slots"])  # same noise, same picks
    loss = (out * torch.tensor(g, device="cuda")).sum() + g_bal * aux["balance_loss"]
    gq, gk, gt = torch.autograd.grad(loss, [tq, params["sub_keys"], params["log_temperature"]])
    torch.cuda.synchronize()

    gum = res_gpu["gumbel"].cpu().numpy()
    res = ol.lookup_forward(q, keys, vals, float(log_t), top_k_=k, gumbel=gum, noise_coef=1.0, dtype=np.float64)
    ok, _ = ol.near_tie_free_rows(q, keys, float(log_t), top_k_=k, gumbel=gum, noise_coef=1.0)
    assert ok.mean() > 0.5
    slots = res_gpu["slots"].cpu().numpy()
    np.testing.assert_array_equal(np.sort(slots[ok], -1), np.sort(res["slots"][ok], -1))
    sel = _with_selection(res, res_gpu["sub_idx"].cpu().numpy(), res_gpu["flat_idx"].cpu().numpy(), slots)

    # f from the GPU's clean stage-1 top-k, checked against the oracle's
    clean = pool._clean_sub_idx(res_gpu["q"], res_gpu["packed"], res_gpu["score_code"], res_gpu["temperature"],
                                M).cpu().numpy()
    want_clean = ol.top_k(res["scores"], k)[1]
    tf = _stage1_tie_free(res["scores"], k)
    assert tf.mean() > 0.5
    np.testing.assert_array_equal(np.sort(clean[tf], -1), np.sort(want_clean[tf], -1))
    codebook = (np.arange(H)[:, None, None] * 2 + np.arange(2)[None, :, None]) * N_SUB
    f = np.bincount((clean + codebook[None]).reshape(-1), minlength=H * 2 * N_SUB).reshape(H, 2, N_SUB) / (M * k)

    ref = ob.lookup_backward(sel, vals, g, n=N_SUB, g_balance=g_bal, f=f)
    _check(gq.cpu().numpy(), ref["d_queries"], 1e-2, "d_queries")
    _check(gk.cpu().numpy(), ref["d_sub_keys"], 1e-2, "d_sub_keys")
    _check(float(gt), ref["d_log_temperature"], 1e-2, "d_log_temperature",
           float(np.abs(ref["d_cos"] * sel["cos"]).sum()))


@pytest.mark.parametrize("values_dtype,M,k", [(torch.float16, 8192, 16), (torch.float16, 300, 16),
                                              (torch.float32, 1000, 16), (torch.float16, 777, 8)])
def test_fused_query_backward_equals_separate_pass(gpu_lib, monkeypatch, values_dtype, M, k):
    """mpl_lookup_bwd_dense_queries (the routed d q_hat inside the balance
    query pass, then the normalisation backward) against the separate
    passes (mpl_lookup_bwd_dense + mpl_lookup_bwd_queries) on the same
    forward: d queries within 2e-3 of max |d q| in fp16 (the routed term
    rides the fp16 MFMA operand there) and 1e-5 in fp32; the sub-key and
    log-temperature gradients are those of the separate path bit for bit."""
    from model_amd import memory as mem
    pool = MemoryPool(N_SUB if values_dtype == torch.float16 else 64, H, D_KEY, D, k, routing_noise=1.0,
                      values_dtype=values_dtype)
    params = make_params(pool, 77, key_std=(D_KEY // 2) ** -0.5, value_std=0.02)
    g = torch.Generator(device="cuda").manual_seed(78)
    q = torch.randn((M, H, D_KEY), generator=g, device="cuda")
    g_out = torch.randn((M, D), generator=g, device="cuda") * 1e-3
    g_bal = torch.full((), 0.01, device="cuda")
    print(f"fused query backward {values_dtype} M={M}", flush=True)
    out = {}
    for fused in (True, False):
        monkeypatch.setattr(mem, "FUSED_QUERY_BWD", fused)
        o, aux, grads = pool.forward_backward(params, q, g_out, g_bal, train=True, rngs={"routing": 5})
        out[fused] = [t.clone() for t in grads]
    torch.cuda.synchronize()
    (dqa, dka, dla), (dqb, dkb, dlb) = out[True], out[False]
    tol = 2e-3 if values_dtype == torch.float16 else 1e-5
    err = float((dqa - dqb).abs().max()) / float(dqb.abs().max())
    assert err <= tol, f"d queries: {err:.3g} of max |d q| > {tol}"
    assert torch.equal(dka, dkb) and torch.equal(dla, dlb)


@pytest.mark.parametrize("d_key", [256, 128])
def test_raw_query_pack_equals_q_hat_pack(gpu_lib, monkeypatch, d_key):
    """The fused query pass with its fp16 operand packs made from the raw
    queries (normalised inside the pack) gives the gradients of the same
    pass fed the fp32 q_hat of mpl_l2_normalize, bit for bit (half = 128
    and 64)."""
    from model_amd import memory as mem
    M, k = 1000, 16
    pool = MemoryPool(128, H, d_key, 64, k, routing_noise=1.0, values_dtype=torch.float16)
    params = make_params(pool, 91, key_std=(d_key // 2) ** -0.5, value_std=0.02)
    g = torch.Generator(device="cuda").manual_seed(92)
    q = torch.randn((M, H, d_key), generator=g, device="cuda") * 3.0
    g_out = torch.randn((M, 64), generator=g, device="cuda") * 1e-3
    g_bal = torch.full((), 0.01, device="cuda")
    print(f"raw query pack d_key={d_key}", flush=True)
    out = {}
    for raw in (True, False):
        monkeypatch.setattr(mem, "RAW_QUERY_PACK", raw)
        _, _, grads = pool.forward_backward(params, q, g_out, g_bal, train=True, rngs={"routing": 9})
        out[raw] = [t.clone() for t in grads]
    torch.cuda.synchronize()
    for a, b in zip(out[True], out[False]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("values_dtype,query_scale", [(torch.float16, False), (torch.float32, False),
                                                      (torch.float16, True)])
def test_forward_backward_with_key_diversity(gpu_lib, values_dtype, query_scale):
    """forward_backward(g_diversity=c) against forward_backward() plus
    key_diversity_value_and_grad(c) added: d sub_keys within 1e-5 of max
    |d sub_keys| (the fused pass sums the two terms before one
    normalisation backward), the loss bit for bit, d queries and
    d log-temperature unchanged."""
    from model_amd.memory import key_diversity_value_and_grad
    k, M = 16, 2048
    n = 512 if values_dtype == torch.float16 else 128
    pool = MemoryPool(n, H, D_KEY, 64, k, routing_noise=1.0, values_dtype=values_dtype, query_scale=query_scale)
    params = make_params(pool, 95, key_std=(D_KEY // 2) ** -0.5, value_std=0.02)
    g = torch.Generator(device="cuda").manual_seed(96)
    q = torch.randn((M, H, D_KEY), generator=g, device="cuda")
    g_out = torch.randn((M, 64), generator=g, device="cuda") * 1e-3
    g_bal = torch.full((), 0.01, device="cuda")
    g_div = torch.full((), 0.05, device="cuda")
    print(f"forward_backward + key diversity {values_dtype} query_scale={query_scale}", flush=True)
    _, aux, (dqa, dka, dla) = pool.forward_backward(params, q, g_out, g_bal, train=True, rngs={"routing": 3},
                                                    g_diversity=g_div)
    _, _, (dqb, dkb, dlb) = pool.forward_backward(params, q, g_out, g_bal, train=True, rngs={"routing": 3})
    loss, ddk = key_diversity_value_and_grad(params["params"]["sub_keys"] if "params" in params
                                             else params["sub_keys"], g_div, pool.score_dtype)
    torch.cuda.synchronize()
    ref = dkb + ddk
    err = float((dka - ref).abs().max()) / float(ref.abs().max())
    assert err <= 1e-5, f"d sub_keys: {err:.3g}"
    assert torch.equal(aux["key_diversity_loss"].reshape(()), loss.reshape(()))
    assert torch.equal(dqa, dqb) and torch.equal(dla, dlb)


@pytest.mark.parametrize("values_dtype", [torch.float16, torch.float32])
def test_forward_backward_on_dq_hook(gpu_lib, values_dtype):
    """forward_backward(on_dq=hook): the dense backward runs as its query
    phase, the hook, then its sub-key phase (fp16 operands; the fp32 pool
    takes the separate query pass and calls the hook after it).  The hook
    gets the finished d queries: a copy it starts on another stream equals
    the returned d queries, and every gradient and the diversity loss equal
    those of the call without the hook bit for bit."""
    k, M = 16, 2048
    n = 512 if values_dtype == torch.float16 else 128
    pool = MemoryPool(n, H, D_KEY, 64, k, routing_noise=1.0, values_dtype=values_dtype)
    params = make_params(pool, 97, key_std=(D_KEY // 2) ** -0.5, value_std=0.02)
    g = torch.Generator(device="cuda").manual_seed(98)
    q = torch.randn((M, H, D_KEY), generator=g, device="cuda")
    g_out = torch.randn((M, 64), generator=g, device="cuda") * 1e-3
    g_bal = torch.full((), 0.01, device="cuda")
    g_div = torch.full((), 0.05, device="cuda")
    print(f"forward_backward on_dq hook {values_dtype}", flush=True)
    side = torch.cuda.Stream()
    seen = {}

    def hook(dq):
        cur = torch.cuda.current_stream()
        side.wait_stream(cur)
        dq.record_stream(side)
        with torch.cuda.stream(side):
            seen["copy"] = dq.clone()
        seen["calls"] = seen.get("calls", 0) + 1

    _, aux_a, (dqa, dka, dla) = pool.forward_backward(params, q, g_out, g_bal, train=True, rngs={"routing": 4},
                                                      g_diversity=g_div, on_dq=hook)
    torch.cuda.current_stream().wait_stream(side)
    _, aux_b, (dqb, dkb, dlb) = pool.forward_backward(params, q, g_out, g_bal, train=True, rngs={"routing": 4},
                                                      g_diversity=g_div)
    torch.cuda.synchronize()
    assert seen["calls"] == 1
    assert torch.equal(seen["copy"], dqa)
    assert torch.equal(dqa, dqb) and torch.equal(dka, dkb) and torch.equal(dla, dlb)
    assert torch.equal(aux_a["key_diversity_loss"], aux_b["key_diversity_loss"])
