"""The temperature clamp with the clamp engaged (memory.py:143-146 of the
reference): T = exp(log_t + sg(clip(log_t, ln min, ln max) - log_t)), so the
value is the clamped one and d log_t = T_clamped * dL/dT passes straight
through.  log_temperature is put below the floor (ln 2 with floors 5 and 10)
and above the ceiling (ln 500 with ceiling 100); aux["temperature"], the
slots, weights and out, and d log_t are compared with the oracle (fp64).
Then tests/test_memory_pool.py:79-101 of the reference is restated: the
floor clamps the value but the read still has a non-zero d log_t, and the
balance loss reaches log_t only with balance_temperature_grad.

Tolerances: 1e-5 relative (fp32 scoring, fp32 table) times max(1, T/10),
since a score is cos * T with cos rounded to fp32 and the softmax passes that
error on (at T = 100 the weights sit about 2e-5 from fp64); 1e-2 (fp16 paths);
aux["temperature"] within 1e-6 relative of the fp64 clamp.  The ceiling on
the fp16 path is 30, not 100: fp16 operands put cos about 1e-4 off, so a
score T * 1e-4 off, and at T = 100 the weights of near-equal slots move by
up to 2% (a numpy emulation of the rounding at these inputs)."""

import math

import numpy as np
import pytest
import torch

from model_amd.memory import MemoryPool
from oracle import backward as ob
from oracle import lookup as ol
from tests.gpu_helpers import oracle_check

pytestmark = pytest.mark.gpu


def _inputs(seed, *, n, H, d_key, d, M, values_dtype, log_t):
    rng = np.random.default_rng(seed)
    half = d_key // 2
    keys = (rng.standard_normal((H, 2, n, half)) * 1.3 / np.sqrt(half)).astype(np.float32)
    values = (rng.standard_normal((n * n, d)) * 0.05).astype(np.float32)
    q = rng.standard_normal((M, H, d_key)).astype(np.float32)
    g = rng.standard_normal((M, d)).astype(np.float32)
    params = {
        "sub_keys": torch.tensor(keys, device="cuda", requires_grad=True),
        "values": torch.tensor(values, device="cuda").to(values_dtype).requires_grad_(True),
        "log_temperature": torch.tensor(np.float32(log_t), device="cuda", requires_grad=True),
    }
    tq = torch.tensor(q, device="cuda", requires_grad=True)
    vals_np = params["values"].detach().float().cpu().numpy()
    return params, tq, q, keys, vals_np, g


def _rel(a, ref, scale=None):
    a, ref = np.asarray(a, np.float64), np.asarray(ref, np.float64)
    scale = max(float(np.abs(ref).max()) if scale is None else scale, 1e-30)
    return float(np.abs(a - ref).max()) / scale


CASES = [
    # (score dtype, values dtype, log_t, min_t, max_t, query_scale, btg, g_bal)
    ("f32", torch.float32, math.log(2.0), 5.0, 100.0, False, False, 0.5),
    ("f32", torch.float32, math.log(2.0), 10.0, 100.0, False, True, 0.5),
    ("f32", torch.float32, math.log(500.0), 10.0, 100.0, True, True, 0.3),
    ("f16", torch.float16, math.log(2.0), 5.0, 100.0, False, False, 0.01),
    # fp16 operands give cos about 1e-4 off, so a score T * 1e-4 off: the ceiling
    # is 30 here to keep the fp16 weights inside the 1e-2 rule (T = 100 above on fp32)
    ("f16", torch.float16, math.log(500.0), 10.0, 30.0, True, False, 0.01),
    ("f16", torch.float16, math.log(3.0), 10.0, 100.0, False, True, 0.2),
]


@pytest.mark.parametrize("sd,values_dtype,log_t,min_t,max_t,qs,btg,g_bal", CASES)
def test_clamped_temperature_forward_and_straight_through_gradient(gpu_lib, sd, values_dtype, log_t, min_t,
                                                                   max_t, qs, btg, g_bal):
    if sd == "f32":
        n, H, d_key, d, k, M, score_dtype = 64, 2, 32, 32, 8, 40, torch.float32
    else:  # the text-study widths on fp16 MFMA scoring
        n, H, d_key, d, k, M, score_dtype = 128, 4, 256, 256, 16, 24, torch.float16
    pool = MemoryPool(n, H, d_key, d, k, min_temperature=min_t, max_temperature=max_t, query_scale=qs,
                      balance_temperature_grad=btg, values_dtype=values_dtype, score_dtype=score_dtype)
    params, tq, q, keys, vals, g = _inputs(31, n=n, H=H, d_key=d_key, d=d, M=M, values_dtype=values_dtype,
                                           log_t=log_t)
    t_want = math.exp(min(max(float(np.float32(log_t)), math.log(min_t)), math.log(max_t)))
    assert t_want in (pytest.approx(min_t, rel=1e-6), pytest.approx(max_t, rel=1e-6))  # the clamp is engaged

    res_gpu = pool.lookup(params, tq.detach())
    assert abs(float(res_gpu["aux"]["temperature"]) / t_want - 1.0) <= 1e-6
    # fp32: a score is cos * T with cos rounded to fp32, so the weights' error
    # grows with T; the 1e-5 rule holds up to T = 10 and scales with T above it
    tol = 1e-5 * max(1.0, t_want / 10.0) if sd == "f32" else 1e-2
    # slots, weights and out at the clamped T
    oracle_check(pool, {key: v.detach() for key, v in params.items()}, tq.detach(), res_gpu, tol=tol)

    out, aux = pool.apply({"params": params}, tq, sparse_grad=False)
    loss = (out * torch.tensor(g, device="cuda")).sum() + g_bal * aux["balance_loss"]
    gq, gk, gt, gv = torch.autograd.grad(loss, [tq, params["sub_keys"], params["log_temperature"],
                                                params["values"]])
    res = ol.lookup_forward(q, keys, vals, float(np.float32(log_t)), top_k_=k, query_scale=qs,
                            min_temperature=min_t, max_temperature=max_t, dtype=np.float64)
    # gradients for the GPU's selection (identical on tie-free rows, checked above)
    from tests.test_gpu_backward import _with_selection

    sel = _with_selection(res, res_gpu["sub_idx"].cpu().numpy(), res_gpu["flat_idx"].cpu().numpy(),
                          res_gpu["slots"].cpu().numpy())
    ao = ol.aux_stats(sel, n=n, noisy=False, balance_temperature_grad=btg)
    assert abs(float(aux["balance_loss"].detach()) / ao["balance_loss"] - 1.0) <= tol
    ref = ob.lookup_backward(sel, vals, g, n=n, query_scale=qs, g_balance=g_bal, f=ao["_f"],
                             balance_temperature_grad=btg, dense_values=True)
    assert ref["d_log_temperature"] != 0.0  # straight through: the clamp does not stop the gradient
    lt_scale = float(np.abs(ref["d_cos"] * sel["cos"]).sum())  # d log_t is a sum with cancellation
    assert _rel(float(gt), ref["d_log_temperature"], lt_scale) <= tol, (float(gt), ref["d_log_temperature"])
    assert _rel(gq.cpu().numpy(), ref["d_queries"]) <= tol
    assert _rel(gk.cpu().numpy(), ref["d_sub_keys"]) <= tol
    assert _rel(gv.float().cpu().numpy(), ref["d_values"]) <= tol

    # the autograd-free training path gives the same d log_t bit for bit
    _, _, (dq2, dk2, dlt2) = pool.forward_backward(
        {"params": params}, tq.detach(), torch.tensor(g, device="cuda"),
        torch.tensor([g_bal], device="cuda"), train=False)
    assert torch.equal(dlt2, gt) and torch.equal(dq2, gq) and torch.equal(dk2, gk)


def _temp_grads(pool_kw, log_t):
    """tests/test_memory_pool.py:80-93: (d balance / d log_t, d sum(out^2) /
    d log_t, aux temperature) at the reference test's shapes."""
    n, H, d_key, d, k = 16, 2, 8, 12, 4
    pool = MemoryPool(n, H, d_key, d, k, values_dtype=torch.float32, **pool_kw)
    p = pool.init(1, device="cuda")["params"]
    p["log_temperature"] = torch.tensor(np.float32(log_t), device="cuda")
    p = {key: v.detach().requires_grad_(True) for key, v in p.items()}
    q = torch.randn((3, 5, H, d_key), generator=torch.Generator(device="cuda").manual_seed(0), device="cuda")

    def grad(what):
        out, aux = pool.apply({"params": p}, q)
        loss = aux["balance_loss"] if what == "balance" else (out ** 2).sum()
        (gt,) = torch.autograd.grad(loss, [p["log_temperature"]])
        return float(gt)

    _, aux = pool.apply({"params": p}, q.detach())
    return grad("balance"), grad("read"), float(aux["temperature"])


def test_temperature_floor_and_balance_gradient(gpu_lib):
    # the floor clamps the value but still passes gradient (no dead temperature)
    _, g_read, t = _temp_grads({"min_temperature": 5.0}, math.log(2.0))
    assert abs(t - 5.0) < 1e-4 and g_read != 0.0
    # the balance loss can't lower its value by flattening the router
    g_bal, _, _ = _temp_grads({"balance_temperature_grad": True}, math.log(10.0))
    assert g_bal != 0.0
    g_bal, g_read, _ = _temp_grads({"balance_temperature_grad": False}, math.log(10.0))
    assert g_bal == 0.0 and g_read != 0.0


def test_temperature_kernel_matches_torch_clamp_exp(gpu_lib):
    """mpl_temperature: exp(clip(log_t, ln min, ln max)) bit for bit against
    torch's clamp + exp, inside, below and above the range; NaN stays NaN."""
    import math
    from model_amd import _lib
    from model_amd._lib import check, ptr
    lo, hi = math.log(10.0), math.log(100.0)
    for v in (math.log(20.0), math.log(2.0), math.log(500.0), lo, hi, -30.0, 30.0, float("nan")):
        lt = torch.tensor([v], dtype=torch.float32, device="cuda")
        t = torch.empty(1, device="cuda")
        check(_lib.lib().mpl_temperature(ptr(lt), lo, hi, ptr(t), _lib.stream_ptr(lt.device)), "mpl_temperature")
        ref = torch.exp(lt.clamp(lo, hi))
        torch.cuda.synchronize()
        if math.isnan(v):
            assert torch.isnan(t).all()
        else:
            assert torch.equal(t, ref), (v, float(t), float(ref))
