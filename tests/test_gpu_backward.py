"""Backward of the lookup on the GPU (MemoryPool.apply under torch autograd,
include/mpl.h mpl_lookup_bwd_*) against oracle/backward.py (fp64), which is
itself pinned by torch autograd in tests/test_oracle.py.

loss = <g_out, out> + g_bal * balance_loss; gradients w.r.t. the raw
queries, raw sub_keys, log_temperature and (sparse_grad=False) the values.
Tolerance: 1e-5 relative for fp32 paths, 1e-2 for fp16 paths,
relative to the largest magnitude of each gradient."""

import numpy as np
import pytest
import torch

from model_amd.memory import MemoryPool
from oracle import backward as ob
from oracle import lookup as ol

pytestmark = pytest.mark.gpu


def _setup(seed, *, n, H, d_key, d, k, M, values_dtype, score_dtype, query_scale, btg):
    pool = MemoryPool(n, H, d_key, d, k, query_scale=query_scale, balance_temperature_grad=btg,
                      values_dtype=values_dtype, score_dtype=score_dtype)
    rng = np.random.default_rng(seed)
    half = d_key // 2
    keys = (rng.standard_normal((H, 2, n, half)) * 1.7 / np.sqrt(half)).astype(np.float32)
    values = (rng.standard_normal((n * n, d)) * 0.02).astype(np.float32)
    q = rng.standard_normal((M, H, d_key)).astype(np.float32)
    g = rng.standard_normal((M, d)).astype(np.float32)
    log_t = np.float32(np.log(20.0))
    dev = "cuda"
    params = {
        "sub_keys": torch.tensor(keys, device=dev, requires_grad=True),
        "values": torch.tensor(values, device=dev).to(values_dtype).requires_grad_(True),
        "log_temperature": torch.tensor(log_t, device=dev, requires_grad=True),
    }
    tq = torch.tensor(q, device=dev, requires_grad=True)
    vals_np = params["values"].detach().float().cpu().numpy()  # the table as stored
    return pool, params, tq, q, keys, vals_np, g, log_t


def _check(a, ref, tol, what, scale=None):
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max() if scale is None else scale, 1e-30)
    err = np.abs(a - ref).max() / scale
    assert err <= tol, f"{what}: max error {err:.3g} of max |ref| {scale:.3g} > {tol}"


def _lt_scale(ref, res):
    """d log_t is a sum with cancellation: its error is measured against the
    sum of the magnitudes of its terms (d_sub * sub_scores)."""
    return float(np.abs(ref["d_sub_scores"] * res["sub_scores"]).sum())


@pytest.mark.parametrize("values_dtype,query_scale,btg,g_bal", [
    (torch.float32, False, False, 0.0),
    (torch.float32, False, False, 0.5),
    (torch.float32, True, False, 0.5),
    (torch.float32, False, True, 0.5),
    (torch.float32, True, True, 0.3),
    (torch.float16, False, False, 0.01),
])
def test_backward_matches_oracle_fp32_scoring(gpu_lib, values_dtype, query_scale, btg, g_bal):
    n, H, d_key, d, k, M = 64, 2, 32, 32, 8, 40
    pool, params, tq, q, keys, vals, g, log_t = _setup(
        21, n=n, H=H, d_key=d_key, d=d, k=k, M=M, values_dtype=values_dtype, score_dtype=torch.float32,
        query_scale=query_scale, btg=btg)
    out, aux = pool.apply({"params": params}, tq, sparse_grad=False)
    loss = (out * torch.tensor(g, device="cuda")).sum() + g_bal * aux["balance_loss"]
    gq, gk, gt, gv = torch.autograd.grad(loss, [tq, params["sub_keys"], params["log_temperature"],
                                                params["values"]])
    res = ol.lookup_forward(q, keys, vals, float(log_t), top_k_=k, query_scale=query_scale, dtype=np.float64)
    np.testing.assert_array_equal(aux["slots"].cpu().numpy(), res["slots"])  # same selection
    ao = ol.aux_stats(res, n=n, noisy=False, balance_temperature_grad=btg)
    np.testing.assert_allclose(float(aux["balance_loss"]), ao["balance_loss"], rtol=1e-5)
    ref = ob.lookup_backward(res, vals, g, n=n, query_scale=query_scale, g_balance=g_bal, f=ao["_f"],
                             balance_temperature_grad=btg, dense_values=True)
    tol = 1e-5 if values_dtype == torch.float32 else 1e-2
    _check(gq.cpu().numpy(), ref["d_queries"], tol, "d_queries")
    _check(gk.cpu().numpy(), ref["d_sub_keys"], tol, "d_sub_keys")
    _check(float(gt), ref["d_log_temperature"], tol, "d_log_temperature", _lt_scale(ref, res))
    _check(gv.float().cpu().numpy(), ref["d_values"], tol, "d_values")


def _with_selection(res, sub_idx, flat_idx, slots):
    """The oracle's forward result with the routing replaced by the GPU's
    (stage-1 ids, flat pair ranks, slots); weights re-derived in fp64 from the
    clean scores of that selection (memory.py:163-178).  Gradients are then
    compared for the same discrete selection."""
    r = dict(res)
    k = sub_idx.shape[-1]
    sub_scores = np.take_along_axis(res["scores"], sub_idx.astype(np.int64), axis=-1)
    fa, fb = flat_idx // k, flat_idx % k
    slot_scores = (np.take_along_axis(sub_scores[:, :, 0], fa, -1) + np.take_along_axis(sub_scores[:, :, 1], fb, -1))
    w = np.exp(slot_scores - slot_scores.max(-1, keepdims=True))
    r.update(sub_idx=sub_idx.astype(np.int64), flat_idx=flat_idx.astype(np.int64), slots=slots.astype(np.int64),
             read_slots=slots.astype(np.int64), sub_scores=sub_scores, slot_scores=slot_scores,
             weights=w / w.sum(-1, keepdims=True),
             idx_a=np.take_along_axis(sub_idx[:, :, 0], fa, -1).astype(np.int64),
             idx_b=np.take_along_axis(sub_idx[:, :, 1], fb, -1).astype(np.int64))
    return r


def test_backward_fp16_scoring_text_study_layer(gpu_lib):
    """fp16 values and fp16 MFMA scoring at the training layer's widths
    (H=4, d_key=256, d=256, k=16), n=128, balance coefficient 0.01.  The
    selection is the parity rule's business (exact on near-tie-free rows, which
    is checked); the gradients are compared for the GPU's selection."""
    n, H, d_key, d, k, M = 128, 4, 256, 256, 16, 24
    pool, params, tq, q, keys, vals, g, log_t = _setup(
        5, n=n, H=H, d_key=d_key, d=d, k=k, M=M, values_dtype=torch.float16, score_dtype=torch.float16,
        query_scale=False, btg=False)
    res_gpu = pool.lookup(params, tq.detach())
    out, aux = pool.apply({"params": params}, tq, sparse_grad=False)
    loss = (out * torch.tensor(g, device="cuda")).sum() + 0.01 * aux["balance_loss"]
    gq, gk, gt, gv = torch.autograd.grad(loss, [tq, params["sub_keys"], params["log_temperature"],
                                                params["values"]])
    res = ol.lookup_forward(q, keys, vals, float(log_t), top_k_=k, dtype=np.float64)
    ok, _ = ol.near_tie_free_rows(q, keys, float(log_t), top_k_=k)
    slots = res_gpu["slots"].cpu().numpy()
    np.testing.assert_array_equal(np.sort(slots[ok], -1), np.sort(res["slots"][ok], -1))
    sel = _with_selection(res, res_gpu["sub_idx"].cpu().numpy(), res_gpu["flat_idx"].cpu().numpy(), slots)
    ao = ol.aux_stats(sel, n=n, noisy=False)
    ref = ob.lookup_backward(sel, vals, g, n=n, g_balance=0.01, f=ao["_f"], dense_values=True)
    _check(gq.cpu().numpy(), ref["d_queries"], 1e-2, "d_queries")
    _check(gk.cpu().numpy(), ref["d_sub_keys"], 1e-2, "d_sub_keys")
    _check(float(gt), ref["d_log_temperature"], 1e-2, "d_log_temperature", _lt_scale(ref, sel))
    _check(gv.float().cpu().numpy(), ref["d_values"], 1e-2, "d_values")


def test_sparse_grad_leaves_values_and_matches_dense_rows(gpu_lib):
    """sparse_grad=True: no table gradient from autograd; the probe gradient
    merged by fetched_row_grads equals the dense table gradient's rows
    (tests/test_memory_pool.py:321-344)."""
    from model_amd import rows as R
    n, H, d_key, d, k, M = 32, 2, 16, 16, 4, 30
    pool, params, tq, q, keys, vals, g, log_t = _setup(
        9, n=n, H=H, d_key=d_key, d=d, k=k, M=M, values_dtype=torch.float32, score_dtype=torch.float32,
        query_scale=False, btg=False)
    probe = torch.zeros((M, d), device="cuda", requires_grad=True)
    out, aux = pool.apply({"params": params}, tq, sparse_grad=True)
    loss = ((out + probe) * torch.tensor(g, device="cuda")).sum()
    gq, gp = torch.autograd.grad(loss, [tq, probe])
    uniq, rows = R.fetched_row_grads({"slots": [aux["slots"]], "weights": [aux["weights"]]}, {0: gp}, [0],
                                     n * n)
    out2, _ = pool.apply({"params": params}, tq, sparse_grad=False)
    (gv,) = torch.autograd.grad((out2 * torch.tensor(g, device="cuda")).sum(), [params["values"]])
    u = uniq.cpu().numpy()
    keep = u < n * n
    np.testing.assert_allclose(gv.cpu().numpy()[u[keep]], rows.cpu().numpy()[keep], rtol=1e-6, atol=1e-7)
    untouched = np.setdiff1d(np.arange(n * n), u[keep])
    assert np.all(gv.cpu().numpy()[untouched] == 0)


@pytest.mark.parametrize("n,H,d_key,k,M,qs,btg,g_bal,seed", [
    (100, 2, 64, 8, 77, False, False, 0.0, 61),    # routed term only; n not a multiple of 32 or 128
    (300, 1, 32, 16, 130, True, False, 0.0, 62),   # query_scale; 3 key groups, partial last
    (64, 2, 16, 32, 45, True, True, 0.4, 63),      # k = 32 (1024 routed entries per query block), half = 8
    (512, 4, 256, 16, 200, False, False, 0.01, 64),  # the text-study widths with the balance term
])
def test_dense_sub_key_gradient_fp16_scoring(gpu_lib, n, H, d_key, k, M, qs, btg, g_bal, seed):
    """With fp16 scoring the whole sub-key gradient (routed d sub_scores plus
    the balance term) is one dense MFMA pass (mpl_lookup_bwd_dense) followed
    by the l2-normalisation backward; compared for the GPU's selection."""
    pool, params, tq, q, keys, vals, g, log_t = _setup(
        seed, n=n, H=H, d_key=d_key, d=32, k=k, M=M, values_dtype=torch.float16, score_dtype=torch.float16,
        query_scale=qs, btg=btg)
    res_gpu = pool.lookup(params, tq.detach())
    out, aux = pool.apply({"params": params}, tq, sparse_grad=True)
    loss = (out * torch.tensor(g, device="cuda")).sum()
    if g_bal:
        loss = loss + g_bal * aux["balance_loss"]
    gq, gk, gt = torch.autograd.grad(loss, [tq, params["sub_keys"], params["log_temperature"]])
    res = ol.lookup_forward(q, keys, vals, float(log_t), top_k_=k, query_scale=qs, dtype=np.float64)
    sel = _with_selection(res, res_gpu["sub_idx"].cpu().numpy(), res_gpu["flat_idx"].cpu().numpy(),
                          res_gpu["slots"].cpu().numpy())
    f = ol.aux_stats(sel, n=n, noisy=False, balance_temperature_grad=btg)["_f"]
    ref = ob.lookup_backward(sel, vals, g, n=n, query_scale=qs, g_balance=g_bal, f=f, balance_temperature_grad=btg)
    _check(gk.cpu().numpy(), ref["d_sub_keys"], 1e-2, "d_sub_keys")
    _check(gq.cpu().numpy(), ref["d_queries"], 1e-2, "d_queries")
    _check(float(gt), ref["d_log_temperature"], 1e-2, "d_log_temperature", float(np.abs(ref["d_cos"] * sel["cos"]).sum()))


@pytest.mark.parametrize("with_len,k", [(False, 16), (True, 16), (True, 5), (False, 37)])
def test_queries_backward_16_byte_form_equals_dword_form(gpu_lib, with_len, k):
    """mpl_lookup_bwd_queries at half = 128 runs a kernel with 16-byte loads
    (two key rows per load instruction) when q, k_hat, the extra d q-hat term
    and d_queries are 16-byte aligned, and the dword kernel otherwise.  The
    two differ only in the order the key rows are summed; entries with key
    id -1 (unfilled ranks), every optional input, and entry counts that do
    not fill the half-waves' batches of 8 are exercised."""
    from model_amd import _lib

    L = gpu_lib
    M, H, n, half = 300, 4, 512, 128
    rows = M * H * 2
    g = torch.Generator(device="cuda").manual_seed(71)
    dev = "cuda"
    q = torch.randn((rows, half), generator=g, device=dev)
    k_hat = torch.nn.functional.normalize(torch.randn((2 * H, n, half), generator=g, device=dev), dim=-1)
    sub_idx = torch.randint(0, n, (rows, k), generator=g, device=dev, dtype=torch.int32)
    sub_idx[::7, k - 3:] = -1
    d_sub = torch.randn((rows, k), generator=g, device=dev)
    sub_scores = torch.randn((rows, k), generator=g, device=dev)
    extra = torch.randn((rows, half), generator=g, device=dev) * 0.1
    q_len = (torch.rand((rows,), generator=g, device=dev) + 0.5) if with_len else None
    dlen_extra = torch.randn((rows,), generator=g, device=dev) if with_len else None
    T = torch.full((1,), 7.5, device=dev)
    p = _lib.ptr

    def run(off):
        # copies shifted by `off` floats: off = 1 leaves them 4-byte aligned only
        def place(t):
            buf = torch.zeros(t.numel() + 4, device=dev)
            v = buf[off:off + t.numel()].view(t.shape)
            v.copy_(t)
            return buf, v
        (_, qv), (_, kv), (_, ev), (_, ov) = place(q), place(k_hat), place(extra), place(torch.zeros_like(q))
        _lib.check(L.mpl_lookup_bwd_queries(p(qv), p(q_len), p(kv), p(sub_idx), p(d_sub), p(sub_scores), p(ev),
                                            p(dlen_extra), M, H, n, half, k, p(T), p(ov),
                                            torch.cuda.current_stream().cuda_stream), "queries")
        torch.cuda.synchronize()
        return ov.clone()

    fast, dword = run(0), run(1)
    assert torch.isfinite(fast).all()
    torch.testing.assert_close(fast, dword, rtol=1e-5, atol=1e-5 * float(dword.abs().max()))


@pytest.mark.parametrize("shuffle", [0, 1])
@pytest.mark.parametrize("H,k", [(4, 16), (2, 16), (4, 8)])
@pytest.mark.parametrize("dtype,d", [(torch.float32, 256), (torch.float16, 512)])
def test_route_backward_1k_rows_equal_generic_form(gpu_lib, dtype, d, H, k, shuffle):
    """mpl_lookup_bwd_route with 1 KB value rows (fp32 d = 256, fp16 d = 512)
    reads a row per 16-byte load instruction and reduce-scatters the lane
    dots; with the table 4-byte aligned only it takes the per-element loop.
    The two differ only in the order each dot is summed.  H * k = 64 fills
    the wave; 32 leaves lanes without a row (they read row 0 and drop it);
    shuffle_reads reads (slot + N/2 + 1) % N in both forms."""
    from model_amd import _lib

    M, N = 200, 4096
    g = torch.Generator(device="cuda").manual_seed(d)
    vals = (torch.randn((N, d), generator=g, device="cuda") * 0.05).to(dtype)
    slots = torch.randint(0, N, (M, H, k), generator=g, device="cuda", dtype=torch.int32)
    w = torch.rand((M, H, k), generator=g, device="cuda")
    w = w / w.sum(-1, keepdim=True)
    flat = torch.randint(0, k * k, (M, H, k), generator=g, device="cuda", dtype=torch.int32)
    sub_scores = torch.randn((M, H, 2, k), generator=g, device="cuda")
    g_out = torch.randn((M, d), generator=g, device="cuda") * 1e-3
    vdt = _lib.MPL_F16 if dtype == torch.float16 else _lib.MPL_F32
    p = _lib.ptr

    def run(off):
        buf = torch.zeros(N * d + 8, dtype=dtype, device="cuda")
        v = buf[off:off + N * d].view(N, d)
        v.copy_(vals)
        dw = torch.empty((M, H, k), device="cuda")
        ds = torch.empty((M, H, 2, k), device="cuda")
        lt = torch.empty((M,), device="cuda")
        _lib.check(gpu_lib.mpl_lookup_bwd_route(p(g_out), p(v), vdt, N, d, p(slots), p(w), p(flat), p(sub_scores),
                                                M, H, k, shuffle, p(dw), p(ds), p(lt),
                                                torch.cuda.current_stream().cuda_stream), "route")
        torch.cuda.synchronize()
        return dw, ds, lt

    off = 2 if dtype == torch.float16 else 1  # 4 bytes: not 16-byte aligned
    for a, b in zip(run(0), run(off)):
        assert torch.isfinite(a).all()
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5 * float(b.abs().max()))
