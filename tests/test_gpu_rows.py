"""Sparse row gradients and row-wise optimizers on the GPU against the oracle
(oracle/rows.py restating train.py:146-172, 395-426).

Bit-exact for ids (uniq, counts); fp32 rows within 1e-5 relative of the
fp64 sums (summation order differs from the oracle's np.add.at); the merge
itself is checked to be bitwise reproducible run to run."""

import numpy as np
import pytest
import torch

from model_amd import rows as R
from oracle import rows as orow
from tests.gpu_helpers import zipf_slots

pytestmark = pytest.mark.gpu

TOL32 = 1e-5


def _fp64_rows(slots, w, g, fpt, pool_size):
    """fp64 per-slot sums via a stable sort + reduceat (an independent path)."""
    slots = slots.reshape(-1).astype(np.int64)
    contrib = (w.reshape(-1, 1).astype(np.float64) * np.repeat(g.astype(np.float64), fpt, axis=0))
    order = np.argsort(slots, kind="stable")
    s = slots[order]
    u, start = np.unique(s, return_index=True)
    rows = np.add.reduceat(contrib[order], start, axis=0)
    return u, rows


def _run_merge(slots, w, g, pool_size):
    dev = "cuda"
    m = R.merge_fetches(torch.as_tensor(slots, device=dev), None if w is None else torch.as_tensor(w, device=dev),
                        torch.as_tensor(g, device=dev), pool_size)
    return m


@pytest.mark.parametrize("P_tokens,fpt,d,pool_size,seed", [
    (37, 8, 12, 16, 0),          # reference test shape: n=4 -> 16 slots, many repeats
    (300, 64, 32, 100000, 1),    # sparse: few repeats
    (1000, 64, 256, 4096, 2),    # dense repeats, several radix passes
    (5000, 16, 128, 262144, 3),  # three radix passes, ragged last tile
])
def test_merge_matches_oracle(gpu_lib, P_tokens, fpt, d, pool_size, seed):
    rng = np.random.default_rng(seed)
    P = P_tokens * fpt
    slots = rng.integers(0, pool_size, P).astype(np.int32)
    w = rng.random(P).astype(np.float32)
    g = rng.standard_normal((P_tokens, d)).astype(np.float32)
    m = _run_merge(slots, w, g, pool_size)
    torch.cuda.synchronize()
    # oracle (train.py:146-172)
    uniq_o, rows_o = orow.fetched_row_grads([slots.reshape(P_tokens, 1, fpt)], [w.reshape(P_tokens, 1, fpt)], [g],
                                            pool_size)
    uniq = m.uniq.cpu().numpy()
    np.testing.assert_array_equal(uniq, uniq_o)
    U = int(m.num_unique.cpu()[0])
    assert U == np.unique(slots).shape[0]
    u64, rows64 = _fp64_rows(slots, w, g, fpt, pool_size)
    rows = m.rows.cpu().numpy()
    scale = np.abs(rows64).max()
    np.testing.assert_allclose(rows[:U], rows64, rtol=TOL32, atol=TOL32 * scale)
    np.testing.assert_allclose(rows[:U], rows_o[:U], rtol=TOL32, atol=TOL32 * scale)
    assert np.all(rows[U:] == 0)
    np.testing.assert_allclose(m.row_sq.cpu().numpy()[:U], (rows64 ** 2).sum(-1), rtol=1e-4)


def test_merge_rows_reference_cases(gpu_lib):
    """Padding and cap semantics of jnp.unique(size=cap, fill_value=N)."""
    slots = np.array([5, 1, 5, 3, 1, 1, 0, 2], np.int32)
    contribs = np.arange(16, dtype=np.float32).reshape(8, 2)
    uniq, rows = R.merge_rows(torch.as_tensor(slots, device="cuda"), torch.as_tensor(contribs, device="cuda"), 6)
    assert uniq.cpu().tolist() == [0, 1, 2, 3, 5, 6]
    np.testing.assert_array_equal(rows.cpu().numpy()[1], contribs[1] + contribs[4] + contribs[5])
    np.testing.assert_array_equal(rows.cpu().numpy()[5], [0, 0])
    # every fetch the same slot: one segment spanning many reduce ranges
    slots = np.full(4000, 7, np.int32)
    contribs = np.random.default_rng(3).standard_normal((4000, 8)).astype(np.float32)
    uniq, rows = R.merge_rows(torch.as_tensor(slots, device="cuda"), torch.as_tensor(contribs, device="cuda"), 50)
    assert uniq.cpu().tolist()[:2] == [7, 50] and uniq.shape[0] == 50
    np.testing.assert_allclose(rows.cpu().numpy()[0], contribs.astype(np.float64).sum(0), rtol=1e-5, atol=1e-4)
    assert np.all(rows.cpu().numpy()[1:] == 0)


def test_merge_empty(gpu_lib):
    m = R.merge_fetches(torch.empty(0, dtype=torch.int32, device="cuda"), None,
                        torch.empty((0, 8), device="cuda"), 10)
    assert m.uniq.shape[0] == 0 and int(m.num_unique.cpu()[0]) == 0


def test_merge_tolerates_out_of_range_ids(gpu_lib):
    """Ids outside [0, pool_size) (a caller's bug) give wrong rows but stay
    inside the [cap] outputs: more fetches than slots, so more distinct ids
    than cap can exist."""
    P, N, d = 4096, 64, 16
    bad = torch.as_tensor(np.random.default_rng(0).integers(-5, 6 * N, P).astype(np.int32), device="cuda")
    m = R.merge_fetches(bad, None, torch.ones((P, d), device="cuda"), N)
    torch.cuda.synchronize()
    assert m.uniq.shape[0] == N and 0 < int(m.num_unique.cpu()[0]) <= N
    assert torch.isfinite(m.rows).all()


def test_merge_zipf_training_shape(gpu_lib):
    """8,192 tokens x 4 heads x 16 fetches = 524,288 Zipf(1.1) fetches over
    262,144 slots, d=256: exact distinct-slot set, column sums (linearity:
    sum_u rows[u] = sum_p w_p g_p) and bitwise run-to-run reproducibility."""
    M, H, k, N, d = 8192, 4, 16, 262144, 256
    slots = zipf_slots(M, H, k, N)
    rng = np.random.default_rng(4)
    w = rng.random((M, H, k)).astype(np.float32)
    w /= w.sum(-1, keepdims=True)
    g = (rng.standard_normal((M, d)) * 1e-3).astype(np.float32)
    m1 = _run_merge(slots, w, g, N)
    m2 = _run_merge(slots, w, g, N)
    torch.cuda.synchronize()
    u = np.unique(slots)
    U = int(m1.num_unique.cpu()[0])
    assert U == u.shape[0]
    uniq = m1.uniq.cpu().numpy()
    np.testing.assert_array_equal(uniq[:U], u)
    assert np.all(uniq[U:] == N)
    assert torch.equal(m1.rows, m2.rows) and torch.equal(m1.uniq, m2.uniq)
    colsum = m1.rows.double().sum(0).cpu().numpy()
    ref = (w.reshape(M, H * k).astype(np.float64).sum(1)[:, None] * g.astype(np.float64)).sum(0)
    np.testing.assert_allclose(colsum, ref, rtol=1e-4, atol=1e-6)
    # the hottest row equals its fp64 sum
    cnt = np.bincount(slots.reshape(-1), minlength=N)
    hot = int(np.argmax(cnt))
    sel = slots.reshape(-1) == hot
    hot_ref = (w.reshape(-1)[sel, None].astype(np.float64) * np.repeat(g, H * k, 0)[sel]).sum(0)
    ui = int(np.searchsorted(u, hot))
    np.testing.assert_allclose(m1.rows[ui].cpu().numpy(), hot_ref, rtol=1e-5, atol=1e-5 * np.abs(hot_ref).max())


def test_fetched_row_grads_two_layers(gpu_lib):
    rng = np.random.default_rng(6)
    B, T, H, k, N, d = 2, 9, 2, 4, 64, 12
    aux = {"slots": [], "weights": []}
    probes = {}
    for layer in (1, 3):
        aux["slots"].append(torch.as_tensor(rng.integers(0, N, (B, T, H, k)).astype(np.int32), device="cuda"))
        aux["weights"].append(torch.as_tensor(rng.random((B, T, H, k)).astype(np.float32), device="cuda"))
        probes[layer] = torch.as_tensor(rng.standard_normal((B, T, d)).astype(np.float32), device="cuda")
    uniq, rows = R.fetched_row_grads(aux, probes, [1, 3], N)
    uo, ro = orow.fetched_row_grads([s.cpu().numpy() for s in aux["slots"]],
                                    [w.cpu().numpy() for w in aux["weights"]],
                                    [probes[1].cpu().numpy(), probes[3].cpu().numpy()], N)
    np.testing.assert_array_equal(uniq.cpu().numpy(), uo)
    np.testing.assert_allclose(rows.cpu().numpy(), ro, rtol=TOL32, atol=1e-6)


def test_clip_scale(gpu_lib):
    rows = np.full((2, 8), 1.0, np.float32)
    s = R.clip_scale(torch.as_tensor((rows ** 2).sum(-1), device="cuda"), torch.tensor([9.0], device="cuda"), 1.0)
    so, go = orow.clip_scale(9.0, rows, 1.0)
    np.testing.assert_allclose(s.cpu().numpy(), [so, go], rtol=1e-6)
    s = R.clip_scale(torch.as_tensor([0.01], device="cuda"), None, 1.0)
    assert float(s[0]) == 1.0


def test_sum_squares_fixed_order(gpu_lib):
    """The dense part of the global norm (train.py:395-397) over several
    buffers (ragged sizes, an empty one, one below the chunk count) plus a
    device scalar: the fp64 sum within 1e-7 relative, the empty sum, and the
    same bits on a repeat."""
    rng = np.random.default_rng(8)
    arrs = [rng.standard_normal(n).astype(np.float32) for n in (262144, 0, 7, 524288 + 13, 1)]
    add = np.float32(3.25)
    ts = [torch.as_tensor(a, device="cuda") for a in arrs]
    got = R.sum_squares(ts, torch.tensor([add], device="cuda"))
    want = sum(float((a.astype(np.float64) ** 2).sum()) for a in arrs) + float(add)
    assert abs(float(got) / want - 1.0) < 1e-7
    assert torch.equal(got, R.sum_squares(ts, torch.tensor([add], device="cuda")))
    assert float(R.sum_squares([ts[1]], None)) == 0.0
    assert float(R.sum_squares([], torch.tensor([2.5], device="cuda"))) == 2.5
    # nine buffers: two calls chained through ``add``
    many = R.sum_squares([ts[2]] * 9)
    assert abs(float(many) / (9 * float((arrs[2].astype(np.float64) ** 2).sum())) - 1.0) < 1e-7


def test_adagrad_known_answer(gpu_lib):
    """tests:505-513: ones on rows [3, 7] + padding 1000: only rows 3 and 7
    change, acc[3] == 1.0."""
    values = torch.as_tensor(np.random.default_rng(0).standard_normal((1000, 64)).astype(np.float32), device="cuda")
    before = values.clone()
    acc = torch.zeros(1000, device="cuda")
    R.rowwise_adagrad(values, acc, torch.tensor([3, 7, 1000], dtype=torch.int32, device="cuda"),
                      torch.ones((3, 64), device="cuda"), lr=0.1)
    changed = torch.nonzero((values != before).any(1)).flatten().cpu().tolist()
    assert changed == [3, 7] and float(acc[3]) == 1.0
    np.testing.assert_allclose((values[3] - before[3]).cpu().numpy(), -0.1 / (1 + 1e-8), rtol=1e-6)


@pytest.mark.parametrize("dtype,use_master", [(torch.float32, False), (torch.float16, True), (torch.float16, False)])
def test_adagrad_matches_oracle(gpu_lib, dtype, use_master):
    rng = np.random.default_rng(7)
    N, d, cap = 500, 32, 120
    v0 = (rng.standard_normal((N, d)) * 0.02).astype(np.float32)
    acc0 = rng.random(N).astype(np.float32)
    uniq = np.sort(rng.choice(N, cap - 7, replace=False))
    uniq = np.concatenate([uniq, np.full(7, N)]).astype(np.int32)
    g = rng.standard_normal((cap, d)).astype(np.float32)
    scale = 0.5
    # oracle
    ov = v0.astype(np.float16 if dtype == torch.float16 else np.float32)
    om = v0.copy() if use_master else None
    oa = acc0.copy()
    orow.rowwise_adagrad(ov, oa, uniq, g * np.float32(scale), 0.03, master=om)
    # GPU
    tv = torch.as_tensor(v0, device="cuda").to(dtype)
    tm = torch.as_tensor(v0, device="cuda").clone() if use_master else None
    ta = torch.as_tensor(acc0, device="cuda")
    R.rowwise_adagrad(tv, ta, torch.as_tensor(uniq, device="cuda"), torch.as_tensor(g, device="cuda"), 0.03,
                      master=tm, grad_scale=torch.tensor([scale], device="cuda"))
    np.testing.assert_allclose(ta.cpu().numpy(), oa, rtol=1e-6)
    if use_master:
        np.testing.assert_allclose(tm.cpu().numpy(), om, rtol=1e-6, atol=1e-7)
    tol = 1e-3 if dtype == torch.float16 else 1e-6
    np.testing.assert_allclose(tv.float().cpu().numpy(), ov.astype(np.float32), rtol=tol, atol=tol * 0.02)


@pytest.mark.parametrize("dtype,use_master,step", [(torch.float32, False, 0), (torch.float16, True, 5)])
def test_adam_matches_oracle(gpu_lib, dtype, use_master, step):
    rng = np.random.default_rng(8)
    N, d, cap = 300, 16, 90
    v0 = (rng.standard_normal((N, d)) * 0.02).astype(np.float32)
    m0 = (rng.standard_normal((N, d)) * 1e-3).astype(np.float32)
    s0 = (rng.random((N, d)) * 1e-6).astype(np.float32)
    uniq = np.concatenate([np.sort(rng.choice(N, cap - 3, replace=False)), np.full(3, N)]).astype(np.int32)
    g = (rng.standard_normal((cap, d)) * 1e-3).astype(np.float32)
    ov = v0.astype(np.float16 if dtype == torch.float16 else np.float32)
    om = v0.copy() if use_master else None
    m, v = m0.copy(), s0.copy()
    orow.lazy_adam(ov, m, v, uniq, g, 1e-3, step, master=om)
    tv = torch.as_tensor(v0, device="cuda").to(dtype)
    tmast = torch.as_tensor(v0, device="cuda").clone() if use_master else None
    tm, ts = torch.as_tensor(m0, device="cuda"), torch.as_tensor(s0, device="cuda")
    R.lazy_adam(tv, tm, ts, torch.as_tensor(uniq, device="cuda"), torch.as_tensor(g, device="cuda"), 1e-3, step,
                master=tmast)
    np.testing.assert_allclose(tm.cpu().numpy(), m, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(ts.cpu().numpy(), v, rtol=1e-5, atol=1e-12)
    if use_master:
        np.testing.assert_allclose(tmast.cpu().numpy(), om, rtol=1e-5, atol=1e-7)
    tol = 1e-3 if dtype == torch.float16 else 1e-5
    np.testing.assert_allclose(tv.float().cpu().numpy(), ov.astype(np.float32), rtol=tol, atol=tol * 0.02)


def test_sparse_row_update_step_matches_oracle(gpu_lib):
    """train.py:378-416 on one layer: merge, global clip (with a dense-part
    norm), Adagrad with the warmup-cosine lr, fp32 master + fp16 table."""
    rng = np.random.default_rng(9)
    B, T, H, k, N, d = 4, 32, 4, 8, 4096, 64
    values0 = (rng.standard_normal((N, d)) * 0.02).astype(np.float32)
    slots = rng.integers(0, N, (B, T, H, k)).astype(np.int32)
    w = rng.random((B, T, H, k)).astype(np.float32)
    g = rng.standard_normal((B, T, d)).astype(np.float32)
    tv = torch.as_tensor(values0, device="cuda").half()
    upd = R.SparseRowUpdate(tv, lr=1e-2, pool_lr_mult=3.0, warmup_steps=10, steps=100, grad_clip=1.0)
    upd.step = 20
    out = upd({"slots": [torch.as_tensor(slots, device="cuda")], "weights": [torch.as_tensor(w, device="cuda")]},
              {0: torch.as_tensor(g, device="cuda")}, [0], rest_sq=torch.tensor([4.0], device="cuda"))
    uniq, rows = orow.fetched_row_grads([slots], [w], [g], N)
    scale, gnorm = orow.clip_scale(4.0, rows, 1.0)
    lr = orow.warmup_cosine(20, 1e-2, 10, 100) * 3.0
    ov = values0.astype(np.float16)
    master = ov.astype(np.float32)  # SparseRowUpdate's master starts as the fp16 table's values
    acc = np.zeros(N, np.float32)
    orow.rowwise_adagrad(ov, acc, uniq, rows * np.float32(scale), lr, master=master)
    np.testing.assert_allclose(float(out["grad_norm"]), gnorm, rtol=1e-5)
    assert int(out["rows_updated"]) == np.unique(slots).shape[0]
    np.testing.assert_allclose(upd.acc.cpu().numpy(), acc, rtol=1e-5, atol=1e-12)
    np.testing.assert_allclose(upd.master.cpu().numpy(), master, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(tv.float().cpu().numpy(), ov.astype(np.float32), rtol=1e-3, atol=2e-5)


@pytest.mark.parametrize("zipf", [True, False])
def test_merge_without_zero_padding(gpu_lib, zipf):
    """zero_padding=False (the optimizers' merge) writes the same ids, rows
    and norms for the distinct slots and still pads uniq / row_sq; only the
    padding rows' content is left unwritten."""
    M, H, k, N, d = 2048, 4, 16, 1 << 16, 64
    if zipf:
        slots = torch.tensor(zipf_slots(M, H, k, N, seed=9), device="cuda", dtype=torch.int32)
    else:
        slots = torch.randint(0, N, (M * H * k,), device="cuda", dtype=torch.int32)
    g = torch.randn((M, d), device="cuda")
    w = torch.rand(M * H * k, device="cuda")
    a = R.merge_fetches(slots.reshape(-1), w, g, N)
    b = R.merge_fetches(slots.reshape(-1), w, g, N, zero_padding=False)
    U = int(a.num_unique[0])
    assert int(b.num_unique[0]) == U < a.uniq.shape[0]
    assert torch.equal(a.uniq, b.uniq)
    assert torch.equal(a.rows[:U], b.rows[:U])
    assert torch.equal(a.row_sq, b.row_sq)
    assert bool((a.rows[U:] == 0).all())


@pytest.mark.parametrize("case", ["reference", "uniform", "zipf", "empty"])
def test_merge_slot_counts(gpu_lib, case):
    """mpl_merge_rows_counts: the per-slot fetch counts (memory.py:215,
    np.bincount here) from the merge's segments, exact, written over a
    buffer that held other values; the merged rows are bitwise those of
    mpl_merge_rows."""
    rng = np.random.default_rng(21)
    if case == "reference":      # more fetches than slots: every slot repeats
        M, fpt, N, d = 37, 8, 16, 12
        slots = rng.integers(0, N, M * fpt).astype(np.int32)
    elif case == "uniform":      # fewer fetches than slots
        M, fpt, N, d = 300, 16, 1 << 14, 24
        slots = rng.integers(0, N, M * fpt).astype(np.int32)
    elif case == "zipf":         # the training shape
        M, H, k, N, d = 8192, 4, 16, 262144, 256
        fpt = H * k
        slots = zipf_slots(M, H, k, N).reshape(-1)
    else:
        M, fpt, N, d = 0, 4, 64, 8
        slots = np.zeros(0, np.int32)
    w = rng.random(M * fpt).astype(np.float32)
    g = rng.standard_normal((M, d)).astype(np.float32)
    ts, tw, tg = (torch.as_tensor(x, device="cuda") for x in (slots, w, g))
    counts = torch.full((N,), 7.0, device="cuda")
    a = R.merge_fetches(ts, tw, tg, N, slot_counts=counts)
    b = R.merge_fetches(ts, tw, tg, N)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(counts.cpu().numpy(), np.bincount(slots, minlength=N).astype(np.float32))
    assert torch.equal(a.uniq, b.uniq) and torch.equal(a.rows, b.rows) and torch.equal(a.row_sq, b.row_sq)
    assert int(a.num_unique[0]) == np.unique(slots).shape[0]


def test_sparse_row_update_counts_slots(gpu_lib):
    """SparseRowUpdate(count_slots=True) on two layers: the counts summed
    over the layers (model.py:136), and the update itself unchanged."""
    rng = np.random.default_rng(22)
    B, T, H, k, N, d = 2, 64, 4, 8, 2048, 32
    aux = {"slots": [], "weights": []}
    probes = {}
    for layer in (0, 2):
        aux["slots"].append(torch.as_tensor(rng.integers(0, N, (B, T, H, k)).astype(np.int32), device="cuda"))
        aux["weights"].append(torch.as_tensor(rng.random((B, T, H, k)).astype(np.float32), device="cuda"))
        probes[layer] = torch.as_tensor(rng.standard_normal((B, T, d)).astype(np.float32), device="cuda")
    v0 = torch.as_tensor((rng.standard_normal((N, d)) * 0.02).astype(np.float32), device="cuda")
    va, vb = v0.clone(), v0.clone()
    ua = R.SparseRowUpdate(va, lr=1e-2, grad_clip=1.0)
    ub = R.SparseRowUpdate(vb, lr=1e-2, grad_clip=1.0)
    oa = ua(aux, probes, [0, 2], count_slots=True)
    ob = ub(aux, probes, [0, 2])
    torch.cuda.synchronize()
    assert "slot_counts" not in ob
    ref = sum(np.bincount(s.cpu().numpy().reshape(-1), minlength=N) for s in aux["slots"])
    np.testing.assert_array_equal(oa["slot_counts"].cpu().numpy(), ref.astype(np.float32))
    assert torch.equal(va, vb) and torch.equal(ua.acc, ub.acc)


def test_clip_scale_dense_equals_two_pass(gpu_lib):
    """mpl_clip_scale_dense (the dense gradients' squares in the clip's own
    fp64 pass) against mpl_sum_squares + mpl_clip_scale and an fp64 numpy
    norm: gnorm within 1e-6 relative, scale likewise; empty inputs give
    gnorm 0 and scale 1."""
    rng = np.random.default_rng(31)
    row_sq = torch.as_tensor(rng.random(5000).astype(np.float32) * 1e-3, device="cuda")
    dense = [torch.as_tensor(rng.standard_normal(s).astype(np.float32) * 1e-2, device="cuda")
             for s in ((256, 1024), (4, 2, 512, 128), (1,))]
    a = R.clip_scale(row_sq, None, 1.0, dense)
    b = R.clip_scale(row_sq, R.sum_squares(dense), 1.0)
    torch.cuda.synchronize()
    ref = np.sqrt(float(row_sq.double().sum()) + sum(float((t.double() ** 2).sum()) for t in dense))
    np.testing.assert_allclose(float(a[1]), ref, rtol=1e-6)
    np.testing.assert_allclose(a.cpu().numpy(), b.cpu().numpy(), rtol=1e-6)
    z = R.clip_scale(torch.zeros(0, device="cuda"), None, 1.0, [])
    assert float(z[1]) == 0.0 and float(z[0]) == 1.0


def test_sparse_row_update_dense_grads_equals_rest_sq(gpu_lib):
    """SparseRowUpdate(dense_grads=...) clips like rest_sq=sum_squares(...)."""
    rng = np.random.default_rng(32)
    B, T, H, k, N, d = 2, 64, 4, 8, 2048, 32
    aux = {"slots": [torch.as_tensor(rng.integers(0, N, (B, T, H, k)).astype(np.int32), device="cuda")],
           "weights": [torch.as_tensor(rng.random((B, T, H, k)).astype(np.float32), device="cuda")]}
    probes = {0: torch.as_tensor(rng.standard_normal((B, T, d)).astype(np.float32), device="cuda")}
    dense = [torch.as_tensor(rng.standard_normal((64, 64)).astype(np.float32), device="cuda")]
    v0 = torch.as_tensor((rng.standard_normal((N, d)) * 0.02).astype(np.float32), device="cuda")
    va, vb = v0.clone(), v0.clone()
    oa = R.SparseRowUpdate(va, lr=1e-2, grad_clip=1.0)(aux, probes, [0], dense_grads=dense)
    ob = R.SparseRowUpdate(vb, lr=1e-2, grad_clip=1.0)(aux, probes, [0], rest_sq=R.sum_squares(dense))
    torch.cuda.synchronize()
    np.testing.assert_allclose(float(oa["grad_norm"]), float(ob["grad_norm"]), rtol=1e-6)
    torch.testing.assert_close(va, vb, rtol=1e-5, atol=1e-7)
