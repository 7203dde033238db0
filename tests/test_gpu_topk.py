"""mpl_score_topk (stage 1 alone: memory.py:161-163, and the clean _top_k of
memory.py:207) against mpl_score_select's stage-1 outputs, which the lookup
tests check against the oracle, and against the oracle's top_k directly.

Ids bit-exact; scores bit-exact to mpl_score_select's (the same kernels and
the same exact list merges), and within fp16-scoring rounding of the
oracle's fp64 scores on near-tie-free rows.  Shapes cover one split, split
lists reduced by merge levels (k = 16) and by the pair kernel (k != 16),
routing noise, and fp32 scoring, up to the 67M- and 268M-slot key widths
(n = 8,192 and 16,384) with k = 8, 16 and 32."""

import numpy as np
import pytest
import torch

from model_amd import _lib
from oracle import lookup as ol

pytestmark = pytest.mark.gpu


def _run(M, H, n, d_key, k, score, noise, seed):
    L = _lib.lib()
    half = d_key // 2
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((M, H, 2, half), generator=g).cuda()
    keys = torch.randn((H, 2, n, half), generator=g).cuda()
    gum = None
    if noise:
        gum = -torch.log(-torch.log(torch.rand((M, H, 2, n), generator=g).clamp_(1e-20, 1 - 1e-7))).cuda()
    packed = torch.empty(L.mpl_packed_keys_bytes(H, n, half, score), dtype=torch.uint8, device="cuda")
    khat = torch.empty_like(keys)
    st = _lib.stream_ptr(q.device)
    _lib.check(L.mpl_pack_keys(_lib.ptr(keys), H, n, half, score, _lib.ptr(khat), _lib.ptr(packed), st), "pack")
    mode = _lib.MPL_Q_RAW
    if score == _lib.MPL_F32:  # raw queries are fp16-scoring only: normalise first
        qn = torch.empty_like(q)
        _lib.check(L.mpl_l2_normalize(_lib.ptr(q), M * H * 2, half, 1e-6, _lib.ptr(qn), None, None, st), "norm")
        q, mode = qn, _lib.MPL_Q_NORMALIZED
    T, coef = 10.0, (0.7 if noise else 0.0)
    T_dev = torch.full((1,), T, device="cuda")  # device scalars, as the C ABI takes them
    coef_dev = torch.full((1,), coef, device="cuda") if noise else None
    i32, f32 = torch.int32, torch.float32
    outs = {}
    for name in ("select", "topk"):
        sub_idx = torch.full((M, H, 2, k), -7, dtype=i32, device="cuda")
        sub_sc = torch.full((M, H, 2, k), 7.0, dtype=f32, device="cuda")
        if name == "select":
            wsb = L.mpl_score_select_workspace_bytes(M, H, n, half, k)
            ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
            fi = torch.empty((M, H, k), dtype=i32, device="cuda")
            sl = torch.empty((M, H, k), dtype=i32, device="cuda")
            w = torch.empty((M, H, k), dtype=f32, device="cuda")
            _lib.check(L.mpl_score_select(_lib.ptr(q), mode, None, _lib.ptr(packed), M, H, n, half, k, score,
                                          _lib.ptr(T_dev), _lib.ptr(gum), _lib.ptr(coef_dev), _lib.ptr(ws), wsb, _lib.ptr(sub_idx), _lib.ptr(sub_sc),
                                          _lib.ptr(fi), _lib.ptr(sl), _lib.ptr(w), st), "select")
        else:
            wsb = L.mpl_score_topk_workspace_bytes(M, H, n, half, k)
            ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
            _lib.check(L.mpl_score_topk(_lib.ptr(q), mode, None, _lib.ptr(packed), M, H, n, half, k, score,
                                        _lib.ptr(T_dev), _lib.ptr(gum), _lib.ptr(coef_dev), _lib.ptr(ws), wsb, _lib.ptr(sub_idx), _lib.ptr(sub_sc),
                                        st), "topk")
        torch.cuda.synchronize()
        outs[name] = (sub_idx.cpu().numpy(), sub_sc.cpu().numpy())
    return q, khat, gum, T, coef, outs


@pytest.mark.parametrize("M,H,n,d_key,k,score,noise", [
    (300, 4, 512, 256, 16, _lib.MPL_F16, False),   # text-study keys, one split
    (512, 4, 512, 256, 16, _lib.MPL_F16, False),   # 16 splits: merge levels
    (3, 4, 1024, 256, 16, _lib.MPL_F16, False),    # decode: 32 splits, two levels
    (37, 2, 64, 16, 4, _lib.MPL_F16, False),       # k != 16 with splits: pair kernel
    (5, 2, 640, 32, 16, _lib.MPL_F16, True),       # noise with splits
    (40, 2, 96, 12, 8, _lib.MPL_F32, True),        # fp32 scoring, noise, ragged n
    (256, 4, 8192, 256, 32, _lib.MPL_F16, False),  # k = 32 at the 67M-slot width: split lists, pair kernel
    (64, 4, 8192, 256, 8, _lib.MPL_F16, False),    # k = 8 at n = 8,192
    (300, 4, 8192, 256, 16, _lib.MPL_F16, True),   # routing noise at n = 8,192 (split noisy stage 1)
    (1, 4, 16384, 256, 16, _lib.MPL_F16, False),   # one token at the 268M-slot width: 64 splits
    (100, 2, 4096, 64, 16, _lib.MPL_F32, False),   # fp32 scoring at n = 4,096 with splits
])
def test_topk_equals_select_stage1(gpu_lib, M, H, n, d_key, k, score, noise):
    q, khat, gum, T, coef, outs = _run(M, H, n, d_key, k, score, noise, seed=M + n + k)
    np.testing.assert_array_equal(outs["topk"][0], outs["select"][0])
    np.testing.assert_array_equal(outs["topk"][1], outs["select"][1])
    # against the oracle's top_k of the fp64 select scores, on rows whose k-th
    # and (k+1)-th scores are apart by more than twice the fp16-scoring error:
    # unit rows rounded to fp16 move a cosine by at most 2 * 2^-12, so a score
    # by at most 2^-11 * T
    qn = ol.l2_normalize(q.cpu().numpy().astype(np.float64))
    kn = khat.cpu().numpy().astype(np.float64)
    cos = np.einsum("mhcd,hcnd->mhcn", qn, kn)
    sel = cos * T + (coef * gum.cpu().numpy().astype(np.float64) if gum is not None else 0.0)
    want = ol.top_k(sel, k)[1]
    srt = -np.sort(-sel, axis=-1)
    gap = srt[..., k - 1] - (srt[..., k] if n > k else -np.inf)
    free = gap > 2.5 * 2.0 ** -11 * T
    # wide key ranges crowd the k-th score (n = 8,192, k = 32: about a quarter
    # of the rows are tie-free), so the floor on checked rows drops there
    assert free.mean() > (0.5 if n <= 2048 else 0.2) and free.sum() >= 1
    # the set is fixed there; the order inside it may swap near-tied entries
    got_ids = outs["topk"][0][free]
    np.testing.assert_array_equal(np.sort(got_ids, -1), np.sort(want[free], -1))
    clean = np.take_along_axis((cos * T)[free], got_ids.astype(np.int64), -1)
    np.testing.assert_allclose(outs["topk"][1][free], clean, rtol=0, atol=2.0 ** -11 * T)


@pytest.mark.parametrize("M,n", [(16, 8192), (4096, 8192), (16, 16384), (64, 16384)])
def test_repeated_keys_tie_by_index_across_flushes(gpu_lib, M, n):
    """Exact ties through the select pass's flushes at the 67M- and 268M-slot
    key widths (n = 8,192 and 16,384; at 16 and 64 tokens the short splits of
    4 and 8 blocks): each codebook holds 16 distinct key vectors, each
    repeated n / 16 times at random places, so a query's best score is
    reached by that many keys at once and the lane buffers overflow many
    times.  The top 16 are then the 16 lowest indices holding the best vector
    (lax.top_k's order, memory.py:34-57), which a flush threshold taken from
    both lanes of the query must keep: a later key that ties the k-th best
    loses on its larger index.  Checked on rows whose best and second-best
    distinct vectors are apart by more than the fp16-scoring error."""
    L = _lib.lib()
    H, half, k, nv = 1, 128, 16, 16
    rng = np.random.default_rng(11)
    base = rng.standard_normal((H, 2, nv, half))
    assign = np.stack([np.stack([rng.permutation(n) % nv for _ in range(2)]) for _ in range(H)])  # [H, 2, n]
    keys_np = np.take_along_axis(base, assign[..., None], axis=2)  # [H, 2, n, half]
    q_np = rng.standard_normal((M, H, 2, half))
    keys = torch.tensor(keys_np, dtype=torch.float32, device="cuda")
    q = torch.tensor(q_np, dtype=torch.float32, device="cuda")
    score = _lib.MPL_F16
    packed = torch.empty(L.mpl_packed_keys_bytes(H, n, half, score), dtype=torch.uint8, device="cuda")
    khat = torch.empty_like(keys)
    st = _lib.stream_ptr(q.device)
    _lib.check(L.mpl_pack_keys(_lib.ptr(keys), H, n, half, score, _lib.ptr(khat), _lib.ptr(packed), st), "pack")
    T_dev = torch.full((1,), 10.0, device="cuda")
    wsb = L.mpl_score_topk_workspace_bytes(M, H, n, half, k)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    sub_idx = torch.full((M, H, 2, k), -7, dtype=torch.int32, device="cuda")
    sub_sc = torch.empty((M, H, 2, k), dtype=torch.float32, device="cuda")
    _lib.check(L.mpl_score_topk(_lib.ptr(q), _lib.MPL_Q_RAW, None, _lib.ptr(packed), M, H, n, half, k, score,
                                _lib.ptr(T_dev), None, None, _lib.ptr(ws), wsb, _lib.ptr(sub_idx), _lib.ptr(sub_sc),
                                st), "topk")
    got = sub_idx.cpu().numpy()
    sc = sub_sc.cpu().numpy()
    # fp64 cosine of each query with each distinct vector
    qn = q_np / np.linalg.norm(q_np, axis=-1, keepdims=True)
    bn = base / np.linalg.norm(base, axis=-1, keepdims=True)
    cos = np.einsum("mhcd,hcvd->mhcv", qn, bn)
    order = np.argsort(-cos, axis=-1)
    best = order[..., 0]
    srt = np.take_along_axis(cos, order, -1)
    free = (srt[..., 0] - srt[..., 1]) > 2.5 * 2.0 ** -11
    assert free.mean() > 0.5
    checked = 0
    for m, h, c in zip(*np.nonzero(free)):
        want = np.nonzero(assign[h, c] == best[m, h, c])[0][:k]
        np.testing.assert_array_equal(got[m, h, c], want, err_msg=f"row {m} head {h} codebook {c}")
        assert np.all(sc[m, h, c] == sc[m, h, c, 0])  # one exact score for every copy
        checked += 1
    assert checked >= 1


@pytest.mark.parametrize("M,n,noise", [(8192, 512, False), (8192, 512, True), (4096, 8192, False)])
def test_stage1_repeats_bit_for_bit(gpu_lib, M, n, noise):
    """The stage-1 kernel's LDS key tiles (the bound pass of the register
    path; both passes with routing noise) are overwritten by DMA while the
    waves go on: a read of a tile still in flight when the next block's DMA
    lands returns a torn vector, a score of no key, which can lift the bound
    above the k-th best and drop candidates, differently from run to run.
    Eight launches on the same inputs at the text-study and 67M-slot key
    widths, with and without noise, must give identical ids and scores."""
    L = _lib.lib()
    H, half, k = 4, 128, 16
    g = torch.Generator(device="cuda").manual_seed(n + M + int(noise))
    q = torch.randn((M, H, 2, half), generator=g, device="cuda")
    keys = torch.randn((H, 2, n, half), generator=g, device="cuda") * half ** -0.5
    gum = -torch.log(-torch.log(torch.rand((M, H, 2, n), generator=g, device="cuda").clamp_(1e-20, 1 - 1e-7))) \
        if noise else None
    st = _lib.stream_ptr(q.device)
    packed = torch.empty(L.mpl_packed_keys_bytes(H, n, half, _lib.MPL_F16), dtype=torch.uint8, device="cuda")
    _lib.check(L.mpl_pack_keys(_lib.ptr(keys), H, n, half, _lib.MPL_F16, None, _lib.ptr(packed), st), "pack")
    T = torch.full((1,), 10.0, device="cuda")
    coef = torch.full((1,), 1.0, device="cuda") if noise else None
    wsb = L.mpl_score_topk_workspace_bytes(M, H, n, half, k)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    first = None
    for it in range(8):
        sub_idx = torch.full((M, H, 2, k), -7, dtype=torch.int32, device="cuda")
        sub_sc = torch.full((M, H, 2, k), 7.0, device="cuda")
        _lib.check(L.mpl_score_topk(_lib.ptr(q), _lib.MPL_Q_RAW, None, _lib.ptr(packed), M, H, n, half, k,
                                    _lib.MPL_F16, _lib.ptr(T), _lib.ptr(gum), _lib.ptr(coef), _lib.ptr(ws), wsb,
                                    _lib.ptr(sub_idx), _lib.ptr(sub_sc), st), "topk")
        torch.cuda.synchronize()
        if first is None:
            first = (sub_idx, sub_sc)
            assert bool((sub_idx >= 0).all()) and bool((sub_idx < n).all())
        else:
            assert torch.equal(sub_idx, first[0]), f"run {it}: {int((sub_idx != first[0]).sum())} ids differ"
            assert torch.equal(sub_sc, first[1]), f"run {it}: scores differ"
