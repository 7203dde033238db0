"""Decode-sized stage 1 (score_topk_decode: at most 4 tokens, fp16 scoring,
no routing noise) against the batched stage-1 kernel (score_topk_kernel),
which the other stage-1 tests pin to the oracle: the same queries scored
alone and as the first rows of an 8-token batch must give the same ids and
bit-identical scores (the decode kernel runs the batched kernel's MFMA chain
with the operands swapped), in every query mode, at ragged key counts,
padded key widths, k < 16 and the 67M- and 268M-slot key widths.  Also the
whole lookup at 1-4 tokens (the decode stage 2 and its fused value read:
slots, weights, output rows) against the batch, and exact ties by index
through the decode path."""

import numpy as np
import pytest
import torch

from model_amd import _lib

pytestmark = pytest.mark.gpu


def _pack(L, keys, H, n, half):
    st = _lib.stream_ptr(keys.device)
    packed = torch.empty(L.mpl_packed_keys_bytes(H, n, half, _lib.MPL_F16), dtype=torch.uint8, device="cuda")
    _lib.check(L.mpl_pack_keys(_lib.ptr(keys), H, n, half, _lib.MPL_F16, None, _lib.ptr(packed), st), "pack")
    return packed


def _topk(L, q, mode, qlen, packed, M, H, n, half, k, T):
    """mpl_score_topk on the first M rows of q; returns ids, scores and the
    q_len buffer (written in mode RAW_SCALED)."""
    st = _lib.stream_ptr(q.device)
    wsb = L.mpl_score_topk_workspace_bytes(M, H, n, half, k)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    sub_idx = torch.full((M, H, 2, k), -7, dtype=torch.int32, device="cuda")
    sub_sc = torch.full((M, H, 2, k), 7.0, dtype=torch.float32, device="cuda")
    ql = qlen[:M].clone() if qlen is not None else None
    _lib.check(L.mpl_score_topk(_lib.ptr(q), mode, _lib.ptr(ql), _lib.ptr(packed), M, H, n, half, k, _lib.MPL_F16,
                                _lib.ptr(T), None, None, _lib.ptr(ws), wsb, _lib.ptr(sub_idx), _lib.ptr(sub_sc), st),
               "topk")
    torch.cuda.synchronize()
    return sub_idx.cpu(), sub_sc.cpu(), (ql.cpu() if ql is not None else None)


SHAPES = [
    # H, n, d_key, k
    (4, 8192, 256, 16),   # the 67M-slot key width: 32 decode splits
    (4, 16384, 256, 16),  # the 268M-slot key width: 64 splits
    (2, 100, 16, 8),      # ragged n (a partial block), half 8 padded to 16, k < 16, one split
    (3, 1000, 48, 5),     # ragged n over splits, half 24 padded to 32, k = 5
    (4, 512, 128, 16),    # the text-study key count, half 64
    (1, 64, 256, 16),     # two blocks: one wave of the workgroup has keys
]


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("H,n,d_key,k", SHAPES)
@pytest.mark.parametrize("mode", ["raw", "raw_scaled", "normalized"])
def test_decode_stage1_equals_batched(gpu_lib, M, H, n, d_key, k, mode):
    L = _lib.lib()
    half = d_key // 2
    g = torch.Generator(device="cuda").manual_seed(M * 1000 + n + k + len(mode))
    MB = 8  # the batch: above the decode limit, so score_topk_kernel runs it
    q = torch.randn((MB, H, 2, half), generator=g, device="cuda")
    keys = torch.randn((H, 2, n, half), generator=g, device="cuda") * half ** -0.5
    packed = _pack(L, keys, H, n, half)
    T = torch.full((1,), 10.0, device="cuda")
    qlen = None
    if mode == "raw":
        qm = _lib.MPL_Q_RAW
    elif mode == "raw_scaled":
        qm = _lib.MPL_Q_RAW_SCALED
        qlen = torch.full((MB, H, 2), -3.0, device="cuda")
    else:
        qm = _lib.MPL_Q_NORMALIZED
        qn = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6)
        q = qn.half().contiguous()
        qlen = torch.rand((MB, H, 2), generator=g, device="cuda") + 0.5
    ids_d, sc_d, ql_d = _topk(L, q, qm, qlen, packed, M, H, n, half, k, T)
    ids_b, sc_b, ql_b = _topk(L, q, qm, qlen, packed, MB, H, n, half, k, T)
    np.testing.assert_array_equal(ids_d.numpy(), ids_b[:M].numpy())
    assert torch.equal(sc_d, sc_b[:M]), "decode scores differ from the batched kernel's"
    if ql_d is not None:
        assert torch.equal(ql_d, ql_b[:M])
    assert bool((ids_d >= 0).all()) and bool((ids_d < n).all())


@pytest.mark.parametrize("M,n,d,vdtype,shuffle", [
    (1, 8192, 256, torch.float16, 0),  # the 67M-slot decode lookup: 32 split lists
    (4, 8192, 256, torch.float16, 0),
    (2, 8192, 256, torch.float16, 1),  # shuffled reads
    (1, 8192, 128, torch.float16, 0),  # 4 rows per load instruction
    (1, 4096, 256, torch.float32, 0),  # fp32 rows: one row per instruction, 16 split lists
    (3, 2500, 512, torch.float16, 1),  # 1 KB rows, 10 split lists (ragged), shuffled
])
def test_decode_lookup_equals_batched(gpu_lib, M, n, d, vdtype, shuffle):
    """mpl_lookup at M tokens (decode stage 1, the decode stage 2 over the
    split lists with the fused value read) against the same tokens inside a
    16-token batch (batched stage 1, the wide stage 2): ids, scores, slots,
    weights and output rows bit for bit."""
    L = _lib.lib()
    H, half, k = 4, 128, 16
    g = torch.Generator(device="cuda").manual_seed(77 + M + n + d)
    MB = 16
    q = torch.randn((MB, H, 2, half), generator=g, device="cuda")
    keys = torch.randn((H, 2, n, half), generator=g, device="cuda") * half ** -0.5
    packed = _pack(L, keys, H, n, half)
    T = torch.full((1,), 10.0, device="cuda")
    # a table of n*n rows generated from a hash, so every slot is a real row
    from model_amd.hashinit import hash_normal_
    values = torch.empty((n * n, d), dtype=vdtype, device="cuda")
    hash_normal_(values, 5, 0.02)
    st = _lib.stream_ptr(q.device)
    res = {}
    for m in (M, MB):
        wsb = L.mpl_score_select_workspace_bytes(m, H, n, half, k)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
        i32, f32 = torch.int32, torch.float32
        sub_idx = torch.empty((m, H, 2, k), dtype=i32, device="cuda")
        sub_sc = torch.empty((m, H, 2, k), dtype=f32, device="cuda")
        fi = torch.empty((m, H, k), dtype=i32, device="cuda")
        sl = torch.empty((m, H, k), dtype=i32, device="cuda")
        w = torch.empty((m, H, k), dtype=f32, device="cuda")
        out = torch.empty((m, d), dtype=f32, device="cuda")
        _lib.check(L.mpl_lookup(_lib.ptr(q), _lib.MPL_Q_RAW, None, _lib.ptr(packed), m, H, n, half, k, _lib.MPL_F16,
                                _lib.ptr(T), None, None, _lib.ptr(ws), wsb, _lib.ptr(sub_idx), _lib.ptr(sub_sc),
                                _lib.ptr(fi), _lib.ptr(sl), _lib.ptr(w), _lib.ptr(values),
                                _lib.MPL_F16 if vdtype == torch.float16 else _lib.MPL_F32, d, shuffle,
                                _lib.ptr(out), st), "lookup")
        torch.cuda.synchronize()
        res[m] = (sub_idx.cpu(), sub_sc.cpu(), sl.cpu(), w.cpu(), out.cpu())
    del values
    torch.cuda.empty_cache()
    for a, b in zip(res[M], res[MB]):
        assert torch.equal(a, b[:M])


@pytest.mark.parametrize("M", [1, 3])
def test_decode_ties_by_index(gpu_lib, M):
    """Exact ties through the decode path: each codebook holds 8 distinct key
    vectors, each repeated 1,024 times at random places (n = 8,192), so a
    query's best score is reached by 1,024 keys in every split.  The top 16
    are then the 16 lowest indices holding the best vector (lax.top_k's
    order), however the splits and the workgroup's lists divide them."""
    L = _lib.lib()
    H, n, half, k, nv = 2, 8192, 128, 16, 8
    rng = np.random.default_rng(3 + M)
    base = rng.standard_normal((H, 2, nv, half))
    assign = np.stack([np.stack([rng.permutation(n) % nv for _ in range(2)]) for _ in range(H)])
    keys_np = np.take_along_axis(base, assign[..., None], axis=2)
    q_np = rng.standard_normal((M, H, 2, half))
    keys = torch.tensor(keys_np, dtype=torch.float32, device="cuda")
    q = torch.tensor(q_np, dtype=torch.float32, device="cuda")
    packed = _pack(L, keys, H, n, half)
    T = torch.full((1,), 10.0, device="cuda")
    ids, sc, _ = _topk(L, q, _lib.MPL_Q_RAW, None, packed, M, H, n, half, k, T)
    ids, sc = ids.numpy(), sc.numpy()
    qn = q_np / np.linalg.norm(q_np, axis=-1, keepdims=True)
    bn = base / np.linalg.norm(base, axis=-1, keepdims=True)
    cos = np.einsum("mhcd,hcvd->mhcv", qn, bn)
    order = np.argsort(-cos, axis=-1)
    srt = np.take_along_axis(cos, order, -1)
    free = (srt[..., 0] - srt[..., 1]) > 2.5 * 2.0 ** -11
    assert free.sum() >= 1
    for m, h, c in zip(*np.nonzero(free)):
        want = np.nonzero(assign[h, c] == order[m, h, c, 0])[0][:k]
        np.testing.assert_array_equal(ids[m, h, c], want, err_msg=f"row {m} head {h} codebook {c}")
        assert np.all(sc[m, h, c] == sc[m, h, c, 0])
