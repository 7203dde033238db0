"""GPU parity of the forward lookup (libmpl.so through the C ABI) against the
oracle: tiny reference shapes, the benchmark workloads' shapes, ties, noise,
query_scale, shuffle_reads, ragged token counts and split-key plans."""

import numpy as np
import pytest
import torch

from model_amd.memory import MemoryPool
from oracle import lookup as ol
from tests.gpu_helpers import make_params, oracle_check
from tests.test_oracle import tie_case

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "fp32": torch.float32}


def _queries(M, H, d_key, seed, lead=None):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((M, H, d_key), generator=g, device="cuda")
    return q.reshape(*(lead or (M,)), H, d_key)


@pytest.mark.parametrize("dt", ["fp32", "fp16"])
def test_reference_test_shapes(gpu_lib, dt):
    """tests/test_memory_pool.py:18-37 shapes: n=16, H=2, d_key=8, d=12, k=4."""
    pool = MemoryPool(16, 2, 8, 12, 4, values_dtype=DT[dt])
    params = make_params(pool, 1)
    q = _queries(15, 2, 8, 0, lead=(3, 5))
    res = pool.lookup(params, q)
    assert res["out"].shape == (3, 5, 12)
    assert res["aux"]["slots"].shape == (3, 5, 2, 4)
    oracle_check(pool, params, q, res)
    aux = res["aux"]
    assert float(aux["slot_counts"].sum()) == 3 * 5 * 2 * 4
    np.testing.assert_allclose(aux["subkey_counts"].sum(-1).cpu().numpy(), 3 * 5 * 4)


@pytest.mark.parametrize("dt", ["fp32", "fp16"])
def test_exact_tie_rules(gpu_lib, dt):
    """Hand-built ties: stage-1 lowest sub-key index, stage-2 lowest flat index."""
    q, keys = tie_case()
    pool = MemoryPool(4, 1, 4, 8, 2, values_dtype=DT[dt])
    params = make_params(pool, 2)
    params["sub_keys"] = torch.tensor(keys, device="cuda")
    res = pool.lookup(params, torch.tensor(q, device="cuda"))
    assert res["sub_idx"][0, 0, 0].tolist() == [3, 0]
    assert res["sub_idx"][0, 0, 1].tolist() == [1, 0]
    assert res["slots"][0, 0].tolist() == [13, 12]
    assert res["flat_idx"][0, 0].tolist() == [0, 1]


@pytest.mark.parametrize("dt,n,H,d_key,d,k,M", [
    ("fp32", 128, 4, 256, 256, 16, 1024),   # fact-task layer, 16,384 slots, fp32
    ("fp16", 512, 4, 256, 256, 16, 8192),   # text-study layer, 262,144 slots, fp16
    ("fp16", 64, 4, 64, 128, 16, 777),      # ragged token count
    ("fp16", 32, 2, 16, 32, 8, 100),        # k < 16, small half
    ("fp32", 64, 1, 32, 32, 32, 300),       # k = 32
    ("fp16", 100, 2, 32, 64, 1, 50),        # k = 1, n not a multiple of 32
])
def test_forward_parity(gpu_lib, dt, n, H, d_key, d, k, M):
    pool = MemoryPool(n, H, d_key, d, k, values_dtype=DT[dt])
    params = make_params(pool, 3, key_std=(d_key // 2) ** -0.5, value_std=0.02)
    q = _queries(M, H, d_key, 4)
    oracle_check(pool, params, q, pool.lookup(params, q))


def test_split_key_plan_small_batches(gpu_lib):
    """Few tokens and many sub-keys: the key range is split over workgroups
    and the per-split lists are merged."""
    pool = MemoryPool(2048, 4, 256, 256, 16, values_dtype=torch.float16)
    params = make_params(pool, 5, key_std=128 ** -0.5, value_std=0.02)
    for M in (1, 16, 200):
        q = _queries(M, 4, 256, 6 + M)
        oracle_check(pool, params, q, pool.lookup(params, q), min_tie_free=0.0)


@pytest.mark.parametrize("dt", ["fp32", "fp16"])
def test_exact_zero_scores_tie_by_index(gpu_lib, dt):
    """Keys orthogonal to the query score exactly 0 and fill places 2..k:
    the selection bound is then 0 itself, and those keys must still enter,
    lowest index first (lax.top_k), next to the one key along the query."""
    n, H, d_key, d, k = 64, 1, 16, 8, 4
    half = d_key // 2
    pool = MemoryPool(n, H, d_key, d, k, values_dtype=DT[dt])
    params = make_params(pool, 1)
    keys = torch.zeros((H, 2, n, half))
    keys[..., 1] = 1.0
    keys[..., 2] = 1.0
    keys[:, :, 5] = 0.0
    keys[:, :, 5, 0] = 1.0
    params["sub_keys"] = keys.cuda()
    q = torch.zeros((3, H, d_key))
    q[..., 0] = 1.0
    q[..., half] = 1.0
    res = pool.lookup(params, q.cuda())
    want = ol.top_k(np.einsum("hcnd,d->hcn", keys.numpy().astype(np.float64), np.eye(half)[0]), k)[1]
    assert want[0, 0].tolist() == [5, 0, 1, 2]
    assert res["sub_idx"].cpu().tolist() == [want.tolist()] * 3


@pytest.mark.parametrize("M", [1, 40])
def test_noise_with_split_plan(gpu_lib, M):
    """Decode-sized batches with routing noise: 32 split lists per codebook
    (n = 1,024) reduced in one stage-2 launch (k = 16), against the oracle
    with the same Gumbel draw."""
    n, H, d_key, d, k = 1024, 2, 64, 32, 16
    pool = MemoryPool(n, H, d_key, d, k, routing_noise=1.0, values_dtype=torch.float16)
    params = make_params(pool, 11, key_std=(d_key // 2) ** -0.5)
    q = _queries(M, H, d_key, 12 + M)
    g = torch.Generator(device="cuda").manual_seed(M)
    u = torch.rand((M, H, 2, n), generator=g, device="cuda").clamp_(min=1e-30)
    gumbel = -torch.log(-torch.log(u))
    res = pool.lookup(params, q, train=True, gumbel=gumbel, noise_scale=0.5)
    oracle_check(pool, params, q, res, gumbel=gumbel, noise_coef=0.5, min_tie_free=0.0)


@pytest.mark.parametrize("dt", ["fp32", "fp16"])
def test_noise_selects_on_noisy_scores_and_weights_stay_clean(gpu_lib, dt):
    """memory.py:155-178 with the Gumbel draw given to both sides."""
    pool = MemoryPool(64, 2, 32, 32, 8, routing_noise=1.0, values_dtype=DT[dt])
    params = make_params(pool, 7)
    q = _queries(200, 2, 32, 8)
    g = torch.Generator(device="cuda").manual_seed(9)
    u = torch.rand((200, 2, 2, 64), generator=g, device="cuda").clamp_(min=1e-30)
    gumbel = -torch.log(-torch.log(u))
    res = pool.lookup(params, q, train=True, gumbel=gumbel, noise_scale=0.7)
    oracle_check(pool, params, q, res, gumbel=gumbel, noise_coef=0.7)
    clean = pool.lookup(params, q)
    assert not torch.equal(clean["slots"], res["slots"])
    zero = pool.lookup(params, q, train=True, gumbel=gumbel, noise_scale=0.0)
    tie_free = oracle_check(pool, params, q, zero, gumbel=gumbel, noise_coef=0.0)
    same = (torch.sort(zero["slots"], -1).values == torch.sort(clean["slots"], -1).values).all(-1).cpu().numpy()
    assert same[tie_free].all()


def test_noise_from_generator_changes_picks_only_in_training(gpu_lib):
    """tests:66-76."""
    pool = MemoryPool(16, 2, 8, 12, 4, routing_noise=5.0, values_dtype=torch.float32)
    params = make_params(pool, 1)
    q = _queries(15, 2, 8, 0)
    a = pool.lookup(params, q, train=False, rngs={"routing": 3})
    b = pool.lookup(params, q, train=False, rngs={"routing": 4})
    c = pool.lookup(params, q, train=True, rngs={"routing": 3})
    d = pool.lookup(params, q, train=True, noise_scale=0.0, rngs={"routing": 3})
    assert torch.equal(a["slots"], b["slots"])
    assert not torch.equal(a["slots"], c["slots"])
    assert torch.equal(a["slots"], d["slots"])


def test_query_scale(gpu_lib):
    """memory.py:137,151-152; tests:118-125: scaling the query keeps the picks
    and sharpens the mix."""
    pool = MemoryPool(64, 2, 32, 32, 8, query_scale=True, values_dtype=torch.float32)
    params = make_params(pool, 10)
    q = _queries(120, 2, 32, 11)
    a = pool.lookup(params, q)
    oracle_check(pool, params, q, a)
    b = pool.lookup(params, q * 10.0)
    assert torch.equal(a["slots"], b["slots"])
    assert float(b["aux"]["top1_weight"]) > float(a["aux"]["top1_weight"])
    # q_len from the scoring kernel and the lazily normalised aux queries (memory.py:136-137, :220)
    qn = q.detach().double().cpu().numpy().reshape(120, 2, 2, 16)
    nrm = np.sqrt((qn * qn).sum(-1) + 1e-6)
    np.testing.assert_allclose(a["q_len"].cpu().numpy(), nrm / np.sqrt(16), rtol=1e-6)
    np.testing.assert_allclose(a["aux"]["queries"].cpu().numpy(), qn / nrm[..., None], rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("dt", ["fp32", "fp16"])
def test_shuffle_reads_closed_form(gpu_lib, dt):
    """tests:577-588."""
    pool = MemoryPool(16, 2, 8, 12, 4, values_dtype=DT[dt])
    params = make_params(pool, 12)
    q = _queries(15, 2, 8, 13)
    a = pool.lookup(params, q)
    b = pool.lookup(params, q, shuffle_reads=True)
    assert torch.equal(a["slots"], b["slots"])
    oracle_check(pool, params, q, b, shuffle_reads=True)
    N = 256
    read = (a["slots"].long() + N // 2 + 1) % N
    manual = torch.einsum("mhk,mhkd->md", a["weights"], params["values"][read].float())
    torch.testing.assert_close(b["out"], manual, rtol=1e-5, atol=1e-6)


def test_deterministic_and_empty(gpu_lib):
    pool = MemoryPool(512, 4, 256, 256, 16, values_dtype=torch.float16)
    params = make_params(pool, 14, key_std=128 ** -0.5, value_std=0.02)
    q = _queries(2000, 4, 256, 15)
    a = pool.lookup(params, q)
    b = pool.lookup(params, q)
    for key in ("slots", "weights", "out", "sub_idx", "sub_scores"):
        assert torch.equal(a[key], b[key]), key
    e = pool.lookup(params, q[:0])
    assert e["out"].shape == (0, 256)


def test_balance_loss_detects_collapse(gpu_lib):
    """tests:153-160 on the GPU statistics path."""
    pool = MemoryPool(16, 2, 8, 12, 4, values_dtype=torch.float32)
    params = make_params(pool, 1)
    spread = _queries(4096, 2, 8, 5)
    collapsed = spread[:1].expand_as(spread).contiguous()
    a = pool.lookup(params, spread)["aux"]
    b = pool.lookup(params, collapsed)["aux"]
    assert float(a["balance_loss"]) < 1.5
    assert float(b["balance_loss"]) > 2 * float(a["balance_loss"])
    # against the oracle's statistics
    res = ol.lookup_forward(spread.cpu().numpy(), params["sub_keys"].cpu().numpy(), None, np.log(10.0), top_k_=4)
    want = ol.aux_stats(res, n=16, noisy=False)
    np.testing.assert_allclose(float(a["balance_loss"]), want["balance_loss"], rtol=1e-4)
