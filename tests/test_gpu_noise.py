"""Routing noise (memory.py:155-159) on the GPU: mpl_gumbel_noise against the
oracle's restatement (oracle/noise.py, pinned by MurmurHash3's known answers
in tests/test_oracle.py), and the lookup's use of it.

The uniform grid is integer work, so the samples must agree to the rounding
of two fp32 logs: |g - g_oracle| <= 1e-6 * (1 + |g_oracle|) against the fp64
transform of the same u (a wrong hash, shift or clamp moves g by O(1))."""

import numpy as np
import pytest
import torch

from model_amd import _lib
from model_amd.memory import MemoryPool, routing_seed
from oracle import noise as on
from tests.gpu_helpers import make_params, oracle_check

pytestmark = pytest.mark.gpu


def _fill(seed, rows, n, offset=0):
    buf = torch.full((rows * n + offset + 4,), float("nan"), dtype=torch.float32, device="cuda")
    out = buf[offset:offset + rows * n]
    _lib.check(_lib.lib().mpl_gumbel_noise(seed, rows, n, _lib.ptr(out), _lib.stream_ptr(out.device)),
               "mpl_gumbel_noise")
    torch.cuda.synchronize()
    tail = buf[offset + rows * n:].cpu()
    assert torch.isnan(tail).all(), "wrote past the end"
    return out.reshape(rows, n).cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("seed,rows,n,offset", [
    (0, 64, 512, 0),                 # text-study rows: vector stores
    ((1 << 40) + 77, 37, 1001, 0),   # ragged n: scalar stores, seed high word used
    (123, 16, 4, 1),                 # output not 16-byte aligned: scalar stores
    (5, 3, 1, 0),                    # n = 1
])
def test_gumbel_fill_matches_oracle(gpu_lib, seed, rows, n, offset):
    g = _fill(seed, rows, n, offset)
    want = on.gumbel_noise(seed, rows, n)
    assert np.all(np.isfinite(g))
    np.testing.assert_array_less(np.abs(g - want), 1e-6 * (1.0 + np.abs(want)))


def test_gumbel_fill_full_size_moments(gpu_lib):
    """C4's noise shape (8,192 tokens x 8 codebooks x 512): Gumbel moments,
    support, and a spot check of rows against the oracle."""
    rows, n = 8192 * 8, 512
    g = _fill(2024, rows, n)
    assert abs(g.mean() - np.euler_gamma) < 2e-3
    assert abs(g.var() - np.pi ** 2 / 6) < 5e-3
    assert g.min() >= -np.log(-np.log(np.float64(on.FLT_MIN))) - 1e-5
    assert g.max() <= -np.log(-np.log(1.0 - 2.0 ** -23)) + 1e-5
    for r0 in (0, 4097, rows - 3):
        want = on.gumbel_noise(2024, 3, n, row0=r0)
        np.testing.assert_array_less(np.abs(g[r0:r0 + 3] - want), 1e-6 * (1.0 + np.abs(want)))


def test_lookup_noise_is_the_fill_of_its_seed(gpu_lib):
    """train=True draws its noise with mpl_gumbel_noise: an int rngs seed
    gives the fill of that seed, the selection agrees with the oracle run
    on that noise, and the same seed repeats it."""
    pool = MemoryPool(16, 2, 8, 12, 4, routing_noise=5.0, values_dtype=torch.float32)
    params = make_params(pool, 1)
    g = torch.Generator().manual_seed(3)
    q = torch.randn((15, 2, 8), generator=g).cuda()
    res = pool.lookup(params, q, train=True, noise_scale=0.5, rngs={"routing": 11})
    noise = res["gumbel"].reshape(15 * 2 * 2, 16).cpu().numpy().astype(np.float64)
    want = on.gumbel_noise(routing_seed({"routing": 11}), 15 * 2 * 2, 16)
    np.testing.assert_array_less(np.abs(noise - want), 1e-6 * (1.0 + np.abs(want)))
    oracle_check(pool, params, q, res, gumbel=res["gumbel"], noise_coef=5.0 * 0.5)
    again = pool.lookup(params, q, train=True, noise_scale=0.5, rngs={"routing": 11})
    assert torch.equal(res["slots"], again["slots"])
    other = pool.lookup(params, q, train=True, noise_scale=0.5, rngs={"routing": 12})
    assert not torch.equal(res["gumbel"], other["gumbel"])
