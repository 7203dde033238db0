"""MemoryPool.init (memory.py:60-61, 94-113 of the reference) on the CPU: the
parameter names, shapes and dtypes, sub_keys on the unit sphere (isotropic),
values ~ N(0, d_value^-1/2) in the table dtype, log_temperature =
log(init_temperature) as an fp32 scalar, and no values parameter with a
host pool (memory.py:103-109)."""

import math

import numpy as np
import pytest
import torch

from model_amd.memory import MemoryPool


@pytest.mark.parametrize("values_dtype", [torch.float16, torch.float32])
def test_init_statistics(values_dtype):
    n, H, d_key, d = 64, 4, 32, 96
    pool = MemoryPool(n, H, d_key, d, 8, init_temperature=7.0, values_dtype=values_dtype)
    p = pool.init(3, device="cpu")["params"]
    assert set(p) == {"sub_keys", "values", "log_temperature"}
    keys, values, log_t = p["sub_keys"], p["values"], p["log_temperature"]
    assert keys.shape == (H, 2, n, d_key // 2) and keys.dtype == torch.float32
    assert values.shape == (n * n, d) and values.dtype == values_dtype
    assert log_t.shape == () and log_t.dtype == torch.float32
    assert float(log_t) == np.float32(math.log(7.0))

    # unit sphere: every key has norm 1 (up to the 1e-6 of the normalisation),
    # and the directions are isotropic: mean ~ 0, per-dim variance ~ 1/half
    k64 = keys.double().numpy()
    norms = np.linalg.norm(k64, axis=-1)
    np.testing.assert_allclose(norms, 1.0, atol=1e-5)
    half = d_key // 2
    flat = k64.reshape(-1, half)
    assert np.abs(flat.mean(0)).max() < 4.0 / math.sqrt(flat.shape[0] * half)
    np.testing.assert_allclose(flat.var(0), 1.0 / half, rtol=0.15)

    # values ~ N(0, d^-1/2): mean, standard deviation, and the normal's fourth
    # moment (3 sigma^4) over 393,216 draws
    v = values.double().numpy().reshape(-1)
    sd = d ** -0.5
    assert abs(v.mean()) < 5 * sd / math.sqrt(v.size)
    assert abs(v.std() / sd - 1.0) < 0.01
    assert abs((v ** 4).mean() / sd ** 4 / 3.0 - 1.0) < 0.05


def test_init_seeds_and_host_pool():
    pool = MemoryPool(32, 2, 16, 16, 4)
    a = pool.init(5, device="cpu")["params"]
    b = pool.init(5, device="cpu")["params"]
    c = pool.init(6, device="cpu")["params"]
    assert torch.equal(a["sub_keys"], b["sub_keys"]) and torch.equal(a["values"], b["values"])
    assert not torch.equal(a["sub_keys"], c["sub_keys"])
    # the default temperature is the floor, log(10) (memory.py:77, 110-113)
    assert float(a["log_temperature"]) == np.float32(math.log(10.0))
    hp = MemoryPool(32, 2, 16, 16, 4, host_pool="some_pool")
    p = hp.init(5, device="cpu")["params"]
    assert set(p) == {"sub_keys", "log_temperature"}


def test_init_rejects_odd_d_key_and_top_k_above_n():
    with pytest.raises(AssertionError):
        MemoryPool(32, 2, 15, 16, 4)
    with pytest.raises(AssertionError):
        MemoryPool(8, 2, 16, 16, 9)
