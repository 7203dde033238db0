"""The host tier's memmap mode on the CPU (host_pool.py: the reference's file
layout, initialisation, host-thread gather and optimizer step).  The update
is checked against the oracle's restatement of the trainer's optimizers
(oracle/rows.py, train.py:412-426), whose host_pool.py twin it is; the
initialisation against numpy's published default_rng(0) normals and a single
undivided draw (chunking must not change the stream)."""

import numpy as np
import pytest

from model_amd.host_pool import HostPool, get
from oracle import rows as orow


def test_init_is_the_reference_stream(tmp_path):
    # numpy's Generator(PCG64(0)).standard_normal(3), as printed by numpy
    first = np.array([0.12573022, -0.13210486, 0.64042265])
    pool = HostPool(17, 3, path=str(tmp_path / "a"), seed=0, trainable=False)
    np.testing.assert_allclose(pool.values[0] / 3 ** -0.5, first, rtol=1e-6)  # printed to 8 digits, stored fp32
    # 2^18 + 5 rows are drawn in two chunks: the same stream as one draw
    n, d = (1 << 18) + 5, 2
    big = HostPool(n, d, path=str(tmp_path / "b"), seed=4, trainable=False, dtype=np.float32)
    want = (np.random.default_rng(4).standard_normal((n, d)) * d ** -0.5).astype(np.float32)
    np.testing.assert_array_equal(np.asarray(big.values), want)
    assert get(big.name) is big


def test_reopen_and_shape_check(tmp_path):
    p = str(tmp_path / "pool")
    a = HostPool(64, 8, path=p, seed=1, optimizer="rowwise_adagrad")
    a.values[3] = 7.0
    a.flush()
    b = HostPool(64, 8, path=p, seed=99, optimizer="rowwise_adagrad")  # reopened, not re-initialised
    np.testing.assert_array_equal(np.asarray(b.values), np.asarray(a.values))
    with pytest.raises(ValueError):
        HostPool(65, 8, path=p, optimizer="rowwise_adagrad")


def test_gather_clips_and_converts(tmp_path):
    pool = HostPool(32, 6, path=str(tmp_path / "g"), dtype=np.float16, trainable=False)
    idx = np.array([0, 31, 40, -3, 5])
    got = pool.gather(idx)
    assert got.dtype == np.float32
    np.testing.assert_array_equal(got, np.asarray(pool.values)[[0, 31, 31, 0, 5]].astype(np.float32))


@pytest.mark.parametrize("optimizer,dtype", [("rowwise_adagrad", np.float32), ("rowwise_adagrad", np.float16),
                                             ("adam", np.float32), ("adam", np.float16)])
def test_update_matches_trainer_optimizer(tmp_path, optimizer, dtype):
    """Three steps on overlapping row sets with padding entries, against
    oracle.rows (host step s is the trainer's 0-based step s - 1)."""
    N, d = 50, 12
    pool = HostPool(N, d, path=str(tmp_path / optimizer), dtype=dtype, optimizer=optimizer, seed=3)
    vals = np.asarray(pool.values).copy()
    acc = np.zeros(N, np.float32)
    m = np.zeros((N, d), np.float32)
    v = np.zeros((N, d), np.float32)
    rng = np.random.default_rng(0)
    for step in (1, 2, 3):
        uniq = np.concatenate([np.sort(rng.choice(N, 20, replace=False)), [N, N]]).astype(np.int32)
        g = rng.standard_normal((uniq.size, d)).astype(np.float32)
        lr = 0.01 * step
        pool.update(uniq, g, step, lr)
        if optimizer == "rowwise_adagrad":
            orow.rowwise_adagrad(vals, acc, uniq, g, lr)
        else:
            orow.lazy_adam(vals, m, v, uniq, g, lr, step - 1)
    # host_pool.py takes Adam's bias corrections in Python floats (float64),
    # train.py in fp32: the two references differ by ~1e-5 of an update
    tol = 2e-6 if dtype == np.float32 else 1e-3
    np.testing.assert_allclose(np.asarray(pool.values).astype(np.float64), vals.astype(np.float64), rtol=tol,
                               atol=max(tol * 0.1, 1e-6))
    if optimizer == "rowwise_adagrad":
        np.testing.assert_allclose(np.asarray(pool.acc), acc, rtol=1e-6)
    else:
        # host_pool.py's moments use Python-float betas, train.py's fp32 ones
        np.testing.assert_allclose(np.asarray(pool.m), m, rtol=1e-6, atol=1e-6 * np.abs(m).max())
        np.testing.assert_allclose(np.asarray(pool.v), v, rtol=1e-6, atol=1e-6 * np.abs(v).max())


def test_save_load_roundtrip(tmp_path):
    a = HostPool(40, 4, path=str(tmp_path / "x"), optimizer="adam", seed=2)
    a.update(np.array([1, 5, 40]), np.ones((3, 4), np.float32), 1, 0.1)
    a.save(str(tmp_path / "snap"))
    b = HostPool(40, 4, path=str(tmp_path / "y"), optimizer="adam", seed=9)
    b.load(str(tmp_path / "snap"))
    for k in ("values", "m", "v"):
        np.testing.assert_array_equal(np.asarray(getattr(b, k)), np.asarray(getattr(a, k)))
    assert a.nbytes() == 40 * 4 * 4 * 3
