"""The hash-defined normal table (oracle/hashinit.py, the numpy statement of
mpl_hash_normal_fill) on the CPU.  Pinned by the published SplitMix64
sequence (Rosetta Code's SplitMix64 task: seed 1234567), a
Kolmogorov-Smirnov test of the Box-Muller output against N(0, 1), and the
defining property that any subset of rows equals the same rows of the full
table."""

import numpy as np
from scipy import stats

from oracle import hashinit as hi

GAMMA = 0x9E3779B97F4A7C15


def test_splitmix64_published_sequence():
    # SplitMix64 from state 1234567: the k-th output is the finalizer of state + k * gamma
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
            16408922859458223821]
    got = [int(hi.splitmix64(np.uint64((1234567 + k * GAMMA) % 2 ** 64))[0]) for k in range(5)]
    assert got == want


def test_values_are_standard_normal():
    x = hi.hash_normal_rows(3, np.arange(1000), 256, 1.0, np.float64).reshape(-1)
    assert abs(x.mean()) < 5 / np.sqrt(x.size) and abs(x.std() - 1.0) < 0.005
    assert stats.kstest(x, "norm").pvalue > 1e-3
    # rows and columns are not correlated with their neighbours
    t = x.reshape(1000, 256)
    assert abs(np.corrcoef(t[:, :-1].reshape(-1), t[:, 1:].reshape(-1))[0, 1]) < 0.01
    assert abs(np.corrcoef(t[:-1].reshape(-1), t[1:].reshape(-1))[0, 1]) < 0.01


def test_rows_regenerate_independently():
    full = hi.hash_normal_rows(7, np.arange(300), 40, 0.02)
    pick = np.array([299, 0, 17, 17, 150])
    np.testing.assert_array_equal(hi.hash_normal_rows(7, pick, 40, 0.02), full[pick])
    assert full.dtype == np.float16
    # another seed is another table; the scale multiplies before the fp32 rounding
    assert not np.array_equal(hi.hash_normal_rows(8, pick, 40, 0.02), full[pick])
    one = hi.hash_normal_rows(7, pick, 40, 1.0, np.float64)
    np.testing.assert_allclose(hi.hash_normal_rows(7, pick, 40, 0.02, np.float32), one * 0.02, rtol=2e-7)
    # far rows of a 268M-slot table are as cheap as near ones
    far = hi.hash_normal_rows(3, [(1 << 28) - 1], 256, 0.02)
    assert far.shape == (1, 256) and np.isfinite(far.astype(np.float32)).all()
