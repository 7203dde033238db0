"""The hash-defined normal table of mpl_hash_normal_fill, in numpy.
TEST INFRASTRUCTURE ONLY: the GPU fill (model_amd/csrc/hashinit.hip) is the
product; this module regenerates any rows of such a table on the CPU (the
CPU baseline of bench.py reads the rows a lookup selects from a 34 GB table
that is never materialised on the host), and the tests compare the two.

Element (row, col) of a [rows, cols] table with seed s and scale a:
  index = row * cols + col                          (uint64, wrapping)
  h     = splitmix64(splitmix64(s) ^ index)
  u1    = ((h >> 40) + 1) / 2^24,  u2 = (h & 0xFFFFFF) / 2^24
  value = dtype(float32(sqrt(-2 ln u1) * cos(2 pi u2) * a))   (fp64 math)
splitmix64 is the finalizer of SplitMix64 (Steele, Lea & Flood, "Fast
splittable pseudorandom number generators", OOPSLA 2014): x + 0x9E3779B97F4A7C15,
then z ^= z >> 30; z *= 0xBF58476D1CE4E5B9; z ^= z >> 27; z *= 0x94D049BB133111EB;
z ^= z >> 31.  The memory pool's own init (KumarDev7/model
memory_pool_model/memory.py:104-109) is jax.random.normal * d^-0.5; this
generator stands in for it in the benchmark tables (values ~ N(0, 0.02)).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module.
"""

from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(x) -> np.ndarray:
    """The SplitMix64 finalizer of (an array of) uint64 values."""
    z = np.array(x, dtype=np.uint64, ndmin=1)
    with np.errstate(over="ignore"):
        z = z + GAMMA
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


def hash_normal_rows(seed: int, rows, cols: int, scale: float, dtype=np.float16) -> np.ndarray:
    """Rows `rows` (int array) of the [*, cols] table: [len(rows), cols] in dtype."""
    rows = np.asarray(rows, dtype=np.int64).reshape(-1)
    key = splitmix64(np.uint64(seed))[0]
    with np.errstate(over="ignore"):
        index = rows.astype(np.uint64)[:, None] * np.uint64(cols) + np.arange(cols, dtype=np.uint64)[None, :]
    h = splitmix64(index ^ key).reshape(rows.size, cols)
    u1 = ((h >> np.uint64(40)) + np.uint64(1)).astype(np.float64) * 2.0 ** -24
    u2 = (h & np.uint64(0xFFFFFF)).astype(np.float64) * 2.0 ** -24
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)
    return (z * float(np.float32(scale))).astype(np.float32).astype(dtype)
