"""Routing-noise generator restated in numpy.  TEST INFRASTRUCTURE ONLY.

The reference draws the Gumbel noise of memory.py:155-159 with
``jax.random.gumbel(rng, scores.shape)``: ``-log(-log(u))`` with u uniform on
JAX's float grid {k * 2^-23 : k < 2^23} clamped below at the smallest normal
float.  libmpl's ``mpl_gumbel_noise`` keeps that transform and support but
draws u from a counter-based hash of (seed, row, column), restated here:

  * ``fmix32``          the 32-bit finalizer of MurmurHash3 (Austin Appleby,
                        public domain, smhasher/src/MurmurHash3.cpp);
  * ``murmur3_32``      MurmurHash3_x86_32 built on it, only so that fmix32
                        can be pinned against the hash's published known
                        answers (the tests hold them);
  * ``gumbel_noise``    the fill: row key rk = fmix32(fmix32(lo(row) ^
                        lo(seed)) ^ hi(seed) ^ hi(row)), h = fmix32(rk + j),
                        u = max((h >> 9) * 2^-23, FLT_MIN), g = -log(-log(u)).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only to check results.
"""

from __future__ import annotations

import numpy as np

M32 = 0xFFFFFFFF
FLT_MIN = float(np.finfo(np.float32).tiny)


def fmix32(x):
    """MurmurHash3 fmix32 on uint32 scalars or arrays (wrapping arithmetic)."""
    x = np.asarray(x, dtype=np.uint64) & M32
    x ^= x >> 16
    x = (x * 0x85EBCA6B) & M32
    x ^= x >> 13
    x = (x * 0xC2B2AE35) & M32
    x ^= x >> 16
    return x.astype(np.uint32)


def _rotl32(x: int, r: int) -> int:
    return ((x << r) | (x >> (32 - r))) & M32


def murmur3_32(data: bytes, seed: int = 0) -> int:
    """MurmurHash3_x86_32 of ``data`` (little-endian blocks)."""
    c1, c2 = 0xCC9E2D51, 0x1B873593
    h = seed & M32
    n = len(data)
    for i in range(n // 4):
        k = int.from_bytes(data[4 * i:4 * i + 4], "little")
        k = (k * c1) & M32
        k = _rotl32(k, 15)
        k = (k * c2) & M32
        h ^= k
        h = _rotl32(h, 13)
        h = (h * 5 + 0xE6546B64) & M32
    tail = data[n - n % 4:]
    k = 0
    if len(tail) >= 3:
        k ^= tail[2] << 16
    if len(tail) >= 2:
        k ^= tail[1] << 8
    if len(tail) >= 1:
        k ^= tail[0]
        k = (k * c1) & M32
        k = _rotl32(k, 15)
        k = (k * c2) & M32
        h ^= k
    h ^= n
    return int(fmix32(h))


def row_keys(seed: int, rows) -> np.ndarray:
    rows = np.asarray(rows, dtype=np.uint64)
    lo = (rows & M32).astype(np.uint64)
    hi = (rows >> 32).astype(np.uint64)
    a = fmix32(lo ^ (seed & M32)).astype(np.uint64)
    return fmix32(a ^ ((seed >> 32) & M32) ^ hi)


def uniform_bits(seed: int, rows: int, n: int, row0: int = 0) -> np.ndarray:
    """The 23-bit integers k = h >> 9 of rows row0 .. row0+rows-1, [rows, n]."""
    rk = row_keys(seed, np.arange(row0, row0 + rows, dtype=np.uint64)).astype(np.uint64)
    j = np.arange(n, dtype=np.uint64)
    h = fmix32((rk[:, None] + j[None, :]) & M32)
    return (h >> 9).astype(np.int64)


def gumbel_noise(seed: int, rows: int, n: int, row0: int = 0) -> np.ndarray:
    """g = -log(-log(u)) in float64 for the fill's [rows, n] block."""
    u = np.maximum(uniform_bits(seed, rows, n, row0).astype(np.float64) * 2.0 ** -23, FLT_MIN)
    return -np.log(-np.log(u))
