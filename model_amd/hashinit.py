"""Hash-defined normal tables on the GPU (mpl_hash_normal_fill).

Element (row, col) depends only on (seed, row, col): SplitMix64 of
row * cols + col keyed by the seed, then Box-Muller in fp64, times `scale`,
rounded to fp32 and then to the table dtype.  A table far larger than host
memory (the 67M- and 268M-slot pools) is filled in place on the GPU, and
any of its rows can be regenerated on the CPU from the same definition.
The reference's values init (memory.py:104-109) is jax.random.normal; this
generator is for synthetic tables of the pool's shapes.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import check, ptr


def hash_normal_(table: torch.Tensor, seed: int, scale: float, row0: int = 0) -> torch.Tensor:
    """Fills table [rows, cols] (fp16 or fp32, contiguous, on the GPU) in
    place with rows row0 .. row0 + rows - 1 of the hash table; returns it."""
    if table.device.type != "cuda":
        raise RuntimeError("hash_normal_ runs on the GPU only (libmpl.so)")
    if table.dim() != 2 or not table.is_contiguous():
        raise ValueError("hash_normal_ needs a contiguous [rows, cols] table")
    if table.dtype == torch.float16:
        code = _lib.MPL_F16
    elif table.dtype == torch.float32:
        code = _lib.MPL_F32
    else:
        raise TypeError(f"hash_normal_: unsupported dtype {table.dtype} (float16 or float32)")
    rows, cols = table.shape
    check(_lib.lib().mpl_hash_normal_fill(ptr(table), code, rows, cols, int(seed) & (2 ** 64 - 1), float(scale),
                                          int(row0), _lib.stream_ptr(table.device)), "mpl_hash_normal_fill")
    return table
