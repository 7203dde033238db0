"""mpl_hash_normal_fill (model_amd/csrc/hashinit.hip) against its numpy
statement (oracle/hashinit.py): every element equal, fp16 and fp32, at row
offsets up to the last rows of a 268M-slot table and at widths that are not
multiples of the vector size."""

import numpy as np
import pytest
import torch

from model_amd.hashinit import hash_normal_
from oracle import hashinit as hi

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,np_dtype", [(torch.float16, np.float16), (torch.float32, np.float32)])
@pytest.mark.parametrize("rows,cols,row0,seed", [
    (4096, 256, 0, 3),                    # the first rows of a pool table
    (1000, 256, (1 << 26) - 1000, 3),     # the last rows of the 67M-slot table
    (513, 3, 12345, 2 ** 64 - 1),         # narrow rows, the largest seed
    (7, 1000, (1 << 28) - 7, 11),         # the last rows of the 268M-slot table
])
def test_fill_matches_numpy(gpu_lib, dtype, np_dtype, rows, cols, row0, seed):
    t = torch.full((rows, cols), 9.0, dtype=dtype, device="cuda")
    hash_normal_(t, seed, 0.02, row0)
    want = hi.hash_normal_rows(seed, np.arange(row0, row0 + rows), cols, 0.02, np_dtype)
    np.testing.assert_array_equal(t.cpu().numpy(), want)


def test_fill_in_pieces_equals_one_fill(gpu_lib):
    whole = torch.empty((3000, 64), dtype=torch.float16, device="cuda")
    hash_normal_(whole, 5, 0.02)
    parts = torch.empty_like(whole)
    hash_normal_(parts[:1234], 5, 0.02, 0)
    hash_normal_(parts[1234:], 5, 0.02, 1234)
    assert torch.equal(whole, parts)
