"""A Flax checkpoint (tests/golden/flax_params_small.msgpack, the encoding of
flax.serialization.to_bytes) loaded onto the GPU drives MemoryPool directly:
the lookup from the loaded parameters matches the oracle run on the
fixture's arrays."""

import numpy as np
import pytest
import torch

from model_amd import checkpoint as ck
from model_amd.memory import MemoryPool
from tests.golden.make_flax_params_fixture import OUT, arrays
from tests.gpu_helpers import oracle_check

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("values_dtype", [torch.float16, torch.float32])
def test_lookup_from_loaded_checkpoint(gpu_lib, values_dtype):
    tree = ck.load_params(OUT, device="cuda", values_dtype=values_dtype)
    params = ck.pool_params(tree)
    H, _, n, half = params["sub_keys"].shape
    pool = MemoryPool(n, H, 2 * half, params["values"].shape[1], 4, values_dtype=values_dtype)
    q = torch.randn((33, H, 2 * half), generator=torch.Generator(device="cuda").manual_seed(3), device="cuda")
    res = pool.lookup(params, q)
    np.testing.assert_array_equal(params["sub_keys"].cpu().numpy(), arrays()["pool"]["sub_keys"])
    oracle_check(pool, params, q, res)
