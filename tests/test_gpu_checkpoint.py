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


@pytest.mark.parametrize("optimizer", ["rowwise_adagrad", "adam"])
def test_train_state_resume_continues_the_same_run(gpu_lib, optimizer):
    """train.py:559-583: 3 sparse updates in one go equal 2 updates, a
    TrainState checkpoint, a fresh SparseRowUpdate resumed from it, and the
    third update (bit for bit: table, master, optimizer state, step)."""
    import io

    from model_amd import checkpoint as ck
    from model_amd import rows as R

    N, d, M, H, k = 4096, 64, 128, 4, 8
    rng = np.random.default_rng(11)
    table0 = torch.as_tensor((0.02 * rng.standard_normal((N, d))).astype(np.float16), device="cuda")
    batches = []
    for _ in range(3):
        slots = torch.as_tensor(rng.integers(0, N, (M, H, k)).astype(np.int32), device="cuda")
        w = torch.softmax(torch.as_tensor(rng.standard_normal((M, H, k)).astype(np.float32), device="cuda"), -1)
        g = torch.as_tensor((1e-2 * rng.standard_normal((M, d))).astype(np.float32), device="cuda")
        batches.append(({"slots": [slots], "weights": [w]}, {0: g}))

    def make(table):
        return R.SparseRowUpdate(table, optimizer=optimizer, lr=1e-2, warmup_steps=1, steps=10, grad_clip=1.0)

    a_tab = table0.clone()
    a = make(a_tab)
    for aux, g in batches:
        a(aux, g, [0])

    b_tab = table0.clone()
    b = make(b_tab)
    for aux, g in batches[:2]:
        b(aux, g, [0])
    pool = b.train_state_pool()
    buf = io.BytesIO()
    ck.save_train_state(buf, step=pool["step"], params={"pool": {"values": pool["values"]}}, opt_state={},
                        subkey_usage=torch.zeros(1), slot_usage=torch.zeros(1), pool_m=pool["pool_m"],
                        pool_v=pool["pool_v"])
    c_tab = torch.zeros_like(table0)
    c = make(c_tab)
    c.resume(ck.load_train_state(buf.getvalue(), device="cuda"))
    assert c.step == 2
    aux, g = batches[2]
    c(aux, g, [0])
    torch.cuda.synchronize()
    assert torch.equal(c_tab, a_tab) and torch.equal(c.master, a.master) and c.step == a.step == 3
    for key in ("acc", "m", "v"):
        if getattr(a, key) is not None:
            assert torch.equal(getattr(c, key), getattr(a, key)), key
