"""The host tier on the GPU (host_pool.py): device de-duplication
(mpl_unique_slots) against numpy's unique, row copies from device and pinned
host tables (mpl_gather_rows), fetch in both modes, a MemoryPool reading a
host pool against the same table in HBM (bit-exact: the same rows summed in
the same order), and the pool optimizer step (host_pool.py:134-165) in RAM
and file mode against the trainer's optimizers restated in oracle/rows.py."""

import ctypes

import numpy as np
import pytest
import torch

from model_amd import _lib
from model_amd import host_pool as hp
from model_amd import rows as R
from model_amd.memory import MemoryPool
from oracle import rows as orow
from tests.gpu_helpers import make_params, zipf_slots

pytestmark = pytest.mark.gpu


def _unique(slots: np.ndarray, pool_size: int):
    L = _lib.lib()
    P = slots.size
    s = torch.as_tensor(slots.astype(np.int32), device="cuda")
    uniq = torch.full((max(P, 1),), -9, dtype=torch.int32, device="cuda")
    inv = torch.full((max(P, 1),), -9, dtype=torch.int32, device="cuda")
    num = torch.full((1,), -9, dtype=torch.int32, device="cuda")
    wsb = L.mpl_unique_slots_workspace_bytes(P, pool_size)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    _lib.check(L.mpl_unique_slots(_lib.ptr(s), P, pool_size, _lib.ptr(ws), wsb, _lib.ptr(uniq), _lib.ptr(inv),
                                  _lib.ptr(num), _lib.stream_ptr(s.device)), "mpl_unique_slots")
    torch.cuda.synchronize()
    return uniq.cpu().numpy()[:P], inv.cpu().numpy()[:P], int(num.item())


@pytest.mark.parametrize("P,pool_size,kind", [(1, 7, "uniform"), (1000, 300, "uniform"),
                                              (524288, 262144, "zipf"), (70000, 1 << 26, "uniform")])
def test_unique_slots_matches_numpy(gpu_lib, P, pool_size, kind):
    rng = np.random.default_rng(P)
    if kind == "zipf":
        slots = zipf_slots(P // 64, 4, 16, pool_size).reshape(-1)
    else:
        slots = rng.integers(0, pool_size, P)
    uniq, inv, U = _unique(slots, pool_size)
    want, want_inv = np.unique(slots, return_inverse=True)
    assert U == want.size
    np.testing.assert_array_equal(uniq[:U], want)
    np.testing.assert_array_equal(uniq[U:], pool_size)
    np.testing.assert_array_equal(inv, want_inv.reshape(-1))


def test_unique_slots_edge_inputs(gpu_lib):
    assert _unique(np.zeros(0, np.int64), 10)[2] == 0
    # ids outside [0, pool_size) stay inside the [P] buffers (no ordering promised)
    rng = np.random.default_rng(1)
    bad = rng.integers(-5, 5000, 4096)
    uniq, inv, U = _unique(bad, 100)
    assert 0 < U <= bad.size and inv.min() >= 0 and inv.max() < U


def _gather_rows(table_ptr, dtype_code, N, d, idx, count_dev, out):
    _lib.check(_lib.lib().mpl_gather_rows(table_ptr, dtype_code, N, d, _lib.ptr(idx), idx.numel(),
                                          _lib.ptr(count_dev), _lib.ptr(out), _lib.stream_ptr(out.device)),
               "mpl_gather_rows")
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype,d,pinned,offset", [(torch.float16, 256, False, 0), (torch.float16, 256, True, 0),
                                                   (torch.float32, 64, True, 0), (torch.float16, 6, True, 0),
                                                   (torch.float32, 16, False, 1)])
def test_gather_rows(gpu_lib, dtype, d, pinned, offset):
    N, n = 5000, 3000
    code = _lib.MPL_F16 if dtype == torch.float16 else _lib.MPL_F32
    host = torch.randn((N, d)).to(dtype)
    if pinned:
        table = host.pin_memory()
        dptr = ctypes.c_void_p()
        _lib.check(_lib.lib().mpl_host_device_pointer(ctypes.c_void_p(table.data_ptr()), ctypes.byref(dptr)), "ptr")
        tptr = dptr.value
    else:
        table = host.cuda()
        tptr = table.data_ptr()
    idx_np = np.random.default_rng(d).integers(-3, N + 3, n)
    idx = torch.as_tensor(idx_np.astype(np.int32), device="cuda")
    buf = torch.full((n * d + offset + d,), 7.0, dtype=dtype, device="cuda")
    out = buf[offset:offset + n * d].view(n, d)
    limit = torch.tensor([n - 11], dtype=torch.int32, device="cuda")
    _gather_rows(tptr, code, N, d, idx, limit, out)
    want = host.numpy()[np.clip(idx_np, 0, N - 1)]
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got[:n - 11], want[:n - 11])
    assert np.all(got[n - 11:] == 7.0), "rows past count_dev were written"
    assert torch.all(buf[offset + n * d:] == 7.0)


def test_host_device_pointer_rejects_pageable_memory(gpu_lib):
    t = torch.zeros(1024)  # pageable
    out = ctypes.c_void_p()
    rc = _lib.lib().mpl_host_device_pointer(ctypes.c_void_p(t.data_ptr()), ctypes.byref(out))
    assert rc != 0 and b"not pinned" in _lib.lib().mpl_last_error()


@pytest.mark.parametrize("mode,dtype", [("ram", np.float32), ("ram", np.float16), ("memmap", np.float16),
                                        ("direct", np.float16)])
def test_fetch_matches_take(gpu_lib, tmp_path, mode, dtype):
    N, d = 4096, 32
    pool = hp.HostPool(N, d, path=None if mode == "ram" else str(tmp_path / "pool"), dtype=dtype, seed=5,
                       trainable=False, direct_io=mode == "direct")
    slots = torch.as_tensor(zipf_slots(50, 4, 16, N).astype(np.int32), device="cuda")
    got = hp.fetch(pool.name, slots, d)
    torch.cuda.synchronize()
    want = np.asarray(pool.values)[slots.cpu().numpy()].astype(np.float32)
    assert tuple(got.shape) == (50, 4, 16, d) and got.dtype == torch.float32
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    np.testing.assert_array_equal(pool.gather(slots.cpu().numpy().reshape(-1)), want.reshape(-1, d))


@pytest.mark.parametrize("shuffle,dtype", [(False, np.float16), (True, np.float32)])
def test_memory_pool_on_host_equals_hbm_table(gpu_lib, shuffle, dtype):
    """memory.py:182-193 with a host pool: the same out and gradients as the
    table in HBM (the staged rows are the table's rows, summed in order)."""
    n, H, d_key, d, k = 32, 2, 16, 24, 4
    pool_h = hp.HostPool(n * n, d, dtype=dtype, seed=2, trainable=False)
    tdt = torch.float16 if dtype == np.float16 else torch.float32
    dev_pool = MemoryPool(n, H, d_key, d, k, values_dtype=tdt)
    host_pool = MemoryPool(n, H, d_key, d, k, values_dtype=tdt, host_pool=pool_h.name)
    params = make_params(dev_pool, 3)
    params["values"] = torch.from_numpy(np.asarray(pool_h.values)).cuda()
    hparams = {kk: v for kk, v in params.items() if kk != "values"}
    g = torch.Generator().manual_seed(0)
    q = torch.randn((40, H, d_key), generator=g).cuda()
    a = dev_pool.lookup(params, q, shuffle_reads=shuffle)
    b = host_pool.lookup(hparams, q, shuffle_reads=shuffle)
    assert torch.equal(a["slots"], b["slots"])
    assert torch.equal(a["out"], b["out"])
    # gradients through the route (dw reads the staged rows)
    outs = []
    for pool, prm in ((dev_pool, params), (host_pool, hparams)):
        qq = q.clone().requires_grad_(True)
        keys = prm["sub_keys"].detach().clone().requires_grad_(True)
        p2 = dict(prm, sub_keys=keys)
        out, aux = pool.apply({"params": p2}, qq, sparse_grad=True, shuffle_reads=shuffle)
        loss = (out * torch.linspace(-1, 1, d, device="cuda")).sum() + 0.01 * aux["balance_loss"]
        outs.append(torch.autograd.grad(loss, [qq, keys]))
    for x, y in zip(*outs):
        assert torch.equal(x, y)
    # the same gradients from forward_backward (no autograd), on the host pool
    keys = hparams["sub_keys"].detach().clone().requires_grad_(True)
    g_out = torch.linspace(-1, 1, d, device="cuda").expand(40, d).contiguous()
    _, _, (gq, gk, _) = host_pool.forward_backward({"params": dict(hparams, sub_keys=keys)}, q, g_out,
                                                   torch.full((), 0.01, device="cuda"), train=False,
                                                   shuffle_reads=shuffle)
    assert torch.equal(gq, outs[1][0]) and torch.equal(gk, outs[1][1])
    with pytest.raises(ValueError):
        host_pool.apply({"params": hparams}, q.clone().requires_grad_(True), sparse_grad=False)


@pytest.mark.parametrize("mode", ["ram", "file"])
@pytest.mark.parametrize("optimizer,dtype", [("rowwise_adagrad", np.float32), ("rowwise_adagrad", np.float16),
                                             ("adam", np.float32), ("adam", np.float16)])
def test_update_matches_trainer_optimizer(gpu_lib, tmp_path, mode, optimizer, dtype):
    """Three steps on overlapping row sets with padding entries and a clip
    factor, against oracle/rows.py (train.py:412-426; the pool's step s is
    the trainer's 0-based step s - 1).  RAM mode updates the pinned rows in
    place; file mode stages them from the .npy files and writes them back."""
    N, d = 3000, 64
    pool = hp.HostPool(N, d, path=None if mode == "ram" else str(tmp_path / "pool"), dtype=dtype, seed=7,
                       optimizer=optimizer)
    vals = np.asarray(pool.values).copy()
    acc = np.zeros(N, np.float32)
    m = np.zeros((N, d), np.float32)
    v = np.zeros((N, d), np.float32)
    rng = np.random.default_rng(1)
    for step in (1, 2, 3):
        uniq = np.concatenate([np.sort(rng.choice(N, 900, replace=False)), [N] * 5]).astype(np.int32)
        rng.shuffle(uniq)
        grads = rng.standard_normal((uniq.size, d)).astype(np.float32)
        lr = 0.01 * step
        if step == 2:  # numpy inputs, as the reference's trainer hands them over
            pool.update(uniq, grads * np.float32(0.5), step, lr)
        else:
            pool.update(torch.as_tensor(uniq, device="cuda"), torch.as_tensor(grads, device="cuda"), step, lr,
                        grad_scale=torch.tensor([0.5], device="cuda"))
        if optimizer == "rowwise_adagrad":
            orow.rowwise_adagrad(vals, acc, uniq, grads * np.float32(0.5), lr)
        else:
            orow.lazy_adam(vals, m, v, uniq, grads * np.float32(0.5), lr, step - 1)
    torch.cuda.synchronize()
    tol = dict(rtol=2e-6, atol=1e-6) if dtype == np.float32 else dict(rtol=2e-3, atol=1e-4)
    np.testing.assert_allclose(np.asarray(pool.values).astype(np.float64), vals.astype(np.float64), **tol)
    if optimizer == "rowwise_adagrad":
        np.testing.assert_allclose(np.asarray(pool.acc), acc, rtol=2e-6)
    else:
        np.testing.assert_allclose(np.asarray(pool.m), m, rtol=2e-6, atol=1e-6 * np.abs(m).max())
        np.testing.assert_allclose(np.asarray(pool.v), v, rtol=2e-6, atol=1e-6 * np.abs(v).max())
    if mode == "file":
        # the rows written back are in the files, and a snapshot of them reloads
        np.testing.assert_array_equal(np.load(str(tmp_path / "pool" / "values.npy")), np.asarray(pool.values))
        pool.save(str(tmp_path / "snap"))
        other = hp.HostPool(N, d, path=str(tmp_path / "other"), dtype=dtype, seed=8, optimizer=optimizer)
        other.load(str(tmp_path / "snap"))
        for key in ("values", "acc", "m", "v"):
            if getattr(pool, key) is not None:
                np.testing.assert_array_equal(np.asarray(getattr(other, key)), np.asarray(getattr(pool, key)))
        with pytest.raises(ValueError):
            pool.update(np.array([3, 3], np.int32), np.ones((2, d), np.float32), 4, 0.01)


def test_sparse_row_update_on_host_pool(gpu_lib):
    """train.py:250-258: the trainer's merged, clipped rows applied to a host
    pool equal the same update of the table in HBM (no master copy)."""
    N, d, M, H, k = 4096, 32, 64, 2, 4
    pool = hp.HostPool(N, d, dtype=np.float32, seed=1, optimizer="rowwise_adagrad")
    table = torch.from_numpy(np.asarray(pool.values).copy()).cuda()
    up_h = R.SparseRowUpdate(pool, optimizer="rowwise_adagrad", lr=1e-2, grad_clip=0.5)
    up_d = R.SparseRowUpdate(table, optimizer="rowwise_adagrad", lr=1e-2, grad_clip=0.5, master=False)
    rng = np.random.default_rng(3)
    for _ in range(2):
        slots = torch.as_tensor(rng.integers(0, N, (M, H, k)).astype(np.int32), device="cuda")
        w = torch.softmax(torch.as_tensor(rng.standard_normal((M, H, k)).astype(np.float32), device="cuda"), -1)
        g = torch.as_tensor(rng.standard_normal((M, d)).astype(np.float32), device="cuda")
        aux = {"slots": [slots], "weights": [w]}
        up_h(aux, {0: g}, [0])
        up_d(aux, {0: g}, [0])
    torch.cuda.synchronize()
    np.testing.assert_allclose(np.asarray(pool.values), table.cpu().numpy(), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(np.asarray(pool.acc), up_d.acc.cpu().numpy(), rtol=1e-6)
