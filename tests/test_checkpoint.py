"""Flax msgpack parameter checkpoints (train.py:559-583, 662-665) read and
written by model_amd/checkpoint.py, on the CPU.

tests/golden/flax_params_small.msgpack is encoded from raw msgpack
primitives the way flax.serialization.to_bytes encodes a parameter tree
(tests/golden/make_flax_params_fixture.py): array leaves as ext type 1,
numpy scalars as ext type 3 (read; the writer, like the reference's
to_bytes(device_get(state)), emits only ndarrays), and the value table as a
chunked array."""

import io
import os

import numpy as np
import pytest
import torch

from model_amd import checkpoint as ck
from tests.golden.make_flax_params_fixture import OUT, arrays


def test_reads_the_flax_encoding():
    want = arrays()
    tree = ck.load_params(OUT, device="cpu", values_dtype=None)
    np.testing.assert_array_equal(tree["embed"]["embedding"].numpy(), want["embed"]["embedding"])
    np.testing.assert_array_equal(tree["pos_embed"].numpy(), want["pos_embed"])
    np.testing.assert_array_equal(tree["router_1"]["kernel"].numpy(), want["router_1"]["kernel"])
    np.testing.assert_array_equal(tree["counts"].numpy(), want["counts"])
    assert tree["counts"].dtype == torch.int32
    pool = ck.pool_params(tree)
    np.testing.assert_array_equal(pool["sub_keys"].numpy(), want["pool"]["sub_keys"])
    np.testing.assert_array_equal(pool["values"].numpy(), want["pool"]["values"])  # the chunked leaf
    assert pool["log_temperature"].shape == () and float(pool["log_temperature"]) == pytest.approx(np.log(10.0))
    assert float(tree["scale"]) == 0.5


def test_values_are_cast_on_load():
    """fp32 values of the reference (memory.py:104-109) become the fp16 table
    this library gathers from; other leaves keep their dtype."""
    tree = ck.load_params(OUT, device="cpu")
    pool = ck.pool_params(tree)
    assert pool["values"].dtype == torch.float16 and pool["sub_keys"].dtype == torch.float32
    np.testing.assert_array_equal(pool["values"].numpy(), arrays()["pool"]["values"].astype(np.float16))


def test_round_trip_with_chunking(monkeypatch, tmp_path):
    monkeypatch.setattr(ck, "MAX_CHUNK_SIZE", 64)  # every leaf above 64 bytes is chunked
    rng = np.random.default_rng(1)
    tree = {"pool": {"values": torch.tensor(rng.standard_normal((37, 5)), dtype=torch.float16),
                     "sub_keys": torch.tensor(rng.standard_normal((1, 2, 3, 4)), dtype=torch.float32),
                     "log_temperature": torch.tensor(2.3)},
            "ln_final": {"scale": torch.ones(5), "bias": torch.zeros(5)}}
    path = str(tmp_path / "p.msgpack")
    ck.save_params(path, tree)  # values written as fp32, as the reference stores them
    back = ck.load_params(path, device="cpu", values_dtype=None)
    assert back["pool"]["values"].dtype == torch.float32
    torch.testing.assert_close(back["pool"]["values"], tree["pool"]["values"].float(), rtol=0, atol=0)
    torch.testing.assert_close(back["pool"]["sub_keys"], tree["pool"]["sub_keys"], rtol=0, atol=0)
    torch.testing.assert_close(back["ln_final"]["scale"], tree["ln_final"]["scale"], rtol=0, atol=0)
    buf = io.BytesIO()
    ck.save_params(buf, tree, values_dtype=None)
    again = ck.load_params(buf.getvalue(), device="cpu", values_dtype=None)
    assert again["pool"]["values"].dtype == torch.float16
    torch.testing.assert_close(again["pool"]["values"], tree["pool"]["values"], rtol=0, atol=0)


def test_fixture_is_current():
    """The committed fixture equals what its generator writes."""
    import tempfile

    from tests.golden import make_flax_params_fixture as mk

    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "f.msgpack")
        old = mk.OUT
        mk.OUT = path
        try:
            mk.main()
        finally:
            mk.OUT = old
        assert open(path, "rb").read() == open(OUT, "rb").read()


# ------------------------------------------------------------ train states
from tests.golden import make_flax_train_state_fixture as ts_fix  # noqa: E402


def test_train_state_fixtures_are_the_committed_bytes(tmp_path):
    for opt, path in ts_fix.OUT.items():
        with open(path, "rb") as f:
            committed = f.read()
        ts_fix.OUT[opt] = str(tmp_path / os.path.basename(path))
        try:
            ts_fix.main()
            with open(ts_fix.OUT[opt], "rb") as f:
                assert f.read() == committed
        finally:
            ts_fix.OUT[opt] = path


@pytest.mark.parametrize("opt", ["adagrad", "adam"])
def test_reads_train_state_and_resumes_row_update(opt):
    from model_amd import rows as R

    want = ts_fix.arrays(opt)
    st = ck.load_train_state(ts_fix.OUT[opt], device="cpu")
    assert st["step"] == ts_fix.STEP
    np.testing.assert_array_equal(st["params"]["pool"]["values"].numpy(), want["params"]["pool"]["values"])
    assert st["params"]["pool"]["values"].dtype == torch.float32  # kept fp32: the master copy
    np.testing.assert_array_equal(st["subkey_usage"].numpy(), want["subkey_usage"])
    adamw = st["opt_state"]["0"]
    assert int(adamw["0"]["count"]) == ts_fix.STEP and int(adamw["2"]["count"]) == ts_fix.STEP
    assert adamw["1"] == {"inner_state": {}} and st["opt_state"]["1"] == {}
    assert "values" not in adamw["0"]["mu"]["pool"]
    N, d = want["params"]["pool"]["values"].shape
    table = torch.zeros((N, d), dtype=torch.float16)
    upd = R.SparseRowUpdate(table, optimizer="rowwise_adagrad" if opt == "adagrad" else "adam")
    upd.resume(st)
    assert upd.step == ts_fix.STEP
    np.testing.assert_array_equal(upd.master.numpy(), want["params"]["pool"]["values"])
    np.testing.assert_array_equal(table.numpy(), want["params"]["pool"]["values"].astype(np.float16))
    if opt == "adagrad":
        np.testing.assert_array_equal(upd.acc.numpy(), want["pool_v"])
    else:
        np.testing.assert_array_equal(upd.m.numpy(), want["pool_m"])
        np.testing.assert_array_equal(upd.v.numpy(), want["pool_v"])
    # the wrong optimizer's layout is refused
    other = R.SparseRowUpdate(torch.zeros((N, d)), optimizer="adam" if opt == "adagrad" else "rowwise_adagrad")
    with pytest.raises(ValueError):
        other.resume(st)


def test_train_state_writer_round_trip():
    from model_amd import rows as R

    st = ck.load_train_state(ts_fix.OUT["adam"], device="cpu")
    N, d = st["params"]["pool"]["values"].shape
    upd = R.SparseRowUpdate(torch.zeros((N, d), dtype=torch.float16), optimizer="adam")
    upd.resume(st)
    pool = upd.train_state_pool()
    params = dict(st["params"])
    params["pool"] = dict(params["pool"], values=pool["values"])
    buf = io.BytesIO()
    ck.save_train_state(buf, step=pool["step"], params=params, opt_state=st["opt_state"],
                        subkey_usage=st["subkey_usage"], slot_usage=st["slot_usage"], pool_m=pool["pool_m"],
                        pool_v=pool["pool_v"])
    back = ck.load_train_state(buf.getvalue(), device="cpu")
    assert back["step"] == st["step"]
    for k in ("pool_m", "pool_v", "subkey_usage", "slot_usage"):
        assert torch.equal(back[k], st[k]), k
    assert torch.equal(back["params"]["pool"]["values"], st["params"]["pool"]["values"])
    mu = ("0", "0", "mu", "router_1", "kernel")
    a, b = back["opt_state"], st["opt_state"]
    for k in mu:
        a, b = a[k], b[k]
    assert torch.equal(a, b)
    # every leaf is written as Flax writes device_get'd arrays: ext type 1, the 0-d step too
    import msgpack

    raw = msgpack.unpackb(buf.getvalue(), raw=False, strict_map_key=False)
    assert isinstance(raw["step"], msgpack.ExtType) and raw["step"].code == 1
    assert raw["opt_state"]["0"]["0"]["count"].code == 1
