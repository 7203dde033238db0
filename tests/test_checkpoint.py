"""Flax msgpack parameter checkpoints (train.py:559-583, 662-665) read and
written by model_amd/checkpoint.py, on the CPU.

tests/golden/flax_params_small.msgpack is encoded from raw msgpack
primitives the way flax.serialization.to_bytes encodes a parameter tree
(tests/golden/make_flax_params_fixture.py): array leaves as ext type 1,
numpy scalars as ext type 3, and the value table as a chunked array."""

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
