"""Torch autograd through the lookup under HIP graph capture is refused with
a clear error, before any library call: a captured autograd training step
crashed torch's graph instantiation (the autograd-free form,
MemoryPool.forward_backward, is what captures).  Capture is mocked on the
CPU and the library loader is replaced by one that fails the test if it is
reached."""

import pytest
import torch

from model_amd import memory as mem
from model_amd.memory import MemoryPool


@pytest.fixture
def mocked_capture(monkeypatch):
    monkeypatch.setattr(mem, "_capturing", lambda: True)

    def no_library():
        raise AssertionError("a library call was reached under the mocked capture")

    monkeypatch.setattr(mem._lib, "lib", no_library)


def _params(requires_grad=True):
    pool = MemoryPool(16, 2, 8, 12, 4, values_dtype=torch.float32)
    p = pool.init(0, device="cpu")["params"]
    p = {k: v.detach().requires_grad_(requires_grad) for k, v in p.items()}
    return pool, p, torch.randn((3, 2, 8), requires_grad=requires_grad)


def test_autograd_lookup_refused_under_capture(mocked_capture):
    pool, p, q = _params()
    with pytest.raises(RuntimeError, match="forward_backward"):
        pool.apply({"params": p}, q)
    with pytest.raises(RuntimeError, match="not supported under HIP graph capture"):
        pool.apply({"params": p}, q, train=True, sparse_grad=True)


def test_backward_refused_under_capture(mocked_capture):
    class Ctx:  # the refusal comes before the saved tensors are touched
        @property
        def saved_tensors(self):
            raise AssertionError("saved tensors read under the mocked capture")

    with pytest.raises(RuntimeError, match="forward_backward"):
        mem._LookupFunction.backward(Ctx(), None, None)


def test_no_grad_lookup_is_not_refused(monkeypatch):
    """Without autograd (no_grad, or nothing requiring grad) the lookup is
    not the refused path: the call goes on to the lookup itself."""
    monkeypatch.setattr(mem, "_capturing", lambda: True)
    reached = []

    def fake_lookup(self, params, queries, **kw):
        reached.append(True)
        return {"out": queries, "aux": {}}

    monkeypatch.setattr(MemoryPool, "lookup", fake_lookup)
    pool, p, q = _params()
    with torch.no_grad():
        pool.apply({"params": p}, q)
    pool2, p2, q2 = _params(requires_grad=False)
    pool2.apply({"params": p2}, q2)
    assert reached == [True, True]
