import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def gpu_lib():
    """The built C-ABI library, loaded on a machine with a GPU.  Fails (does not skip)
    when the library is missing: the product path has no fallback."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test collected on a machine without a GPU")
    from model_amd import _lib

    return _lib.lib()


@pytest.fixture(autouse=True)
def _release_gpu_memory(request):
    """After each GPU test, collect reference cycles and return cached blocks,
    so that a test holding a 100+ GB table (the 268M-slot pool) never leaves
    it to the next one."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import gc

    import torch

    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
