"""The lookup captured in a HIP graph (as bench.py and serving loops run it):
every replay, with eager work and synchronisations in between, must equal the
eager result bit for bit."""

import pytest
import torch

from model_amd.memory import MemoryPool
from tests.gpu_helpers import make_params

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M", [8192, 16])
def test_graph_replays_match_eager(gpu_lib, M):
    pool = MemoryPool(512, 4, 256, 256, 16, values_dtype=torch.float16)
    params = make_params(pool, 21, key_std=128 ** -0.5, value_std=0.02)
    q = torch.randn((M, 4, 256), generator=torch.Generator(device="cuda").manual_seed(22), device="cuda")
    eager = pool.lookup(params, q)  # also warms the key/temperature caches
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pool.lookup(params, q)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cap = pool.lookup(params, q)
    for i in range(3):
        cap["out"].zero_()
        cap["slots"].zero_()
        g.replay()
        torch.cuda.synchronize()
        for key in ("out", "slots", "weights", "sub_idx", "sub_scores", "flat_idx"):
            assert torch.equal(cap[key], eager[key]), (i, key)
        # unrelated eager work between replays
        torch.randn(1000, device="cuda").sum().item()
