"""mpl_decode_attention (the decode step of the backbone's attention,
model.py:88-94 in decode mode) against the oracle's causal attention
(oracle/backbone.py:attention, pinned in tests/test_oracle_backbone.py): a
sequence fed one position per launch must give, at every position, the
oracle's attention output of that row, and leave the keys and values of the
positions seen so far in the caches.  Cache entries after the current
position hold large garbage, so a kernel that read them would fail."""

import numpy as np
import pytest
import torch

from model_amd.model import decode_attention
from oracle import backbone as ob

pytestmark = pytest.mark.gpu


def _case(B, H, hd, T, L, seed):
    rng = np.random.default_rng(seed)
    d = H * hd
    p = {nm: {"kernel": rng.standard_normal((d, H, hd)) * d ** -0.5, "bias": rng.standard_normal((H, hd)) * 0.1}
         for nm in ("query", "key", "value")}
    # identity output projection: the oracle then returns the heads' outputs
    p["out"] = {"kernel": np.eye(d).reshape(H, hd, d), "bias": np.zeros(d)}
    h = rng.standard_normal((B, T, d))
    want = ob.attention(p, h)  # [B, T, d]
    w = np.concatenate([p[nm]["kernel"].reshape(d, d) for nm in ("query", "key", "value")], 1)
    b = np.concatenate([p[nm]["bias"].reshape(d) for nm in ("query", "key", "value")])
    qkv = np.einsum("btd,de->bte", h, w) + b  # [B, T, 3 * d]: query, key, value
    return qkv, want


@pytest.mark.parametrize("B,H,hd,T,L", [(3, 4, 64, 40, 48), (2, 2, 16, 12, 16), (2, 2, 128, 9, 9),
                                        (2, 2, 64, 300, 320), (1, 1, 256, 5, 8)])
def test_decode_steps_match_oracle_attention(gpu_lib, B, H, hd, T, L):
    qkv, want = _case(B, H, hd, T, L, seed=B * 1000 + hd + T)
    g = torch.Generator(device="cuda").manual_seed(T)
    cache = {"kt": torch.randn((B, H, hd, L), generator=g, device="cuda") * 1e3,
             "v": torch.randn((B, H, L, hd), generator=g, device="cuda") * 1e3}
    garbage_kt, garbage_v = cache["kt"].clone(), cache["v"].clone()
    pos = torch.zeros(1, dtype=torch.int64, device="cuda")
    x = torch.as_tensor(qkv, dtype=torch.float32, device="cuda")
    got = []
    for t in range(T):
        pos.fill_(t)
        got.append(decode_attention(x[:, t].contiguous(), pos, cache, H, hd ** -0.5))
    got = torch.stack(got, 1).double().cpu().numpy()
    scale = np.abs(want).max()
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5 * scale)
    # the caches hold the keys and values of positions < T, untouched garbage after
    k = qkv[..., H * hd:2 * H * hd].reshape(B, T, H, hd)
    v = qkv[..., 2 * H * hd:].reshape(B, T, H, hd)
    kt = cache["kt"].cpu().numpy()
    vc = cache["v"].cpu().numpy()
    np.testing.assert_array_equal(kt[..., :T], k.astype(np.float32).transpose(0, 2, 3, 1))
    np.testing.assert_array_equal(vc[:, :, :T], v.astype(np.float32).transpose(0, 2, 1, 3))
    assert torch.equal(cache["kt"][..., T:], garbage_kt[..., T:])
    assert torch.equal(cache["v"][:, :, T:], garbage_v[:, :, T:])


@pytest.mark.parametrize("bad", [-1, 16])
def test_position_outside_cache_writes_nothing_and_returns_nan(gpu_lib, bad):
    B, H, hd, L = 2, 2, 32, 16
    cache = {"kt": torch.ones((B, H, hd, L), device="cuda"), "v": torch.ones((B, H, L, hd), device="cuda")}
    x = torch.randn((B, 3 * H * hd), device="cuda")
    out = decode_attention(x, torch.tensor([bad], device="cuda"), cache, H, hd ** -0.5)
    assert torch.isnan(out).all()
    assert bool((cache["kt"] == 1).all()) and bool((cache["v"] == 1).all())


def test_shape_errors_are_raised_on_the_host(gpu_lib):
    cache = {"kt": torch.zeros((2, 2, 24, 8), device="cuda"), "v": torch.zeros((2, 2, 8, 24), device="cuda")}
    pos = torch.zeros(1, dtype=torch.int64, device="cuda")
    with pytest.raises(Exception, match="head_dim=24"):  # 24 does not divide 256
        decode_attention(torch.zeros((2, 144), device="cuda"), pos, cache, 2, 0.2)
    cache = {"kt": torch.zeros((2, 2, 32, 8), device="cuda"), "v": torch.zeros((2, 2, 8, 32), device="cuda")}
    with pytest.raises(ValueError):
        decode_attention(torch.zeros((2, 100), device="cuda"), pos, cache, 2, 0.2)
    with pytest.raises(ValueError):
        decode_attention(torch.zeros((2, 192), device="cuda"), pos.cpu(), cache, 2, 0.2)
