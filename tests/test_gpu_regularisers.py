"""The training-side regularisers of memory.py:230-281 on the GPU
(include/mpl.h mpl_key_diversity, mpl_l2_normalize_bwd, mpl_revive_keys)
against the oracle (oracle/lookup.py key_diversity_loss / revive_dead_keys,
oracle/backward.py key_diversity_backward; fp64).

key_diversity_loss runs on fp16 or fp32 MFMA Gram tiles.  fp16: the loss is
checked to 2e-3 relative and its gradient to 1e-2 of the largest magnitude
(the fp16 path tolerance); fp32: 1e-5 for both.  revive_dead_keys is fp32
elementwise work: 1e-6."""

import numpy as np
import pytest
import torch

from model_amd import memory as mem
from oracle import backward as ob
from oracle import lookup as ol

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,n,half,seed", [
    (4, 512, 128, 1),   # the text-study codebooks
    (2, 100, 32, 2),    # n not a multiple of 32, query range split
    (1, 64, 8, 3),      # half = 8
    (1, 2, 16, 4),      # two keys
    (2, 1000, 64, 5),
])
def test_key_diversity_loss_and_gradient(gpu_lib, H, n, half, seed):
    rng = np.random.default_rng(seed)
    raw = (rng.standard_normal((H, 2, n, half)) * 0.7).astype(np.float32)
    t = torch.tensor(raw, device="cuda", requires_grad=True)
    loss = mem.key_diversity_loss(t)
    (g,) = torch.autograd.grad(3.0 * loss, [t])
    want = ol.key_diversity_loss(raw)
    np.testing.assert_allclose(float(loss), want, rtol=2e-3)
    ref = 3.0 * ob.key_diversity_backward(raw)
    err = np.abs(g.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= 1e-2, f"d sub_keys: max error {err:.3g} of the largest magnitude"


@pytest.mark.parametrize("H,n,half,seed", [
    (4, 128, 128, 11),  # the fact-task codebooks
    (2, 100, 10, 12),   # half = 10: only the fp32 tiles take it
    (1, 300, 3, 13),    # half = 3, query range split
    (1, 2, 64, 14),     # two keys
])
def test_key_diversity_fp32(gpu_lib, H, n, half, seed):
    rng = np.random.default_rng(seed)
    raw = (rng.standard_normal((H, 2, n, half)) * 0.7).astype(np.float32)
    t = torch.tensor(raw, device="cuda", requires_grad=True)
    loss = mem.key_diversity_loss(t, torch.float32)
    (g,) = torch.autograd.grad(3.0 * loss, [t])
    np.testing.assert_allclose(float(loss), ol.key_diversity_loss(raw), rtol=1e-5)
    ref = 3.0 * ob.key_diversity_backward(raw)
    err = np.abs(g.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= 1e-5, f"d sub_keys: max error {err:.3g} of the largest magnitude"
    if half % 8:
        with pytest.raises(ValueError):
            mem.key_diversity_loss(t, torch.float16)


def test_key_diversity_collapsed_codebook_is_one(gpu_lib):
    """memory.py:230-240 closed form: every off-diagonal cosine of a codebook
    of one repeated direction is 1, so the loss is 1 and the gradient along
    the keys' own direction vanishes after the normalisation backward."""
    d = torch.randn(64, device="cuda")
    keys = d.expand(2, 2, 40, 64).contiguous().requires_grad_(True)
    loss = mem.key_diversity_loss(keys)
    np.testing.assert_allclose(float(loss), 1.0, rtol=2e-3)
    (g,) = torch.autograd.grad(loss, [keys])
    assert float(g.abs().max()) <= 1e-2 * float(d.abs().max()) / float(d.norm())


@pytest.mark.parametrize("score_dtype", [torch.float16, torch.float32])
def test_key_diversity_value_and_grad_equals_autograd(gpu_lib, score_dtype):
    """key_diversity_value_and_grad (no torch autograd, for captured training
    steps) runs the same kernels as key_diversity_loss + autograd: equal bit
    for bit, loss and gradient, for an upstream gradient of 0.01."""
    raw = torch.randn((2, 2, 256, 64), device="cuda").requires_grad_(True)
    g = torch.full((), 0.01, device="cuda")
    loss = mem.key_diversity_loss(raw, score_dtype)
    (ga,) = torch.autograd.grad(loss, [raw], grad_outputs=[g])
    lm, gm = mem.key_diversity_value_and_grad(raw, g, score_dtype)
    assert torch.equal(loss.detach(), lm)
    assert gm.dtype == ga.dtype and torch.equal(ga, gm)


def test_key_diversity_without_grad(gpu_lib):
    raw = torch.randn((1, 2, 96, 32), device="cuda")
    with torch.no_grad():
        a = mem.key_diversity_loss(raw)
    np.testing.assert_allclose(float(a), ol.key_diversity_loss(raw.cpu().numpy()), rtol=2e-3)


@pytest.mark.parametrize("H,n,d,M", [(2, 64, 16, 300), (4, 512, 128, 37), (1, 5, 3, 2)])
def test_revive_dead_keys_matches_oracle(gpu_lib, H, n, d, M):
    rng = np.random.default_rng(n)
    keys = rng.standard_normal((H, 2, n, d)).astype(np.float32)
    usage = rng.random((H, 2, n)).astype(np.float32)
    usage[..., ::3] *= 1e-3  # a third of the keys far below threshold / n
    usage /= usage.sum(-1, keepdims=True)
    q = rng.standard_normal((M, H, 2, d)).astype(np.float32)
    q /= np.sqrt((q * q).sum(-1, keepdims=True))
    pick = rng.integers(0, M, (H, 2, n)).astype(np.int32)
    normal = rng.standard_normal((H, 2, n, d)).astype(np.float32)
    dev = "cuda"
    nk, nu, dead = mem.revive_dead_keys(torch.tensor(keys, device=dev), torch.tensor(usage, device=dev),
                                        torch.tensor(q, device=dev), None, 0.1, 0.05,
                                        pick=torch.tensor(pick, device=dev), normal=torch.tensor(normal, device=dev))
    wk, wu, wd = ol.revive_dead_keys(keys, usage, q, pick, normal, 0.1, 0.05)
    np.testing.assert_array_equal(dead.cpu().numpy(), wd)
    assert wd.any() and not wd.all()
    np.testing.assert_allclose(nk.cpu().numpy(), wk, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(nu.cpu().numpy(), wu, rtol=1e-6)
    np.testing.assert_allclose(nu.sum(-1).cpu().numpy(), 1.0, rtol=1e-6)


def test_revive_draws_from_generator(gpu_lib):
    """The rng path: revived keys are unit-norm; live keys are unchanged."""
    keys = torch.randn((2, 2, 32, 16), device="cuda")
    usage = torch.full((2, 2, 32), 1.0 / 32, device="cuda")
    usage[0, 1, 5] = 0.0
    q = torch.nn.functional.normalize(torch.randn((50, 2, 2, 16), device="cuda"), dim=-1)
    nk, nu, dead = mem.revive_dead_keys(keys, usage, q, 7, 0.1)
    assert dead.sum().item() == 1 and bool(dead[0, 1, 5])
    np.testing.assert_allclose(float(nk[0, 1, 5].norm()), 1.0, rtol=1e-5)
    live = ~dead
    assert torch.equal(nk[live], keys[live])
