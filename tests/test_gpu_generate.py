"""The backbone mirror and token-by-token generation on the GPU
(model_amd/model.py, model_amd/generate.py) with the memory reads in
libmpl.so: KV-cache decoding reproduces the full forward
(tests/test_memory_pool.py:486-502 of the reference, atol 1e-4), the
HIP-graph decode step equals the eager one, and a parameter tree survives a
Flax-format checkpoint round trip."""

import io

import numpy as np
import pytest
import torch

from model_amd import checkpoint as ck
from model_amd.generate import Generator
from model_amd.model import MemoryPoolLM, ModelConfig

pytestmark = pytest.mark.gpu


def _cfg(dt):
    return ModelConfig(vocab_size=50, max_len=16, d_model=32, n_heads=2, n_sub_keys=8, pool_heads=2, d_key=16,
                       d_value=32, top_k=4, memory_layers=(0, 1), values_dtype=dt)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
@pytest.mark.parametrize("graph", [True, False])
def test_kv_cache_decoding_matches_full_forward(gpu_lib, dt, graph):
    cfg = _cfg(dt)
    toks = torch.tensor(np.random.default_rng(0).integers(0, 50, (2, 12)), device="cuda")
    model = MemoryPoolLM(cfg)
    params = model.init(1)
    with torch.no_grad():
        full, _ = model.apply(params, toks)
    res = Generator(cfg, params, batch_size=2, graph=graph).generate(toks.cpu().numpy(), n_new=3)
    np.testing.assert_allclose(res["logits"][:, :12].cpu().numpy(), full.cpu().numpy(), atol=1e-4)
    assert res["tokens"].shape == (2, 3)


def test_graph_step_equals_eager_step(gpu_lib):
    cfg = ModelConfig(vocab_size=300, max_len=40, d_model=64, n_heads=4, n_layers=3, ffn_mult=2, n_sub_keys=64,
                      pool_heads=4, d_key=64, d_value=64, top_k=8, memory_layers=(1, 2))
    params = MemoryPoolLM(cfg).init(3)
    prompt = np.random.default_rng(1).integers(0, 300, (5, 10))
    a = Generator(cfg, params, batch_size=5, graph=True).generate(prompt, n_new=20)
    b = Generator(cfg, params, batch_size=5, graph=False).generate(prompt, n_new=20)
    assert torch.equal(a["tokens"], b["tokens"])
    assert torch.equal(a["logits"], b["logits"])
    # a second generation on the same graph starts from a clean cache
    c = Generator(cfg, params, batch_size=5, graph=True)
    c.generate(prompt[:, ::-1].copy(), n_new=5)
    assert torch.equal(c.generate(prompt, n_new=20)["tokens"], a["tokens"])


def test_checkpoint_round_trip_drives_the_backbone(gpu_lib):
    cfg = _cfg(torch.float16)
    model = MemoryPoolLM(cfg)
    params = model.init(4)
    buf = io.BytesIO()
    ck.save_params(buf, params["params"])  # values written as fp32, as the reference stores them
    back = ck.load_params(buf.getvalue(), device="cuda", values_dtype=torch.float16)
    toks = torch.tensor(np.random.default_rng(2).integers(0, 50, (3, 9)), device="cuda")
    with torch.no_grad():
        a, _ = model.apply(params, toks)
        b, _ = model.apply({"params": back}, toks)
    assert torch.equal(a, b)


def test_generator_follows_pool_parameters_changed_in_place(gpu_lib):
    """The captured decode step bakes in the packed sub-keys and the clamped
    temperature; after an in-place update of sub_keys or log_temperature (an
    optimizer step) the next generate() must use the new values, as an eager
    step does."""
    cfg = ModelConfig(vocab_size=300, max_len=40, d_model=64, n_heads=4, n_layers=2, ffn_mult=2, n_sub_keys=64,
                      pool_heads=4, d_key=64, d_value=64, top_k=8, memory_layers=(0, 1))
    params = MemoryPoolLM(cfg).init(5)
    prompt = np.random.default_rng(3).integers(0, 300, (4, 10))
    gen = Generator(cfg, params, batch_size=4, graph=True)
    before = gen.generate(prompt, n_new=8)
    pool = params["params"]["pool"]
    with torch.no_grad():
        pool["sub_keys"].mul_(-1.0).add_(0.3)  # in place: same storage, new version
        pool["log_temperature"].add_(1.0)
    after = gen.generate(prompt, n_new=8)
    eager = Generator(cfg, params, batch_size=4, graph=False).generate(prompt, n_new=8)
    assert torch.equal(after["logits"], eager["logits"])
    assert not torch.equal(after["logits"], before["logits"])


def test_generator_follows_attention_weights_changed_in_place(gpu_lib):
    """The GPU decode step reads the query/key/value weights through one
    fused copy made before capture; after an in-place update of one of them
    the next generate() must re-capture and use the new weights."""
    cfg = ModelConfig(vocab_size=300, max_len=40, d_model=64, n_heads=4, n_layers=2, ffn_mult=2, n_sub_keys=64,
                      pool_heads=4, d_key=64, d_value=64, top_k=8, memory_layers=(1,))
    params = MemoryPoolLM(cfg).init(6)
    prompt = np.random.default_rng(4).integers(0, 300, (3, 10))
    gen = Generator(cfg, params, batch_size=3, graph=True)
    before = gen.generate(prompt, n_new=6)
    with torch.no_grad():
        params["params"]["attn_0"]["query"]["kernel"].mul_(-2.0)
        params["params"]["attn_1"]["value"]["bias"].add_(0.5)
    after = gen.generate(prompt, n_new=6)
    eager = Generator(cfg, params, batch_size=3, graph=False).generate(prompt, n_new=6)
    assert torch.equal(after["logits"], eager["logits"])
    assert not torch.equal(after["logits"], before["logits"])


@pytest.mark.parametrize("V", [1000, 999, 16384])
def test_next_token_kernel_matches_torch(gpu_lib, V):
    """mpl_decode_next_token (the greedy graph's token step, generate.py:44-61):
    the prompt's next token while it lasts, then torch.argmax of the logits
    (first maximal index, ties and NaN included, all -inf gives 0), the
    generated tokens written in order, and the position advanced by one per
    call with the workgroup count left at 0."""
    from model_amd import _lib

    B, Lmax, P = 7, 12, 3
    g = torch.Generator(device="cuda").manual_seed(9)
    prompt = torch.randint(0, V, (B, Lmax), generator=g, device="cuda")
    plen = torch.full((1,), P, dtype=torch.int64, device="cuda")
    pos = torch.zeros(1, dtype=torch.int64, device="cuda")
    tok = torch.zeros(B, dtype=torch.int64, device="cuda")
    out = torch.full((B, Lmax), -1, dtype=torch.int64, device="cuda")
    done = torch.zeros(1, dtype=torch.int32, device="cuda")
    want_out = []
    for step in range(8):
        logits = torch.randn((B, V), generator=g, device="cuda")
        logits[0, 17] = logits[0, V - 90] = 50.0  # a tie: the first index wins
        logits[1, :] = 3.0  # all equal: index 0
        logits[2, 555] = float("nan")  # NaN counts as the maximum
        logits[3, :] = float("-inf")  # nothing above -inf: index 0
        logits[4, V - 1] = 99.0  # the last element
        _lib.check(_lib.lib().mpl_decode_next_token(
            _lib.ptr(logits), B, V, _lib.ptr(prompt), Lmax, _lib.ptr(plen), _lib.ptr(pos), _lib.ptr(tok),
            _lib.ptr(out), Lmax, Lmax, _lib.ptr(done), _lib.stream_ptr(logits.device)), "next_token")
        want = prompt[:, step + 1] if step + 1 < P else torch.argmax(logits, -1)
        if step + 1 >= P:
            want_out.append(want)
        assert torch.equal(tok, want), step
        assert int(pos.item()) == step + 1 and int(done.item()) == 0
    assert torch.equal(out[:, :len(want_out)], torch.stack(want_out, 1))
    assert bool((out[:, len(want_out):] == -1).all())
    assert tok[0].item() in (17,) and tok[1].item() == 0 and tok[2].item() == 555 and tok[3].item() == 0


@pytest.mark.parametrize("B,V,P,d", [(64, 16384, 512, 256), (3, 17, 9, 8)])
def test_decode_embed_matches_torch(gpu_lib, B, V, P, d):
    """mpl_decode_embed (the decode step's input rows in one launch) equals
    emb[tokens] + pos_emb[position] bit for bit, and an out-of-range token
    or position gives NaN rows rather than a read outside the tables."""
    from model_amd.model import decode_embed

    g = torch.Generator(device="cuda").manual_seed(B + V)
    emb = torch.randn((V, d), generator=g, device="cuda")
    pos_emb = torch.randn((P, d), generator=g, device="cuda")
    tok = torch.randint(0, V, (B,), generator=g, device="cuda")
    for p in (0, P - 1, P // 2):
        pos = torch.tensor([p], dtype=torch.int64, device="cuda")
        assert torch.equal(decode_embed(emb, pos_emb, tok, pos), emb[tok] + pos_emb[pos])
    bad = tok.clone()
    bad[0] = V
    out = decode_embed(emb, pos_emb, bad, torch.tensor([1], dtype=torch.int64, device="cuda"))
    assert torch.isnan(out[0]).all() and torch.isfinite(out[1:]).all()
    out = decode_embed(emb, pos_emb, tok, torch.tensor([P], dtype=torch.int64, device="cuda"))
    assert torch.isnan(out).all()
