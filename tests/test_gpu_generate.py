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


@pytest.mark.parametrize("mode", ["ram", "file"])
@pytest.mark.parametrize("graph", [True, False])
def test_kv_cache_decoding_matches_full_forward_host_pool(gpu_lib, tmp_path, mode, graph):
    """tests/test_memory_pool.py:486-502 [host]: an fp16 HostPool (generate.py
    over host_pool.py:206-220): decode logits equal the full forward at atol
    1e-4, and tokens and logits equal a generator over the same table in HBM.
    RAM mode captures the decode step (the GPU reads the pinned table); file
    mode runs it eagerly whatever ``graph`` says."""
    from model_amd import host_pool as hp

    base = _cfg(torch.float16)
    pool = hp.HostPool(base.pool_size, base.d_value, path=None if mode == "ram" else str(tmp_path / "pool"),
                       trainable=False, dtype=np.float16, seed=4)
    cfg = ModelConfig(**{**base.__dict__, "host_pool": pool.name})
    toks = torch.tensor(np.random.default_rng(0).integers(0, 50, (2, 12)), device="cuda")
    model = MemoryPoolLM(cfg)
    params = model.init(1)
    assert "values" not in params["params"]["pool"]
    with torch.no_grad():
        full, _ = model.apply(params, toks)
    gen = Generator(cfg, params, batch_size=2, graph=graph)
    res = gen.generate(toks.cpu().numpy(), n_new=3)
    np.testing.assert_allclose(res["logits"][:, :12].cpu().numpy(), full.cpu().numpy(), atol=1e-4)
    assert res["tokens"].shape == (2, 3)
    assert (gen.graph is not None) == (graph and mode == "ram")
    # the same parameters with the pool's table in HBM
    hbm = {"params": dict(params["params"])}
    hbm["params"]["pool"] = dict(params["params"]["pool"],
                                 values=torch.from_numpy(np.asarray(pool.values)).to("cuda"))
    ref = Generator(base, hbm, batch_size=2, graph=graph).generate(toks.cpu().numpy(), n_new=3)
    assert torch.equal(res["tokens"], ref["tokens"])
    np.testing.assert_allclose(res["logits"].cpu().numpy(), ref["logits"].cpu().numpy(), rtol=0, atol=1e-6)
    # a second generation over the captured step starts clean
    again = gen.generate(toks.cpu().numpy(), n_new=3)
    assert torch.equal(again["tokens"], res["tokens"]) and torch.equal(again["logits"], res["logits"])


def test_generator_follows_pool_parameters_replaced(gpu_lib):
    """A pool parameter replaced by a new tensor of the same shape between
    generate() calls (possibly at the freed tensor's address, where its
    version counter starts again at 0) is a change: the next generate()
    uses the new keys and temperature, as an eager step does."""
    cfg = ModelConfig(vocab_size=300, max_len=40, d_model=64, n_heads=4, n_layers=2, ffn_mult=2, n_sub_keys=64,
                      pool_heads=4, d_key=64, d_value=64, top_k=8, memory_layers=(0, 1))
    params = MemoryPoolLM(cfg).init(7)
    prompt = np.random.default_rng(5).integers(0, 300, (4, 10))
    gen = Generator(cfg, params, batch_size=4, graph=True)
    before = gen.generate(prompt, n_new=8)
    pool = params["params"]["pool"]
    new_keys = (pool["sub_keys"] * -1.0 + 0.3).contiguous()
    new_lt = pool["log_temperature"] + 0.7
    del pool["sub_keys"], pool["log_temperature"]
    pool["sub_keys"], pool["log_temperature"] = new_keys, new_lt
    after = gen.generate(prompt, n_new=8)
    eager = Generator(cfg, params, batch_size=4, graph=False).generate(prompt, n_new=8)
    assert torch.equal(after["logits"], eager["logits"])
    assert not torch.equal(after["logits"], before["logits"])


def test_generation_at_the_268M_slot_shapes(gpu_lib):
    """A short greedy generation at the 268M-slot decode shapes: n_sub_keys
    16,384 (268,435,456 fp16 slots, 137 GB), vocab 16,384, d_model 256, 4
    layers with memory layers 1 and 3, 64 streams, 16 prompt tokens and 8
    new ones.  The captured step equals the eager one bit for bit, and the
    decode logits equal the full forward over the same tokens within the
    fp16 rule (1e-2 of the largest |logit|: near-tied slots may be chosen
    differently by the two paths' query rounding)."""
    n, d, B, P, new = 16384, 256, 64, 16, 8
    cfg = ModelConfig(vocab_size=16384, max_len=P + new, d_model=256, n_layers=4, n_heads=4, ffn_mult=4,
                      memory_layers=(1, 3), n_sub_keys=n, pool_heads=4, d_key=256, d_value=d, top_k=16,
                      values_dtype=torch.float16)
    free, _ = torch.cuda.mem_get_info()
    if free < 150 * 2 ** 30:
        pytest.skip(f"needs 150 GiB of free device memory, {free / 2 ** 30:.0f} GiB free")
    g = torch.Generator(device="cuda").manual_seed(17)
    values = torch.empty((n * n, d), dtype=torch.float16, device="cuda")
    values.normal_(0.0, 0.02, generator=g)
    print("268M-slot table filled", flush=True)
    try:
        model = MemoryPoolLM(cfg)
        params = model.init(0, pool_values=values)
        prompt = torch.randint(0, cfg.vocab_size, (B, P), generator=g, device="cuda")
        a = Generator(cfg, params, batch_size=B, graph=True).generate(prompt, n_new=new)
        b = Generator(cfg, params, batch_size=B, graph=False).generate(prompt, n_new=new)
        print("graph and eager generations done", flush=True)
        assert torch.equal(a["tokens"], b["tokens"]) and torch.equal(a["logits"], b["logits"])
        seq = torch.cat([prompt, a["tokens"][:, :-1]], 1)  # the tokens every decode step was fed
        with torch.no_grad():
            full, _ = model.apply(params, seq)
        lg = a["logits"].float()
        assert lg.shape == full.shape == (B, P + new - 1, cfg.vocab_size)
        scale = float(full.abs().max())
        err = float((lg - full).abs().max())
        assert err <= 1e-2 * scale, (err, scale)
        close = ((lg - full).abs().amax(-1) <= 1e-4 * scale).float().mean()
        print(f"max |decode - full| {err:.3g} of max |logit| {scale:.3g}; positions within 1e-4 of it: "
              f"{float(close):.1%}", flush=True)
    finally:
        del values
        params = None
        torch.cuda.empty_cache()


def test_next_token_embed_writes_next_input_rows(gpu_lib):
    """mpl_decode_next_token_embed: the same tokens, outputs and position as
    mpl_decode_next_token, and x_next equal to mpl_decode_embed of the chosen
    tokens at the advanced position bit for bit (prompt tokens first, then
    argmax picks); past the position table the rows are NaN."""
    from model_amd import _lib
    from model_amd.model import decode_embed

    B, V, Lmax, P, d = 5, 777, 6, 3, 64
    g = torch.Generator(device="cuda").manual_seed(17)
    emb = torch.randn((V, d), generator=g, device="cuda")
    pe = torch.randn((Lmax, d), generator=g, device="cuda")
    prompt = torch.randint(0, V, (B, Lmax), generator=g, device="cuda")
    plen = torch.full((1,), P, dtype=torch.int64, device="cuda")
    st = {}
    for fused in (False, True):
        st[fused] = {"pos": torch.zeros(1, dtype=torch.int64, device="cuda"),
                     "tok": torch.zeros(B, dtype=torch.int64, device="cuda"),
                     "out": torch.full((B, Lmax), -1, dtype=torch.int64, device="cuda"),
                     "done": torch.zeros(1, dtype=torch.int32, device="cuda")}
    x_next = torch.empty((B, d), device="cuda")
    p_ = _lib.ptr
    for step in range(Lmax):
        logits = torch.randn((B, V), generator=g, device="cuda")
        for fused in (False, True):
            s = st[fused]
            head = (p_(logits), B, V, p_(prompt), Lmax, p_(plen), p_(s["pos"]), p_(s["tok"]), p_(s["out"]), Lmax,
                    Lmax, p_(s["done"]))
            if fused:
                pos_before = s["pos"].clone()
                _lib.check(_lib.lib().mpl_decode_next_token_embed(*head, p_(emb), V, p_(pe), Lmax, d, p_(x_next),
                                                                  _lib.stream_ptr(logits.device)), "embed")
            else:
                _lib.check(_lib.lib().mpl_decode_next_token(*head, _lib.stream_ptr(logits.device)), "next")
        torch.cuda.synchronize()
        for key in ("pos", "tok", "out", "done"):
            assert torch.equal(st[True][key], st[False][key]), (step, key)
        if step + 1 < Lmax:
            want = decode_embed(emb, pe, st[True]["tok"], pos_before + 1)
            assert torch.equal(x_next, want), step
        else:  # position past the table: NaN rows, nothing read outside it
            assert torch.isnan(x_next).all()
