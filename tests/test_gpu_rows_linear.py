"""mpl_rows_linear (the backbone's dense layers of a decode step, with the
layer norm before them, the activation and the residual add after them
fused in; model.py:29-127) against the oracle's layer_norm, dense,
gelu_tanh and silu (oracle/backbone.py, pinned in
tests/test_oracle_backbone.py) in fp64: fp32 accumulation within 2e-5 of
the result's largest magnitude, over row counts around the tile heights (16
and 64 rows), K up to 1024, outputs up to the vocabulary width and of odd
width, both weight layouts, and every optional operand on and off."""

import numpy as np
import pytest
import torch

from model_amd.model import rows_linear
from oracle import backbone as ob

pytestmark = pytest.mark.gpu

CASES = [
    # rows, K, N, out_in, ln, mul, act, bias, residual
    (1, 256, 768, False, True, False, None, True, False),
    (5, 16, 4, False, False, False, None, True, True),
    (64, 256, 1024, False, True, False, "gelu_tanh", True, False),
    (64, 1024, 256, False, False, False, None, True, True),
    (70, 256, 256, False, True, False, "silu", True, False),
    (17, 256, 48, False, False, True, None, True, True),
    (64, 256, 4096, True, True, False, None, False, False),
    (130, 64, 2048, True, False, False, None, False, False),
    (3, 32, 300, True, True, False, None, False, False),
    (33, 128, 96, False, True, True, "silu", False, True),
    (2, 32, 51, False, True, False, None, True, True),  # odd N: column pairs split
    (4, 32, 50, True, True, False, None, False, False),
    (19, 64, 50, False, False, False, "gelu_tanh", True, False),
]


@pytest.mark.parametrize("rows,K,N,out_in,ln,mul,act,bias,residual", CASES)
def test_rows_linear_matches_oracle(gpu_lib, rows, K, N, out_in, ln, mul, act, bias, residual):
    rng = np.random.default_rng(rows * 7919 + K * 31 + N)
    x = rng.standard_normal((rows, K)) * 1.5 + 0.3
    W = rng.standard_normal((N, K) if out_in else (K, N)) * K ** -0.5
    b = rng.standard_normal(N) * 0.1 if bias else None
    lnp = {"scale": 1.0 + 0.1 * rng.standard_normal(K), "bias": 0.1 * rng.standard_normal(K)} if ln else None
    m = rng.standard_normal((rows, K)) if mul else None
    res = rng.standard_normal((rows, N)) if residual else None
    f32 = [t.astype(np.float32) if t is not None else None for t in (x, W, b, m, res)]
    x, W, b, m, res = [t.astype(np.float64) if t is not None else None for t in f32]  # the inputs as stored
    if lnp is not None:
        lnp = {k: v.astype(np.float32).astype(np.float64) for k, v in lnp.items()}

    a = ob.layer_norm(x, lnp) if ln else x
    if mul:
        a = a * m
    want = ob.dense(a, {"kernel": W.T if out_in else W, "bias": b if b is not None else np.zeros(N)})
    if act == "gelu_tanh":
        want = ob.gelu_tanh(want)
    elif act == "silu":
        want = ob.silu(want)
    if residual:
        want = want + res

    cuda = [torch.as_tensor(t, device="cuda") if t is not None else None for t in f32]
    xt, Wt, bt, mt, rt = cuda
    lnt = {k: torch.as_tensor(v, dtype=torch.float32, device="cuda") for k, v in lnp.items()} if ln else None
    got = rows_linear(xt, Wt, bt, out_in=out_in, ln=lnt, x_mul=mt, act=act, residual=rt)
    assert got.shape == (rows, N)
    err = np.abs(got.double().cpu().numpy() - want).max() / np.abs(want).max()
    assert err <= 2e-5, f"relative error {err:.3g}"


@pytest.mark.parametrize("K,mul,out_in", [(1024, False, False), (256, False, False), (256, True, False),
                                          (1024, False, True), (640, False, False)])
def test_narrow_tiles_equal_wide_tiles(gpu_lib, K, mul, out_in):
    """A narrow product (N = 256 at 64 rows, no layer norm) runs on 4-row
    tiles; the same columns inside a wide product (N = 2,048: 16-row tiles)
    come out bit for bit the same, since each element's K-slice sums are
    added in the same order on both."""
    g = torch.Generator(device="cuda").manual_seed(K + 7 * mul + 3 * out_in)
    x = torch.randn((64, K), generator=g, device="cuda")
    W = torch.randn((2048, K) if out_in else (K, 2048), generator=g, device="cuda") * K ** -0.5
    b = torch.randn(2048, generator=g, device="cuda")
    r = torch.randn((64, 2048), generator=g, device="cuda")
    m = torch.randn((64, K), generator=g, device="cuda") if mul else None
    wide = rows_linear(x, W, b, out_in=out_in, x_mul=m, residual=r)
    Wn = (W[:256] if out_in else W[:, :256]).contiguous()
    narrow = rows_linear(x, Wn, b[:256].contiguous(), out_in=out_in, x_mul=m, residual=r[:, :256].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(wide[:, :256], narrow)


def test_rows_linear_is_deterministic_and_accepts_residual_as_output(gpu_lib):
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn((64, 1024), generator=g, device="cuda")
    W = torch.randn((1024, 256), generator=g, device="cuda")
    r = torch.randn((64, 256), generator=g, device="cuda")
    a = rows_linear(x, W, residual=r)
    b = rows_linear(x, W, residual=r)
    assert torch.equal(a, b)


def test_rows_linear_rejects_bad_operands(gpu_lib):
    x = torch.zeros((4, 30), device="cuda")
    with pytest.raises(Exception, match="multiple of 4"):
        rows_linear(x, torch.zeros((30, 8), device="cuda"))
    x = torch.zeros((4, 32), device="cuda")
    with pytest.raises(ValueError):
        rows_linear(x, torch.zeros((32, 8), device="cuda"), torch.zeros(7, device="cuda"))
    with pytest.raises(ValueError):
        rows_linear(x.half(), torch.zeros((32, 8), device="cuda"))
    with pytest.raises(Exception, match="16-byte aligned"):
        rows_linear(torch.zeros(4 * 32 + 1, device="cuda")[1:].view(4, 32), torch.zeros((32, 8), device="cuda"))


@pytest.mark.parametrize("rows,K,n1,n2,ln,act1,act2,bias", [
    (64, 256, 1024, 256, True, None, "silu", True),  # the memory layer's router and gate
    (5, 16, 12, 8, True, None, "silu", True),
    (37, 64, 20, 44, False, "gelu_tanh", None, False),  # tiles across the split, no layer norm
    (70, 128, 17, 15, True, "silu", "gelu_tanh", True),  # odd widths: column pairs across the split
])
def test_rows_linear_pair_equals_two_layers(gpu_lib, rows, K, n1, n2, ln, act1, act2, bias):
    """mpl_rows_linear_pair against mpl_rows_linear of each layer: the same
    bits, since every output column is the same product in both."""
    from model_amd.model import rows_linear_pair

    g = torch.Generator(device="cuda").manual_seed(rows + K + n1)
    x = torch.randn((rows, K), generator=g, device="cuda")
    w1 = torch.randn((K, n1), generator=g, device="cuda") * K ** -0.5
    w2 = torch.randn((K, n2), generator=g, device="cuda") * K ** -0.5
    b1 = torch.randn(n1, generator=g, device="cuda") if bias else None
    b2 = torch.randn(n2, generator=g, device="cuda") if bias else None
    lnp = {"scale": torch.rand(K, generator=g, device="cuda") + 0.5,
           "bias": torch.randn(K, generator=g, device="cuda")} if ln else None
    w = torch.cat([w1, w2], 1).contiguous()
    b = torch.cat([b1, b2]) if bias else None
    o1, o2 = rows_linear_pair(x, w, b, n1, ln=lnp, act1=act1, act2=act2)
    r1 = rows_linear(x, w1, b1, ln=lnp, act=act1)
    r2 = rows_linear(x, w2, b2, ln=lnp, act=act2)
    torch.cuda.synchronize()
    assert o1.shape == (rows, n1) and o2.shape == (rows, n2)
    assert torch.equal(o1, r1) and torch.equal(o2, r2)


@pytest.mark.parametrize("rows,d,V", [(64, 256, 16384), (5, 64, 300), (2, 32, 50), (64, 256, 1000), (1, 128, 64)])
def test_vocab_logits_matches_torch(gpu_lib, rows, d, V):
    """mpl_vocab_logits against torch's layer_norm + linear in fp64 on the
    same fp32 inputs: within fp32 rounding (1e-5 of the largest |logit|)."""
    import torch.nn.functional as F
    from model_amd.model import LN_EPS, vocab_logits
    g = torch.Generator(device="cuda").manual_seed(rows * 31 + d + V)
    x = torch.randn((rows, d), generator=g, device="cuda") * 2.0 + 0.5
    sc = torch.rand(d, generator=g, device="cuda") + 0.5
    bi = torch.randn(d, generator=g, device="cuda") * 0.1
    emb = torch.randn((V, d), generator=g, device="cuda") * 0.05
    print(f"vocab logits rows={rows} d={d} V={V}", flush=True)
    out = vocab_logits(x, sc, bi, emb)
    torch.cuda.synchronize()
    ref = F.linear(F.layer_norm(x.double(), (d,), sc.double(), bi.double(), LN_EPS), emb.double())
    err = float((out.double() - ref).abs().max()) / float(ref.abs().max())
    assert err <= 1e-5, err
