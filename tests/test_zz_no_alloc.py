"""mpl_lookup_static (the lookup that allocates nothing: its scratch is a
fixed device array) against mpl_lookup with a caller workspace, through the
C ABI: every output bit for bit, on two calls in a row, the second with a
smaller batch (a different split plan), one with routing noise.  Also: a
batch whose scratch would exceed the fixed array is refused before any
launch."""

import numpy as np
import pytest
import torch

from model_amd import _lib

pytestmark = pytest.mark.gpu

H, D_KEY, D, K, N_SUB = 4, 256, 256, 16, 2048
HALF = D_KEY // 2


@pytest.fixture(scope="module")
def table(gpu_lib):
    L = gpu_lib
    g = torch.Generator(device="cuda").manual_seed(90)
    keys = torch.randn((H, 2, N_SUB, HALF), generator=g, device="cuda") * HALF ** -0.5
    packed = torch.empty(L.mpl_packed_keys_bytes(H, N_SUB, HALF, _lib.MPL_F16), dtype=torch.uint8, device="cuda")
    _lib.check(L.mpl_pack_keys(_lib.ptr(keys), H, N_SUB, HALF, _lib.MPL_F16, None, _lib.ptr(packed),
                               _lib.stream_ptr(keys.device)), "pack")
    values = torch.empty((N_SUB * N_SUB, D), dtype=torch.float16, device="cuda").normal_(0.0, 0.02, generator=g)
    return packed, values


def _outputs(M):
    i32, f32 = torch.int32, torch.float32
    return {
        "sub_idx": torch.full((M, H, 2, K), -5, dtype=i32, device="cuda"),
        "sub_scores": torch.full((M, H, 2, K), 5.0, dtype=f32, device="cuda"),
        "flat_idx": torch.full((M, H, K), -5, dtype=i32, device="cuda"),
        "slots": torch.full((M, H, K), -5, dtype=i32, device="cuda"),
        "weights": torch.full((M, H, K), 5.0, dtype=f32, device="cuda"),
        "out": torch.full((M, D), 5.0, dtype=f32, device="cuda"),
    }


def _call(L, static, q, packed, values, gumbel, coef):
    M = q.shape[0]
    o = _outputs(M)
    p = _lib.ptr
    st = _lib.stream_ptr(q.device)
    T = torch.full((1,), 10.0, device="cuda")  # device scalars, as the C ABI takes them
    c = torch.full((1,), coef, device="cuda") if gumbel is not None else None
    head = (p(q), _lib.MPL_Q_RAW, None, p(packed), M, H, N_SUB, HALF, K, _lib.MPL_F16, p(T), p(gumbel), p(c))
    tail = (p(o["sub_idx"]), p(o["sub_scores"]), p(o["flat_idx"]), p(o["slots"]), p(o["weights"]), p(values),
            _lib.MPL_F16, D, 0, p(o["out"]), st)
    if static:
        _lib.check(L.mpl_lookup_static(*head, *tail), "mpl_lookup_static")
    else:
        wsb = L.mpl_score_select_workspace_bytes(M, H, N_SUB, HALF, K)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
        _lib.check(L.mpl_lookup(*head, p(ws), wsb, *tail), "mpl_lookup")
    torch.cuda.synchronize()
    return o


def test_static_lookup_equals_lookup(gpu_lib, table):
    L = gpu_lib
    packed, values = table
    assert L.mpl_lookup_static_scratch_bytes() == 32 << 20
    g = torch.Generator(device="cuda").manual_seed(91)
    # first call: 1,500 tokens with noise (6 key splits, stage 2 fused with the
    # read); second call: 5 tokens without (64 splits, one-launch wide merge)
    for M, noisy in ((1500, True), (5, False)):
        print(f"static lookup vs lookup: {M} tokens, noise={noisy}", flush=True)
        q = torch.randn((M, H, 2, HALF), generator=g, device="cuda")
        gumbel = None
        if noisy:
            u = torch.rand((M, H, 2, N_SUB), generator=g, device="cuda").clamp_(1e-30, 1 - 1e-7)
            gumbel = -torch.log(-torch.log(u))
        coef = 0.5 if noisy else 0.0
        want = _call(L, False, q, packed, values, gumbel, coef)
        got = _call(L, True, q, packed, values, gumbel, coef)
        for key in want:
            assert torch.equal(got[key], want[key]), f"{key} differs at M={M}"
        assert int(got["slots"].min()) >= 0


def test_static_lookup_refuses_oversized_batch(gpu_lib, table):
    """A batch whose selection scratch exceeds the fixed array fails with
    MPL_EWORKSPACE before anything is launched (no buffer is touched)."""
    L = gpu_lib
    M, n = 70000, 512
    need = L.mpl_score_select_workspace_bytes(M, H, n, HALF, K)
    assert need > L.mpl_lookup_static_scratch_bytes()
    rc = L.mpl_lookup_static(None, _lib.MPL_Q_RAW, None, None, M, H, n, HALF, K, _lib.MPL_F16, None, None, None,
                             None, None, None, None, None, None, _lib.MPL_F16, D, 0, None, None)
    assert rc == 3  # MPL_EWORKSPACE
    assert b"scratch" in L.mpl_last_error()
