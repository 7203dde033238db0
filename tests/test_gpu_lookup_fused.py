"""mpl_lookup (selection and value read in one call) against mpl_score_select
followed by mpl_gather_wsum, through the C ABI: every output bit for bit.
Covers the fused stage-2 + read kernel (H = 4, k = 16: fp16 rows of 128, 256
and 512 elements, fp32 rows, shuffled reads, split-key plans whose lists are
merged before stage 2), the plans with 9-64 split lists (decode sizes),
whose lists the fused decode stage 2 (pair_decode_read_k16) reduces, and the
shapes that fall back to two launches (other H or k, row widths without a
fused variant)."""

import pytest
import torch

from model_amd import _lib
from model_amd._lib import ptr

pytestmark = pytest.mark.gpu


def _run(M, H, n, d_key, d, k, vdt, shuffle, seed):
    L = _lib.lib()
    half = d_key // 2
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((M, H, 2, half), generator=g, device="cuda")
    keys = torch.randn((H, 2, n, half), generator=g, device="cuda") * half ** -0.5
    values = (torch.randn((n * n, d), generator=g, device="cuda") * 0.02).to(vdt)
    vcode = _lib.MPL_F16 if vdt == torch.float16 else _lib.MPL_F32
    packed = torch.empty(L.mpl_packed_keys_bytes(H, n, half, _lib.MPL_F16), dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    _lib.check(L.mpl_pack_keys(ptr(keys), H, n, half, _lib.MPL_F16, None, ptr(packed), s), "pack")
    wsb = L.mpl_score_select_workspace_bytes(M, H, n, half, k)
    T = torch.full((1,), 10.0, device="cuda")  # the clamped temperature, a device scalar
    outs = []
    for fused in (False, True):
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
        o = {"sub_idx": torch.full((M, H, 2, k), -7, dtype=torch.int32, device="cuda"),
             "sub_scores": torch.full((M, H, 2, k), 7.0, device="cuda"),
             "flat_idx": torch.full((M, H, k), -7, dtype=torch.int32, device="cuda"),
             "slots": torch.full((M, H, k), -7, dtype=torch.int32, device="cuda"),
             "weights": torch.full((M, H, k), 7.0, device="cuda"),
             "out": torch.full((M, d), 7.0, device="cuda")}
        sel = (ptr(q), _lib.MPL_Q_RAW, None, ptr(packed), M, H, n, half, k, _lib.MPL_F16, ptr(T), None, None,
               ptr(ws), wsb, ptr(o["sub_idx"]), ptr(o["sub_scores"]), ptr(o["flat_idx"]), ptr(o["slots"]),
               ptr(o["weights"]))
        if fused:
            _lib.check(L.mpl_lookup(*sel, ptr(values), vcode, d, shuffle, ptr(o["out"]), s), "mpl_lookup")
        else:
            _lib.check(L.mpl_score_select(*sel, s), "mpl_score_select")
            _lib.check(L.mpl_gather_wsum(ptr(values), vcode, n * n, d, ptr(o["slots"]), ptr(o["weights"]), M,
                                         H * k, shuffle, ptr(o["out"]), s), "mpl_gather_wsum")
        outs.append(o)
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("M,H,n,d_key,d,k,vdt,shuffle", [
    (8192, 4, 512, 256, 256, 16, torch.float16, 0),   # text-study layer: fused, one split
    (777, 4, 64, 64, 128, 16, torch.float16, 0),      # ragged token count, 128-wide fp16 rows
    (1000, 4, 128, 256, 256, 16, torch.float32, 0),   # fp32 rows (fact-task layer)
    (333, 4, 128, 128, 512, 16, torch.float16, 1),    # 512-wide rows, shuffled reads
    (64, 4, 1024, 256, 256, 16, torch.float16, 0),    # split-key plan merged before stage 2
    (16, 4, 1024, 256, 256, 16, torch.float16, 1),
    (1, 4, 1024, 256, 256, 16, torch.float16, 0),     # decode: one token, 4 split lists
    (5, 4, 1024, 256, 256, 16, torch.float32, 1),     # 32 split lists, fp32 rows, shuffled reads
    (3, 4, 2048, 128, 128, 16, torch.float16, 0),     # decode: 8 split lists, 128-wide rows
    (2, 4, 4096, 256, 128, 16, torch.float16, 1),     # decode: 16 split lists, shuffled reads
    (20, 4, 4096, 256, 128, 16, torch.float16, 0),    # 64 split lists
    (9, 4, 2500, 256, 256, 16, torch.float32, 0),     # 40 split lists (ragged n), fp32 rows
    (300, 2, 128, 64, 256, 16, torch.float16, 0),     # H = 2: two launches
    (300, 4, 128, 64, 256, 8, torch.float16, 0),      # k = 8: two launches
    (300, 4, 128, 64, 96, 16, torch.float16, 0),      # 96-wide rows: two launches
])
def test_lookup_equals_select_then_gather(gpu_lib, M, H, n, d_key, d, k, vdt, shuffle):
    ref, got = _run(M, H, n, d_key, d, k, vdt, shuffle, seed=M + n)
    for name in ref:
        assert torch.equal(ref[name], got[name]), name
    assert bool((got["slots"] >= 0).all()) and bool((got["slots"] < n * n).all())


def test_lookup_zero_tokens_and_errors(gpu_lib):
    L = _lib.lib()
    s = torch.cuda.current_stream().cuda_stream
    # M = 0 launches nothing and succeeds
    assert L.mpl_lookup(None, _lib.MPL_Q_RAW, None, None, 0, 4, 64, 64, 16, _lib.MPL_F16, None, None, None,
                        None, 0, None, None, None, None, None, None, _lib.MPL_F16, 256, 0, None, s) == 0
    # a bad values dtype is reported, not launched
    rc = L.mpl_lookup(None, _lib.MPL_Q_RAW, None, None, 4, 4, 64, 64, 16, _lib.MPL_F16, None, None, None,
                      None, 0, None, None, None, None, None, None, 99, 256, 0, None, s)
    assert rc != 0 and b"values_dtype" in L.mpl_last_error()
