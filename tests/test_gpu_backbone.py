"""The backbone mirror with its memory layers on the GPU (model_amd/model.py
with libmpl.so reads) against the numpy oracle of model.py:29-127
(oracle/backbone.py, pinned in tests/test_oracle_backbone.py).  The seeds
give inputs whose every memory-layer row is tie free under the parity rule
(checked here), so the selections must agree and the logits match within
1e-4 relative for an fp32 table (fp32 scoring) and 1e-2 for fp16."""

import numpy as np
import pytest
import torch

from model_amd.model import MemoryPoolLM
from oracle import backbone as ob
from oracle import lookup as ol
from tests.test_oracle_backbone import _cpu_params, _np_tree, _pool_cfg

pytestmark = pytest.mark.gpu


def _to_cuda(t, values_dtype):
    if isinstance(t, dict):
        return {k: (_to_cuda(v, values_dtype) if k != "values" else v.to("cuda", values_dtype)) for k, v in t.items()}
    return t.cuda()


@pytest.mark.parametrize("seed,dt,tol", [(5, torch.float32, 1e-4), (6, torch.float16, 1e-2)])
def test_logits_match_oracle(gpu_lib, seed, dt, tol):
    cfg = _pool_cfg(values_dtype=dt)
    cpu = _cpu_params(cfg, seed)
    params = {"params": _to_cuda(cpu, dt)}
    toks = np.random.default_rng(seed).integers(0, 40, (2, 10))
    with torch.no_grad():
        got, aux = MemoryPoolLM(cfg).apply(params, torch.as_tensor(toks, device="cuda"))
    ref = _np_tree(cpu)
    ref["pool"]["values"] = params["params"]["pool"]["values"].cpu().numpy()  # the table as stored
    want, queries = ob.forward(ref, toks, cfg)
    for q in queries:
        tie_free, _ = ol.near_tie_free_rows(q, ref["pool"]["sub_keys"], float(ref["pool"]["log_temperature"]),
                                            top_k_=cfg.top_k)
        assert tie_free.all()
    got = got.double().cpu().numpy()
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err <= tol, f"logits relative error {err:.3g} > {tol}"
    assert len(aux["slots"]) == len(cfg.memory_layers)
