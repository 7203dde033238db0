"""Writes tests/golden/train_state_{adagrad,adam}.msgpack: small TrainState
checkpoints laid out as the reference's save_checkpoint writes them
(train.py:36-44, 559-571: flax.serialization.to_bytes of the TrainState
dataclass, fields step, params, opt_state, subkey_usage, slot_usage, pool_m,
pool_v).  Built from raw msgpack primitives only, as flax >= 0.8.5 encodes
them (maps; arrays as ext type 1 holding msgpack((shape, dtype name, C-order
bytes))), so the reader is checked against the published encoding, not
against its own writer.  The reference writes to_bytes(jax.device_get(state)):
device_get turns every jax array, the 0-d int32 step and optax's counts
included, into a numpy ndarray, which Flax writes as ext type 1 (ext type 3
is for numpy scalars, which such a state does not hold).
Row-wise Adagrad keeps its accumulator in pool_v [N] with an empty pool_m
(train.py:284-285); lazy Adam keeps both moments [N, d] (train.py:286-287).

opt_state restates the layout of the sparse-mode optimizer (train.py:106-132,
clip=False): optax.chain(optax.adamw(schedule, mask=...), scale_pool_values),
a tuple of (adamw's chain state, EmptyState).  adamw's state is the tuple
(ScaleByAdamState(count, mu, nu), MaskedState(inner_state=EmptyState) of the
masked weight decay, ScaleByScheduleState(count)).  Flax writes a tuple as a
map with keys "0", "1", ..., a NamedTuple as a map of its fields and an
EmptyState as an empty map.  optax is absent here, so this nesting is
restated from optax's published sources (>= 0.2.3, requirements.txt:3) and
is an approximation of what a given optax version writes; the reader treats
opt_state as an opaque nested tree, so its layout does not change what is
read.

Run: python tests/golden/make_flax_train_state_fixture.py
"""
import os

import msgpack
import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = {opt: os.path.join(HERE, f"train_state_{opt}.msgpack") for opt in ("adagrad", "adam")}
STEP = 7


def arrays(opt: str):
    rng = np.random.default_rng(77 if opt == "adagrad" else 78)
    H, n, half, d = 2, 8, 4, 6
    N = n * n
    params = {
        "router_1": {"kernel": rng.standard_normal((5, H * 2 * half)).astype(np.float32),
                     "bias": np.zeros(H * 2 * half, np.float32)},
        "pool": {"sub_keys": rng.standard_normal((H, 2, n, half)).astype(np.float32),
                 "values": (0.02 * rng.standard_normal((N, d))).astype(np.float32),
                 "log_temperature": np.array(np.log(10.0), dtype=np.float32)},
    }
    if opt == "adagrad":
        pool_m = np.zeros((0,), np.float32)
        pool_v = np.abs(rng.standard_normal(N)).astype(np.float32) * 1e-3
    else:
        pool_m = (1e-3 * rng.standard_normal((N, d))).astype(np.float32)
        pool_v = np.abs(1e-5 * rng.standard_normal((N, d))).astype(np.float32)
    return {
        "params": params,
        "subkey_usage": np.full((H, 2, n), 1.0 / n, np.float32),
        "slot_usage": np.full((N,), 1.0 / N, np.float32),
        "pool_m": pool_m,
        "pool_v": pool_v,
    }


def _ext(a: np.ndarray, code: int = 1) -> msgpack.ExtType:
    return msgpack.ExtType(code, msgpack.packb((a.shape, a.dtype.name, a.tobytes("C")), use_bin_type=True))


def _enc(tree):
    if isinstance(tree, dict):
        return {k: _enc(v) for k, v in tree.items()}
    return _ext(tree)


def main():
    for opt, path in OUT.items():
        a = arrays(opt)
        step = _ext(np.array(STEP, dtype=np.int32))
        # chain(adamw, scale_pool_values) over the dense params (the pool values
        # are split out in sparse mode, train.py:76-87)
        dense = {"router_1": a["params"]["router_1"],
                 "pool": {k: v for k, v in a["params"]["pool"].items() if k != "values"}}
        count = _ext(np.array(STEP, dtype=np.int32))
        adamw = {"0": {"count": count, "mu": _enc(dense), "nu": _enc(dense)},  # ScaleByAdamState
                 "1": {"inner_state": {}},                                   # MaskedState(EmptyState)
                 "2": {"count": count}}                                      # ScaleByScheduleState
        opt_state = {"0": adamw, "1": {}}
        state = {"step": step, "params": _enc(a["params"]), "opt_state": opt_state,
                 "subkey_usage": _ext(a["subkey_usage"]), "slot_usage": _ext(a["slot_usage"]),
                 "pool_m": _ext(a["pool_m"]), "pool_v": _ext(a["pool_v"])}
        with open(path, "wb") as f:
            f.write(msgpack.packb(state, use_bin_type=True))


if __name__ == "__main__":
    main()
