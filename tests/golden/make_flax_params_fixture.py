"""Writes tests/golden/flax_params_small.msgpack: a small MemoryPoolLM-style
parameter tree encoded the way flax.serialization.to_bytes encodes it
(flax >= 0.8.5, flax/serialization.py: msgpack maps; array leaves as ext
type 1 holding msgpack((shape, dtype name, C-order bytes)); numpy scalars as
ext type 3; large arrays as {"__msgpack_chunked_array__": True, "shape":
{"0": ...}, "chunks": {"0": flat ext-1 array, ...}}).  Built from raw msgpack
primitives only (not from model_amd.checkpoint), so the reader is checked
against the published encoding rather than against its own writer.  The
pool's value table is stored chunked (chunks of 100 elements) to exercise
that path; Flax's reader concatenates chunks of any length.

Run: python tests/golden/make_flax_params_fixture.py
"""
import os

import msgpack
import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "flax_params_small.msgpack")


def arrays():
    rng = np.random.default_rng(2024)
    H, n, half, d, vocab, dm = 2, 8, 4, 6, 11, 5
    return {
        "embed": {"embedding": rng.standard_normal((vocab, dm)).astype(np.float32)},
        "pos_embed": (0.02 * rng.standard_normal((7, dm))).astype(np.float32),
        "pool": {
            "sub_keys": rng.standard_normal((H, 2, n, half)).astype(np.float32),
            "values": (0.02 * rng.standard_normal((n * n, d))).astype(np.float32),
            "log_temperature": np.array(np.log(10.0), dtype=np.float32),
        },
        "router_1": {"kernel": rng.standard_normal((dm, H * 2 * half)).astype(np.float32),
                     "bias": np.zeros(H * 2 * half, np.float32)},
        "counts": np.arange(6, dtype=np.int32).reshape(2, 3),
    }


def _ext(a: np.ndarray, code: int = 1) -> msgpack.ExtType:
    return msgpack.ExtType(code, msgpack.packb((a.shape, a.dtype.name, a.tobytes("C")), use_bin_type=True))


def encode(tree):
    if isinstance(tree, dict):
        return {k: encode(v) for k, v in tree.items()}
    return _ext(tree)


def main():
    t = arrays()
    enc = encode(t)
    v = t["pool"]["values"].reshape(-1)
    enc["pool"]["values"] = {
        "__msgpack_chunked_array__": True,
        "shape": {str(i): int(s) for i, s in enumerate(t["pool"]["values"].shape)},
        "chunks": {str(i): _ext(v[o:o + 100]) for i, o in enumerate(range(0, v.size, 100))},
    }
    enc["scale"] = _ext(np.array(np.float32(0.5)), code=3)  # a numpy scalar leaf
    with open(OUT, "wb") as f:
        f.write(msgpack.packb(enc, use_bin_type=True))


if __name__ == "__main__":
    main()
