"""Flax parameter checkpoints of the reference read into (and written from)
this library's tensors.

The reference saves ``flax.serialization.to_bytes(params)``
(memory_pool_model/train.py:559-571, 662-665): a msgpack map of the
parameter tree whose array leaves use msgpack extension types (flax >= 0.8.5,
flax/serialization.py, as pinned by requirements.txt:2):

  * ext 1 (ndarray): the msgpack encoding of (shape, dtype name, C-order
    bytes);
  * ext 3 (numpy scalar): the same encoding of a 0-d array;
  * arrays above 2**30 bytes are stored as a map
    {"__msgpack_chunked_array__": True, "shape": {"0": d0, ...},
     "chunks": {"0": flat chunk, "1": ...}} of flat chunks of
    2**30 / itemsize elements.

``load_params`` streams the file: each array leaf goes to the device as it
is decoded, and the pool's value table (``params["pool"]["values"]``, fp32 in
the reference, memory.py:104-109) is converted chunk by chunk into the
requested dtype (fp16 by default), so a table larger than host memory is
never held whole on the host.  ``pool_params`` returns the MemoryPool
parameter dict of a loaded tree; ``save_params`` writes the same format.
``load_train_state`` / ``save_train_state`` do the same for the trainer's
resumable TrainState checkpoint (train.py:36-44, 559-583), whose pool
optimizer state SparseRowUpdate.resume / .train_state_pool map.
"""

from __future__ import annotations

import io
import os
from typing import Any, Dict, Optional, Union

import msgpack
import numpy as np
import torch

EXT_NDARRAY = 1
EXT_NATIVE_COMPLEX = 2
EXT_NPSCALAR = 3
MAX_CHUNK_SIZE = 2 ** 30  # bytes per flat chunk of a large array
CHUNKED = "__msgpack_chunked_array__"
POOL_PATH = ("pool", "values")

_TORCH_DTYPES = {
    "float32": torch.float32, "float16": torch.float16, "float64": torch.float64, "bfloat16": torch.bfloat16,
    "int32": torch.int32, "int64": torch.int64, "int16": torch.int16, "int8": torch.int8, "uint8": torch.uint8,
    "bool": torch.bool,
}


def _decode_ndarray(data: bytes, device) -> torch.Tensor:
    shape, dtype_name, buf = msgpack.unpackb(data, raw=False)
    shape = tuple(shape)
    if dtype_name not in _TORCH_DTYPES:
        raise ValueError(f"unsupported array dtype {dtype_name!r} in checkpoint")
    if dtype_name == "bfloat16":  # numpy has no bfloat16: reinterpret the raw 16-bit words
        host = torch.frombuffer(bytearray(buf), dtype=torch.int16).view(torch.bfloat16)
    else:
        host = torch.from_numpy(np.frombuffer(buf, dtype=np.dtype(dtype_name)).copy())
    return host.reshape(shape).to(device)


class _Hook:
    """ext_hook for msgpack's Unpacker: array leaves become device tensors."""

    def __init__(self, device):
        self.device = device

    def __call__(self, code: int, data: bytes):
        if code in (EXT_NDARRAY, EXT_NPSCALAR):
            return _decode_ndarray(data, self.device)
        if code == EXT_NATIVE_COMPLEX:
            re, im = msgpack.unpackb(data)
            return complex(re, im)
        return msgpack.ExtType(code, data)


def _leaf_dtype(path, stored: torch.dtype, values_dtype):
    return values_dtype if (path[-2:] == POOL_PATH and values_dtype is not None) else stored


def _read_chunked(up, path, device, values_dtype) -> torch.Tensor:
    """The rest of a chunked-array map after its marker entry: "shape", then
    "chunks", whose flat pieces are copied into the output as they arrive."""
    out = shape = None
    for _ in range(2):
        key = up.unpack()
        if key == "shape":
            n = up.read_map_header()
            dims = {}
            for _ in range(n):
                k = up.unpack()
                dims[k] = int(up.unpack())
            shape = tuple(dims[str(i)] for i in range(n))
        elif key == "chunks":
            if shape is None:
                raise ValueError(f"chunked array {'/'.join(path)}: chunks before shape")
            n = up.read_map_header()
            o = 0
            for _ in range(n):
                up.unpack()  # "0", "1", ... in order
                c = up.unpack()
                if out is None:
                    out = torch.empty(int(np.prod(shape)), dtype=_leaf_dtype(path, c.dtype, values_dtype),
                                      device=device)
                out[o:o + c.numel()].copy_(c.reshape(-1))
                o += c.numel()
                del c
            if out is None or o != out.numel():
                raise ValueError(f"chunked array {'/'.join(path)}: {o} elements for shape {shape}")
        else:
            raise ValueError(f"chunked array {'/'.join(path)}: unexpected entry {key!r}")
    return out.reshape(shape)


def _walk(up, path, device, values_dtype):
    try:
        n = up.read_map_header()
    except ValueError:  # not a map: one leaf (the header byte is not consumed)
        leaf = up.unpack()
        if isinstance(leaf, torch.Tensor):
            return leaf.to(_leaf_dtype(path, leaf.dtype, values_dtype))
        return leaf
    d: Dict[str, Any] = {}
    for i in range(n):
        key = up.unpack()
        if i == 0 and key == CHUNKED:
            up.unpack()  # True
            return _read_chunked(up, path, device, values_dtype)
        d[key] = _walk(up, path + (key,), device, values_dtype)
    return d


def load_params(src: Union[str, bytes, io.BufferedIOBase], device: Union[str, torch.device] = "cuda",
                values_dtype: Optional[torch.dtype] = torch.float16) -> Dict[str, Any]:
    """Parameter tree of a Flax msgpack checkpoint (train.py:662-665) as
    nested dicts of tensors on ``device``; ``pool/values`` is cast to
    ``values_dtype`` (None keeps the stored dtype).  The file is walked one
    leaf at a time, so host memory holds at most one array (or one 1 GiB
    chunk of a large one)."""
    f = open(src, "rb") if isinstance(src, (str, os.PathLike)) else (io.BytesIO(src) if isinstance(src, bytes) else src)
    try:
        up = msgpack.Unpacker(f, ext_hook=_Hook(device), raw=False, strict_map_key=False,
                              max_buffer_size=2 ** 31 - 1)
        return _walk(up, (), device, values_dtype)
    finally:
        if f is not src:
            f.close()


def pool_params(tree: Dict[str, Any]) -> Dict[str, torch.Tensor]:
    """The MemoryPool parameter dict {sub_keys, values, log_temperature} of a
    loaded model tree (the module is named "pool", model.py:70-84)."""
    p = tree["params"] if "params" in tree and "pool" not in tree else tree
    pool = p["pool"]
    out = {"sub_keys": pool["sub_keys"], "log_temperature": pool["log_temperature"]}
    if "values" in pool:  # absent with a host pool (memory.py:103-109)
        out["values"] = pool["values"]
    return out


def _ndarray_bytes(arr: np.ndarray) -> bytes:
    return msgpack.packb((list(arr.shape), arr.dtype.name, arr.tobytes("C")), use_bin_type=True)


def _to_numpy(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16:
            raise ValueError("bfloat16 leaves are not written by this writer")
        return t.numpy()
    return np.asarray(t)


def _pack_tree(tree, path, values_dtype):
    if isinstance(tree, dict):
        return {str(k): _pack_tree(v, path + (str(k),), values_dtype) for k, v in tree.items()}
    # every leaf, 0-d ones included, is an ndarray (ext 1): the reference writes
    # to_bytes(jax.device_get(state)), and device_get turns each jax array,
    # the int32 step and optax's counts among them, into an ndarray
    arr = _to_numpy(tree)
    if path[-2:] == POOL_PATH and values_dtype is not None:
        arr = arr.astype(values_dtype)
    arr = np.ascontiguousarray(arr)
    if arr.size * arr.dtype.itemsize > MAX_CHUNK_SIZE:
        per = max(1, MAX_CHUNK_SIZE // arr.dtype.itemsize)
        flat = arr.reshape(-1)
        chunks = {str(i): msgpack.ExtType(EXT_NDARRAY, _ndarray_bytes(flat[o:o + per]))
                  for i, o in enumerate(range(0, flat.size, per))}
        return {CHUNKED: True, "shape": {str(i): int(d) for i, d in enumerate(arr.shape)}, "chunks": chunks}
    return msgpack.ExtType(EXT_NDARRAY, _ndarray_bytes(arr))


def save_params(dst: Union[str, io.BufferedIOBase], tree: Dict[str, Any],
                values_dtype: Optional[np.dtype] = np.float32) -> None:
    """Write a parameter tree in the format of flax.serialization.to_bytes;
    ``pool/values`` is written as ``values_dtype`` (fp32 as the reference
    stores it; None keeps the tensor's dtype)."""
    payload = msgpack.packb(_pack_tree(tree, (), values_dtype), use_bin_type=True)
    if isinstance(dst, (str, os.PathLike)):
        tmp = str(dst) + ".tmp"
        with open(tmp, "wb") as f:
            f.write(payload)
        os.replace(tmp, dst)
    else:
        dst.write(payload)


# ------------------------------------------------------------ train states
TRAIN_STATE_KEYS = ("step", "params", "opt_state", "subkey_usage", "slot_usage", "pool_m", "pool_v")


def load_train_state(src: Union[str, bytes, io.BufferedIOBase], device: Union[str, torch.device] = "cuda",
                     values_dtype: Optional[torch.dtype] = None) -> Dict[str, Any]:
    """The resumable checkpoint of train.py:559-583: the msgpack of the
    TrainState dataclass (train.py:36-44), fields {step, params, opt_state,
    subkey_usage, slot_usage, pool_m, pool_v}, read leaf by leaf like
    load_params.  ``values_dtype`` None keeps the stored fp32 value table
    (the master copy a resumed sparse update needs; SparseRowUpdate.resume
    derives the fp16 table from it).  ``step`` is returned as an int."""
    state = load_params(src, device=device, values_dtype=values_dtype)
    missing = [k for k in TRAIN_STATE_KEYS if k not in state]
    if missing:
        raise ValueError(f"not a TrainState checkpoint: missing {missing}")
    step = state["step"]
    state["step"] = int(step.item() if isinstance(step, torch.Tensor) else step)
    return state


def save_train_state(dst: Union[str, io.BufferedIOBase], *, step: int, params: Dict[str, Any],
                     opt_state: Any, subkey_usage: torch.Tensor, slot_usage: torch.Tensor,
                     pool_m: torch.Tensor, pool_v: torch.Tensor) -> None:
    """Writes a TrainState checkpoint in the reference's layout (field order
    of train.py:36-44; ``step`` an int32 scalar; the pool table fp32)."""
    tree = {
        "step": np.array(int(step), dtype=np.int32),
        "params": params,
        "opt_state": opt_state if opt_state is not None else {},
        "subkey_usage": subkey_usage,
        "slot_usage": slot_usage,
        "pool_m": pool_m,
        "pool_v": pool_v,
    }
    save_params(dst, tree, values_dtype=np.float32)
