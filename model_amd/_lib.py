"""ctypes binding of libmpl.so (include/mpl.h).

The product path has no fallback: if the library is missing or fails to load
this module raises, so a GPU run can never silently use another code path.
"""

from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmpl.so")

MPL_F32, MPL_F16 = 0, 1
MPL_OK, MPL_EINVAL, MPL_EHIP, MPL_EWORKSPACE, MPL_EUNSUPPORTED = 0, 1, 2, 3, 4  # include/mpl.h status codes
MPL_Q_NORMALIZED, MPL_Q_RAW, MPL_Q_RAW_SCALED = 0, 1, 2
MPL_ACT_NONE, MPL_ACT_GELU_TANH, MPL_ACT_SILU = 0, 1, 2
MPL_W_IN_OUT, MPL_W_OUT_IN = 0, 1

# name -> (restype, argtypes); the C ABI of include/mpl.h
_P, _I, _I64, _F, _SZ = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t
_U64 = C.c_uint64
SIGNATURES = {
    "mpl_version": (_I, []),
    "mpl_last_error": (C.c_char_p, []),
    "mpl_l2_normalize": (_I, [_P, _I64, _I, _F, _P, _P, _P, _P]),
    "mpl_packed_keys_bytes": (_SZ, [_I, _I, _I, _I]),
    "mpl_pack_keys": (_I, [_P, _I, _I, _I, _I, _P, _P, _P]),
    "mpl_score_select_workspace_bytes": (_SZ, [_I64, _I, _I, _I, _I]),
    "mpl_score_select": (_I, [_P, _I, _P, _P, _I64, _I, _I, _I, _I, _I, _P, _P, _P, _P, _SZ,
                              _P, _P, _P, _P, _P, _P]),
    "mpl_gather_wsum": (_I, [_P, _I, _I64, _I, _P, _P, _I64, _I, _I, _P, _P]),
    "mpl_lookup": (_I, [_P, _I, _P, _P, _I64, _I, _I, _I, _I, _I, _P, _P, _P, _P, _SZ,
                        _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P]),
    "mpl_rowfile_open": (_I, [C.c_char_p, _I64, _I64, _I64, _I, C.POINTER(C.c_void_p)]),
    "mpl_rowfile_read": (_I, [_P, _P, _I64, _P, _I]),
    "mpl_rowfile_read_direct": (_I, [_P, _P, _I64, _P, _I]),
    "mpl_rowfile_direct_supported": (_I, [_P]),
    "mpl_rowfile_write": (_I, [_P, _P, _I64, _P, _I]),
    "mpl_rowfile_sync": (_I, [_P]),
    "mpl_rowfile_evict": (_I, [_P]),
    "mpl_rowfile_close": (_I, [_P]),
    "mpl_lookup_static_scratch_bytes": (_SZ, []),
    "mpl_lookup_static": (_I, [_P, _I, _P, _P, _I64, _I, _I, _I, _I, _I, _P, _P, _P,
                               _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P]),
    "mpl_gumbel_noise": (_I, [_U64, _I64, _I, _P, _P]),
    "mpl_unique_slots_workspace_bytes": (_SZ, [_I64, _I64]),
    "mpl_unique_slots": (_I, [_P, _I64, _I64, _P, _SZ, _P, _P, _P, _P]),
    "mpl_gather_rows": (_I, [_P, _I, _I64, _I, _P, _I64, _P, _P, _P]),
    "mpl_host_device_pointer": (_I, [_P, C.POINTER(C.c_void_p)]),
    "mpl_score_topk_workspace_bytes": (_SZ, [_I64, _I, _I, _I, _I]),
    "mpl_score_topk": (_I, [_P, _I, _P, _P, _I64, _I, _I, _I, _I, _I, _P, _P, _P, _P, _SZ, _P, _P, _P]),
    "mpl_merge_rows_workspace_bytes": (_SZ, [_I64, _I, _I64]),
    "mpl_merge_rows": (_I, [_P, _P, _I64, _I, _P, _I, _I64, _P, _SZ, _P, _P, _P, _P, _I, _P]),
    "mpl_merge_rows_counts": (_I, [_P, _P, _I64, _I, _P, _I, _I64, _P, _SZ, _P, _P, _P, _P, _I, _P, _P]),
    "mpl_clip_scale_workspace_bytes": (_SZ, []),
    "mpl_clip_scale": (_I, [_P, _I64, _P, _F, _P, _P, _SZ, _P]),
    "mpl_clip_scale_dense": (_I, [_P, _I64, _P, _P, _I, _F, _P, _P, _SZ, _P]),
    "mpl_sum_squares_workspace_bytes": (_SZ, []),
    "mpl_sum_squares": (_I, [_P, _P, _I, _P, _P, _P, _SZ, _P]),
    "mpl_row_adagrad": (_I, [_P, _I, _P, _P, _P, _P, _I64, _I, _I64, _F, _P, _P]),
    "mpl_row_adam": (_I, [_P, _I, _P, _P, _P, _P, _P, _I64, _I, _I64, _F, _I, _P, _P]),
    "mpl_lookup_bwd_route": (_I, [_P, _P, _I, _I64, _I, _P, _P, _P, _P, _I64, _I, _I, _I, _P, _P, _P, _P]),
    "mpl_lookup_bwd_queries": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I, _I, _I, _I, _P, _P, _P]),
    "mpl_lookup_bwd_keys_workspace_bytes": (_SZ, [_I64, _I, _I, _I, _I]),
    "mpl_lookup_bwd_keys": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I, _I, _I, _I, _P, _P, _SZ, _P, _P]),
    "mpl_sum": (_I, [_P, _I64, _P, _P, _P]),
    "mpl_temperature": (_I, [_P, _F, _F, _P, _P]),
    "mpl_l2_normalize_bwd": (_I, [_P, _P, _I64, _I, _F, _P, _P, _P]),
    "mpl_key_diversity_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "mpl_key_diversity": (_I, [_P, _P, _I, _I, _I, _I, _P, _SZ, _P, _P, _P]),
    "mpl_revive_keys": (_I, [_P, _P, _P, _I64, _P, _P, _I, _I, _I, _F, _F, _P, _P]),
    "mpl_route_counts": (_I, [_P, _P, _I64, _I, _I, _I, _P, _P, _P, _P]),
    "mpl_hash_normal_fill": (_I, [_P, _I, _I64, _I, _U64, _F, _I64, _P]),
    "mpl_decode_attention": (_I, [_P, _I64, _I, _I, _I, _P, _P, _P, _P, _F, _P]),
    "mpl_decode_next_token": (_I, [_P, _I64, _I64, _P, _I64, _P, _P, _P, _P, _I64, _I64, _P, _P]),
    "mpl_decode_next_token_embed": (_I, [_P, _I64, _I64, _P, _I64, _P, _P, _P, _P, _I64, _I64, _P, _P, _I64, _P,
                                         _I64, _I, _P, _P]),
    "mpl_decode_embed": (_I, [_P, _I64, _P, _I64, _I, _P, _P, _I64, _P, _P]),
    "mpl_rows_linear": (_I, [_P, _P, _P, _P, _F, _P, _I, _P, _I, _P, _I64, _I, _I, _P, _P]),
    "mpl_vocab_logits": (_I, [_P, _P, _P, _F, _P, _I64, _I, _I64, _P, _P]),
    "mpl_rows_linear_pair": (_I, [_P, _P, _P, _F, _P, _P, _I, _I, _I64, _I, _I, _I, _P, _P, _P]),
    "mpl_balance_state_bytes": (_SZ, [_I64, _I]),
    "mpl_balance_fwd": (_I, [_P, _I, _P, _P, _I64, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    "mpl_lookup_bwd_dense_workspace_bytes": (_SZ, [_I64, _I, _I, _I, _I]),
    "mpl_lookup_bwd_dense": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I64, _I, _I, _I, _I, _I, _P, _P,
                                  _SZ, _P, _P, _P, _P, _P]),
    "mpl_lookup_bwd_dense_queries": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I, _I, _I, _I, _I, _P, _P,
                                         _SZ, _F, _P, _P, _P, _P, _SZ, _P, _P, _I, _P]),
}

_lib = None


class MplError(RuntimeError):
    pass


def lib() -> C.CDLL:
    """The loaded library (raises MplError if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MplError(f"{LIB_PATH} is missing: build it with `python -m model_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().mpl_last_error().decode(errors="replace")
        raise MplError(f"{what or 'libmpl'} failed (code {rc}): {msg}")


def ptr(t) -> int | None:
    """Device pointer of a torch tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_ptr(device) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream
