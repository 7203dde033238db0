"""CPU checks of the C ABI: the built library loads and exports every symbol
declared in include/mpl.h, with the ctypes signatures the host mirror uses.
No compute call is made (there is no GPU here)."""

import ctypes
import os
import re

import pytest

from model_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "mpl.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mpl_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "mpl_score_select" in syms and "mpl_gather_wsum" in syms
    assert set(syms) == set(_lib.SIGNATURES), "ctypes table and header disagree"


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libmpl.so is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, f"missing exports: {missing}"


def test_size_queries_without_gpu():
    L = _lib.lib()
    assert L.mpl_version() >= 100
    assert L.mpl_packed_keys_bytes(4, 512, 128, _lib.MPL_F16) == 8 * 16 * 32 * 128 * 2
    assert L.mpl_packed_keys_bytes(4, 100, 4, _lib.MPL_F32) == 8 * 4 * 32 * 8 * 4
    assert L.mpl_packed_keys_bytes(4, 512, 200, _lib.MPL_F16) == 0  # half > 128 unsupported
    assert L.mpl_score_select_workspace_bytes(8192, 4, 512, 128, 16) > 0


def test_invalid_arguments_are_reported_not_launched():
    L = _lib.lib()
    rc = L.mpl_score_select(None, 0, None, None, 10, 4, 8, 128, 20, _lib.MPL_F16, None, None, None,
                            None, 0, None, None, None, None, None, None, None)
    assert rc == 4  # MPL_EUNSUPPORTED: k > n
    assert b"k <= min(n, 32)" in L.mpl_last_error()
    rc = L.mpl_gather_wsum(None, 7, 10, 4, None, None, 1, 4, 0, None, None)
    assert rc == 1 and b"null buffer" in L.mpl_last_error()


def test_row_entry_points_validate_before_launch():
    L = _lib.lib()
    P, d, N = 524288, 256, 262144
    ws = L.mpl_merge_rows_workspace_bytes(P, d, N)
    # keys/values ping-pong (4 x P x 4 B) + segment ids (P x 4 B) + partial rows
    assert ws >= 5 * P * 4 + (P // 128) * 2 * d * 4
    assert L.mpl_merge_rows_workspace_bytes(0, d, N) == 0
    rc = L.mpl_merge_rows(None, None, 64, 16, None, 2000, N, None, 0, None, None, None, None, 1, None)
    assert rc == 4 and b"<= 1024" in L.mpl_last_error()
    rc = L.mpl_merge_rows(None, None, -1, 16, None, 8, N, None, 0, None, None, None, None, 1, None)
    assert rc == 1
    rc = L.mpl_merge_rows(None, None, 64, 16, None, 8, N, None, 0, None, None, None, None, 1, None)
    assert rc == 1 and b"null buffer" in L.mpl_last_error()
    rc = L.mpl_merge_rows_counts(None, None, 64, 16, None, 8, N, None, 0, None, None, None, None, 1, None, None)
    assert rc == 1 and b"null slot_counts" in L.mpl_last_error()
    rc = L.mpl_row_adagrad(None, 5, None, None, None, None, 10, 8, N, 0.1, None, None)
    assert rc == 1 and b"values_dtype" in L.mpl_last_error()
    rc = L.mpl_row_adam(None, _lib.MPL_F16, None, None, None, None, None, 10, 8, N, 0.1, -1, None, None)
    assert rc == 1
    assert L.mpl_clip_scale_workspace_bytes() >= 8
    rc = L.mpl_clip_scale(None, 10, None, 1.0, None, None, 0, None)
    assert rc == 1
    assert L.mpl_sum_squares_workspace_bytes() >= 8
    rc = L.mpl_sum_squares(None, None, 9, None, None, None, 0, None)
    assert rc == 1 and b"at most 8" in L.mpl_last_error()
