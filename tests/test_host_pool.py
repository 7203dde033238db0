"""The host tier's file mode on the CPU: the reference's pool directory
layout and initial table, reopening, the host read of rows, snapshots, and
the library's row-file reader/writer (mpl_rowfile_*) against numpy on .npy
files.  The optimizer step runs on the GPU in both modes and is tested in
tests/test_gpu_host_pool.py.  The initial table is checked against numpy's
published default_rng(0) normals and against one undivided draw (the
reference draws 2^18 rows at a time; chunking must not change the stream)."""

import ctypes

import numpy as np
import pytest

from model_amd import _lib
from model_amd.host_pool import HostPool, get


def test_init_is_the_reference_stream(tmp_path):
    # numpy's Generator(PCG64(0)).standard_normal(3), as printed by numpy
    first = np.array([0.12573022, -0.13210486, 0.64042265])
    pool = HostPool(17, 3, path=str(tmp_path / "a"), seed=0, trainable=False)
    np.testing.assert_allclose(pool.values[0] / 3 ** -0.5, first, rtol=1e-6)  # printed to 8 digits, stored fp32
    n, d = (1 << 18) + 5, 2
    big = HostPool(n, d, path=str(tmp_path / "b"), seed=4, trainable=False, dtype=np.float32)
    want = (np.random.default_rng(4).standard_normal((n, d)) * d ** -0.5).astype(np.float32)
    np.testing.assert_array_equal(np.asarray(big.values), want)
    assert get(big.name) is big
    # the files are plain .npy arrays of the reference's layout
    np.testing.assert_array_equal(np.load(str(tmp_path / "b" / "values.npy")), want)


def test_state_files_per_optimizer(tmp_path):
    a = HostPool(10, 4, path=str(tmp_path / "adam"), optimizer="adam")
    assert sorted(p.name for p in (tmp_path / "adam").iterdir()) == ["m.npy", "v.npy", "values.npy"]
    assert a.acc is None and np.asarray(a.m).shape == (10, 4) and not np.asarray(a.m).any()
    b = HostPool(10, 4, path=str(tmp_path / "ada"), optimizer="rowwise_adagrad", dtype=np.float16)
    assert sorted(p.name for p in (tmp_path / "ada").iterdir()) == ["acc.npy", "values.npy"]
    assert np.asarray(b.acc).shape == (10,) and b.values.dtype == np.float16
    assert b.nbytes() == 10 * 4 * 2 + 10 * 4
    c = HostPool(10, 4, path=str(tmp_path / "frozen"), trainable=False)
    assert [p.name for p in (tmp_path / "frozen").iterdir()] == ["values.npy"]
    with pytest.raises(ValueError):
        HostPool(10, 4, optimizer="sgd")


def test_reopen_and_shape_check(tmp_path):
    p = str(tmp_path / "pool")
    a = HostPool(64, 8, path=p, seed=1, optimizer="rowwise_adagrad")
    a.values[3] = 7.0
    a.flush()
    b = HostPool(64, 8, path=p, seed=99, optimizer="rowwise_adagrad")  # reopened, not re-initialised
    np.testing.assert_array_equal(np.asarray(b.values), np.asarray(a.values))
    with pytest.raises(ValueError):
        HostPool(65, 8, path=p, optimizer="rowwise_adagrad")
    with pytest.raises(ValueError):
        HostPool(64, 8, path=p, optimizer="rowwise_adagrad", dtype=np.float16)


def test_gather_clips_and_converts(tmp_path):
    pool = HostPool(32, 6, path=str(tmp_path / "g"), dtype=np.float16, trainable=False)
    idx = np.array([0, 31, 40, -3, 5])
    got = pool.gather(idx)
    assert got.dtype == np.float32
    np.testing.assert_array_equal(got, np.asarray(pool.values)[[0, 31, 31, 0, 5]].astype(np.float32))
    assert pool.pop_gather_seconds() > 0 and pool.pop_gather_seconds() == 0


def test_gather_direct_io_equals_mapped(tmp_path):
    """A file-mode pool with direct_io reads its rows with O_DIRECT (no page
    cache): the same rows as the mapped reads."""
    mapped = HostPool(3000, 40, path=str(tmp_path / "d"), dtype=np.float16, trainable=False, seed=7)
    if not mapped._arrays["values"].direct_supported:
        with pytest.raises(OSError):
            HostPool(3000, 40, path=str(tmp_path / "d"), dtype=np.float16, trainable=False, direct_io=True)
        pytest.skip("this file system refuses O_DIRECT")
    direct = HostPool(3000, 40, path=str(tmp_path / "d"), dtype=np.float16, trainable=False, direct_io=True)
    idx = np.concatenate([np.unique(np.random.default_rng(1).integers(0, 3000, 900)), [2999, 0, 17]])
    np.testing.assert_array_equal(direct.gather(idx), mapped.gather(idx))


def test_save_load_roundtrip(tmp_path):
    a = HostPool(40, 4, path=str(tmp_path / "x"), optimizer="adam", seed=2)
    a.values[5] = 3.0
    a.m[1] = 0.25
    a.v[39] = 0.5
    a.save(str(tmp_path / "snap"))
    assert sorted(p.name for p in (tmp_path / "snap").iterdir()) == ["m.npy", "v.npy", "values.npy"]
    b = HostPool(40, 4, path=str(tmp_path / "y"), optimizer="adam", seed=9)
    b.load(str(tmp_path / "snap"))
    for k in ("values", "m", "v"):
        np.testing.assert_array_equal(np.asarray(getattr(b, k)), np.asarray(getattr(a, k)))
    assert a.nbytes() == 40 * 4 * 4 * 3
    with pytest.raises(ValueError):
        HostPool(41, 4, path=str(tmp_path / "z"), optimizer="adam").load(str(tmp_path / "snap"))
    b.evict_page_cache()  # advisory; the contents stay
    np.testing.assert_array_equal(np.asarray(b.values), np.asarray(a.values))


# --------------------------------------------------- native row-file I/O
def _open(path, offset, row_bytes, rows, writable=1):
    h = ctypes.c_void_p()
    _lib.check(_lib.lib().mpl_rowfile_open(str(path).encode(), offset, row_bytes, rows, writable, ctypes.byref(h)),
               "open")
    return h.value


def _npy(tmp_path, arr):
    f = tmp_path / "t.npy"
    np.save(f, arr)
    mm = np.load(f, mmap_mode="r")
    return f, mm.offset


@pytest.mark.parametrize("dtype,d", [(np.float16, 256), (np.float32, 3), (np.float32, 64)])
def test_rowfile_read_matches_numpy(tmp_path, dtype, d):
    rng = np.random.default_rng(d)
    N = 5000
    arr = rng.standard_normal((N, d)).astype(dtype)
    f, off = _npy(tmp_path, arr)
    h = _open(f, off, d * np.dtype(dtype).itemsize, N, 0)
    L = _lib.lib()
    try:
        # random ids with repeats, a long consecutive run, and single rows at both ends
        ids = np.concatenate([rng.integers(0, N, 3000), np.arange(1000, 1900), [0, N - 1, N - 1]]).astype(np.int64)
        for threads in (1, 7):
            out = np.full((ids.size, d), 9, dtype)
            _lib.check(L.mpl_rowfile_read(h, ids.ctypes.data, ids.size, out.ctypes.data, threads), "read")
            np.testing.assert_array_equal(out, arr[ids])
        # out-of-range ids are refused before anything is read
        bad = np.array([3, N], dtype=np.int64)
        out = np.zeros((2, d), dtype)
        assert L.mpl_rowfile_read(h, bad.ctypes.data, 2, out.ctypes.data, 1) != 0
        assert b"outside" in L.mpl_last_error() and not out.any()
        # a read-only file refuses writes
        assert L.mpl_rowfile_write(h, ids.ctypes.data, 1, out.ctypes.data, 1) != 0
    finally:
        L.mpl_rowfile_close(h)


@pytest.mark.parametrize("dtype,d,N", [(np.float16, 256, 5000), (np.float32, 3, 5000), (np.float32, 64, 5000),
                                       (np.float32, 1500, 900)])
def test_rowfile_read_direct_matches_numpy(tmp_path, dtype, d, N):
    """O_DIRECT reads (no page cache) return the rows numpy reads: sorted
    unique ids (the host tier's lookups), ids out of order and repeated, a
    long consecutive run (spans merged up to 1 MiB), rows that cross 4 KiB
    blocks (the .npy header shifts the rows), rows larger than a block
    (d = 1500 fp32: 6,000 bytes), and the last row of the file, whose span
    ends past the end of the file."""
    rng = np.random.default_rng(d + N)
    arr = rng.standard_normal((N, d)).astype(dtype)
    f, off = _npy(tmp_path, arr)
    row_bytes = d * np.dtype(dtype).itemsize
    h = _open(f, off, row_bytes, N, 0)
    L = _lib.lib()
    try:
        if not L.mpl_rowfile_direct_supported(h):
            ids = np.arange(3, dtype=np.int64)
            out = np.zeros((3, d), dtype)
            assert L.mpl_rowfile_read_direct(h, ids.ctypes.data, 3, out.ctypes.data, 1) == _lib.MPL_EUNSUPPORTED
            pytest.skip("this file system refuses O_DIRECT")
        uniq = np.unique(rng.integers(0, N, N // 3)).astype(np.int64)
        mixed = np.concatenate([rng.integers(0, N, 700), np.arange(100, 600), [0, N - 1, N - 1, 5, 4]])
        for ids in (uniq, mixed.astype(np.int64), np.array([N - 1], np.int64)):
            for threads in (1, 7):
                out = np.full((ids.size, d), 9, dtype)
                _lib.check(L.mpl_rowfile_read_direct(h, ids.ctypes.data, ids.size, out.ctypes.data, threads),
                           "read_direct")
                np.testing.assert_array_equal(out, arr[ids])
        bad = np.array([3, -1], dtype=np.int64)
        out = np.zeros((2, d), dtype)
        assert L.mpl_rowfile_read_direct(h, bad.ctypes.data, 2, out.ctypes.data, 1) != 0
        assert b"outside" in L.mpl_last_error() and not out.any()
    finally:
        L.mpl_rowfile_close(h)


def test_rowfile_read_direct_sees_rows_written_through_the_mapping(tmp_path):
    """Rows written through the shared mapping and not yet synced are what a
    direct read returns (the kernel writes the dirty range back first)."""
    rng = np.random.default_rng(4)
    N, d = 4000, 64
    arr = rng.standard_normal((N, d)).astype(np.float32)
    f, off = _npy(tmp_path, arr)
    h = _open(f, off, d * 4, N)
    L = _lib.lib()
    try:
        if not L.mpl_rowfile_direct_supported(h):
            pytest.skip("this file system refuses O_DIRECT")
        ids = np.unique(rng.integers(0, N, 500)).astype(np.int64)
        new = rng.standard_normal((ids.size, d)).astype(np.float32)
        _lib.check(L.mpl_rowfile_write(h, ids.ctypes.data, ids.size, new.ctypes.data, 4), "write")
        out = np.zeros_like(new)
        _lib.check(L.mpl_rowfile_read_direct(h, ids.ctypes.data, ids.size, out.ctypes.data, 4), "read_direct")
        np.testing.assert_array_equal(out, new)
    finally:
        L.mpl_rowfile_close(h)


def test_rowfile_write_matches_numpy(tmp_path):
    rng = np.random.default_rng(0)
    N, d = 3000, 40
    arr = rng.standard_normal((N, d)).astype(np.float32)
    f, off = _npy(tmp_path, arr)
    h = _open(f, off, d * 4, N)
    L = _lib.lib()
    try:
        ids = np.unique(np.concatenate([rng.integers(0, N, 800), np.arange(10, 600)])).astype(np.int64)
        new = rng.standard_normal((ids.size, d)).astype(np.float32)
        _lib.check(L.mpl_rowfile_write(h, ids.ctypes.data, ids.size, new.ctypes.data, 5), "write")
        _lib.check(L.mpl_rowfile_sync(h), "sync")
    finally:
        L.mpl_rowfile_close(h)
    arr[ids] = new
    np.testing.assert_array_equal(np.load(f), arr)


def test_rowfile_open_checks_size(tmp_path):
    f, off = _npy(tmp_path, np.zeros((10, 4), np.float32))
    h = ctypes.c_void_p()
    assert _lib.lib().mpl_rowfile_open(str(f).encode(), off, 16, 11, 0, ctypes.byref(h)) != 0
    assert _lib.lib().mpl_rowfile_open(str(tmp_path / "missing.npy").encode(), 0, 16, 1, 0, ctypes.byref(h)) != 0
