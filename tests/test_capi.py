"""The C-ABI library loads and exports every symbol include/quiver_hip.h declares."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    text = (ROOT / "include" / "quiver_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qv_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    from quiver import _lib

    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding declares a signature for each of them
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_search_defaults_follow_reference_cli():
    from quiver import _lib

    o = _lib.default_search_opts()
    # bin/quiver_search.cu:202-205 (gpruning 10/8), search.cu:980 (admit 32)
    assert (o.early_exit, o.gpruning_warmup, o.gpruning_patience) == (_lib.QV_EXIT_GPRUNING, 10, 8)
    assert o.admit_min_batch == 32 and o.prefeed == 0 and o.queries_per_block == 1
    p = _lib.default_build_params()
    assert (p.R, p.L, round(p.alpha, 3), p.num_chunks, p.kmeans_iters) == (64, 100, 1.2, 32, 15)


def test_open_errors_are_reported_not_thrown(tmp_path):
    from quiver import _lib

    lib = _lib.load()
    h = C.c_void_p()
    rc = lib.qv_index_open(str(tmp_path / "missing").encode(), b"uint8", b"heap", None, 0, C.byref(h))
    assert rc == _lib.QV_EIO and b"does not exist" in lib.qv_last_error()
    rc = lib.qv_index_open(str(tmp_path).encode(), b"complex64", b"heap", None, 0, C.byref(h))
    assert rc == _lib.QV_EINVAL and b"Unsupported data type" in lib.qv_last_error()
    rc = lib.qv_index_open(str(tmp_path).encode(), b"uint8", b"mmap", None, 0, C.byref(h))
    assert rc == _lib.QV_EIO  # no index files in an empty directory
    rc = lib.qv_index_open_ex(str(tmp_path).encode(), b"uint8", b"heap", None, 0, 7, C.byref(h))
    assert rc == _lib.QV_EINVAL and b"graph placement" in lib.qv_last_error()
    rc = lib.qv_index_open(str(tmp_path).encode(), b"uint8", b"disk", None, 0, C.byref(h))
    assert rc == _lib.QV_EINVAL
    lib.qv_index_close(None)  # accepted


def test_mmap_backend_checks_file_size(tmp_path):
    """--memory-backend mmap rejects an index file shorter than its pages, with
    the reference's message (mem_loader.cpp:63-71), before any device work."""
    import os

    import numpy as np
    from index_fixtures import exact_pq, write_index
    from quiver import _lib

    v = np.random.default_rng(0).integers(0, 256, (50, 8), dtype=np.uint8)
    piv, cen, off, codes = exact_pq(v)
    write_index(tmp_path / "t", v, [[(i + 1) % 50] for i in range(50)], 0, 4, piv, cen, off, codes)
    f = tmp_path / "t_disk.index"
    os.truncate(f, f.stat().st_size - 100)
    lib = _lib.load()
    h = C.c_void_p()
    rc = lib.qv_index_open(str(tmp_path).encode(), b"uint8", b"mmap", None, 0, C.byref(h))
    assert rc == _lib.QV_EIO
    assert b"is too small: size=8092 required=8192" in lib.qv_last_error()


def test_null_arguments_rejected():
    from quiver import _lib

    lib = _lib.load()
    assert lib.qv_search(None, None, 1, 1, 1, 1, None, None, None, None, None) == _lib.QV_EINVAL
    assert lib.qv_dev_copy(None, None, 16, 0) == _lib.QV_EINVAL


def test_cpu_builder_rejects_bad_params(tmp_path):
    import numpy as np
    import quiver
    from quiver import QuiverError

    base = np.zeros((10, 8), np.uint8)
    with pytest.raises(QuiverError, match="R must be"):
        quiver.build_index(base, tmp_path / "x", R=129, L=160)
    with pytest.raises(QuiverError, match="L must be"):
        quiver.build_index(base, tmp_path / "x", R=8, L=4)
