"""The neighbour code table (qv_index_neighbour_codes) changes only where a
hop reads its code rows: results with it must equal the oracle's (ids,
distances, found counts, hops) on the same cases as without it (runs on the
MI355X)."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import qv_oracle as O

pytestmark = pytest.mark.gpu
K = 10


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def opened(small_u8_index):
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    L = _lib.load()
    h = C.c_void_p()
    _lib.check(L.qv_index_open(str(small_u8_index["dir"]).encode(), b"uint8", b"heap", None, 0, C.byref(h)))
    _say("[gpu] building the neighbour code table")
    _lib.check(L.qv_index_neighbour_codes(h, 1))
    yield _lib, L, h, O.HostIndex.from_files(small_u8_index["dir"], "uint8"), small_u8_index
    L.qv_index_close(h)


def _search(lib, L, h, q, ef, policy, kernel, pipe):
    n = q.shape[0]
    ids = np.empty((n, K), np.int32)
    dists = np.empty((n, K), np.float32)
    found = np.empty(n, np.int32)
    hops = np.empty(n, np.int32)
    o = lib.default_search_opts()
    o.early_exit = lib.QV_EXIT_GPRUNING if policy == "gpruning" else lib.QV_EXIT_NONE
    o.pipe_width = pipe
    o.kernel = lib.KERNEL_NAMES[kernel]
    o.num_blocks = 256
    lib.check(L.qv_search(h, q.ctypes.data, n, q.shape[1], K, ef, C.byref(o), ids.ctypes.data, dists.ctypes.data,
                          found.ctypes.data, None))
    lib.check(L.qv_last_hops(h, hops.ctypes.data, n))
    return ids, dists, found, hops


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
@pytest.mark.parametrize("pipe", [1, 2])
@pytest.mark.parametrize("policy", ["none", "gpruning"])
@pytest.mark.parametrize("ef", [24, 100, 300, 700])
def test_with_neighbour_codes_matches_oracle(opened, ef, policy, pipe, kernel):
    lib, L, h, host, ix = opened
    q = np.ascontiguousarray(ix["queries"], np.float32)
    _say(f"[gpu] neighbour codes ef={ef} policy={policy} pipe={pipe} kernel={kernel}")
    got = _search(lib, L, h, q, ef, policy, kernel, pipe)
    want = O.search(host, q, K, ef, pipe_width=pipe,
                    early_exit=O.EXIT_GPRUNING if policy == "gpruning" else O.EXIT_NONE)
    for g, w, what in zip(got, want, ("ids", "dists", "found", "hops")):
        np.testing.assert_array_equal(g, w, err_msg=what)


def test_table_can_be_dropped_and_rebuilt(opened):
    lib, L, h, host, ix = opened
    q = np.ascontiguousarray(ix["queries"][:64], np.float32)
    with_table = _search(lib, L, h, q, 64, "none", "shared-pivots", 1)
    lib.check(L.qv_index_neighbour_codes(h, 0))
    without = _search(lib, L, h, q, 64, "none", "shared-pivots", 1)
    lib.check(L.qv_index_neighbour_codes(h, 1))
    for a, b in zip(with_table, without):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
def test_float_index_with_neighbour_codes(small_f32_index, kernel):
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    L = _lib.load()
    h = C.c_void_p()
    _lib.check(L.qv_index_open(str(small_f32_index["dir"]).encode(), b"float", b"heap", None, 0, C.byref(h)))
    try:
        _lib.check(L.qv_index_neighbour_codes(h, 1))  # M = 48 rows of 48 bytes
        q = np.ascontiguousarray(small_f32_index["queries"], np.float32)
        _say(f"[gpu] neighbour codes float kernel={kernel}")
        got = _search(_lib, L, h, q, 90, "none", kernel, 1)
        want = O.search(O.HostIndex.from_files(small_f32_index["dir"], "float"), q, K, 90, early_exit=O.EXIT_NONE)
        for g, w, what in zip(got, want, ("ids", "dists", "found", "hops")):
            np.testing.assert_array_equal(g, w, err_msg=what)
    finally:
        L.qv_index_close(h)
