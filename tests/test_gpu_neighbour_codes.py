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
@pytest.mark.parametrize("pipe", [1, 2, 4])
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


@pytest.mark.parametrize("dim,R,msg", [(4, 8, "M = 32 or 48"), (16, 8, "M = 32 or 48"), (64, 8, "M = 32 or 48"),
                                       (32, 128, "R <= 64")])
def test_unsupported_shapes_are_refused(tmp_path, dim, R, msg):
    from index_fixtures import exact_pq, write_index
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    rng = np.random.default_rng(dim)
    n = 200
    vecs = rng.integers(0, 256, size=(n, dim)).astype(np.uint8)
    adj = [sorted({(v + 1 + j) % n for j in range(R)}) for v in range(n)]
    write_index(tmp_path / "x", vecs, adj, 0, R, *exact_pq(vecs))  # M = dim one-dimension chunks
    L = _lib.load()
    h = C.c_void_p()
    _lib.check(L.qv_index_open(str(tmp_path).encode(), b"uint8", b"heap", None, 0, C.byref(h)))
    try:
        _say(f"[gpu] neighbour codes refused: M={dim} R={R}")
        assert L.qv_index_neighbour_codes(h, 1) == _lib.QV_EUNSUPPORTED
        assert msg in L.qv_last_error().decode()
        # the handle still searches, without the table
        q = vecs[:8].astype(np.float32)
        got = _search(_lib, L, h, q, 32, "none", "lut", 1)
        want = O.search(O.HostIndex.from_files(tmp_path, "uint8"), q, K, 32, early_exit=O.EXIT_NONE)
        for g, w, what in zip(got, want, ("ids", "dists", "found", "hops")):
            np.testing.assert_array_equal(g, w, err_msg=what)
    finally:
        L.qv_index_close(h)


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
def test_python_api_option(small_u8_index, kernel):
    import quiver

    ix = small_u8_index
    _say(f"[gpu] IndexQuiver(neighbour_codes=True) kernel={kernel}")
    index = quiver.IndexQuiver(ix["dir"], data_type="uint8", pipe_width=1, num_blocks=256, search_kernel=kernel,
                               neighbour_codes=True)
    try:
        ids, dists = index.search(ix["queries"], topk=K, ef_search=120, early_exit_policy="none")
    finally:
        index.close()
    oids, odists, _, _ = O.search(O.HostIndex.from_files(ix["dir"], "uint8"), ix["queries"].astype(np.float32), K,
                                  120, early_exit=O.EXIT_NONE)
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(dists, odists)


def test_cli_flag(small_u8_index, tmp_path):
    import struct
    import subprocess
    from pathlib import Path

    cli = Path(__file__).resolve().parents[1] / "quiver-ae_amd" / "bin" / "quiver_search"
    if not cli.is_file():
        pytest.fail(f"{cli} not built")
    ix = small_u8_index
    q = ix["queries"][:100]
    qf = tmp_path / "q.u8bin"
    qf.write_bytes(struct.pack("<ii", *q.shape) + q.tobytes())
    _say("[gpu] CLI --neighbour-codes")
    r = subprocess.run([str(cli), "--index-dir", str(ix["dir"]), "--query", str(qf), "--data-type", "uint8",
                        "--ef-search", "80", "--repeat", "1", "--pipe-width", "1", "--early-exit-policy", "none",
                        "--search-kernel", "shared-pivots", "--neighbour-codes", "--result-prefix",
                        str(tmp_path / "res")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    ids = np.fromfile(tmp_path / "res_ids.bin", dtype="<i4")
    assert tuple(ids[:2]) == (100, 10)
    oids, _, _, _ = O.search(O.HostIndex.from_files(ix["dir"], "uint8"), q.astype(np.float32), K, 80,
                             early_exit=O.EXIT_NONE)
    np.testing.assert_array_equal(ids[2:].reshape(100, 10), oids)
