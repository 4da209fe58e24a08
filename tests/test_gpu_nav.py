"""Nav-graph entry on the MI355X vs the oracle: each query's entry node comes
from the in-kernel nav search (inkernel_nav_entry,
src/quiver/kernel_core/inkernel_nav.cuh:61-200), then the beam search runs
from it.  Ids, distances, found counts and hop counts must equal the oracle's
(the hop count changes with the entry node, so it checks the entry too)."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import qv_oracle as O
from index_fixtures import write_nav

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    return _lib


def _gpu_search(ix, nav_dir, ef, *, policy="none", pipe_width=1, skip_nav=False, dtype=b"uint8",
                q=None):
    from quiver import _lib

    L = _lib.load()
    h = C.c_void_p()
    _lib.check(L.qv_index_open(str(ix["dir"]).encode(), dtype, b"heap", None, 0, C.byref(h)))
    try:
        if nav_dir is not None:
            _lib.check(L.qv_index_load_nav(h, str(nav_dir).encode()))
        info = _lib.IndexInfo()
        _lib.check(L.qv_index_get_info(h, C.byref(info)))
        q = np.ascontiguousarray(ix["queries"] if q is None else q, dtype=np.float32)
        n, dim = q.shape
        ids = np.empty((n, 10), np.int32)
        dists = np.empty((n, 10), np.float32)
        found = np.empty(n, np.int32)
        hops = np.empty(n, np.int32)
        opts = _lib.default_search_opts()
        opts.pipe_width = pipe_width
        opts.early_exit = _lib.QV_EXIT_GPRUNING if policy == "gpruning" else _lib.QV_EXIT_NONE
        opts.skip_nav = 1 if skip_nav else 0
        rep = _lib.SearchReport()
        _lib.check(L.qv_search(h, q.ctypes.data, n, dim, 10, ef, C.byref(opts), ids.ctypes.data,
                               dists.ctypes.data, found.ctypes.data, C.byref(rep)))
        _lib.check(L.qv_last_hops(h, hops.ctypes.data, n))
    finally:
        L.qv_index_close(h)
    return ids, dists, found, hops, info


def _check(ix, nav_dir, ef, data_type="uint8", **kw):
    ids, dists, found, hops, info = _gpu_search(ix, nav_dir, ef, dtype=data_type.encode(), **kw)
    host = O.HostIndex.from_files(ix["dir"], data_type)
    nav = None if (nav_dir is None or kw.get("skip_nav")) else O.HostNav.from_dir(nav_dir, data_type)
    q = np.ascontiguousarray(ix["queries"] if kw.get("q") is None else kw["q"], np.float32)
    oids, odists, ofound, ohops = O.search(
        host, q, 10, ef, pipe_width=kw.get("pipe_width", 1),
        early_exit=O.EXIT_GPRUNING if kw.get("policy") == "gpruning" else O.EXIT_NONE, nav=nav)
    mism = np.nonzero(np.any(ids != oids, axis=1))[0]
    assert mism.size == 0, f"{mism.size} queries differ, first {mism[:5]}"
    np.testing.assert_array_equal(dists, odists)
    np.testing.assert_array_equal(found, ofound)
    np.testing.assert_array_equal(hops, ohops)
    return hops, ohops, info


@pytest.fixture(scope="module")
def u8_nav(small_u8_index, tmp_path_factory):
    import quiver

    base = small_u8_index["base"]
    sample = np.arange(3, base.shape[0], 10, dtype=np.int32)
    d = tmp_path_factory.mktemp("nav_u8") / "nav"
    quiver.build_nav(base[sample], sample, d, R=28, L=64, threads=0)
    return d


@pytest.mark.parametrize("pipe_width", [1, 4])
@pytest.mark.parametrize("policy", ["none", "gpruning"])
@pytest.mark.parametrize("ef", [32, 100, 256])
def test_nav_entry_u8_matches_oracle(lib, small_u8_index, u8_nav, pipe_width, policy, ef):
    _say(f"[gpu] nav u8 pipe_width={pipe_width} policy={policy} ef={ef}")
    hops, _, info = _check(small_u8_index, u8_nav, ef, pipe_width=pipe_width, policy=policy)
    assert info.nav_nodes == 2000 and info.nav_max_m == 28


def test_skip_nav_is_the_medoid_path(lib, small_u8_index, u8_nav):
    _say("[gpu] nav loaded, skip_nav")
    _check(small_u8_index, u8_nav, 64, skip_nav=True)


def test_nav_entry_reduces_hops(lib, small_u8_index, u8_nav):
    _say("[gpu] nav hop reduction")
    with_nav, _, _ = _check(small_u8_index, u8_nav, 64)
    without, _, _ = _check(small_u8_index, None, 64)
    assert with_nav.mean() < without.mean()


def test_nav_entry_f32_matches_oracle(lib, small_f32_index, tmp_path):
    import quiver

    base = small_f32_index["base"]
    sample = np.arange(0, base.shape[0], 8, dtype=np.int32)
    quiver.build_nav(base[sample], sample, tmp_path / "nav", R=28, L=48, threads=0)
    _say("[gpu] nav f32 ef=64")
    _check(small_f32_index, tmp_path / "nav", 64, data_type="float")


def test_hand_nav_graphs(lib, small_u8_index, tmp_path):
    """Hand graphs whose entry behaviour the oracle's known-answer tests fix:
    a complete graph, rows narrower than the 28 reads (spill into later rows),
    and a one-node self loop whose queue ends with slot 0 empty (entry falls
    back to the medoid)."""
    base = small_u8_index["base"]
    rng = np.random.default_rng(17)
    cases = []
    ids = rng.choice(base.shape[0], 29, replace=False).astype(np.int32)
    g = np.full((29, 28), -1, np.int32)
    for i in range(29):
        g[i, :28] = [j for j in range(29) if j != i]
    cases.append(("complete29", ids, g, 5))
    ids = rng.choice(base.shape[0], 40, replace=False).astype(np.int32)
    g = np.full((40, 4), -1, np.int32)
    for i in range(40):
        deg = 1 + i % 4
        g[i, :deg] = rng.choice([j for j in range(40) if j != i], deg, replace=False)
    cases.append(("narrow40", ids, g, 0))
    cases.append(("selfloop1", np.array([123], np.int32), np.array([[0, -1]], np.int32), 0))
    for name, nid, graph, start in cases:
        d = tmp_path / name
        write_nav(d, base[nid], graph, nid, start)
        _say(f"[gpu] hand nav {name}")
        _check(small_u8_index, d, 64)
