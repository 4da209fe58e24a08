"""Indexes of max degree up to 128 and beams of up to 2048 entries on the GPU,
against the oracle: ids, distances, found counts and hop counts identical
(runs on the MI355X).

* R = 128 (the reference's own index layouts are R = 128, ae/scripts/
  common.sh:118-121): two neighbour slots per lane.  A CPU-built uint8 index
  (d = 128, M = 32) and float index (d = 96, M = 48), both kernels, pipe
  widths 1 and 2, gpruning and none, ef from 30 (the reference's dedicated
  R = 128, ef = 30 merge, kernel_helpers.cuh:188-230, which yields the generic
  merge's result) to 800; the star of degree 128 whose answers are derived
  by hand in test_oracle_wide.py.
* ef in (448, 1024] (Q = 10 and 16 beam positions per lane) on the R = 32
  and R = 64 fixtures and on the R = 128 index; ef in (1024, 2048] (Q = 32,
  per-query-LUT kernel only) on the uint8, float and R = 128 indexes.
* The ef limits: 2048 overall, 1024 for a forced shared-pivot search.
* Graph validation at open on R = 128 records (slots 64..127).
"""
from __future__ import annotations

import ctypes as C
import struct
import sys

import numpy as np
import pytest

import qv_oracle as O
from index_fixtures import exact_pq, write_index

pytestmark = pytest.mark.gpu
K = 10


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    return _lib


class Opened:
    def __init__(self, lib, directory, dtype):
        self.lib, self.L = lib, lib.load()
        self.h = C.c_void_p()
        lib.check(self.L.qv_index_open(str(directory).encode(), dtype.encode(), b"heap", None, 0, C.byref(self.h)))
        self.host = O.HostIndex.from_files(directory, dtype)

    def search(self, q, ef, policy="none", kernel="auto", pipe=1, k=K):
        n, dim = q.shape
        ids = np.empty((n, k), np.int32)
        dists = np.empty((n, k), np.float32)
        found = np.empty(n, np.int32)
        hops = np.empty(n, np.int32)
        o = self.lib.default_search_opts()
        o.early_exit = self.lib.QV_EXIT_GPRUNING if policy == "gpruning" else self.lib.QV_EXIT_NONE
        o.pipe_width = pipe
        o.kernel = self.lib.KERNEL_NAMES[kernel]
        o.num_blocks = 256
        rep = self.lib.SearchReport()
        qq = np.ascontiguousarray(q, np.float32)
        self.lib.check(self.L.qv_search(self.h, qq.ctypes.data, n, dim, k, ef, C.byref(o), ids.ctypes.data,
                                        dists.ctypes.data, found.ctypes.data, C.byref(rep)))
        self.lib.check(self.L.qv_last_hops(self.h, hops.ctypes.data, n))
        return ids, dists, found, hops, rep

    def close(self):
        self.L.qv_index_close(self.h)


def _same(got, want, what):
    ids, dists, found, hops = got[:4]
    oids, odists, ofound, ohops = want
    bad = np.nonzero(np.any(ids != oids, axis=1))[0]
    assert bad.size == 0, f"{what}: {bad.size} queries with other ids, first {bad[:5]}"
    np.testing.assert_array_equal(dists, odists, err_msg=what)
    np.testing.assert_array_equal(found, ofound, err_msg=what)
    np.testing.assert_array_equal(hops, ohops, err_msg=what)


def _policy(p):
    return O.EXIT_GPRUNING if p == "gpruning" else O.EXIT_NONE


def _degrees(host):
    v = np.arange(host.n)
    off = (v // host.npp) * 4096 + (v % host.npp) * host.node_size + host.data_size
    return host.pages.view(np.uint8)[off[:, None] + np.arange(4)].copy().view("<u4").ravel()


@pytest.fixture(scope="module")
def r128_u8(tmp_path_factory, lib):
    import quiver

    d = tmp_path_factory.mktemp("r128u8")
    base = quiver.mixture(12000, 128, num_centers=48, seed=0x128)
    q = quiver.mixture(240, 128, num_centers=48, seed=0x128, first_row=10**7).astype(np.float32)
    _say("[gpu] building the R=128 uint8 index on the CPU")
    quiver.build_index(base, d / "r128", R=128, L=160, num_chunks=32, threads=0)
    ix = Opened(lib, d, "uint8")
    assert ix.host.R == 128 and _degrees(ix.host).max() > 64  # second slots are used
    yield ix, q
    ix.close()


@pytest.fixture(scope="module")
def r128_f32(tmp_path_factory, lib):
    import quiver

    d = tmp_path_factory.mktemp("r128f32")
    base = quiver.mixture(5000, 96, data_type="float", num_centers=32, seed=0x129, sigma=1.0)
    q = quiver.mixture(160, 96, data_type="float", num_centers=32, seed=0x129, sigma=1.0, first_row=10**7)
    _say("[gpu] building the R=128 float index on the CPU")
    quiver.build_index(base, d / "r128f", R=128, L=160, num_chunks=48, threads=0)
    ix = Opened(lib, d, "float")
    assert ix.host.R == 128 and _degrees(ix.host).max() > 64
    yield ix, np.ascontiguousarray(q, np.float32)
    ix.close()


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
@pytest.mark.parametrize("policy", ["none", "gpruning"])
@pytest.mark.parametrize("ef", [30, 64, 200, 448, 800])
def test_r128_u8_matches_oracle(r128_u8, ef, policy, kernel):
    ix, q = r128_u8
    _say(f"[gpu] R=128 u8 ef={ef} policy={policy} kernel={kernel}")
    got = ix.search(q, ef, policy, kernel)
    assert got[4].kernel == ix.lib.KERNEL_NAMES[kernel]
    _same(got, O.search(ix.host, q, K, ef, early_exit=_policy(policy)), f"R=128 u8 ef={ef} {policy} {kernel}")


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
@pytest.mark.parametrize("pipe", [2, 4])
def test_r128_pipe_lanes(r128_u8, pipe, kernel):
    ix, q = r128_u8
    _say(f"[gpu] R=128 u8 pipe={pipe} kernel={kernel}")
    got = ix.search(q, 100, "gpruning", kernel, pipe)
    _same(got, O.search(ix.host, q, K, 100, pipe_width=pipe, early_exit=O.EXIT_GPRUNING),
          f"R=128 pipe {pipe} {kernel}")


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
@pytest.mark.parametrize("ef", [40, 300, 600])
def test_r128_f32_matches_oracle(r128_f32, ef, kernel):
    ix, q = r128_f32
    _say(f"[gpu] R=128 f32 ef={ef} kernel={kernel}")
    got = ix.search(q, ef, "none", kernel)
    _same(got, O.search(ix.host, q, K, ef, early_exit=O.EXIT_NONE), f"R=128 f32 ef={ef} {kernel}")


@pytest.mark.parametrize("ef", [64, 128, 200, 1000])
def test_star_of_degree_128(lib, tmp_path, ef):
    rng = np.random.default_rng(128)
    vecs = np.empty((129, 4), np.uint8)
    vecs[0] = 200
    vecs[1:] = 100 + rng.integers(-12, 13, size=(128, 4))
    adj = [list(range(1, 129))] + [[0] for _ in range(128)]
    write_index(tmp_path / "star", vecs, adj, 0, 128, *exact_pq(vecs))
    ix = Opened(lib, tmp_path, "uint8")
    try:
        q = np.full((3, 4), 100, np.float32)
        q[1] += 3
        q[2] -= 5
        _say(f"[gpu] star of degree 128 ef={ef}")
        _same(ix.search(q, ef, "none", "lut"), O.search(ix.host, q, K, ef, early_exit=O.EXIT_NONE),
              f"star ef={ef}")
    finally:
        ix.close()


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
@pytest.mark.parametrize("policy", ["none", "gpruning"])
@pytest.mark.parametrize("ef", [449, 640, 641, 1024])
def test_deep_beam_u8(lib, small_u8_index, ef, policy, kernel):
    ix = Opened(lib, small_u8_index["dir"], "uint8")
    try:
        q = small_u8_index["queries"].astype(np.float32)
        _say(f"[gpu] deep beam u8 ef={ef} policy={policy} kernel={kernel}")
        got = ix.search(q, ef, policy, kernel)
        assert got[4].kernel == ix.lib.KERNEL_NAMES[kernel]
        _same(got, O.search(ix.host, q, K, ef, early_exit=_policy(policy)), f"deep u8 ef={ef} {policy} {kernel}")
    finally:
        ix.close()


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
@pytest.mark.parametrize("ef", [500, 1024])
def test_deep_beam_f32(lib, small_f32_index, ef, kernel):
    ix = Opened(lib, small_f32_index["dir"], "float")
    try:
        q = np.ascontiguousarray(small_f32_index["queries"], np.float32)
        _say(f"[gpu] deep beam f32 ef={ef} kernel={kernel}")
        _same(ix.search(q, ef, "none", kernel), O.search(ix.host, q, K, ef, early_exit=O.EXIT_NONE),
              f"deep f32 ef={ef} {kernel}")
    finally:
        ix.close()


@pytest.mark.parametrize("policy", ["none", "gpruning"])
@pytest.mark.parametrize("ef", [1025, 1500, 2048])
def test_xl_beam_u8(lib, small_u8_index, ef, policy):
    """ef in (1024, 2048] (the reference sizes its frontier from ef,
    search.cu:391): 32 beam positions per lane in the per-query-LUT kernel,
    which `auto` takes; pipe widths 1 and 2, and a top-100 at ef = 1500."""
    ix = Opened(lib, small_u8_index["dir"], "uint8")
    try:
        q = small_u8_index["queries"][:120].astype(np.float32)
        for pipe in (1, 2):
            _say(f"[gpu] xl beam u8 ef={ef} policy={policy} W={pipe}")
            got = ix.search(q, ef, policy, "auto", pipe=pipe)
            assert got[4].kernel == ix.lib.KERNEL_NAMES["lut"]
            _same(got, O.search(ix.host, q, K, ef, pipe_width=pipe, early_exit=_policy(policy)),
                  f"xl u8 ef={ef} {policy} W={pipe}")
        if ef == 1500:
            _say(f"[gpu] xl beam u8 ef={ef} policy={policy} topk=100")
            _same(ix.search(q, ef, policy, "auto", k=100), O.search(ix.host, q, 100, ef, early_exit=_policy(policy)),
                  f"xl u8 ef={ef} {policy} topk=100")
    finally:
        ix.close()


def test_xl_beam_f32_and_r128(lib, small_f32_index, r128_u8):
    q = np.ascontiguousarray(small_f32_index["queries"][:100], np.float32)
    ix = Opened(lib, small_f32_index["dir"], "float")
    try:
        _say("[gpu] xl beam f32 ef=2048")
        _same(ix.search(q, 2048, "none"), O.search(ix.host, q, K, 2048, early_exit=O.EXIT_NONE), "xl f32 ef=2048")
    finally:
        ix.close()
    ix, q = r128_u8
    _say("[gpu] xl beam R=128 u8 ef=1200")
    _same(ix.search(q[:100], 1200, "gpruning"), O.search(ix.host, q[:100], K, 1200, early_exit=O.EXIT_GPRUNING),
          "xl R=128 ef=1200")


def test_wide_topk_r128_and_float(lib, small_f32_index, r128_u8):
    """A top-k above 64 (entries past the 64th in LDS) with two neighbour
    slots per lane and with 2-dim PQ chunks."""
    ix, q = r128_u8
    _say("[gpu] R=128 u8 topk=100 ef=300 W=2 gpruning")
    _same(ix.search(q[:120], 300, "gpruning", pipe=2, k=100),
          O.search(ix.host, q[:120], 100, 300, pipe_width=2, early_exit=O.EXIT_GPRUNING), "R=128 topk=100")
    qf = np.ascontiguousarray(small_f32_index["queries"][:100], np.float32)
    fx = Opened(lib, small_f32_index["dir"], "float")
    try:
        _say("[gpu] float topk=80 ef=200")
        _same(fx.search(qf, 200, "none", k=80), O.search(fx.host, qf, 80, 200, early_exit=O.EXIT_NONE),
              "float topk=80")
    finally:
        fx.close()


def test_ef_limits(lib, small_u8_index):
    """ef above 2048 is rejected; a forced shared-pivot search above 1024 is
    unsupported (its beams stop at 1024)."""
    ix = Opened(lib, small_u8_index["dir"], "uint8")
    try:
        q = small_u8_index["queries"][:4].astype(np.float32)
        with pytest.raises(lib.QuiverError, match=r"ef_search must be in \[1, 2048\]"):
            ix.search(q, 2049)
        with pytest.raises(lib.QuiverError, match=r"beams of at most 1024"):
            ix.search(q, 1025, kernel="shared-pivots")
    finally:
        ix.close()


@pytest.mark.parametrize("slot,value,what", [(100, None, "duplicate"), (127, 10**6, "range")])
def test_r128_graph_validation(lib, tmp_path, slot, value, what):
    rng = np.random.default_rng(7)
    n = 300
    vecs = rng.integers(0, 256, size=(n, 4)).astype(np.uint8)
    adj = [sorted({(v + 1 + j) % n for j in range(128)}) for v in range(n)]
    write_index(tmp_path / "bad", vecs, adj, 0, 128, *exact_pq(vecs))
    path = tmp_path / "bad_disk.index"
    raw = bytearray(path.read_bytes())
    node_size = 4 + 4 + 4 * 128
    npp = 4096 // node_size
    v = 5
    off = 4096 * (1 + v // npp) + (v % npp) * node_size + 4 + 4 * (1 + slot)
    bad = adj[v][3] if value is None else value  # repeats slot 3's id, or points past the graph
    struct.pack_into("<I", raw, off, bad)
    path.write_bytes(bytes(raw))
    L = lib.load()
    h = C.c_void_p()
    _say(f"[gpu] R=128 validation: {what} in slot {slot}")
    rc = L.qv_index_open(str(tmp_path).encode(), b"uint8", b"heap", None, 0, C.byref(h))
    if rc == 0:
        L.qv_index_close(h)
    assert rc == lib.QV_EINDEX
