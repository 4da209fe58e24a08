"""On-disk formats and the host half of the setup path (CPU only)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

import qv_oracle as O
from index_fixtures import exact_pq, write_index


@pytest.fixture(scope="module")
def L():
    from quiver import _lib

    return _lib


def test_page_indexing_matches_reference_loader_fixture(tmp_path, L):
    # src/shared/io/mem_loader_test.cpp:22-79: a zero header page then pages
    # filled with 0x40 + k; page k of the image is file page k + 1.
    path = tmp_path / "disk.index"
    with path.open("wb") as f:
        f.write(bytes(4096))
        for k in range(3):
            f.write(bytes([0x40 + k]) * 4096)
    img = np.empty(3 * 4096, np.uint8)
    L.check(L.load().qv_read_index_pages(str(path).encode(), 3, img.ctypes.data))
    for k in range(3):
        assert (img[k * 4096:(k + 1) * 4096] == 0x40 + k).all()
    assert L.load().qv_read_index_pages(str(path).encode(), 4, img.ctypes.data) == L.QV_EIO
    assert b"Mem Index Load FAILED" in L.load().qv_last_error()


def test_discovery_symlink_and_fallbacks(tmp_path, L):
    # bin/common/search_setup_test.cpp:89-96 and index_discovery.hpp:57-103
    lib = L.load()
    idx = C.create_string_buffer(4096)
    pq = C.create_string_buffer(4096)
    d = tmp_path / "sym"
    d.mkdir()
    (d / "ann.index").write_bytes(bytes(8192))
    os.symlink(d / "ann.index", d / "deep1b_disk.index")
    (d / "deep1b_pq_pivots.bin").write_bytes(b"x")
    L.check(lib.qv_find_index_files(str(d).encode(), idx, pq, 4096))
    assert idx.value.decode() == str(d / "deep1b_disk.index")
    assert pq.value.decode() == str(d / "deep1b_pq")
    (d / "other_disk.index").write_bytes(b"")
    assert lib.qv_find_index_files(str(d).encode(), idx, pq, 4096) == L.QV_EIO
    assert b"Multiple *_disk.index" in lib.qv_last_error()
    f = tmp_path / "fallback"
    f.mkdir()
    (f / "disk.index").write_bytes(b"")
    (f / "pq_pivots.bin").write_bytes(b"")
    L.check(lib.qv_find_index_files(str(f).encode(), idx, pq, 4096))
    assert idx.value.decode() == str(f / "disk.index")
    assert pq.value.decode() == str(f / "pq")
    e = tmp_path / "empty"
    e.mkdir()
    assert lib.qv_find_index_files(str(e).encode(), idx, pq, 4096) == L.QV_EIO
    assert lib.qv_find_index_files(str(tmp_path / "nope").encode(), idx, pq, 4096) == L.QV_EIO


@pytest.mark.parametrize("dtype,dim,R", [(np.uint8, 128, 64), (np.float32, 96, 64), (np.int8, 16, 5)])
def test_metadata_layout(tmp_path, L, dtype, dim, R):
    rng = np.random.default_rng(9)
    n = 37
    if dtype == np.float32:
        vecs = rng.standard_normal((n, dim)).astype(np.float32)
    else:
        vecs = rng.integers(0, 100, (n, dim)).astype(dtype)
    adj = [[(v + 1) % n] for v in range(n)]
    pv, ce, co, _ = exact_pq(np.zeros((n, dim), np.uint8))
    write_index(tmp_path / "m", vecs, adj, 5, R, pv, ce, co, np.zeros((n, dim), np.uint8))
    info = L.IndexInfo()
    name = {np.uint8: b"uint8", np.float32: b"float", np.int8: b"int8"}[dtype]
    L.check(L.load().qv_read_layout(str(tmp_path / "m_disk.index").encode(), name, C.byref(info)))
    esz = np.dtype(dtype).itemsize
    assert (info.num_data, info.num_dims, info.enter_point) == (n, dim, 5)
    assert info.max_m0 == R  # (node_len - d*size)/4 - 1, metadata.hpp:49-50
    assert info.node_size == dim * esz + 4 + 4 * R
    assert info.nodes_per_page == 4096 // info.node_size
    assert info.num_pages == -(-n // info.nodes_per_page)
    host = O.HostIndex.from_files(tmp_path, name.decode())
    for v in range(n):
        np.testing.assert_array_equal(host.vector(v), vecs[v])
        np.testing.assert_array_equal(host.neighbors(v), adj[v])


def test_builder_files_round_trip(tmp_path):
    import quiver

    base = quiver.mixture(3000, 64, num_centers=16, seed=4)
    quiver.build_index(base, tmp_path / "b", R=24, L=40, num_chunks=16, threads=0)
    host = O.HostIndex.from_files(tmp_path, "uint8")
    assert host.n == 3000 and host.dim == 64 and host.R == 24 and host.M == 16
    np.testing.assert_array_equal(host.base(), base)
    mean = base.astype(np.float64).mean(0)
    d = ((base.astype(np.float64) - mean.astype(np.float32).astype(np.float64)) ** 2).sum(1)
    assert d[host.medoid] == d.min()
    for v in range(host.n):
        nb = host.neighbors(v)
        assert len(nb) <= 24 and len(set(nb.tolist())) == len(nb) and (nb < host.n).all() and v not in nb
    # codes are the nearest pivot of each centred sub-vector
    for v in range(0, 3000, 97):
        x = base[v].astype(np.float32) - host.centroid
        for m in range(16):
            o0, o1 = host.chunk_offsets[m], host.chunk_offsets[m + 1]
            dd = ((host.pivots[:, o0:o1] - x[o0:o1]) ** 2).sum(1)
            assert dd[host.codes[v, m]] == dd.min()


def test_mixture_generator_properties():
    import quiver

    a = quiver.mixture(500, 128, num_centers=8, seed=1)
    b = quiver.mixture(100, 128, num_centers=8, seed=1, first_row=400)
    np.testing.assert_array_equal(a[400:], b)          # rows depend only on their index
    assert a.dtype == np.uint8 and 60 < a.mean() < 200
    f = quiver.mixture(200, 96, data_type="float", num_centers=8, seed=2, sigma=1.0)
    np.testing.assert_allclose(np.linalg.norm(f.astype(np.float64), axis=1), 1.0, atol=1e-6)
