"""HIP path vs the oracle on the same seeded inputs (runs on the MI355X).

Bars: bit-exact ids, PQ/exact distances for uint8; float within the 1e-5
relative tolerance of the task (the float path mirrors the reference's
summation order, so it is expected to be bit-exact too and is asserted so
first, with the tolerance as the documented bar).
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import qv_oracle as O

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


KERNELS = {"lut": 1, "shared-pivots": 2}


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
@pytest.mark.parametrize("pipe_width", [1, 2, 4])
@pytest.mark.parametrize("policy", ["none", "gpruning"])
@pytest.mark.parametrize("ef", [24, 64, 100, 150, 200, 300, 350, 448])
def test_search_u8_bit_exact(lib, small_u8_index, pipe_width, policy, ef, kernel):
    import quiver

    ix = small_u8_index
    _say(f"[gpu] search u8 kernel={kernel} pipe_width={pipe_width} policy={policy} ef={ef}")
    index = quiver.IndexQuiver(ix["dir"], data_type="uint8", pipe_width=pipe_width, num_blocks=512,
                               search_kernel=kernel)
    ids, dists = index.search(ix["queries"], topk=10, ef_search=ef, early_exit_policy=policy)
    assert index.last_report["kernel"] == KERNELS[kernel]
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, odists, ofound, ohops = O.search(
        host, ix["queries"].astype(np.float32), 10, ef, pipe_width=pipe_width,
        early_exit=O.EXIT_GPRUNING if policy == "gpruning" else O.EXIT_NONE)
    index.close()
    mism = np.nonzero(np.any(ids != oids, axis=1))[0]
    assert mism.size == 0, f"{mism.size} queries differ, first {mism[:5]}"
    np.testing.assert_array_equal(dists, odists)
    assert abs(O.recall(ids, ix["gt"], 10) - O.recall(oids, ix["gt"], 10)) <= 0.002


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
@pytest.mark.parametrize("pipe_width", [1, 2])
@pytest.mark.parametrize("ef", [32, 90])
def test_search_f32(lib, small_f32_index, pipe_width, ef, kernel):
    import quiver

    ix = small_f32_index
    _say(f"[gpu] search f32 kernel={kernel} pipe_width={pipe_width} ef={ef}")
    index = quiver.IndexQuiver(ix["dir"], data_type="float32", pipe_width=pipe_width, num_blocks=256,
                               search_kernel=kernel)
    ids, dists = index.search(ix["queries"], topk=10, ef_search=ef, early_exit_policy="none")
    assert index.last_report["kernel"] == KERNELS[kernel]
    host = O.HostIndex.from_files(ix["dir"], "float")
    oids, odists, _, _ = O.search(host, ix["queries"], 10, ef, pipe_width=pipe_width,
                                  early_exit=O.EXIT_NONE)
    index.close()
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_allclose(dists, odists, rtol=1e-5, atol=0)
    np.testing.assert_array_equal(dists, odists)


@pytest.fixture(scope="module")
def small_i8_index(tmp_path_factory):
    """6k x 128 int8 (the uint8 mixture shifted by -128), M = 32."""
    import quiver

    d = tmp_path_factory.mktemp("i8")
    base = (quiver.mixture(6000, 128, num_centers=32, seed=21).astype(np.int16) - 128).astype(np.int8)
    queries = (quiver.mixture(150, 128, num_centers=32, seed=21, first_row=10**6).astype(np.int16)
               - 128).astype(np.int8)
    quiver.build_index(base, d / "i8", R=32, L=48, num_chunks=32, threads=0)
    return {"dir": d, "queries": queries}


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
@pytest.mark.parametrize("policy", ["none", "gpruning"])
@pytest.mark.parametrize("ef", [64, 200])
def test_search_i8_bit_exact(lib, small_i8_index, kernel, policy, ef):
    """Signed 8-bit vectors (exact distances on sign-extended elements) through
    both kernels, against the oracle."""
    import quiver

    ix = small_i8_index
    _say(f"[gpu] search i8 kernel={kernel} policy={policy} ef={ef}")
    index = quiver.IndexQuiver(ix["dir"], data_type="int8", pipe_width=1, num_blocks=512, search_kernel=kernel)
    ids, dists = index.search(ix["queries"], topk=10, ef_search=ef, early_exit_policy=policy)
    assert index.last_report["kernel"] == KERNELS[kernel]
    index.close()
    host = O.HostIndex.from_files(ix["dir"], "int8")
    oids, odists, _, _ = O.search(host, ix["queries"].astype(np.float32), 10, ef,
                                  early_exit=O.EXIT_GPRUNING if policy == "gpruning" else O.EXIT_NONE)
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(dists, odists)


@pytest.fixture(scope="module")
def uneven_u8_index(tmp_path_factory):
    """3k x 100 uint8, M = 32: PQ chunks of 3 and 4 dims."""
    import quiver

    d = tmp_path_factory.mktemp("uneven")
    base = quiver.mixture(3000, 100, num_centers=16, seed=11)
    queries = quiver.mixture(120, 100, num_centers=16, seed=11, first_row=10**6)
    quiver.build_index(base, d / "u", R=24, L=40, num_chunks=32, threads=0)
    return {"dir": d, "queries": queries}


def test_uneven_chunks_take_the_lut_kernel(lib, uneven_u8_index):
    """Chunks of unequal width: auto picks the per-query LUT kernel (bit-exact
    against the oracle) and a forced shared-pivot search is refused."""
    import quiver
    from quiver._lib import QuiverError

    ix = uneven_u8_index
    _say("[gpu] uneven chunks auto + forced shared-pivots")
    index = quiver.IndexQuiver(ix["dir"], data_type="uint8", pipe_width=1, num_blocks=128)
    ids, dists = index.search(ix["queries"], topk=10, ef_search=64, early_exit_policy="none")
    assert index.last_report["kernel"] == KERNELS["lut"]
    index.close()
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, odists, _, _ = O.search(host, ix["queries"].astype(np.float32), 10, 64, early_exit=O.EXIT_NONE)
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(dists, odists)
    forced = quiver.IndexQuiver(ix["dir"], data_type="uint8", pipe_width=1, num_blocks=128,
                                search_kernel="shared-pivots")
    with pytest.raises(QuiverError, match="shared-pivot kernel needs"):
        forced.search(ix["queries"], topk=10, ef_search=64, early_exit_policy="none")
    forced.close()


def test_auto_kernel_follows_queries_in_flight(lib, small_u8_index):
    """Auto takes the per-query LUT kernel while its resident slots (4 per CU
    at ef = 64: 1024 on 256 CUs) hold every query the call can have in flight,
    and the shared-pivot kernel (8 per CU) beyond that; answers are the
    oracle's either way."""
    import quiver

    ix = small_u8_index
    q8 = np.ascontiguousarray(np.concatenate([ix["queries"]] * 8))  # 2400 queries
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, odists, _, _ = O.search(host, q8.astype(np.float32), 10, 64, early_exit=O.EXIT_NONE)
    # num_blocks 4096: more slots than the device holds (the launch stops at capacity)
    for nq, num_blocks, want in ((300, 4096, "lut"), (2400, 4096, "shared-pivots"), (2400, 512, "lut")):
        _say(f"[gpu] auto kernel nq={nq} num_blocks={num_blocks}")
        index = quiver.IndexQuiver(ix["dir"], data_type="uint8", pipe_width=1, num_blocks=num_blocks)
        ids, dists = index.search(q8[:nq], topk=10, ef_search=64, early_exit_policy="none")
        assert index.last_report["kernel"] == KERNELS[want], (nq, num_blocks)
        # slots launched: no more than the queries (whole workgroups of at most 16 waves)
        assert min(nq, num_blocks) <= index.last_report["num_blocks"] < min(nq, num_blocks) + 16
        index.close()
        np.testing.assert_array_equal(ids, oids[:nq])
        np.testing.assert_array_equal(dists, odists[:nq])


def test_search_batch_admission_and_hops(lib, small_u8_index):
    """Whole-batch admission gives the same answers; hop counts match the oracle."""
    from quiver import _lib

    ix = small_u8_index
    _say("[gpu] batch admission + hops")
    h = C.c_void_p()
    _lib.check(_lib.load().qv_index_open(str(ix["dir"]).encode(), b"uint8", b"heap", None, 0, C.byref(h)))
    q = np.ascontiguousarray(ix["queries"], dtype=np.float32)
    n = q.shape[0]
    ids = np.empty((n, 10), np.int32)
    dists = np.empty((n, 10), np.float32)
    found = np.empty(n, np.int32)
    hops = np.empty(n, np.int32)
    opts = _lib.default_search_opts()
    opts.admission = _lib.QV_ADMIT_BATCH
    opts.early_exit = _lib.QV_EXIT_NONE
    rep = _lib.SearchReport()
    _lib.check(_lib.load().qv_search(h, q.ctypes.data, n, 128, 10, 64, C.byref(opts), ids.ctypes.data,
                                     dists.ctypes.data, found.ctypes.data, C.byref(rep)))
    _lib.check(_lib.load().qv_last_hops(h, hops.ctypes.data, n))
    _lib.load().qv_index_close(h)
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, odists, ofound, ohops = O.search(host, q, 10, 64, early_exit=O.EXIT_NONE)
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(found, ofound)
    np.testing.assert_array_equal(hops, ohops)
    assert rep.qps > 0 and rep.lat_p99_ms >= rep.lat_p50_ms > 0


@pytest.mark.parametrize("backend,placement", [("mmap", "hbm"), ("heap", "host"), ("mmap", "host")])
def test_backends_and_graph_placement(lib, small_u8_index, backend, placement):
    """The mmap backend and the page image in pinned host memory give the
    oracle's answers, hop for hop."""
    import quiver

    ix = small_u8_index
    _say(f"[gpu] backend={backend} placement={placement}")
    index = quiver.IndexQuiver(ix["dir"], data_type="uint8", pipe_width=1, num_blocks=512,
                               memory_backend=backend, graph_placement=placement)
    ids, dists = index.search(ix["queries"], topk=10, ef_search=100, early_exit_policy="none")
    info = index.info()
    index.close()
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, odists, _, _ = O.search(host, ix["queries"].astype(np.float32), 10, 100, early_exit=O.EXIT_NONE)
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(dists, odists)
    pages = info["num_pages"] * 4096
    assert (info["device_bytes"] < pages) == (placement == "host")


def test_place_graph_round_trip(lib, small_u8_index):
    """qv_index_place_graph moves the page image HBM -> host -> HBM; every
    placement answers identically (ids, distances, hops)."""
    from quiver import _lib

    ix = small_u8_index
    _say("[gpu] place_graph round trip")
    L = _lib.load()
    h = C.c_void_p()
    _lib.check(L.qv_index_open(str(ix["dir"]).encode(), b"uint8", b"heap", None, 0, C.byref(h)))
    q = np.ascontiguousarray(ix["queries"], dtype=np.float32)
    n = q.shape[0]
    outs = []
    try:
        for placement in (_lib.QV_GRAPH_HBM, _lib.QV_GRAPH_HOST, _lib.QV_GRAPH_HBM):
            _lib.check(L.qv_index_place_graph(h, placement))
            ids = np.empty((n, 10), np.int32)
            dists = np.empty((n, 10), np.float32)
            hops = np.empty(n, np.int32)
            opts = _lib.default_search_opts()
            opts.early_exit = _lib.QV_EXIT_NONE
            rep = _lib.SearchReport()
            _lib.check(L.qv_search(h, q.ctypes.data, n, 128, 10, 64, C.byref(opts), ids.ctypes.data,
                                   dists.ctypes.data, None, C.byref(rep)))
            _lib.check(L.qv_last_hops(h, hops.ctypes.data, n))
            outs.append((ids, dists, hops))
    finally:
        L.qv_index_close(h)
    for ids, dists, hops in outs[1:]:
        np.testing.assert_array_equal(ids, outs[0][0])
        np.testing.assert_array_equal(dists, outs[0][1])
        np.testing.assert_array_equal(hops, outs[0][2])


@pytest.mark.parametrize("num_blocks,qpb", [(64, 2), (100, 8), (500, 3)])
def test_queries_per_block_slots(lib, small_u8_index, num_blocks, qpb):
    """--queries-per-block Q gives num_blocks x Q query slots (search.cu:393-399);
    answers are the oracle's for every slot count, and the launch is capped at
    the device's resident capacity."""
    from quiver import _lib

    ix = small_u8_index
    _say(f"[gpu] queries_per_block={qpb} num_blocks={num_blocks}")
    L = _lib.load()
    h = C.c_void_p()
    _lib.check(L.qv_index_open(str(ix["dir"]).encode(), b"uint8", b"heap", None, 0, C.byref(h)))
    q = np.ascontiguousarray(np.concatenate([ix["queries"]] * 8), dtype=np.float32)
    n = q.shape[0]
    ids = np.empty((n, 10), np.int32)
    dists = np.empty((n, 10), np.float32)
    hops = np.empty(n, np.int32)
    info = _lib.IndexInfo()
    try:
        _lib.check(L.qv_index_get_info(h, C.byref(info)))
        opts = _lib.default_search_opts()
        opts.early_exit = _lib.QV_EXIT_GPRUNING
        opts.num_blocks = num_blocks
        opts.queries_per_block = qpb
        rep = _lib.SearchReport()
        _lib.check(L.qv_search(h, q.ctypes.data, n, 128, 10, 64, C.byref(opts), ids.ctypes.data,
                               dists.ctypes.data, None, C.byref(rep)))
        _lib.check(L.qv_last_hops(h, hops.ctypes.data, n))
        ncu = C.c_int32()
        mem = C.c_int64()
        _lib.check(L.qv_device_info(0, None, 0, C.byref(ncu), C.byref(mem)))
        # whole workgroups: less than one workgroup's waves (at most 16) above the request
        want = min(num_blocks * qpb, info.slots_per_cu * ncu.value)
        assert want <= rep.num_blocks < want + 16 and rep.num_blocks <= info.slots_per_cu * ncu.value
        assert rep.max_inflight == min(n, num_blocks * qpb)
        opts.queries_per_block = 9
        assert L.qv_search(h, q.ctypes.data, n, 128, 10, 64, C.byref(opts), ids.ctypes.data,
                           dists.ctypes.data, None, C.byref(rep)) == _lib.QV_EINVAL
    finally:
        L.qv_index_close(h)
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, odists, _, ohops = O.search(host, q, 10, 64, early_exit=O.EXIT_GPRUNING)
    np.testing.assert_array_equal(ids, oids)
    np.testing.assert_array_equal(dists, odists)
    np.testing.assert_array_equal(hops, ohops)


def test_lut_matches_oracle(lib, small_u8_index):
    from quiver import _lib

    ix = small_u8_index
    _say("[gpu] LUT build")
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    q = np.ascontiguousarray(ix["queries"][:64], dtype=np.float32)
    M = host.M
    dq = _lib.DeviceBuffer(q.nbytes).upload(q)
    dc = _lib.DeviceBuffer(host.centroid.nbytes).upload(host.centroid)
    dp = _lib.DeviceBuffer(host.pivots_t.nbytes).upload(host.pivots_t)
    do = _lib.DeviceBuffer(host.chunk_offsets.nbytes).upload(host.chunk_offsets)
    dl = _lib.DeviceBuffer(64 * M * 256 * 4)
    du = _lib.DeviceBuffer(q.nbytes)
    _lib.check(_lib.load().qv_lut_build_raw(dc.ptr, dp.ptr, do.ptr, 128, M, dq.ptr, 64, dl.ptr, du.ptr, 0))
    luts = dl.download(np.float32, (64, M, 256))
    qu = du.download(np.float32, (64, 128))
    for i in range(64):
        ol, oq = O.lut(128, host.centroid, host.pivots_t, host.chunk_id, q[i])
        np.testing.assert_array_equal(luts[i], ol)
        np.testing.assert_array_equal(qu[i], oq)


@pytest.mark.parametrize("M", [32, 48, 20])
def test_adc_bench_matches_oracle(lib, M):
    from quiver import _lib

    _say(f"[gpu] ADC bench M={M}")
    rng = np.random.default_rng(M)
    nq, per_q, ncodes, k = 24, 64 * 37 + 5, 50000, 10
    luts = rng.random((nq, M, 256), dtype=np.float32) * 100
    codes = rng.integers(0, 256, (ncodes, M), dtype=np.uint8)
    ids = rng.integers(0, ncodes, (nq, per_q), dtype=np.int32)
    ids[:, 100:110] = ids[:, 0:10]  # repeated ids: ties broken by position
    dl = _lib.DeviceBuffer(luts.nbytes).upload(luts)
    dc = _lib.DeviceBuffer(codes.nbytes).upload(codes)
    di = _lib.DeviceBuffer(ids.nbytes).upload(ids)
    doi = _lib.DeviceBuffer(nq * k * 4)
    dod = _lib.DeviceBuffer(nq * k * 4)
    dsum = _lib.DeviceBuffer(nq * 8)
    ms = C.c_float(0)
    _lib.check(_lib.load().qv_adc_bench(dl.ptr, M, dc.ptr, ncodes, di.ptr, nq, per_q, k, doi.ptr, dod.ptr,
                                        dsum.ptr, 0, C.byref(ms)))
    gi = doi.download(np.int32, (nq, k))
    gd = dod.download(np.float32, (nq, k))
    gs = dsum.download(np.float64, (nq,))
    for i in range(nq):
        oi, od, osum = O.adc_topk(luts[i], codes, ids[i], k)
        np.testing.assert_array_equal(gd[i], od)
        np.testing.assert_array_equal(gi[i], oi)
        assert abs(gs[i] - osum) <= 1e-9 * abs(osum)


def test_gather_bench_fold(lib):
    from quiver import _lib

    _say("[gpu] gather bench fold")
    rng = np.random.default_rng(9)
    nrows, n = 5000, 64 * 300 + 37
    rows = rng.integers(0, 2**32, (nrows, 8), dtype=np.uint32)
    ids = rng.integers(0, nrows, n, dtype=np.int32)
    nblk = (2 * n + 255) // 256
    dr = _lib.DeviceBuffer(rows.nbytes).upload(rows)
    di = _lib.DeviceBuffer(ids.nbytes).upload(ids)
    df = _lib.DeviceBuffer(nblk * 4)
    ms = C.c_float(0)
    _lib.check(_lib.load().qv_gather_bench(dr.ptr, nrows, di.ptr, n, df.ptr, 0, C.byref(ms)))
    got = df.download(np.uint32, (nblk,))
    # workgroup b covers ids [128 b, 128 b + 128): the XOR of all words of those rows
    want = np.zeros(nblk, np.uint32)
    for b in range(nblk):
        sel = rows[ids[128 * b: 128 * b + 128]]
        want[b] = np.bitwise_xor.reduce(sel.reshape(-1)) if sel.size else 0
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("nwords", [300 * 256 + 17, 4096 * 256 * 5 + 1234])
def test_stream_read_bench_fold(lib, nwords):
    """Workgroup b of the streaming read folds every 16-byte word w with
    (w mod 256 B) // 256 == b, B = min(4096, ceil(nwords / 256)) workgroups."""
    from quiver import _lib

    _say(f"[gpu] stream read fold nwords={nwords}")
    rng = np.random.default_rng(nwords)
    words = rng.integers(0, 2**32, (nwords, 4), dtype=np.uint32)
    blocks = min(_lib.QV_STREAM_READ_BLOCKS, (nwords + 255) // 256)
    src = _lib.DeviceBuffer(words.nbytes).upload(words)
    fold = _lib.DeviceBuffer(blocks * 4)
    ms = C.c_float(0)
    _lib.check(_lib.load().qv_stream_read_bench(src.ptr, words.nbytes, fold.ptr, 0, C.byref(ms)))
    got = fold.download(np.uint32, (blocks,))
    per_word = np.bitwise_xor.reduce(words, axis=1)
    owner = (np.arange(nwords) % (blocks * 256)) // 256
    want = np.zeros(blocks, np.uint32)
    np.bitwise_xor.at(want, owner, per_word)
    np.testing.assert_array_equal(got, want)
    assert ms.value > 0
    assert _lib.load().qv_stream_read_bench(src.ptr, 24, fold.ptr, 0, None) == _lib.QV_EINVAL


def test_mixture_device_matches_host(lib):
    import quiver
    from quiver import _lib

    _say("[gpu] mixture device vs host")
    for dt, dim, extra in (("uint8", 128, {}), ("float", 96, {"sigma": 1.0})):
        host = quiver.mixture(3000, dim, data_type=dt, num_centers=100, seed=5, first_row=12345, **extra)
        m = _lib.Mixture(5, 100, dim, _lib.QV_UINT8 if dt == "uint8" else _lib.QV_FLOAT, 32.0, 224.0,
                         extra.get("sigma", 20.0), 1)
        buf = _lib.DeviceBuffer(host.nbytes)
        _lib.check(_lib.load().qv_mixture_fill_device(C.byref(m), 12345, 3000, buf.ptr, 0))
        dev = buf.download(host.dtype, host.shape)
        np.testing.assert_array_equal(dev, host)


@pytest.mark.parametrize("row", [32, 64, 128, 256])
def test_gather_sweep_fold(lib, row):
    """The access-rate matrix's gather: every shape reads exactly the rows its
    ids map to (the XOR of all words read, against numpy)."""
    from quiver import _lib

    _say(f"[gpu] gather sweep fold row={row}")
    rng = np.random.default_rng(row)
    nrows, n, id_range = 3001, 64 * 500 + 29, 1_000_000
    table = rng.integers(0, 2**32, (nrows, row // 4), dtype=np.uint32)
    ids = rng.integers(0, id_range, n, dtype=np.int32)
    mul = (nrows << 32) // id_range
    rows = np.minimum((ids.astype(np.uint64) * np.uint64(mul)) >> np.uint64(32), nrows - 1).astype(np.int64)
    want = np.bitwise_xor.reduce(table[rows].reshape(-1))
    dt = _lib.DeviceBuffer(table.nbytes).upload(table)
    di = _lib.DeviceBuffer(ids.nbytes).upload(ids)
    df = _lib.DeviceBuffer(4)
    L = _lib.load()
    for per in (1, 2, 4):
        for waves in (8, 16, 32):
            for nt in (0, 1):
                df.clear()
                ms, launched = C.c_float(0), C.c_int32(0)
                _lib.check(L.qv_gather_sweep_bench(dt.ptr, nrows, row, di.ptr, n, id_range, per, waves, nt, df.ptr,
                                                   0, C.byref(ms), C.byref(launched)))
                assert df.download(np.uint32, (1,))[0] == want, (per, waves, nt)
                assert launched.value % 4 == 0 and launched.value <= 256 * waves
