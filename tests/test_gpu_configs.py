"""The HIP path against the oracle at the benchmark shape (runs on the MI355X).

Workload: 1M uint8 vectors of dimension 128 from the seeded mixture (1024
centres in [32, 224], sigma 20), a Vamana graph R=64 / L=100 / alpha=1.2 with
PQ 32x256 built on the GPU -- the shape every quoted throughput number uses
(node records of 388 B, 10 per page, 32-byte code rows, all 64 neighbour lanes
of a wave in use).  2000 queries from the same mixture, top-10.

For every case ids, distances, found counts and hop counts must equal the
oracle's (deterministic mode: pipe width 1 unless stated, one query per wave),
and Recall@10 against the GPU brute force must be within 0.002 of the
oracle's.  Also covered: the latency mode (open-loop batches of 1, 16 and 256
queries, streaming admission, automatic kernel choice) and the host-forced
give-up path (a deadline that fires mid-batch, then a search on the same handle).
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import qv_oracle as O

pytestmark = pytest.mark.gpu

N, DIM, NQ, K = 1_000_000, 128, 2000, 10
KERNEL = {"lut": 1, "shared-pivots": 2, "auto": 0}


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def c1():
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    L = _lib.load()
    _say("[gpu] C1: 1M x 128 u8 mixture, GPU build R=64 L=100 alpha=1.2 PQ 32x256")
    mix = _lib.Mixture(0x5EED_0001, 1024, DIM, _lib.QV_UINT8, 32.0, 224.0, 20.0, 1)
    d_base = _lib.DeviceBuffer(N * DIM)
    _lib.check(L.qv_mixture_fill_device(C.byref(mix), 0, N, d_base.ptr, 0))
    q = np.empty((NQ + 8000, DIM), np.uint8)  # the last 8000 only feed the give-up test
    _lib.check(L.qv_mixture_fill_host(C.byref(mix), 1 << 40, q.shape[0], q.ctypes.data))
    qf = q.astype(np.float32)
    p = _lib.default_build_params()
    p.R, p.L, p.alpha, p.num_chunks, p.kmeans_iters, p.passes = 64, 100, 1.2, 32, 15, 2
    h = C.c_void_p()
    _lib.check(L.qv_build_index_gpu(d_base.ptr, _lib.QV_UINT8, N, DIM, C.byref(p), 0, C.byref(h)))
    info = _lib.IndexInfo()
    _lib.check(L.qv_index_get_info(h, C.byref(info)))
    assert (info.max_m0, info.node_size, info.nodes_per_page, info.num_chunks) == (64, 388, 10, 32)
    d_q = _lib.DeviceBuffer(NQ * DIM * 4).upload(qf[:NQ])
    d_gi, d_gd = _lib.DeviceBuffer(NQ * K * 4), _lib.DeviceBuffer(NQ * K * 4)
    _lib.check(L.qv_ground_truth(d_base.ptr, _lib.QV_UINT8, N, DIM, d_q.ptr, NQ, K, d_gi.ptr, d_gd.ptr, 0))
    gt = d_gi.download(np.int32, (NQ, K))
    d_base.close()
    pages = np.empty(info.num_pages * 4096, np.uint8)
    codes = np.empty((N, 32), np.uint8)
    centroid = np.empty(DIM, np.float32)
    pivots = np.empty((256, DIM), np.float32)
    offs = np.empty(33, np.int32)
    _lib.check(L.qv_index_copy_out(h, pages.ctypes.data, codes.ctypes.data, centroid.ctypes.data,
                                   pivots.ctypes.data, offs.ctypes.data))
    host = O.HostIndex.from_arrays(O.UINT8, DIM, N, 64, int(info.enter_point), pages, codes, centroid,
                                   pivots, offs)
    degs = pages.reshape(-1, 4096)[:, :3880].reshape(-1, 10, 388)[:, :, 128:132].copy().view(np.uint32).ravel()[:N]
    assert degs.max() <= 64 and degs.mean() > 30, "the R=64 graph must fill most neighbour lanes"
    yield {"lib": _lib, "L": L, "h": h, "q": qf, "gt": gt, "host": host, "cache": {}}
    L.qv_index_close(h)


def _search(c, queries, ef, policy, kernel="auto", pipe=1, num_blocks=0, timeout=0.0, k=K):
    lib, L = c["lib"], c["L"]
    n = queries.shape[0]
    ids = np.empty((n, k), np.int32)
    dists = np.empty((n, k), np.float32)
    found = np.empty(n, np.int32)
    o = lib.default_search_opts()
    o.early_exit = lib.QV_EXIT_GPRUNING if policy == "gpruning" else lib.QV_EXIT_NONE
    o.pipe_width = pipe
    o.kernel = KERNEL[kernel]
    o.num_blocks = num_blocks
    o.timeout_s = timeout
    rep = lib.SearchReport()
    q = np.ascontiguousarray(queries, np.float32)
    rc = L.qv_search(c["h"], q.ctypes.data, n, DIM, k, ef, C.byref(o), ids.ctypes.data, dists.ctypes.data,
                     found.ctypes.data, C.byref(rep))
    if rc != 0:
        return rc, None
    hops = np.empty(n, np.int32)
    lib.check(L.qv_last_hops(c["h"], hops.ctypes.data, n))
    return rc, (ids, dists, found, hops, rep)


def _oracle(c, ef, policy, pipe=1, n=NQ, k=K):
    key = (ef, policy, pipe, n, k)
    if key not in c["cache"]:
        c["cache"][key] = O.search(c["host"], c["q"][:n], k, ef, pipe_width=pipe,
                                   early_exit=O.EXIT_GPRUNING if policy == "gpruning" else O.EXIT_NONE)
    return c["cache"][key]


class _CodeTable:
    """The neighbour code table on the C1 handle for the duration of a test."""

    def __init__(self, c):
        self.c = c

    def __enter__(self):
        self.c["lib"].check(self.c["L"].qv_index_neighbour_codes(self.c["h"], 1))
        return self

    def __exit__(self, *exc):
        self.c["lib"].check(self.c["L"].qv_index_neighbour_codes(self.c["h"], 0))
        return False


def _percentiles_are_order_statistics(rep, lat):
    """The report's P50 / P90 / P99 / P99.9 / max are the per-query latencies'
    elements of ranks n 50 / 100, n 90 / 100, n 99 / 100 (integer), floor(n 0.999)
    and n - 1 in ascending order, exactly as the reference indexes its sorted
    latencies (search.cu:1141-1145)."""
    s = np.sort(lat)
    n = len(s)
    for r, got in ((n * 50 // 100, rep.lat_p50_ms), (n * 90 // 100, rep.lat_p90_ms),
                   (n * 99 // 100, rep.lat_p99_ms), (min(n - 1, int(n * 0.999)), rep.lat_p999_ms)):
        assert got == s[r], (r, got)
    assert rep.lat_max_ms == s[-1]
    assert abs(rep.lat_avg_ms - s.mean()) <= 1e-9 * s.mean()


def _same(got, want, what):
    ids, dists, found, hops = got[:4]
    oids, odists, ofound, ohops = want
    bad = np.nonzero(np.any(ids != oids, axis=1))[0]
    assert bad.size == 0, f"{what}: {bad.size} queries with other ids, first {bad[:5]}"
    np.testing.assert_array_equal(dists, odists, err_msg=what)
    np.testing.assert_array_equal(found, ofound, err_msg=what)
    np.testing.assert_array_equal(hops, ohops, err_msg=what)


@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
@pytest.mark.parametrize("policy", ["none", "gpruning"])
@pytest.mark.parametrize("ef", [45, 64, 128, 240, 256, 288])
def test_c1_matches_oracle(c1, kernel, policy, ef):
    _say(f"[gpu] C1 kernel={kernel} policy={policy} ef={ef}")
    rc, got = _search(c1, c1["q"][:NQ], ef, policy, kernel)
    assert rc == 0, c1["lib"].load().qv_last_error()
    assert got[4].kernel == KERNEL[kernel]
    want = _oracle(c1, ef, policy)
    _same(got, want, f"{kernel} {policy} ef={ef}")
    r_gpu, r_ora = O.recall(got[0], c1["gt"], K), O.recall(want[0], c1["gt"], K)
    assert abs(r_gpu - r_ora) <= 0.002
    if policy == "none" and ef >= 240:
        assert r_gpu >= 0.90, f"Recall@10 {r_gpu:.4f} at ef={ef}"


@pytest.mark.parametrize("pipe,ef,policy", [(2, 128, "gpruning"), (4, 128, "gpruning"), (2, 256, "none"),
                                             (3, 45, "none")])
def test_c1_pipe_lanes_match_oracle(c1, pipe, ef, policy):
    """Pipe lanes, whose expansions request the record and code rows of the
    expansion expected next (a wrong guess is fetched again)."""
    _say(f"[gpu] C1 pipe_width={pipe} ef={ef} policy={policy}")
    for kernel in ("lut", "shared-pivots"):
        rc, got = _search(c1, c1["q"][:500], ef, policy, kernel, pipe=pipe)
        assert rc == 0
        _same(got, _oracle(c1, ef, policy, pipe=pipe, n=500), f"{kernel} W={pipe} ef={ef} {policy}")


@pytest.mark.parametrize("batch", [1, 16, 256])
def test_c1_latency_mode_batches(c1, batch):
    """Open-loop arrival at a fixed batch size: each batch is one qv_search
    call (streaming admission, automatic kernel); answers do not depend on
    how queries are batched."""
    n = 200 if batch == 1 else 1024
    _say(f"[gpu] C1 latency mode batch={batch} queries={n}")
    ids = np.empty((n, K), np.int32)
    dists = np.empty((n, K), np.float32)
    found = np.empty(n, np.int32)
    hops = np.empty(n, np.int32)
    for s in range(0, n, batch):
        rc, got = _search(c1, c1["q"][s:s + batch], 240, "none", "auto")
        assert rc == 0
        ids[s:s + batch], dists[s:s + batch], found[s:s + batch], hops[s:s + batch] = got[:4]
        assert got[4].lat_max_ms > 0
    want = tuple(a[:n] for a in _oracle(c1, 240, "none"))
    _same((ids, dists, found, hops), want, f"batch {batch}")


def test_deadline_gives_up_then_next_search_is_exact(c1):
    """A deadline that fires mid-batch: qv_search returns QV_ETIMEDOUT once
    the host has raised the terminate word and every wave has left on its own;
    the handle stays usable and the next search on it equals the oracle."""
    lib = c1["lib"]
    _say("[gpu] deadline: 10k queries, ef=448, 32 query slots, 5 ms limit")
    for kernel in ("lut", "shared-pivots"):
        rc, _ = _search(c1, c1["q"], 448, "none", kernel, num_blocks=32, timeout=0.005)
        assert rc == lib.QV_ETIMEDOUT, (kernel, rc)
        assert "timeout" in lib.load().qv_last_error().decode()
        rc, got = _search(c1, c1["q"][:NQ], 128, "none", "lut")
        assert rc == 0
        _same(got, _oracle(c1, 128, "none"), f"LUT kernel after a {kernel} give-up")


@pytest.mark.parametrize("threshold", [0.8, 1.0])
def test_c1_step_recall_matches_oracle(c1, threshold):
    """Per-step recall on the benchmark shape: each query stops once
    ceil(threshold k) of its top-10 ids are in its ground-truth row; steps,
    hits, ids and hop counts equal the oracle's."""
    lib, L = c1["lib"], c1["L"]
    n = 1000
    _say(f"[gpu] C1 per-step recall threshold={threshold}")
    gt = np.ascontiguousarray(c1["gt"][:n], np.int32)
    for kernel in ("lut", "shared-pivots"):
        o = lib.default_search_opts()
        o.early_exit = lib.QV_EXIT_NONE
        o.kernel = KERNEL[kernel]
        step = np.empty(n, np.int32)
        hits = np.empty(n, np.int32)
        o.step_recall_gt, o.step_recall_gt_width, o.step_recall_gt_count = gt.ctypes.data, K, n
        o.step_recall_threshold = threshold
        o.step_recall_step, o.step_recall_hits = step.ctypes.data, hits.ctypes.data
        q = np.ascontiguousarray(c1["q"][:n], np.float32)
        ids = np.empty((n, K), np.int32)
        dists = np.empty((n, K), np.float32)
        found = np.empty(n, np.int32)
        lib.check(L.qv_search(c1["h"], q.ctypes.data, n, DIM, K, 128, C.byref(o), ids.ctypes.data,
                              dists.ctypes.data, found.ctypes.data, None))
        hops = np.empty(n, np.int32)
        lib.check(L.qv_last_hops(c1["h"], hops.ctypes.data, n))
        oids, odists, ofound, ohops, ostep, ohits = O.search(
            c1["host"], c1["q"][:n], K, 128, early_exit=O.EXIT_NONE,
            step_recall=(gt, O.required_hits(threshold, K)))
        _same((ids, dists, found, hops), (oids, odists, ofound, ohops), f"step recall {kernel}")
        np.testing.assert_array_equal(step, ostep)
        np.testing.assert_array_equal(hits, ohits)
        assert 0 < (step >= 0).sum() < n  # both outcomes occur


@pytest.mark.parametrize("blocks", [64, 640])
@pytest.mark.parametrize("kernel", ["lut", "shared-pivots"])
def test_c1_static_batches(c1, kernel, blocks):
    """Static dispatch (run_static_batch_search, search.cu:1703-1796): batches
    of num_blocks queries, each admitted when the previous has completed, every
    query of a batch taking the batch's wall time as its latency; answers equal
    the oracle's.  64 slots are one-wave workgroups of the shared-pivot kernel
    (no tail mode: a wave whose workgroup has no other wave may still get
    queries), 640 slots three-wave ones (tail mode in the last batch)."""
    lib, L = c1["lib"], c1["L"]
    n = 1000
    _say(f"[gpu] C1 static batches kernel={kernel} blocks={blocks}")
    o = lib.default_search_opts()
    o.early_exit = lib.QV_EXIT_NONE
    o.kernel = KERNEL[kernel]
    o.num_blocks = blocks
    o.admission = lib.QV_ADMIT_STATIC
    q = np.ascontiguousarray(c1["q"][:n], np.float32)
    ids = np.empty((n, K), np.int32)
    dists = np.empty((n, K), np.float32)
    found = np.empty(n, np.int32)
    rep = lib.SearchReport()
    lib.check(L.qv_search(c1["h"], q.ctypes.data, n, DIM, K, 128, C.byref(o), ids.ctypes.data,
                          dists.ctypes.data, found.ctypes.data, C.byref(rep)))
    hops = np.empty(n, np.int32)
    lib.check(L.qv_last_hops(c1["h"], hops.ctypes.data, n))
    _same((ids, dists, found, hops), _oracle(c1, 128, "none", n=n), f"static {kernel}")
    assert rep.max_inflight == blocks
    if kernel == "lut" or blocks == 64:
        assert rep.tail_queries == 0
    lat = np.empty(n, np.float64)
    lib.check(L.qv_last_latencies(c1["h"], lat.ctypes.data, n))
    batches = [lat[b:b + blocks] for b in range(0, n, blocks)]
    assert len(batches) == (n + blocks - 1) // blocks
    for bl in batches:
        assert bl.min() == bl.max() > 0  # one wall time per batch


@pytest.mark.parametrize("pipe", [1, 2])
@pytest.mark.parametrize("ef", [32, 288, 416])
def test_c1_headline_path_with_code_table(c1, pipe, ef):
    """The path the throughput benchmark times: uint8, R = 64, M = 32, the
    neighbour code table (2 KB blocks of the 64 neighbours' code rows), the
    shared-pivot kernel (forced, and picked by `auto` for 2000 queries), pipe
    widths 1 and 2, both early-exit policies.  Beams past 64 (ef 288, 416)
    finish the last query of a workgroup in tail mode (the pivot table turned
    into that wave's own LUT): the report counts such queries, and their
    answers are the oracle's like every other."""
    with _CodeTable(c1):
        for kernel in ("shared-pivots", "auto"):
            for policy in ("none", "gpruning"):
                _say(f"[gpu] C1 code table kernel={kernel} ef={ef} W={pipe} policy={policy}")
                rc, got = _search(c1, c1["q"][:NQ], ef, policy, kernel, pipe=pipe)
                assert rc == 0, c1["lib"].load().qv_last_error()
                assert got[4].kernel == KERNEL["shared-pivots"]
                if ef > 64:
                    assert 0 < got[4].tail_queries < NQ, got[4].tail_queries
                else:
                    assert got[4].tail_queries == 0
                want = _oracle(c1, ef, policy, pipe=pipe)
                _same(got, want, f"table {kernel} ef={ef} W={pipe} {policy}")
                assert abs(O.recall(got[0], c1["gt"], K) - O.recall(want[0], c1["gt"], K)) <= 0.002


@pytest.mark.parametrize("k", [1, 20, 33, 64])
def test_c1_topk_matches_oracle(c1, k):
    """top-k other than 10: k = 1, k = 20 and 33 (the reference's k > 32
    insert, gpu_primitives.cuh:99-138, has the same first-found-wins order)
    and k = 64; both kernels, with and without the code table."""
    n = 1000
    want = _oracle(c1, 128, "none", n=n, k=k)
    for table in (False, True):
        for kernel in ("lut", "shared-pivots"):
            _say(f"[gpu] C1 topk={k} kernel={kernel} table={table}")
            if table:
                with _CodeTable(c1):
                    rc, got = _search(c1, c1["q"][:n], 128, "none", kernel, k=k)
            else:
                rc, got = _search(c1, c1["q"][:n], 128, "none", kernel, k=k)
            assert rc == 0, c1["lib"].load().qv_last_error()
            _same(got, want, f"topk={k} {kernel} table={table}")
            if kernel == "lut":
                assert got[4].tail_queries == 0


@pytest.mark.parametrize("k", [65, 100, 200, 1024])
def test_c1_wide_topk_matches_oracle(c1, k):
    """top-k above 64 (retset_push_32, gpu_primitives.cuh:99-138, for any k):
    the per-query-LUT kernel keeps entries 64 .. k - 1 in LDS.  `auto` takes
    that kernel whatever the number of queries; a forced shared-pivot search
    is refused.  Pipe widths 1 and 2, both early-exit policies (gpruning reads
    entry k - 1), ef below and above k (k = 1024 at ef = 64 leaves most of the
    list as -1 / +inf padding), and the code table on."""
    n = 300 if k < 1024 else 100
    cases = [(1, "none", 128), (2, "gpruning", 256), (2, "none", 64)]
    if k == 100:
        cases.append((1, "gpruning", 416))
    for pipe, policy, ef in cases:
        _say(f"[gpu] C1 wide topk={k} W={pipe} {policy} ef={ef}")
        want = _oracle(c1, ef, policy, pipe=pipe, n=n, k=k)
        rc, got = _search(c1, c1["q"][:n], ef, policy, "auto", pipe=pipe, k=k)
        assert rc == 0, c1["lib"].load().qv_last_error()
        assert got[4].kernel == KERNEL["lut"]
        _same(got, want, f"wide topk={k} W={pipe} {policy} ef={ef}")
        assert np.all(got[2] <= k)
        pad = np.arange(k)[None, :] >= got[2][:, None]
        assert np.all(got[0][pad] == -1) and np.all(np.isinf(got[1][pad]))
    with _CodeTable(c1):
        rc, got = _search(c1, c1["q"][:n], 128, "none", "auto", k=k)
        assert rc == 0, c1["lib"].load().qv_last_error()
        _same(got, _oracle(c1, 128, "none", n=n, k=k), f"wide topk={k} table")
    rc, _ = _search(c1, c1["q"][:8], 128, "none", "shared-pivots", k=k)
    assert rc == c1["lib"].QV_EUNSUPPORTED
    assert "at most 64 results" in c1["lib"].load().qv_last_error().decode()


def test_c1_wide_topk_per_step_recall(c1):
    """Per-step recall over a top-100 (its entries past 64 read from LDS):
    each query stops once 50 of its top-100 ids are in its ground-truth row,
    here the oracle's top-128 at ef = 512; steps, hits and results equal the
    oracle's."""
    lib, L = c1["lib"], c1["L"]
    n, k, width, need = 200, 100, 128, 50
    gt = np.ascontiguousarray(_oracle(c1, 512, "none", n=n, k=width)[0])
    want = O.search(c1["host"], c1["q"][:n], k, 256, early_exit=O.EXIT_NONE, step_recall=(gt, need))
    o = lib.default_search_opts()
    o.early_exit = lib.QV_EXIT_NONE
    o.pipe_width = 1
    o.kernel = KERNEL["auto"]
    step, hits = np.full(n, -7, np.int32), np.full(n, -7, np.int32)
    o.step_recall_gt, o.step_recall_gt_width, o.step_recall_gt_count = gt.ctypes.data, width, n
    o.step_recall_threshold = need / k
    o.step_recall_step, o.step_recall_hits = step.ctypes.data, hits.ctypes.data
    ids = np.empty((n, k), np.int32)
    dists = np.empty((n, k), np.float32)
    found = np.empty(n, np.int32)
    q = np.ascontiguousarray(c1["q"][:n], np.float32)
    _say("[gpu] C1 wide topk=100 per-step recall")
    lib.check(L.qv_search(c1["h"], q.ctypes.data, n, DIM, k, 256, C.byref(o), ids.ctypes.data,
                          dists.ctypes.data, found.ctypes.data, None))
    hops = np.empty(n, np.int32)
    lib.check(L.qv_last_hops(c1["h"], hops.ctypes.data, n))
    _same((ids, dists, found, hops), want[:4], "wide topk per-step recall")
    np.testing.assert_array_equal(step, want[4])
    np.testing.assert_array_equal(hits, want[5])
    assert np.any(step > 0) and np.any(hits >= need)


@pytest.mark.parametrize("batch,rate", [(1, 2e5), (16, 1e6), (256, 4e6)])
def test_c1_open_loop_arrival(c1, batch, rate):
    """Open-loop arrival into one launch: groups of `batch` queries admitted on
    a fixed clock (arrival_qps), whatever is in flight.  Answers equal the
    oracle's; the search lasts at least until the last group's scheduled
    arrival; every latency is positive."""
    lib, L = c1["lib"], c1["L"]
    n = NQ
    _say(f"[gpu] C1 open loop batch={batch} rate={rate:.0f}")
    o = lib.default_search_opts()
    o.early_exit = lib.QV_EXIT_NONE
    o.arrival_qps = rate
    o.arrival_batch = batch
    q = np.ascontiguousarray(c1["q"][:n], np.float32)
    ids = np.empty((n, K), np.int32)
    dists = np.empty((n, K), np.float32)
    found = np.empty(n, np.int32)
    rep = lib.SearchReport()
    lib.check(L.qv_search(c1["h"], q.ctypes.data, n, DIM, K, 128, C.byref(o), ids.ctypes.data,
                          dists.ctypes.data, found.ctypes.data, C.byref(rep)))
    hops = np.empty(n, np.int32)
    lib.check(L.qv_last_hops(c1["h"], hops.ctypes.data, n))
    _same((ids, dists, found, hops), _oracle(c1, 128, "none"), f"open loop batch={batch}")
    last_arrival = ((n + batch - 1) // batch - 1) * batch / rate
    assert rep.search_time_s >= last_arrival
    lat = np.empty(n, np.float64)
    lib.check(L.qv_last_latencies(c1["h"], lat.ctypes.data, n))
    assert lat.min() > 0 and rep.lat_p99_ms > 0
    _percentiles_are_order_statistics(rep, lat)
    # the static and batch admissions refuse an arrival rate
    o.admission = lib.QV_ADMIT_STATIC
    rc = L.qv_search(c1["h"], q.ctypes.data, 16, DIM, K, 128, C.byref(o), ids.ctypes.data, dists.ctypes.data,
                     None, None)
    assert rc == lib.QV_EINVAL and b"open-loop" in L.qv_last_error()


@pytest.mark.parametrize("admission", ["streaming", "static"])
def test_c1_host_queries_change_between_calls(c1, admission):
    """A host-buffer call copies its queries into the index's pinned staging
    buffer a chunk at a time while the kernel already runs, and the kernel
    reads each query there.  Consecutive calls with different queries (a later
    slice, another one, then the first queries in reverse order; 1,500, 1,000
    and 700 queries, so both kernels) must each return what the device-buffer
    path returns for the same queries; the results come back through the
    pinned buffer the kernel writes them into, and the report's percentiles are
    the order statistics of the per-query latencies (ties included: a static
    batch's queries share one latency)."""
    lib, L = c1["lib"], c1["L"]
    adm = lib.QV_ADMIT_STREAMING if admission == "streaming" else lib.QV_ADMIT_STATIC
    sets = [c1["q"][NQ:NQ + 1500], c1["q"][NQ + 1500:NQ + 2500], c1["q"][:700][::-1]]
    for i, qs in enumerate(sets):
        qs = np.ascontiguousarray(qs, np.float32)
        n = qs.shape[0]
        _say(f"[gpu] host queries call {i}: {n} queries, admission={admission}")
        o = lib.default_search_opts()
        o.early_exit = lib.QV_EXIT_NONE
        o.admission = adm
        ids = np.empty((n, K), np.int32)
        dists = np.empty((n, K), np.float32)
        rep = lib.SearchReport()
        lib.check(L.qv_search(c1["h"], qs.ctypes.data, n, DIM, K, 128, C.byref(o), ids.ctypes.data,
                              dists.ctypes.data, None, C.byref(rep)))
        lat = np.empty(n, np.float64)
        lib.check(L.qv_last_latencies(c1["h"], lat.ctypes.data, n))
        _percentiles_are_order_statistics(rep, lat)
        d_q = lib.DeviceBuffer(qs.nbytes).upload(qs)
        d_i, d_d = lib.DeviceBuffer(n * K * 4), lib.DeviceBuffer(n * K * 4)
        o.device_buffers = 1
        lib.check(L.qv_search(c1["h"], d_q.ptr, n, DIM, K, 128, C.byref(o), d_i.ptr, d_d.ptr, None, None))
        want_i, want_d = d_i.download(np.int32, (n, K)), d_d.download(np.float32, (n, K))
        for b in (d_q, d_i, d_d):
            b.close()
        assert np.array_equal(ids, want_i) and np.array_equal(dists, want_d), f"call {i}"
