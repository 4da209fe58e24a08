"""qv_search_noalloc (the allocation-free search entry point) against
qv_search through the C ABI (runs on the MI355X).

Each case runs qv_search on device buffers with every query admitted at
launch, then qv_search_noalloc twice in a row -- the full input, then a
smaller one -- and requires ids, distances, found counts, the hop and
evaluation totals and the early-exit count to equal qv_search's for the same
queries (integer and index work: bit-exact), and the device's free memory to
be the same before and after every call but the process's first (which may
load the entry's kernels).  Also: a 600k-point index with 1024 query slots of
either kernel, and the entry's argument limits.
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

K = 10
_WARM = {"calls": 0}  # noalloc calls made so far in this process


def _free_bytes(lib) -> int:
    free, total = C.c_int64(), C.c_int64()
    lib.check(lib.load().qv_device_mem_info(0, C.byref(free), C.byref(total)))
    return free.value


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    return _lib


class _Dev:
    """Device query and output buffers for up to n queries."""

    def __init__(self, lib, queries, k=K):
        self.n, self.dim = queries.shape
        self.k = k
        self.q = lib.DeviceBuffer(queries.nbytes).upload(np.ascontiguousarray(queries, np.float32))
        self.ids = lib.DeviceBuffer(self.n * k * 4)
        self.dists = lib.DeviceBuffer(self.n * k * 4)
        self.found = lib.DeviceBuffer(self.n * 4)

    def fetch(self, n):
        return (self.ids.download(np.int32, (n, self.k)), self.dists.download(np.float32, (n, self.k)),
                self.found.download(np.int32, (n,)))


def _opts(lib, kernel, num_blocks=0, policy="none"):
    o = lib.default_search_opts()
    o.kernel = {"auto": 0, "lut": 1, "shared-pivots": 2}[kernel]
    o.num_blocks = num_blocks
    o.early_exit = lib.QV_EXIT_NONE if policy == "none" else lib.QV_EXIT_GPRUNING
    o.device_buffers = 1
    o.admission = lib.QV_ADMIT_BATCH
    return o


def _pair(lib, h, dev, n, ef, kernel, num_blocks=0, policy="none"):
    """(qv_search's answer, qv_search_noalloc's answer, both reports) for the first n queries."""
    L = lib.load()
    o = _opts(lib, kernel, num_blocks, policy)
    r0, r1 = lib.SearchReport(), lib.SearchReport()
    dev.ids.clear()
    lib.check(L.qv_search(h, dev.q.ptr, n, dev.dim, dev.k, ef, C.byref(o), dev.ids.ptr, dev.dists.ptr,
                          dev.found.ptr, C.byref(r0)))
    want = dev.fetch(n)
    dev.ids.clear()
    dev.dists.clear()
    dev.found.clear()
    free0 = _free_bytes(lib)
    lib.check(L.qv_search_noalloc(h, dev.q.ptr, n, dev.dim, dev.k, ef, C.byref(o), dev.ids.ptr, dev.dists.ptr,
                                  dev.found.ptr, C.byref(r1)))
    free1 = _free_bytes(lib)
    if _WARM["calls"] > 0:
        assert free1 == free0, f"device memory changed across a warm qv_search_noalloc: {free0 - free1} bytes"
    _WARM["calls"] += 1
    return want, dev.fetch(n), r0, r1


def _check(want, got, r0, r1, what):
    for a, b, name in zip(want, got, ("ids", "dists", "found")):
        np.testing.assert_array_equal(b, a, err_msg=f"{what}: {name}")
    assert (r1.total_hops, r1.total_evals) == (r0.total_hops, r0.total_evals), what
    assert r1.early_stopped == r0.early_stopped, what
    assert r1.kernel == r0.kernel, what


def _open_small(lib, ix):
    h = C.c_void_p()
    lib.check(lib.load().qv_index_open(str(ix["dir"]).encode(), ix["dtype"].encode(), b"heap", None, 0,
                                       C.byref(h)))
    return h


@pytest.mark.parametrize("kernel", ["auto", "lut", "shared-pivots"])
def test_noalloc_equals_search_u8(lib, small_u8_index, kernel):
    ix = small_u8_index
    h = _open_small(lib, ix)
    dev = _Dev(lib, ix["queries"].astype(np.float32))
    try:
        stops = 0
        for n, ef, policy in ((dev.n, 128, "none"), (37, 64, "gpruning")):  # second call smaller
            _say(f"[gpu] noalloc u8 kernel={kernel} n={n} ef={ef} {policy}")
            want, got, r0, r1 = _pair(lib, h, dev, n, ef, kernel, policy=policy)
            _check(want, got, r0, r1, f"u8 {kernel} n={n}")
            stops += r1.early_stopped
        assert stops > 0, "gpruning stopped no query: the early-exit count went untested"
    finally:
        lib.load().qv_index_close(h)


def test_noalloc_equals_search_float(lib, small_f32_index):
    ix = small_f32_index
    h = _open_small(lib, ix)
    dev = _Dev(lib, ix["queries"])
    try:
        for kernel in ("lut", "shared-pivots"):
            for n in (dev.n, 5):
                _say(f"[gpu] noalloc float kernel={kernel} n={n}")
                _check(*_pair(lib, h, dev, n, 96, kernel), f"float {kernel} n={n}")
    finally:
        lib.load().qv_index_close(h)


def test_noalloc_wide_topk(lib, small_u8_index):
    """A top-100 (entries past the 64th in the per-query-LUT kernel's LDS,
    no scratch of their own): equal to qv_search on calls in a row, each
    smaller than the one before, both policies, the last with a beam of 1500
    (32 positions per lane)."""
    ix = small_u8_index
    h = _open_small(lib, ix)
    dev = _Dev(lib, ix["queries"].astype(np.float32), k=100)
    try:
        for n, ef, policy in ((dev.n, 128, "none"), (23, 256, "gpruning"), (17, 1500, "none")):
            _say(f"[gpu] noalloc u8 topk=100 n={n} ef={ef} {policy}")
            want, got, r0, r1 = _pair(lib, h, dev, n, ef, "auto", policy=policy)
            _check(want, got, r0, r1, f"u8 topk=100 n={n}")
            assert r1.kernel == 1
    finally:
        lib.load().qv_index_close(h)


def test_noalloc_many_slots_on_a_larger_index(lib):
    """600k points and 1024 requested query slots: each kernel launches all of
    them (the scratch holds only counts, nothing per slot or per point) and
    equals qv_search; at ef = 128 the shared-pivot launch (four-wave
    workgroups) finishes queries in tail mode, its ended-wave counts in the
    fixed array too."""
    import quiver  # noqa: F401

    L = lib.load()
    n, dim = 600_000, 128
    mix = lib.Mixture(0x5EED_0A11, 256, dim, lib.QV_UINT8, 32.0, 224.0, 20.0, 1)
    base = lib.DeviceBuffer(n * dim)
    lib.check(L.qv_mixture_fill_device(C.byref(mix), 0, n, base.ptr, 0))
    p = lib.default_build_params()
    p.R, p.L, p.num_chunks, p.passes = 32, 48, 32, 1
    h = C.c_void_p()
    _say("[gpu] noalloc: build 600k u8 index")
    lib.check(L.qv_build_index_gpu(base.ptr, lib.QV_UINT8, n, dim, C.byref(p), 0, C.byref(h)))
    base.close()
    q = np.empty((3000, dim), np.uint8)
    lib.check(L.qv_mixture_fill_host(C.byref(mix), 1 << 40, q.shape[0], q.ctypes.data))
    dev = _Dev(lib, q.astype(np.float32))
    try:
        for n_q in (3000, 1500):
            for kernel in ("lut", "shared-pivots"):
                _say(f"[gpu] noalloc 600k points kernel={kernel} 1024 slots n={n_q}")
                want, got, r0, r1 = _pair(lib, h, dev, n_q, 64, kernel, num_blocks=1024)
                _check(want, got, r0, r1, f"{kernel} 1024 slots n={n_q}")
                assert r0.num_blocks == r1.num_blocks == 1024
        for n_q in (3000, 1500):
            _say(f"[gpu] noalloc 600k points shared-pivots ef=128 1024 slots n={n_q}")
            want, got, r0, r1 = _pair(lib, h, dev, n_q, 128, "shared-pivots", num_blocks=1024)
            _check(want, got, r0, r1, f"shared-pivots ef=128 1024 slots n={n_q}")
            assert 0 < r1.tail_queries < n_q and 0 < r0.tail_queries < n_q, (r0.tail_queries, r1.tail_queries)
    finally:
        L.qv_index_close(h)


def test_noalloc_rejects_out_of_range_calls(lib, small_u8_index):
    ix = small_u8_index
    h = _open_small(lib, ix)
    dev = _Dev(lib, ix["queries"][:4].astype(np.float32))
    L = lib.load()
    try:
        o = _opts(lib, "auto")
        too_many = lib.QV_NOALLOC_MAX_QUERIES + 1  # rejected before any device access
        rc = L.qv_search_noalloc(h, dev.q.ptr, too_many, dev.dim, K, 64, C.byref(o), dev.ids.ptr, dev.dists.ptr,
                                 None, None)
        assert rc == lib.QV_EINVAL and b"queries per call" in L.qv_last_error()
        o.timeout_s = 1.0
        rc = L.qv_search_noalloc(h, dev.q.ptr, 4, dev.dim, K, 64, C.byref(o), dev.ids.ptr, dev.dists.ptr,
                                 None, None)
        assert rc == lib.QV_EINVAL and b"no deadline" in L.qv_last_error()
        o.timeout_s = 0.0
        rc = L.qv_search_noalloc(h, dev.q.ptr, 4, dev.dim, K, 2049, C.byref(o), dev.ids.ptr, dev.dists.ptr,
                                 None, None)
        assert rc == lib.QV_EINVAL
        # still usable afterwards
        _check(*_pair(lib, h, dev, 4, 64, "auto"), "after rejected calls")
    finally:
        L.qv_index_close(h)
