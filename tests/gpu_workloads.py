"""GPU-built benchmark workloads for the parity tests, and a search helper.

Each workload is the seeded mixture of one benchmark configuration, built on
the GPU (Vamana R / L / alpha = 1.2 and PQ M x 256), with its queries taken
from the same mixture beyond the base rows (row 2^40 on) and brute-force
ground truth from the GPU.  The handle's page image, codes and PQ tables are
copied back into a host index for the oracle.
"""
from __future__ import annotations

import ctypes as C
import sys
import time

import numpy as np

import qv_oracle as O

KERNEL = {"lut": 1, "shared-pivots": 2, "auto": 0}


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


class Workload:
    """One GPU-built index with its queries, ground truth and host copy."""

    def __init__(self, *, n: int, dim: int, dtype: str, centers: int, sigma: float, seed: int, R: int, L: int,
                 M: int, nq: int, k: int = 10, lo: float = 32.0, hi: float = 224.0):
        from quiver import _lib

        self.lib, self.L = _lib, _lib.load()
        self.n, self.dim, self.nq = n, dim, nq
        is_u8 = dtype == "uint8"
        code = _lib.QV_UINT8 if is_u8 else _lib.QV_FLOAT
        t = time.time()
        mix = _lib.Mixture(seed, centers, dim, code, lo, hi, sigma, 1)
        d_base = _lib.DeviceBuffer(n * dim * (1 if is_u8 else 4))
        _lib.check(self.L.qv_mixture_fill_device(C.byref(mix), 0, n, d_base.ptr, 0))
        q = np.empty((nq, dim), np.uint8 if is_u8 else np.float32)
        _lib.check(self.L.qv_mixture_fill_host(C.byref(mix), 1 << 40, nq, q.ctypes.data))
        self.q = np.ascontiguousarray(q, np.float32)
        p = _lib.default_build_params()
        p.R, p.L, p.alpha, p.num_chunks, p.kmeans_iters, p.passes = R, L, 1.2, M, 15, 2
        h = C.c_void_p()
        _lib.check(self.L.qv_build_index_gpu(d_base.ptr, code, n, dim, C.byref(p), 0, C.byref(h)))
        self.h = h
        say(f"[gpu] built {n} x {dim} {dtype} R={R} M={M} in {time.time() - t:.1f}s")
        info = _lib.IndexInfo()
        _lib.check(self.L.qv_index_get_info(h, C.byref(info)))
        self.info = info
        d_q = _lib.DeviceBuffer(self.q.nbytes).upload(self.q)
        d_gi, d_gd = _lib.DeviceBuffer(nq * k * 4), _lib.DeviceBuffer(nq * k * 4)
        _lib.check(self.L.qv_ground_truth(d_base.ptr, code, n, dim, d_q.ptr, nq, k, d_gi.ptr, d_gd.ptr, 0))
        self.gt = d_gi.download(np.int32, (nq, k))
        for b in (d_base, d_q, d_gi, d_gd):
            b.close()
        t = time.time()
        pages = np.empty(info.num_pages * 4096, np.uint8)
        codes = np.empty((n, M), np.uint8)
        centroid = np.empty(dim, np.float32)
        pivots = np.empty((256, dim), np.float32)
        offs = np.empty(M + 1, np.int32)
        _lib.check(self.L.qv_index_copy_out(h, pages.ctypes.data, codes.ctypes.data, centroid.ctypes.data,
                                            pivots.ctypes.data, offs.ctypes.data))
        self.host = O.HostIndex.from_arrays(code, dim, n, R, int(info.enter_point), pages, codes, centroid,
                                            pivots, offs)
        del pages, codes
        say(f"[gpu] host copy for the oracle ({info.num_pages * 4096 / 2**30:.1f} GiB pages) "
            f"in {time.time() - t:.1f}s")
        self.cache: dict = {}

    def close(self) -> None:
        if self.h:
            self.L.qv_index_close(self.h)
            self.h = None
        self.host = None
        self.cache.clear()

    def neighbour_codes(self, enable: bool) -> None:
        self.lib.check(self.L.qv_index_neighbour_codes(self.h, 1 if enable else 0))

    def search(self, queries, ef, policy, kernel="auto", pipe=1, k=10, num_blocks=0, timeout=0.0,
               device_buffers=False):
        """(rc, (ids, dists, found, hops, report)) of one qv_search call."""
        lib, L = self.lib, self.L
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
        rc = L.qv_search(self.h, q.ctypes.data, n, self.dim, k, ef, C.byref(o), ids.ctypes.data,
                         dists.ctypes.data, found.ctypes.data, C.byref(rep))
        if rc != 0:
            return rc, None
        hops = np.empty(n, np.int32)
        lib.check(L.qv_last_hops(self.h, hops.ctypes.data, n))
        return rc, (ids, dists, found, hops, rep)

    def oracle(self, ef, policy, pipe=1, n=None, k=10):
        n = self.nq if n is None else n
        key = (ef, policy, pipe, n, k)
        if key not in self.cache:
            self.cache[key] = O.search(self.host, self.q[:n], k, ef, pipe_width=pipe,
                                       early_exit=O.EXIT_GPRUNING if policy == "gpruning" else O.EXIT_NONE)
        return self.cache[key]


def same(got, want, what: str) -> None:
    """ids, distances, found counts and hop counts equal, query by query."""
    ids, dists, found, hops = got[:4]
    oids, odists, ofound, ohops = want[:4]
    bad = np.nonzero(np.any(ids != oids, axis=1))[0]
    assert bad.size == 0, f"{what}: {bad.size} queries with other ids, first {bad[:5]}"
    np.testing.assert_array_equal(dists, odists, err_msg=what)
    np.testing.assert_array_equal(found, ofound, err_msg=what)
    np.testing.assert_array_equal(hops, ohops, err_msg=what)
