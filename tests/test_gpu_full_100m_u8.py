"""Large-scale uint8 configuration at its full size (runs on the MI355X).

100M uint8 vectors of dimension 128 from the seeded mixture with 65536
centres, a Vamana graph R=64 / L=100 / alpha=1.2 and PQ 32x256 built on the
GPU: a 38.7 GiB page image (byte offsets past 2^32), 3.2 GB of codes and the
204.8 GB neighbour code table (block offsets past 2^37), all in HBM; 1000
queries from the same mixture, top-10.  The throughput benchmark's own point
(ef 288, pipe width 2, early exit off, code table, shared pivots) and its
Recall@10 >= 0.95 point (ef 416), gpruning, the per-query-LUT kernel, and
latency-mode batches of 1, 16 and 256 queries: ids, distances, found counts
and hop counts identical to the oracle in every case.
"""
from __future__ import annotations

import numpy as np
import pytest

import qv_oracle as O
from gpu_workloads import Workload, same, say

pytestmark = pytest.mark.gpu

NQ = 1000


@pytest.fixture(scope="module")
def w():
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    say("[gpu] 100M u8: 65536 centres, GPU build R=64 L=100 PQ 32x256")
    wl = Workload(n=100_000_000, dim=128, dtype="uint8", centers=65536, sigma=20.0, seed=0x5EED_0002, R=64,
                  L=100, M=32, nq=NQ)
    assert wl.info.num_pages * 4096 > 1 << 32
    say("[gpu] 100M u8: neighbour code table")
    wl.neighbour_codes(True)
    yield wl
    wl.close()


@pytest.mark.parametrize("ef,pipe,policy", [(288, 2, "none"), (416, 2, "none"), (288, 1, "none"),
                                            (288, 1, "gpruning")])
def test_100m_benchmark_points(w, ef, pipe, policy):
    want = w.oracle(ef, policy, pipe=pipe)
    say(f"[gpu] 100M ef={ef} W={pipe} {policy} shared pivots + code table")
    rc, got = w.search(w.q, ef, policy, "shared-pivots", pipe=pipe)
    assert rc == 0, w.L.qv_last_error()
    same(got, want, f"100M ef={ef} W={pipe} {policy}")
    r = O.recall(got[0], w.gt, 10)
    assert abs(r - O.recall(want[0], w.gt, 10)) <= 0.002
    if policy == "none":
        assert r >= (0.95 if ef == 416 else 0.89), r


def test_100m_lut_kernel(w):
    """The per-query-LUT kernel (auto takes it for 1000 queries: they fit its
    resident slots), reading the code table's blocks."""
    say("[gpu] 100M ef=288 W=2 auto (per-query LUT)")
    rc, got = w.search(w.q, 288, "none", "auto", pipe=2)
    assert rc == 0, w.L.qv_last_error()
    assert got[4].kernel == 1
    same(got, w.oracle(288, "none", pipe=2), "100M LUT kernel")


@pytest.mark.parametrize("batch", [1, 16, 256])
def test_100m_latency_batches(w, batch):
    """One qv_search call per batch of queries (streaming admission, automatic
    kernel): the answers do not depend on how the queries are batched."""
    n = 64 if batch == 1 else 512
    say(f"[gpu] 100M latency batch={batch} queries={n}")
    ids = np.empty((n, 10), np.int32)
    dists = np.empty((n, 10), np.float32)
    found = np.empty(n, np.int32)
    hops = np.empty(n, np.int32)
    for s in range(0, n, batch):
        rc, got = w.search(w.q[s:s + batch], 288, "none", "auto", pipe=2)
        assert rc == 0, w.L.qv_last_error()
        ids[s:s + batch], dists[s:s + batch], found[s:s + batch], hops[s:s + batch] = got[:4]
    want = tuple(a[:n] for a in w.oracle(288, "none", pipe=2))
    same((ids, dists, found, hops), want, f"100M batch {batch}")
