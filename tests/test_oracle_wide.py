"""Known answers for the oracle at degree 128 and at ef above 448 (CPU only).

Neither shape appears in the reference's own tests, so the expected values
below come from what the search rules fix, not from running the oracle:

* the star: node 0 (the entry) links to nodes 1..128 and each of them links
  back to node 0 only; PQ is exact (one chunk per dimension, pivots 0..255), so
  a beam key is (exact squared distance, id).  The query sits among nodes
  1..128 and node 0 is far from all of them.  Expanding the entry evaluates
  all 128 neighbours at once (persistent_merge_data, kernel_helpers.cuh:
  232-357, with deg = 128) and keeps the first ef of them in (distance, id)
  order; every later expansion offers only node 0, which ranks last, so it
  enters the beam only while the beam has room.  The trace is therefore the
  entry, then the kept nodes in key order, then (with room) the entry again.
  A candidate dropped from a 128-wide merge, a wrong tie order or a wrong
  truncation fails one of the cases.
* exhaustive search: with ef at least the number of nodes of a connected
  graph the beam never drops an entry, so every node is expanded once, the
  entry twice (it is expanded at the start without entering the beam, then
  enters as a neighbour), and the top-k equals brute force.  A beam capped
  below ef fails it.
"""
from __future__ import annotations

import numpy as np
import pytest

import qv_oracle as O
from index_fixtures import exact_pq, write_index

Q = np.full(4, 100, np.float32)


def _star(tmp_path):
    rng = np.random.default_rng(128)
    vecs = np.empty((129, 4), np.uint8)
    vecs[0] = 200
    vecs[1:] = 100 + rng.integers(-12, 13, size=(128, 4))
    adj = [list(range(1, 129))] + [[0] for _ in range(128)]
    write_index(tmp_path / "star", vecs, adj, 0, 128, *exact_pq(vecs))
    d = ((vecs.astype(np.int64) - 100) ** 2).sum(axis=1)
    ids = np.arange(1, 129)
    order = ids[np.lexsort((ids, d[1:]))]
    return O.HostIndex.from_files(tmp_path, "uint8"), d, order


@pytest.mark.parametrize("ef,extra", [(64, []), (100, []), (128, []), (200, [0]), (1000, [0])])
def test_star_of_degree_128(tmp_path, ef, extra):
    ix, d, order = _star(tmp_path)
    assert len(np.unique(d[1:])) < 128  # ties exist, so the id order matters
    kept = list(order[:min(ef, 128)])
    # node 0 enters the beam only if a slot is free once 128 nodes are in it
    want = [0] + kept + (extra if ef > 128 else [])
    ids, dists, found, hops, trace = O.search_trace(ix, Q, 10, ef, early_exit=O.EXIT_NONE)
    assert trace == want
    assert hops == len(want)
    assert list(ids) == list(order[:10])
    assert list(dists) == [float(d[i]) for i in order[:10]]
    assert found == 10


@pytest.mark.parametrize("ef", [700, 1024])
def test_exhaustive_beyond_448(tmp_path, ef):
    n, dim = 700, 8
    rng = np.random.default_rng(448)
    vecs = rng.integers(0, 256, size=(n, dim)).astype(np.uint8)
    adj = []
    for v in range(n):
        nb = {(v + 1) % n, (v - 1) % n}  # a ring keeps the graph connected
        nb.update(int(x) for x in rng.choice(n, size=14, replace=False) if x != v)
        adj.append(sorted(nb)[:16])
    write_index(tmp_path / "rand", vecs, adj, 0, 16, *exact_pq(vecs))
    ix = O.HostIndex.from_files(tmp_path, "uint8")
    q = rng.integers(0, 256, size=dim).astype(np.float32)
    ids, dists, found, hops, trace = O.search_trace(ix, q, 10, ef, early_exit=O.EXIT_NONE)
    assert hops == n + 1
    assert sorted(trace) == sorted(list(range(n)) + [0])
    d = ((vecs.astype(np.int64) - q.astype(np.int64)) ** 2).sum(axis=1)
    want = np.lexsort((np.arange(n), d))[:10]
    assert list(ids) == list(want)
    assert list(dists) == [float(d[i]) for i in want]
    # one position short of every node: the search is no longer exhaustive
    _, _, _, hops_short, _ = O.search_trace(ix, q, 10, 64, early_exit=O.EXIT_NONE)
    assert hops_short < n
