"""Known-answer checks of the oracle's beam search (CPU only).

Hand graphs whose traversal can be followed step by step pin the merge cap
(2*ef), the duplicate compaction, the truncation to ef, the first-unvisited
selection, the stable top-k and the reference's entry-revisit quirk (the entry
node is expanded but never inserted into the beam, so a neighbour linking back
to it makes it selectable again: kernel_q1.cuh:264-287, kernel_helpers.cuh:279).
"""
from __future__ import annotations

import numpy as np
import pytest

import qv_oracle as O
from index_fixtures import exact_pq, write_index


def _line_index(tmp_path):
    vecs = np.array([[10 * v] * 4 for v in range(6)], np.uint8)
    adj = [[1]] + [[v - 1, v + 1] for v in range(1, 5)] + [[4]]
    write_index(tmp_path / "line", vecs, adj, 0, 4, *exact_pq(vecs))
    return O.HostIndex.from_files(tmp_path, "uint8")


def test_line_graph_revisits_entry(tmp_path):
    ix = _line_index(tmp_path)
    q = np.full((1, 4), 50, np.float32)
    ids, dists, found, hops = O.search(ix, q, 3, 10, early_exit=O.EXIT_NONE)
    # expansion order 0,1,2,3,4,5 then the entry 0 again (it entered the beam
    # unvisited as a neighbour of 1): 7 hops
    assert hops[0] == 7
    np.testing.assert_array_equal(ids[0], [5, 4, 3])
    np.testing.assert_array_equal(dists[0], [0, 400, 1600])
    assert found[0] == 3


def test_line_graph_truncation_to_ef_drops_entry(tmp_path):
    ix = _line_index(tmp_path)
    q = np.full((1, 4), 50, np.float32)
    # with ef = 5 the beam [5,4,3,2,1,0] is cut to five entries after node 4's
    # expansion, which drops the unvisited entry: 6 hops
    _, _, _, hops = O.search(ix, q, 3, 5, early_exit=O.EXIT_NONE)
    assert hops[0] == 6


def test_complete_graph_known_answer(tmp_path):
    rng = np.random.default_rng(8)
    n, dim = 40, 8
    vecs = rng.integers(0, 256, (n, dim), dtype=np.uint8)
    adj = [[u for u in range(n) if u != v] for v in range(n)]
    entry = 17
    write_index(tmp_path / "full", vecs, adj, entry, n - 1, *exact_pq(vecs))
    ix = O.HostIndex.from_files(tmp_path, "uint8")
    qs = rng.integers(0, 256, (20, dim)).astype(np.float32)
    k = 12
    ids, dists, found, hops = O.search(ix, qs, k, 64, early_exit=O.EXIT_NONE)
    for i in range(qs.shape[0]):
        exact = ((vecs.astype(np.int64) - qs[i].astype(np.int64)) ** 2).sum(1)
        # every node expanded once, the entry twice
        assert hops[i] == n + 1
        expect = np.sort(np.concatenate([exact, [exact[entry]]]))[:k]
        np.testing.assert_array_equal(dists[i], expect.astype(np.float32))
        for j in range(k):
            assert exact[ids[i, j]] == dists[i, j]


def test_duplicate_adjacency_is_outside_the_domain(tmp_path):
    vecs = np.array([[0] * 4, [10] * 4, [20] * 4], np.uint8)
    adj = [[1, 1], [0, 2], [1]]
    write_index(tmp_path / "dup", vecs, adj, 0, 4, *exact_pq(vecs))
    ix = O.HostIndex.from_files(tmp_path, "uint8")
    with pytest.raises(RuntimeError):
        O.search(ix, np.zeros((1, 4), np.float32), 2, 8, early_exit=O.EXIT_NONE)


def test_gpruning_invariants(small_u8_index):
    ix = O.HostIndex.from_files(small_u8_index["dir"], "uint8")
    q = small_u8_index["queries"].astype(np.float32)
    ids_n, _, _, hops_n = O.search(ix, q, 10, 96, early_exit=O.EXIT_NONE)
    ids_g, _, _, hops_g = O.search(ix, q, 10, 96, early_exit=O.EXIT_GPRUNING)
    assert (hops_g <= hops_n).all()
    # warmup 10 + patience 8: the earliest stop is at step 17
    assert (hops_g >= np.minimum(17, hops_n)).all()
    ids_p, _, _, hops_p = O.search(ix, q, 10, 96, early_exit=O.EXIT_GPRUNING, patience=10**6)
    np.testing.assert_array_equal(hops_p, hops_n)
    np.testing.assert_array_equal(ids_p, ids_n)


def test_recall_grows_with_ef(small_u8_index):
    ix = O.HostIndex.from_files(small_u8_index["dir"], "uint8")
    q = small_u8_index["queries"].astype(np.float32)
    r = []
    for ef in (16, 48, 160):
        ids, _, _, _ = O.search(ix, q, 10, ef, early_exit=O.EXIT_NONE)
        r.append(O.recall(ids, small_u8_index["gt"], 10))
    assert r[0] < r[1] < r[2]
    assert r[2] >= 0.9


def test_pipe_width_lanes_expand_more_per_round(small_u8_index):
    ix = O.HostIndex.from_files(small_u8_index["dir"], "uint8")
    q = small_u8_index["queries"].astype(np.float32)[:50]
    _, _, _, h1 = O.search(ix, q, 10, 64, pipe_width=1, early_exit=O.EXIT_NONE)
    _, _, _, h4 = O.search(ix, q, 10, 64, pipe_width=4, early_exit=O.EXIT_NONE)
    # speculative lanes expand at least as many nodes in total
    assert h4.sum() >= h1.sum()


def test_timed_search_matches_untimed(small_u8_index):
    """The CPU baseline's timed search returns the same answers and one positive
    wall time per query."""
    ix = small_u8_index
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    q = ix["queries"][:64].astype(np.float32)
    ids0, d0, f0, h0 = O.search(host, q, 10, 64, early_exit=O.EXIT_NONE)
    secs = np.zeros(q.shape[0], np.float64)
    ids1, d1, f1, h1 = O.search(host, q, 10, 64, early_exit=O.EXIT_NONE, seconds=secs)
    np.testing.assert_array_equal(ids0, ids1)
    np.testing.assert_array_equal(d0, d1)
    np.testing.assert_array_equal(h0, h1)
    assert (secs > 0).all() and (secs < 10).all()
    with pytest.raises(ValueError):
        O.search(host, q, 10, 64, seconds=np.zeros(3))
