"""The oracle's nav-graph entry search (inkernel_nav_entry,
src/quiver/kernel_core/inkernel_nav.cuh:61-200) against known answers:

- complete nav graphs (every node lists all others, n <= 29 so one 28-wide row
  read covers them): the first hop sees every node, so the entry is the exact
  nearest nav node;
- chains and a trap: a 4-wide beam that only expands its four best ends at the
  best node reachable through them;
- 1-, 2- and 3-node graphs, traced by hand: with fewer than four distinct
  nodes a selection round swaps an empty slot into slot 0 (all candidates
  +inf, the argmin stays at lane 0); the shuffle-down tournament's tie rule
  decides whether slot 0 is refilled;
- rows narrower than 28 (max_m = 4): the 28 reads of one node span the next
  six rows, each warp's seven stop at its first -1 only.

Plus the nav files written by the library's builder, read back by the
oracle's own NumPy reader.
"""
from __future__ import annotations

import numpy as np
import pytest

import qv_oracle as O


def _complete(n: int) -> np.ndarray:
    g = np.full((n, 28), -1, np.int32)
    for i in range(n):
        others = [j for j in range(n) if j != i]
        g[i, :len(others)] = others
    return g


def _l2_64(q: np.ndarray, x: np.ndarray) -> np.ndarray:
    return ((x.astype(np.float64) - q.astype(np.float64)[None, :]) ** 2).sum(axis=1)


@pytest.mark.parametrize("n", [5, 12, 29])
@pytest.mark.parametrize("dtype", ["uint8", "float"])
def test_complete_graph_finds_nearest(n, dtype):
    rng = np.random.default_rng(100 + n)
    dim = 100 if dtype == "uint8" else 24
    if dtype == "uint8":
        data = rng.integers(0, 256, (n, dim), dtype=np.uint8)
    else:
        data = rng.standard_normal((n, dim)).astype(np.float32)
    mapping = rng.permutation(10 * n)[:n].astype(np.int32)
    for start in (0, n - 1):
        nav = O.HostNav.from_arrays(data, _complete(n), mapping, start=start)
        for t in range(40):
            if dtype == "uint8":
                q = rng.integers(0, 256, dim).astype(np.float32)  # integer sums: exact in fp32
            else:
                q = rng.standard_normal(dim).astype(np.float32)
            d = _l2_64(q, data)
            got = O.nav_entry(nav, q, fallback=-7)
            best = np.flatnonzero(d == d.min())
            assert got in set(mapping[best].tolist()), (start, t)


def _hand_chain_nav(n: int, width: int = 28):
    """Chain 0-1-...-(n-1) on the line, rows padded with -1 to `width`."""
    data = (np.arange(n, dtype=np.float32) * 10.0)[:, None].repeat(2, axis=1)
    g = np.full((n, width), -1, np.int32)
    for i in range(n):
        nb = [j for j in (i - 1, i + 1) if 0 <= j < n]
        g[i, :len(nb)] = nb
    return data, g


@pytest.mark.parametrize("k", [4, 9, 17])
def test_full_width_chain(k):
    data, g = _hand_chain_nav(18)
    mapping = np.arange(18, dtype=np.int32) + 500
    nav = O.HostNav.from_arrays(data, g, mapping, start=0)
    q = np.full(2, 10.0 * k + 2.0, np.float32)
    assert O.nav_entry(nav, q) == 500 + k


def test_beam_of_four_stops_at_local_minimum():
    # Start 0 at the origin; six cluster nodes 1..6 at x = 1..6 hang off it.
    # Node 1 (the cluster node farthest from the query) is the only way to the
    # bridge B = 7 (x = 50) and the target T = 8 (x = 100).  The query sits at
    # x = 99: the beam keeps nodes 6, 5, 4, 3 as its best four and never
    # expands node 1, so the entry is node 6 although T is nearer.
    x = np.array([0, 1, 2, 3, 4, 5, 6, 50, 100], np.float32)
    data = x[:, None].repeat(3, axis=1)
    adj = {0: [1, 2, 3, 4, 5, 6], 1: [0, 7], 2: [0], 3: [0], 4: [0], 5: [0], 6: [0], 7: [1, 8], 8: [7]}
    g = np.full((9, 28), -1, np.int32)
    for i, nb in adj.items():
        g[i, :len(nb)] = nb
    mapping = np.arange(9, dtype=np.int32) * 3
    nav = O.HostNav.from_arrays(data, g, mapping, start=0)
    assert O.nav_entry(nav, np.full(3, 99.0, np.float32)) == 6 * 3
    # the same graph with the bridge on node 6 reaches T
    adj[1], adj[6], adj[7] = [0], [0, 7], [6, 8]
    g[:] = -1
    for i, nb in adj.items():
        g[i, :len(nb)] = nb
    nav = O.HostNav.from_arrays(data, g, mapping, start=0)
    assert O.nav_entry(nav, np.full(3, 99.0, np.float32)) == 8 * 3


@pytest.mark.parametrize("n", [2, 3])
def test_tiny_graph_traced(n):
    # Nodes at x = 0, 10, 20 (complete graph), query x = 1, start 0; traced
    # by hand.  Hop 1 ends with round 3 (n = 3; round 2 for n = 2) seeing
    # every slot >= i at +inf: the argmin result stays lane 0 and, as
    # +inf != 1, slot 0 (node 0) swaps with the empty slot i.  Hop 2 writes
    # node 0 (unvisited) into slot 4, level with node 0's old copy in slot 2
    # (n = 2) or 3 (n = 3).  The shuffle-down tournament keeps the lower lane
    # of each pair on ties, so at offset 4 lane 0 takes slot 4's copy and at
    # offset 1 it keeps it against lane 1's (slot 2 or 3): slot 4 wins
    # (a first-index argmin would pick the older copy).  Round 1's duplicate
    # merge then gives slot 0 the visited bit and sets the old copy to +inf,
    # and the later empty-slot swap moves that +inf copy (id 0) into slot 0,
    # so the entry is node 0 again.  A first-index argmin ends with slot 0
    # empty for n = 2.
    data = (np.arange(n, dtype=np.float32) * 10.0)[:, None]
    nav = O.HostNav.from_arrays(data, _complete(n), np.arange(n, dtype=np.int32) + 40, start=0)
    assert O.nav_entry(nav, np.array([1.0], np.float32), fallback=-3) == 40


def test_self_loop_single_node_ends_empty():
    # One node whose only neighbour is itself: hop 1 writes it into slot 4
    # (tied with slot 0, lane 0 keeps slot 0), round 1 turns the copy into a
    # duplicate (+inf) and swaps slot 0 with empty slot 1, nothing refills
    # slot 0, and the search stops with slot 0 empty.  The reference reads
    # nav_mapping[0x7fffffff] there; the restatement returns the fallback.
    data = np.array([[3.0, 4.0]], np.float32)
    g = np.array([[0, -1, -1]], np.int32)
    nav = O.HostNav.from_arrays(data, g, np.array([9], np.int32), start=0)
    assert O.nav_entry(nav, np.array([0.0, 0.0], np.float32), fallback=-3) == -3


def test_four_node_graph_has_no_empty_slot():
    data = (np.arange(4, dtype=np.float32) * 10.0)[:, None]
    nav = O.HostNav.from_arrays(data, _complete(4), np.arange(4, dtype=np.int32) + 40, start=0)
    for qx, want in ((1.0, 40), (12.0, 41), (19.0, 42), (33.0, 43)):
        assert O.nav_entry(nav, np.array([qx], np.float32), fallback=-3) == want


def test_narrow_rows_read_into_following_rows():
    # max_m = 4, 8 nodes.  The 28 reads from node u start at row u and span
    # rows u..u+6; warp w takes reads [7w, 7w+7) and stops at its first -1.
    # From node 0: warp 0 reads row 0 = [1] and stops; warp 1 reads row 1[3],
    # row 2, row 3[0..1]; warp 2 reads row 3[2..3] = [2, 7], row 4, row 5[0];
    # warp 3 reads row 5[1..3], row 6.  Node 7 (x = 500) sits at the query.
    x = np.array([0, 200, 210, 300, 220, 230, 240, 500], np.float32)
    data = x[:, None].repeat(2, axis=1)
    rows = {0: [1], 1: [0], 2: [1, 4], 3: [0, 1, 2, 7], 4: [1, 2], 5: [4], 6: [5], 7: [3]}
    g = np.full((8, 4), -1, np.int32)
    for i, nb in rows.items():
        g[i, :len(nb)] = nb
    mapping = np.arange(8, dtype=np.int32) + 70
    nav = O.HostNav.from_arrays(data, g, mapping, start=0)
    # Through listed neighbours alone, 0 and 1 only reach each other (entry
    # node 1 = 71); the spill-over of warp 2 shows node 7 at the first hop.
    assert O.nav_entry(nav, np.full(2, 490.0, np.float32)) == 77
    # Row 3 cut to [0]: warp 2 now reads row 3[2] = -1 and stops, warp 1 reads
    # row 1[3] = -1 and stops, warp 3 reads row 5[1] = -1; node 1's reads
    # (rows 1..7) reach nodes 4 and 2 (warp 1: row 2 = [1, 4]; ...) but never 7.
    g[3, 1:] = -1
    nav = O.HostNav.from_arrays(data, g, mapping, start=0)
    got = O.nav_entry(nav, np.full(2, 490.0, np.float32))
    assert got != 77


def test_nav_files_round_trip(tmp_path):
    import quiver

    rng = np.random.default_rng(5)
    rows = rng.integers(0, 256, (600, 32), dtype=np.uint8)
    ids = (np.arange(600, dtype=np.int32) * 7 + 3)
    quiver.build_nav(rows, ids, tmp_path / "nav", R=28, L=48, threads=4)
    nav = O.HostNav.from_dir(tmp_path / "nav", "uint8")
    assert nav.num_node == 600 and nav.dim == 32 and nav.max_m == 28
    np.testing.assert_array_equal(nav.data, rows)
    np.testing.assert_array_equal(nav.mapping, ids)
    assert 0 <= nav.start < 600
    deg = (nav.graph >= 0).sum(axis=1)
    assert deg.min() >= 1 and deg.max() <= 28
    # -1 only after each degree, no self loops, no repeated neighbours
    for i in range(600):
        r = nav.graph[i]
        assert (r[:deg[i]] >= 0).all() and (r[deg[i]:] == -1).all()
        assert i not in r[:deg[i]] and len(set(r[:deg[i]].tolist())) == deg[i]
    # the graph is navigable: the nav search finds the exact nearest sample
    # for most queries drawn near sample rows
    hits = 0
    for t in range(100):
        q = (rows[rng.integers(600)].astype(np.float32) + rng.normal(0, 2, 32)).astype(np.float32)
        d = _l2_64(q, rows)
        hits += O.nav_entry(nav, q) == ids[int(d.argmin())]
    assert hits >= 80


def test_search_with_nav_entry_beats_medoid_hops(small_u8_index, tmp_path):
    """Whole oracle search started from the nav entry: same or better recall
    and fewer hops than from the medoid on the clustered 20k index."""
    import quiver

    ix = small_u8_index
    base = ix["base"]
    sample = np.arange(0, base.shape[0], 10, dtype=np.int32)
    quiver.build_nav(base[sample], sample, tmp_path / "nav", R=28, L=64, threads=0)
    nav = O.HostNav.from_dir(tmp_path / "nav", "uint8")
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    q = ix["queries"][:150].astype(np.float32)
    ids0, _, _, hops0 = O.search(host, q, 10, 64, early_exit=O.EXIT_NONE)
    ids1, _, _, hops1 = O.search(host, q, 10, 64, early_exit=O.EXIT_NONE, nav=nav)
    r0 = O.recall(ids0, ix["gt"][:150], 10)
    r1 = O.recall(ids1, ix["gt"][:150], 10)
    assert r1 >= r0 - 0.01
    assert hops1.mean() < hops0.mean()
    # every query's entry is a sampled node
    for i in range(20):
        e = O.nav_entry(nav, q[i], fallback=-1)
        assert e in set(sample.tolist())
