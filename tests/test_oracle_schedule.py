"""Hand-traced known answers for the oracle's gpruning stop rule and its
pipe-width (W >= 2) lane schedule (CPU only).

The reference rules being pinned:
* gpruning (kernel_q1.cuh:294-315 after the boot hop, :524-545 after every
  pipe hop): the step counter is 1 after the entry's expansion and grows by one
  per expansion; "improved" is found count up, or top-1 distance down, or the
  k-th distance down (all strict); before step `warmup` the no-improvement
  count is reset, from step `warmup` on it counts consecutive steps without
  improvement, and the query stops at the first step >= warmup whose count
  reaches `patience` (patience 0 never stops).
* the pipe (kernel_q1.cuh:367-372, 462-653): after the boot expansion, lanes
  1..W-1 take select_next_no_compact (the first unvisited beam entry,
  kernel_helpers.cuh:491-518); every iteration expands each lane holding a
  node, in lane order, and each expansion selects that lane's next node; a
  lane whose expansion found nothing sits out the rest of that iteration and
  asks select_next_no_compact in the next one; the query ends when no lane
  holds a node.  A stop requested by one lane does not skip the lanes after it
  in the same iteration (the stop is tested after the lane loop, :602).

Every expected value below was derived by hand from those rules -- the
derivations are in the comments -- not by running the oracle.  PQ is exact here
(one chunk per dimension, pivots 0..255), so beam keys are exact squared
distances, ties broken by node id.  An off-by-one in the stop step, a `<=` in
an improvement test, a dropped improvement term, a warmup that counts one step
late, a stop that skips the remaining lanes, or a different lane order each
fails at least one case.
"""
from __future__ import annotations

import numpy as np
import pytest

import qv_oracle as O
from index_fixtures import exact_pq, write_index


def _index(tmp_path, name, xs, adj, entry):
    vecs = np.array([[x] * 4 for x in xs], np.uint8)
    R = max(len(a) for a in adj)
    write_index(tmp_path / name, vecs, adj, entry, R, *exact_pq(vecs))
    return O.HostIndex.from_files(tmp_path, "uint8")


def _q(x):
    return np.full(4, x, np.float32)


# ---- the line 0 - 1 - ... - 39, node v at 6v, entry 0 ------------------------
# A query at node m is at squared distance 144 (v - m)^2 from node v.  From the
# entry the beam walks up the line one node per step.  The entry re-enters the
# beam unvisited as a neighbour of node 1 (it is expanded but never inserted)
# and is taken again once it is the beam's first unvisited entry.

@pytest.fixture()
def line40(tmp_path):
    adj = [[1]] + [[v - 1, v + 1] for v in range(1, 39)] + [[38]]
    return _index(tmp_path, "line40", [6 * v for v in range(40)], adj, 0)


def test_line_without_early_exit(line40):
    # q at node 20: d(0) = 57600 is above every node up the line, so nodes
    # 0..39 in order, then the entry again, then nothing unvisited: 41 hops.
    ids, dists, found, hops, order = O.search_trace(line40, _q(120), 1, 64, early_exit=O.EXIT_NONE)
    assert hops == 41
    assert order == list(range(40)) + [0]
    assert (ids[0], dists[0], found) == (20, 0.0, 1)


@pytest.mark.parametrize("patience,stop", [(8, 29), (9, 30), (1, 22), (19, 40), (20, 41), (0, 41)])
def test_gpruning_stop_is_patience_steps_after_the_last_improvement(line40, patience, stop):
    # k = 1, q at node 20, warmup 10: the top-1 distance falls at steps 1..21
    # (node 20 is expanded at step 21) and never again, so steps 22, 23, ...
    # count 1, 2, ... and the stop is step 21 + patience.  Patience 20 fires at
    # step 41, the walk's last step; patience 0 never fires.
    _, _, _, hops, order = O.search_trace(line40, _q(120), 1, 64, early_exit=O.EXIT_GPRUNING,
                                          warmup=10, patience=patience)
    assert hops == stop
    assert order == (list(range(40)) + [0])[:stop]


@pytest.mark.parametrize("warmup,patience,stop", [(25, 2, 26), (25, 1, 25), (10, 2, 11), (3, 2, 8)])
def test_gpruning_counts_nothing_before_warmup(line40, warmup, patience, stop):
    # k = 1, q at node 5: the last improvement is step 6 (node 5 expanded).
    # Steps below warmup reset the count, so it is 1 at step max(warmup, 7) and
    # the stop is at max(warmup, 7) + patience - 1:
    #   (25, 2): 25 -> 1, 26 -> 2: stop 26      (25, 1): stop 25
    #   (10, 2): 10 -> 1, 11 -> 2: stop 11      (3, 2): 7 -> 1, 8 -> 2: stop 8
    _, _, _, hops, _ = O.search_trace(line40, _q(30), 1, 64, early_exit=O.EXIT_GPRUNING,
                                      warmup=warmup, patience=patience)
    assert hops == stop


def test_gpruning_kth_distance_counts_as_improvement(line40):
    # k = 3, q at node 5 (d = 3600, 2304, 1296, 576, 144, 0, 144, 576, 1296, 2304,
    # 3600 for nodes 0..10).  Steps 1-3 fill the top-k, steps 4-6 lower the
    # top-1.  Step 7 expands node 6 (144): top-3 [5:0, 4:144, 3:576] becomes
    # [5:0, 4:144, 6:144] (ties keep the first found first) and only the 3rd
    # distance improves (576 -> 144).  Steps 8, 9, 10 (nodes 7, 8, 9) improve
    # nothing; step 11 takes the entry (3600, ties node 10 and wins on id).
    # warmup 2, patience 4: counts 1..4 at steps 8..11 -> stop at 11.  Without
    # the k-th-distance term the count would start at step 7 and stop at 10.
    ids, dists, found, hops, order = O.search_trace(line40, _q(30), 3, 64, early_exit=O.EXIT_GPRUNING,
                                                    warmup=2, patience=4)
    assert hops == 11
    assert order == [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 0]
    assert list(ids) == [5, 4, 6] and list(dists) == [0, 144, 144] and found == 3


def test_gpruning_found_count_counts_as_improvement(line40):
    # k = 3, q at node 0.  Step 1 expands 0 (d 0); step 2 expands 1 (144), and
    # the entry re-enters the beam at distance 0, so step 3 expands 0 again
    # (the top-k then holds it twice: [0:0, 0:0, 1:144]); step 4 expands 2
    # (576 > 144).  Step 2 improves only by the found count (top-1 stays 0, the
    # 3rd distance stays +inf); step 3 by the count and the 3rd distance.
    # warmup 0, patience 1: step 4 is the first without improvement -> stop 4.
    # Without the found-count term step 2 would stop the query.
    ids, dists, found, hops, order = O.search_trace(line40, _q(0), 3, 64, early_exit=O.EXIT_GPRUNING,
                                                    warmup=0, patience=1)
    assert hops == 4
    assert order == [0, 1, 0, 2]
    assert list(ids) == [0, 0, 1] and list(dists) == [0, 0, 144] and found == 3


# ---- a branching graph for the pipe lanes -------------------------------------
# node:      0      1     2      3      4    5     6
# position:  0      60    50     40     90   70    100     query at 100
# d:         40000  6400  10000  14400  400  3600  0
# edges:     0:[1,2,3]  1:[0,4]  2:[0,5]  3:[0]  4:[1]  5:[2,6]  6:[5]   entry 0

@pytest.fixture()
def branch(tmp_path):
    adj = [[1, 2, 3], [0, 4], [0, 5], [0], [1], [2, 6], [5]]
    return _index(tmp_path, "branch", [0, 60, 50, 40, 90, 70, 100], adj, 0)


# W = 1: 0 (beam 1 2 3) -> 1 (adds 4, 0) -> 4 -> 2 (adds 5) -> 5 (adds 6) -> 6
#        -> 3 -> 0 (revisit) -> nothing: 8 hops.
# W = 2: boot expands 0 and selects 1; lane 1 takes 2 (first unvisited).
#   it1: lane 0 expands 1 (adds 4, 0; selects 4), lane 1 expands 2 (adds 5;
#        selects 5)
#   it2: lane 0 expands 4 (selects 3), lane 1 expands 5 (adds 6; selects 6)
#   it3: lane 0 expands 3 (selects the entry 0), lane 1 expands 6 (nothing)
#   it4: lane 0 expands 0 (nothing); lane 1 asks again: nothing.  8 hops.
# W = 3: boot selects 1; lanes 1, 2 take 2 and 3.
#   it1: 1 (adds 4, 0; selects 4), 2 (adds 5; selects 5), 3 (selects 0)
#   it2: 4 (nothing), 5 (adds 6; selects 6), 0 (nothing)
#   it3: 6 (nothing); lanes 0 and 2 ask again next: nothing.  8 hops.
SCHEDULES = {
    1: [0, 1, 4, 2, 5, 6, 3, 0],
    2: [0, 1, 2, 4, 5, 3, 6, 0],
    3: [0, 1, 2, 3, 4, 5, 0, 6],
}


@pytest.mark.parametrize("width", [1, 2, 3])
def test_pipe_lane_schedule(branch, width):
    ids, dists, found, hops, order = O.search_trace(branch, _q(100), 3, 16, pipe_width=width,
                                                    early_exit=O.EXIT_NONE)
    assert order == SCHEDULES[width]
    assert hops == 8
    assert list(ids) == [6, 4, 5] and list(dists) == [0, 400, 3600]


# gpruning with warmup 0, patience 1 (top-3 after each step):
# W = 1: [0] [1 0] [4 1 0] [4 1 2] [4 5 1] [6 4 5] then 3 improves nothing:
#        stop at step 7 -> [6 4 5].
# W = 2: [0] [1 0] [1 2 0] [4 1 2] [4 5 1], step 6 (node 3) improves nothing
#        and requests the stop, but lane 1 of the same iteration still expands
#        6 at step 7 -> [6 4 5], 7 hops.
# W = 3: [0] [1 0] [1 2 0] [1 2 3] [4 1 2] [4 5 1], step 7 (the entry, third
#        lane of iteration 2) improves nothing -> stop; node 6 is never reached
#        -> [4 5 1].
@pytest.mark.parametrize("width,order,ids,dists", [
    (1, [0, 1, 4, 2, 5, 6, 3], [6, 4, 5], [0, 400, 3600]),
    (2, [0, 1, 2, 4, 5, 3, 6], [6, 4, 5], [0, 400, 3600]),
    (3, [0, 1, 2, 3, 4, 5, 0], [4, 5, 1], [400, 3600, 6400]),
])
def test_pipe_lanes_with_gpruning(branch, width, order, ids, dists):
    got_ids, got_dists, _, hops, got_order = O.search_trace(branch, _q(100), 3, 16, pipe_width=width,
                                                            early_exit=O.EXIT_GPRUNING, warmup=0, patience=1)
    assert got_order == order
    assert hops == len(order)
    assert list(got_ids) == ids and list(got_dists) == dists


# ---- per-step recall (kernel_q1.cuh:354-364, 662-667) ---------------------------
# q at node 20 (x = 120), k = 3, no early exit: step s <= 21 expands node s - 1,
# so the top-3 after step s is {s-1, s-2, s-3}; step 22 expands 21 (144), which
# ties 19 and enters: [20, 19, 21].  Hits count top-3 ids found anywhere in the
# ground-truth row:
#   row A = [20, 19, 21, 18, 22]: step 19 {18, 17, 16} -> 1, step 20 -> 2, step 21 -> 3
#   row B = [20, 21, 22]:         step 21 -> 1, step 22 -> 2, never 3 (19 stays in the top-3)
ROW_A = [20, 19, 21, 18, 22]
ROW_B = [20, 21, 22]


@pytest.mark.parametrize("row,required,step,hits,hops", [
    (ROW_A, 1, 19, 1, 19), (ROW_A, 2, 20, 2, 20), (ROW_A, 3, 21, 3, 21),
    (ROW_B, 1, 21, 1, 21), (ROW_B, 2, 22, 2, 22), (ROW_B, 3, -1, 2, 41),
])
def test_step_recall_stop(line40, row, required, step, hits, hops):
    out = O.search_trace(line40, _q(120), 3, 64, early_exit=O.EXIT_NONE,
                         step_recall=(np.array(row, np.int32), required))
    assert out[3] == hops
    assert out[5:] == (step, hits)


def test_step_recall_after_gpruning(line40):
    # gpruning (warmup 10, patience 8, k = 3): the last improvement is step 22
    # (the 3rd distance, 576 -> 144), steps 23..30 count 1..8, so the query
    # stops at step 30, before row B's 3 hits are ever reached: step -1 and the
    # final hit count 2
    out = O.search_trace(line40, _q(120), 3, 64, early_exit=O.EXIT_GPRUNING, warmup=10, patience=8,
                         step_recall=(np.array(ROW_B, np.int32), 3))
    assert out[3] == 30 and out[5:] == (-1, 2)


def test_step_recall_batch_rows_and_width_one_only(line40):
    # query i takes ground-truth row i % count
    q = np.stack([_q(120), _q(120), _q(120)])
    gt = np.array([ROW_A, ROW_B[:2] + [-1, -1, -1]], np.int32)
    ids, _, _, hops, step, hits = O.search(line40, q, 3, 64, early_exit=O.EXIT_NONE, step_recall=(gt, 2))
    assert list(step) == [20, 22, 20] and list(hits) == [2, 2, 2] and list(hops) == [20, 22, 20]
    with pytest.raises(RuntimeError):
        O.search(line40, q, 3, 64, pipe_width=2, early_exit=O.EXIT_NONE, step_recall=(gt, 2))


def test_required_hits_known_values():
    # search.cu:100-102 at the CLI's default threshold and k = 10
    assert [O.required_hits(t, 10) for t in (0.9, 0.95, 1.0, 0.1, 0.01, 0.5)] == [9, 10, 10, 1, 1, 5]
