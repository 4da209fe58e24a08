"""The HIP search against hand-traced answers of the gpruning stop rule and of
the pipe-lane schedule (runs on the MI355X).

The graphs, queries and expected values are the ones derived by hand in
tests/test_oracle_schedule.py (a 40-node line and a 7-node branching graph with
exact PQ); here the GPU kernel must reproduce the ids, distances and hop counts
of those traces directly.
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

from index_fixtures import exact_pq, write_index

pytestmark = pytest.mark.gpu


def _open(lib, tmp_path, name, xs, adj, entry):
    vecs = np.array([[x] * 4 for x in xs], np.uint8)
    d = tmp_path / name
    d.mkdir()
    write_index(d / "g", vecs, adj, entry, max(len(a) for a in adj), *exact_pq(vecs))
    h = C.c_void_p()
    lib.check(lib.load().qv_index_open(str(d).encode(), b"uint8", b"heap", None, 0, C.byref(h)))
    return h


def _run(lib, h, x, k, ef, width, policy, warmup=10, patience=8, sr=None):
    """One query at position x; sr = (ground-truth row, threshold) turns on
    per-step recall and appends (step, hits) to the result."""
    o = lib.default_search_opts()
    o.pipe_width = width
    o.early_exit = lib.QV_EXIT_GPRUNING if policy == "gpruning" else lib.QV_EXIT_NONE
    o.gpruning_warmup, o.gpruning_patience = warmup, patience
    if sr is not None:
        gt = np.ascontiguousarray(np.array(sr[0], np.int32).reshape(1, -1))
        sr_out = np.full(2, -7, np.int32)
        o.step_recall_gt, o.step_recall_gt_width, o.step_recall_gt_count = gt.ctypes.data, gt.shape[1], 1
        o.step_recall_threshold = sr[1]
        o.step_recall_step, o.step_recall_hits = sr_out.ctypes.data, sr_out.ctypes.data + 4
    q = np.full((1, 4), x, np.float32)
    ids = np.empty((1, k), np.int32)
    dists = np.empty((1, k), np.float32)
    found = np.empty(1, np.int32)
    lib.check(lib.load().qv_search(h, q.ctypes.data, 1, 4, k, ef, C.byref(o), ids.ctypes.data,
                                   dists.ctypes.data, found.ctypes.data, None))
    hops = np.empty(1, np.int32)
    lib.check(lib.load().qv_last_hops(h, hops.ctypes.data, 1))
    out = (list(ids[0]), list(dists[0]), int(found[0]), int(hops[0]))
    return out + (int(sr_out[0]), int(sr_out[1])) if sr is not None else out


@pytest.fixture(scope="module")
def lib():
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    return _lib


def test_line_gpruning_known_answers(lib, tmp_path):
    print("[gpu] line graph gpruning known answers", flush=True)
    adj = [[1]] + [[v - 1, v + 1] for v in range(1, 39)] + [[38]]
    h = _open(lib, tmp_path, "line", [6 * v for v in range(40)], adj, 0)
    try:
        assert _run(lib, h, 120, 1, 64, 1, "none") == ([20], [0.0], 1, 41)
        for patience, stop in ((8, 29), (9, 30), (1, 22), (19, 40), (20, 41), (0, 41)):
            assert _run(lib, h, 120, 1, 64, 1, "gpruning", 10, patience)[3] == stop, patience
        for warmup, patience, stop in ((25, 2, 26), (25, 1, 25), (10, 2, 11), (3, 2, 8)):
            assert _run(lib, h, 30, 1, 64, 1, "gpruning", warmup, patience)[3] == stop, (warmup, patience)
        assert _run(lib, h, 30, 3, 64, 1, "gpruning", 2, 4) == ([5, 4, 6], [0.0, 144.0, 144.0], 3, 11)
        assert _run(lib, h, 0, 3, 64, 1, "gpruning", 0, 1) == ([0, 0, 1], [0.0, 0.0, 144.0], 3, 4)
        # per-step recall (k = 3: thresholds 0.3 / 0.6 / 0.9 need 1 / 2 / 3 hits)
        row_a, row_b = [20, 19, 21, 18, 22], [20, 21, 22]
        for row, t, step, hits, hops in ((row_a, 0.3, 19, 1, 19), (row_a, 0.6, 20, 2, 20), (row_a, 0.9, 21, 3, 21),
                                         (row_b, 0.3, 21, 1, 21), (row_b, 0.6, 22, 2, 22), (row_b, 1.0, -1, 2, 41)):
            got = _run(lib, h, 120, 3, 64, 1, "none", sr=(row, t))
            assert (got[3], got[4], got[5]) == (hops, step, hits), (row, t)
        got = _run(lib, h, 120, 3, 64, 1, "gpruning", 10, 8, sr=(row_b, 1.0))
        assert (got[3], got[4], got[5]) == (30, -1, 2)
    finally:
        lib.load().qv_index_close(h)


def test_branching_pipe_lanes_known_answers(lib, tmp_path):
    print("[gpu] branching graph pipe-lane known answers", flush=True)
    adj = [[1, 2, 3], [0, 4], [0, 5], [0], [1], [2, 6], [5]]
    h = _open(lib, tmp_path, "branch", [0, 60, 50, 40, 90, 70, 100], adj, 0)
    try:
        for width in (1, 2, 3):
            assert _run(lib, h, 100, 3, 16, width, "none") == ([6, 4, 5], [0.0, 400.0, 3600.0], 3, 8), width
        assert _run(lib, h, 100, 3, 16, 1, "gpruning", 0, 1) == ([6, 4, 5], [0.0, 400.0, 3600.0], 3, 7)
        assert _run(lib, h, 100, 3, 16, 2, "gpruning", 0, 1) == ([6, 4, 5], [0.0, 400.0, 3600.0], 3, 7)
        assert _run(lib, h, 100, 3, 16, 3, "gpruning", 0, 1) == ([4, 5, 1], [400.0, 3600.0, 6400.0], 3, 7)
    finally:
        lib.load().qv_index_close(h)
