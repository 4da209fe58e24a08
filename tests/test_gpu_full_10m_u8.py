"""Mid-scale uint8 throughput configuration at its full size (runs on the MI355X).

10M uint8 vectors of dimension 128 from the seeded mixture with 8192 centres
(sigma 20, centres in [32, 224]), a Vamana graph R=64 / L=100 / alpha=1.2 and
PQ 32x256 built on the GPU (320 MB of codes, a 3.9 GiB page image, the 20.5 GB
neighbour code table), 2000 queries from the same mixture, top-10, ef over
the sweep range 32-160.  Every case must give ids, distances, found counts and
hop counts identical to the oracle, and Recall@10 within 0.002 of it.
"""
from __future__ import annotations

import numpy as np
import pytest

import qv_oracle as O
from gpu_workloads import Workload, same, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def w():
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    say("[gpu] 10M u8: 8192 centres, GPU build R=64 L=100 PQ 32x256")
    wl = Workload(n=10_000_000, dim=128, dtype="uint8", centers=8192, sigma=20.0, seed=0x5EED_0002, R=64, L=100,
                  M=32, nq=2000)
    assert (wl.info.max_m0, wl.info.node_size, wl.info.nodes_per_page) == (64, 388, 10)
    yield wl
    wl.close()


@pytest.mark.parametrize("policy", ["none", "gpruning"])
@pytest.mark.parametrize("ef", [32, 96, 160])
def test_10m_u8_sweep_points(w, ef, policy):
    want = w.oracle(ef, policy)
    for kernel in ("lut", "shared-pivots"):
        say(f"[gpu] 10M u8 ef={ef} {policy} kernel={kernel} (no code table)")
        rc, got = w.search(w.q, ef, policy, kernel)
        assert rc == 0, w.L.qv_last_error()
        same(got, want, f"10M {kernel} ef={ef} {policy}")
    assert abs(O.recall(got[0], w.gt, 10) - O.recall(want[0], w.gt, 10)) <= 0.002


@pytest.mark.parametrize("pipe", [1, 2])
@pytest.mark.parametrize("ef", [32, 96, 160])
def test_10m_u8_code_table(w, ef, pipe):
    """The neighbour code table with the shared-pivot kernel (the throughput
    path), pipe widths 1 and 2, early exit off and gpruning."""
    w.neighbour_codes(True)
    try:
        for policy in ("none", "gpruning"):
            say(f"[gpu] 10M u8 code table ef={ef} W={pipe} {policy}")
            rc, got = w.search(w.q, ef, policy, "shared-pivots", pipe=pipe)
            assert rc == 0, w.L.qv_last_error()
            same(got, w.oracle(ef, policy, pipe=pipe), f"10M table ef={ef} W={pipe} {policy}")
    finally:
        w.neighbour_codes(False)


def test_10m_u8_recall_at_sweep_top(w):
    """Recall@10 rises with ef over the sweep, and the oracle and the GPU agree
    on it at every point (both use the same ids)."""
    rs = [O.recall(w.oracle(ef, "none")[0], w.gt, 10) for ef in (32, 96, 160)]
    assert rs[0] < rs[1] < rs[2]
    assert rs[2] > 0.8, rs
