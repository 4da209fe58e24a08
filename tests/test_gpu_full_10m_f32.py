"""Float configuration at its full size (runs on the MI355X).

10M float vectors of dimension 96 from the seeded mixture with 4096 centres
and unit-variance noise, each row L2-normalised; a Vamana graph R=64 / L=100 /
alpha=1.2 and PQ 48x256 (2 dims per chunk) built on the GPU; 2000 queries from
the same mixture; top-10; ef 45-200.  ids, distances, found counts and hop
counts must equal the oracle's.  The fp32 exact distances are bit-identical to
the oracle's (the reference's lane order), and within 1e-5 relative of the
float64 squared distance of the same pair.
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
    say("[gpu] 10M f32 d96: 4096 centres, GPU build R=64 L=100 PQ 48x256")
    wl = Workload(n=10_000_000, dim=96, dtype="float", centers=4096, sigma=1.0, seed=0x5EED_0003, R=64, L=100,
                  M=48, nq=2000)
    assert (wl.info.max_m0, wl.info.node_size, wl.info.nodes_per_page) == (64, 644, 6)
    yield wl
    wl.close()


@pytest.mark.parametrize("ef", [45, 128, 200])
def test_10m_f32_matches_oracle(w, ef):
    want = w.oracle(ef, "none")
    for kernel in ("lut", "shared-pivots"):
        say(f"[gpu] 10M f32 ef={ef} kernel={kernel}")
        rc, got = w.search(w.q, ef, "none", kernel)
        assert rc == 0, w.L.qv_last_error()
        same(got, want, f"10M f32 {kernel} ef={ef}")
    # rerank tolerance of the float path: 1e-5 relative against float64
    ids, dists = got[0], got[1]
    for i in range(0, w.nq, 97):
        for j in range(10):
            x = w.host.vector(int(ids[i, j])).astype(np.float64)
            ref = float(np.sum((w.q[i].astype(np.float64) - x) ** 2))
            assert abs(float(dists[i, j]) - ref) <= 1e-5 * max(ref, 1e-30), (i, j, dists[i, j], ref)


@pytest.mark.parametrize("pipe,policy", [(1, "gpruning"), (2, "none"), (2, "gpruning")])
def test_10m_f32_code_table(w, pipe, policy):
    """48-byte code rows from the neighbour code table (3 KB blocks)."""
    w.neighbour_codes(True)
    try:
        for ef in (96, 200):
            say(f"[gpu] 10M f32 code table ef={ef} W={pipe} {policy}")
            rc, got = w.search(w.q, ef, policy, "shared-pivots", pipe=pipe)
            assert rc == 0, w.L.qv_last_error()
            same(got, w.oracle(ef, policy, pipe=pipe), f"10M f32 table ef={ef} W={pipe} {policy}")
    finally:
        w.neighbour_codes(False)
