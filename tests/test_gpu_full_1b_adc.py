"""Billion-point ADC microbenchmark configuration at its full size (runs on
the MI355X).

1B x 32-byte PQ code rows (32 GB of uniform random bytes) in HBM, 10k query
LUTs (M = 32 x 256 fp32, built from 128-d uint8 queries), 200 hops x 64
uniform ids per query: the ADC gather-sum with top-10 over all 128M
evaluations in one launch, as the benchmark runs it.  For a sample of queries
the top-10 (ids and distances) must equal the oracle's sequential ADC over the
same rows, and each query's float64 distance sum must agree to 1e-9.  The
code rows the oracle reads are produced on the host by an independent numpy
restatement of the counter-based generator (SplitMix64, Steele, Lea and Flood
2014), itself checked against the first rows of the device table.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import qv_oracle as O
from gpu_workloads import say

pytestmark = pytest.mark.gpu

NCODES, M, NQ, HOPS, K = 1_000_000_000, 32, 10_000, 200, 10
PER_Q = HOPS * 64
SEED_CODES, SEED_IDS, STREAM_BYTES = 0xC0DE, 0x1D5, 4
_U = np.uint64


def _mix64(z):
    z = z + _U(0x9E3779B97F4A7C15)
    z = (z ^ (z >> _U(30))) * _U(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> _U(27))) * _U(0x94D049BB133111EB)
    return z ^ (z >> _U(31))


def _rng_u64(seed: int, stream: int, counter):
    with np.errstate(over="ignore"):
        s = _mix64(np.array([(seed + stream * 0xD1B54A32D192ED03) % 2**64], np.uint64))
        return _mix64(s ^ np.asarray(counter, np.uint64))


def _rows(ids: np.ndarray) -> np.ndarray:
    """Code rows [len(ids), 32] of the table: 8-byte word w is rng_u64(seed, 4, w)."""
    words = (ids.astype(np.uint64)[:, None] * _U(4) + np.arange(4, dtype=np.uint64)[None, :]).ravel()
    return _rng_u64(SEED_CODES, STREAM_BYTES, words).view(np.uint8).reshape(len(ids), 32)


def test_adc_1b_codes_matches_oracle():
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    L = _lib.load()
    say("[gpu] ADC 1B x 32 B codes: fill 32 GB, 128M ids, 10k LUTs")
    codes = _lib.DeviceBuffer(NCODES * M)
    _lib.check(L.qv_fill_uniform_bytes(codes.ptr, NCODES * M, SEED_CODES, 0))
    ids = _lib.DeviceBuffer(NQ * PER_Q * 4)
    _lib.check(L.qv_fill_uniform_ids(ids.ptr, NQ * PER_Q, NCODES, SEED_IDS, 0))
    rng = np.random.default_rng(5)
    pivots_t = (rng.random((128, 256), dtype=np.float32) * 255).astype(np.float32)
    centroid = np.full(128, 128.0, np.float32)
    offs = np.arange(0, 129, 4, dtype=np.int32)
    qs = rng.integers(0, 256, (NQ, 128)).astype(np.float32)
    d_p = _lib.DeviceBuffer(pivots_t.nbytes).upload(pivots_t)
    d_c = _lib.DeviceBuffer(centroid.nbytes).upload(centroid)
    d_o = _lib.DeviceBuffer(offs.nbytes).upload(offs)
    d_q = _lib.DeviceBuffer(qs.nbytes).upload(qs)
    luts = _lib.DeviceBuffer(NQ * M * 256 * 4)
    _lib.check(L.qv_lut_build_raw(d_c.ptr, d_p.ptr, d_o.ptr, 128, M, d_q.ptr, NQ, luts.ptr, None, 0))
    oi, od, osum = _lib.DeviceBuffer(NQ * K * 4), _lib.DeviceBuffer(NQ * K * 4), _lib.DeviceBuffer(NQ * 8)
    ms = C.c_float()
    say("[gpu] ADC 1B: one launch over all 10k queries")
    _lib.check(L.qv_adc_bench(luts.ptr, M, codes.ptr, NCODES, ids.ptr, NQ, PER_Q, K, oi.ptr, od.ptr, osum.ptr, 0,
                              C.byref(ms)))
    assert ms.value > 0
    # the host restatement of the table against its first 4096 rows and its last row
    head = codes.download(np.uint8, (4096, M))
    np.testing.assert_array_equal(head, _rows(np.arange(4096)))
    gi, gd = oi.download(np.int32, (NQ, K)), od.download(np.float32, (NQ, K))
    gs = osum.download(np.float64, (NQ,))
    all_ids = ids.download(np.int32, (NQ, PER_Q))
    assert all_ids.min() >= 0 and all_ids.max() < NCODES and all_ids.max() > NCODES - NCODES // 1000
    all_luts = luts.download(np.float32, (NQ, M, 256))
    sample = list(range(0, NQ, 157)) + [NQ - 1]
    say(f"[gpu] ADC 1B: oracle over {len(sample)} queries")
    for i in sample:
        rows = _rows(all_ids[i])
        pos, dist, dsum = O.adc_topk(all_luts[i], rows, np.arange(PER_Q, dtype=np.int32), K)
        np.testing.assert_array_equal(gd[i], dist, err_msg=f"query {i}")
        np.testing.assert_array_equal(gi[i], all_ids[i][pos], err_msg=f"query {i}")
        assert abs(gs[i] - dsum) <= 1e-9 * abs(dsum), i
    for b in (codes, ids, luts, oi, od, osum, d_p, d_c, d_o, d_q):
        b.close()
