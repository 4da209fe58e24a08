"""Pins of the oracle's arithmetic (CPU only).

Each check is chosen so that a plausible slip -- a dropped centroid, a wrong
chunk index, a tree instead of a sequential sum, a missing fused multiply-add,
an unstable top-k -- fails it.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

import qv_oracle as O


def f32_round(x: Fraction) -> np.float32:
    """Round an exact rational to the nearest float32 (ties to even)."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    q, r = divmod(a, ulp)
    q = int(q)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return np.float32(sign * float(q * ulp))


def exact_lut(q, centroid, pivots_t, chunk_id):
    """The reference's LUT loop (pq_device.cuh:18-31) evaluated with exact
    rationals: q' = fl(q - mu); cell = fl(fma(d, d, cell)) with d = fl(q' - p),
    dimensions in ascending order."""
    dim = q.shape[0]
    M = int(chunk_id.max()) + 1
    lut = [[np.float32(0.0)] * 256 for _ in range(M)]
    qc = [np.float32(np.float32(q[i]) - np.float32(centroid[i])) for i in range(dim)]
    for i in range(dim):
        m = int(chunk_id[i])
        for j in range(256):
            d = np.float32(qc[i] - np.float32(pivots_t[i, j]))
            lut[m][j] = f32_round(Fraction(float(d)) * Fraction(float(d)) + Fraction(float(lut[m][j])))
    return np.array(lut, dtype=np.float32)


def test_lut_exact_rounding_and_closed_form():
    rng = np.random.default_rng(1)
    dim, M = 8, 4
    chunk_id = np.repeat(np.arange(M, dtype=np.int32), dim // M)
    centroid = (rng.random(dim) * 100).astype(np.float32)
    pivots = (rng.standard_normal((256, dim)) * 37.3).astype(np.float32)
    q = rng.integers(0, 256, dim).astype(np.float32)
    lut, q_used = O.lut(dim, centroid, np.ascontiguousarray(pivots.T), chunk_id, q)
    np.testing.assert_array_equal(lut, exact_lut(q, centroid, pivots.T, chunk_id))
    # the same loop without the fused multiply-add rounds differently somewhere
    unfused = np.zeros((M, 256), np.float32)
    for i in range(dim):
        d = np.float32(np.float32(q[i]) - centroid[i]) - pivots[:, i]
        unfused[chunk_id[i]] = unfused[chunk_id[i]] + d * d
    assert (unfused != lut).any()
    # closed form in float64: sum over the chunk of (q - mu - P)^2
    ref = np.zeros((M, 256))
    for i in range(dim):
        ref[chunk_id[i]] += (np.float64(q[i]) - centroid[i] - pivots[:, i].astype(np.float64)) ** 2
    np.testing.assert_allclose(lut, ref, rtol=1e-5)
    assert (lut >= 0).all()
    np.testing.assert_array_equal(q_used, (q - centroid) + centroid)


def test_lut_zero_at_pivot_and_centroid_matters():
    dim = 16
    chunk_id = np.repeat(np.arange(4, dtype=np.int32), 4)
    centroid = np.full(dim, 10.0, np.float32)
    pivots = np.arange(256 * dim, dtype=np.float32).reshape(256, dim) % 50
    q = (centroid + pivots[77]).astype(np.float32)
    lut, _ = O.lut(dim, centroid, np.ascontiguousarray(pivots.T), chunk_id, q)
    assert (lut[:, 77] == 0).all()
    # without the centroid the same query would not hit pivot 77 exactly
    lut0, _ = O.lut(dim, np.zeros(dim, np.float32), np.ascontiguousarray(pivots.T), chunk_id, q)
    assert (lut0[:, 77] > 0).all()


def test_adc_is_sequential_fp32():
    M = 32
    lut = np.zeros((M, 256), np.float32)
    lut[0, 5] = 2.0 ** 24
    lut[1:, 7] = 1.0
    code = np.array([5] + [7] * (M - 1), np.uint8)
    # sequential fp32: 2^24 + 1 rounds back to 2^24 at every step
    assert O.adc(lut, code) == 2.0 ** 24
    # integers below 2^24 are exact in any order
    lut2 = np.arange(M * 256, dtype=np.float32).reshape(M, 256)
    code2 = np.arange(M, dtype=np.uint8) * 3
    assert O.adc(lut2, code2) == sum(int(lut2[m, code2[m]]) for m in range(M))
    rng = np.random.default_rng(2)
    lut3 = rng.random((M, 256), dtype=np.float32) * 1000
    code3 = rng.integers(0, 256, M, dtype=np.uint8)
    exact = sum(float(lut3[m, code3[m]]) for m in range(M))
    assert abs(O.adc(lut3, code3) - exact) <= M * 2 ** -24 * exact


@pytest.mark.parametrize("dtype", [np.uint8, np.int8])
def test_exact_l2_integer_types_bit_exact(dtype):
    rng = np.random.default_rng(3)
    for dim in (128, 100, 17):
        lo, hi = (0, 256) if dtype == np.uint8 else (-128, 128)
        x = rng.integers(lo, hi, dim).astype(dtype)
        q = rng.integers(lo, hi, dim).astype(np.float32)
        ref = int(np.sum((q.astype(np.int64) - x.astype(np.int64)) ** 2))
        assert O.exact_l2(q, x) == ref


def test_exact_l2_float_bound():
    rng = np.random.default_rng(4)
    for dim in (96, 128, 33):
        x = rng.standard_normal(dim).astype(np.float32)
        q = rng.standard_normal(dim).astype(np.float32)
        ref = float(np.sum((q.astype(np.float64) - x) ** 2))
        assert abs(O.exact_l2(q, x) - ref) <= 1e-5 * ref


def test_exact_l2_float_uses_strided_lanes_then_tree():
    # Lane 0 holds 2^24 and lanes 1..31 hold 1.  A sequential sum over the
    # dimensions stays at 2^24 (each +1 is a tie rounded to even).  The
    # shuffle-down tree first adds lane 16 to lane 0 (again a tie: 2^24), then
    # partial sums 2, 4, 8, 16 that are exact: 2^24 + 2 + 4 + 8 + 16.
    q = np.zeros(32, np.float32)
    x = np.ones(32, np.float32)
    x[0] = np.float32(2.0 ** 12)
    got = O.exact_l2(q, x)
    assert got == 2.0 ** 24 + 30


def test_recall_reference_known_answer():
    # bin/common/search_setup_test.cpp:67-81
    results = np.array([[1, 2, 3], [8, 9, 10]], np.int32)
    gt = np.array([[3, 2, 1, 4], [7, 8, 11, 12]], np.int32)
    assert O.recall(results[:1], gt[:1], 3) == 1.0
    assert abs(O.recall(results[1:], gt[1:], 3) - 1 / 3) < 1e-12
    assert abs(O.recall(results, gt, 3) - 4 / 6) < 1e-12


def test_recall_against_reference_header():
    ref = O.reference_recall_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    rng = np.random.default_rng(5)
    res = rng.integers(0, 50, (200, 10)).astype(np.int32)
    gt = rng.integers(0, 50, (200, 20)).astype(np.int32)
    want = ref.ref_calc_recall(res.ctypes.data, gt.ctypes.data, 200, 20, 10)
    assert O.recall(res, gt, 10) == want


def test_adc_topk_matches_sort_by_dist_then_position():
    rng = np.random.default_rng(6)
    M = 16
    lut = (rng.integers(0, 8, (M, 256))).astype(np.float32)  # many ties
    codes = rng.integers(0, 256, (300, M), dtype=np.uint8)
    ids = rng.integers(0, 300, 2000).astype(np.int32)
    gi, gd, gs = O.adc_topk(lut, codes, ids, 10)
    d = np.array([O.adc(lut, codes[i]) for i in ids], np.float32)
    order = np.lexsort((np.arange(ids.size), d))[:10]
    np.testing.assert_array_equal(gi, ids[order])
    np.testing.assert_array_equal(gd, d[order])
    assert abs(gs - d.astype(np.float64).sum()) < 1e-6 * gs


def test_ground_truth_brute_force():
    rng = np.random.default_rng(7)
    base = rng.integers(0, 256, (500, 24), dtype=np.uint8)
    q = rng.integers(0, 256, (5, 24)).astype(np.float32)
    ids, dists = O.ground_truth(base, q, 7)
    for i in range(5):
        d = ((base.astype(np.int64) - q[i].astype(np.int64)) ** 2).sum(1)
        order = np.lexsort((np.arange(500), d))[:7]
        np.testing.assert_array_equal(ids[i], order)
        np.testing.assert_array_equal(dists[i], d[order].astype(np.float32))
