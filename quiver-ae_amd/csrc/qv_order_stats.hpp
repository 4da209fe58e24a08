// Order statistics of a search's per-query latencies (the report's P50 /
// P90 / P99 / P99.9 / max): several ranks of one array by radix selection.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <vector>

namespace qv {

// Unsigned key whose order is the double's order (NaN excluded): negative
// values flip every bit, the others set the sign bit.
inline uint64_t order_key(double x) {
  uint64_t b;
  std::memcpy(&b, &x, sizeof(b));
  return (b >> 63) ? ~b : (b | (1ull << 63));
}

inline double from_order_key(uint64_t k) {
  const uint64_t b = (k >> 63) ? (k & ~(1ull << 63)) : ~k;
  double x;
  std::memcpy(&x, &b, sizeof(x));
  return x;
}

// out[j] = the element of rank r[j] (0-based, ascending) of v[0, n), for
// j < m; every r[j] < n, v holds no NaN and is not modified.  Three passes
// over v -- the keys and their range, a histogram of the 11 key bits below
// the highest bit on which the keys differ, and the gathering of the buckets
// that hold the ranks -- then a selection inside each such bucket.  (Four
// nth_element passes over the latencies of a 10k-query search cost several
// times as much.)
inline void select_ranks(const double* v, size_t n, const size_t* r, int m, double* out) {
  if (n == 0 || m <= 0) return;
  std::vector<uint64_t> keys(n);
  uint64_t lo = ~0ull, hi = 0;
  for (size_t i = 0; i < n; i++) {
    const uint64_t k = order_key(v[i]);
    keys[i] = k;
    lo = std::min(lo, k);
    hi = std::max(hi, k);
  }
  if (lo == hi) {
    for (int j = 0; j < m; j++) out[j] = v[0];
    return;
  }
  constexpr int kBits = 11;
  const int top = 63 - __builtin_clzll(lo ^ hi);  // highest differing bit
  const int shift = std::max(0, top + 1 - kBits);
  const uint64_t mask = (top + 1 - shift >= 64) ? ~0ull : ((1ull << (top + 1 - shift)) - 1);
  std::vector<uint32_t> start((1u << kBits) + 1, 0);
  for (size_t i = 0; i < n; i++) start[((keys[i] >> shift) & mask) + 1]++;
  for (size_t b = 1; b < start.size(); b++) start[b] += start[b - 1];
  // the bucket of each rank; each wanted bucket gathered once
  std::vector<int> bucket_of(m);
  std::vector<int> slot((size_t)1 << kBits, -1);
  std::vector<std::vector<uint64_t>> got;
  for (int j = 0; j < m; j++) {
    const int b = (int)(std::upper_bound(start.begin(), start.end(), (uint32_t)r[j]) - start.begin()) - 1;
    bucket_of[j] = b;
    if (slot[(size_t)b] < 0) {
      slot[(size_t)b] = (int)got.size();
      got.emplace_back();
      got.back().reserve(start[(size_t)b + 1] - start[(size_t)b]);
    }
  }
  for (size_t i = 0; i < n; i++) {
    const int s = slot[(size_t)((keys[i] >> shift) & mask)];
    if (s >= 0) got[(size_t)s].push_back(keys[i]);
  }
  for (int j = 0; j < m; j++) {
    const int b = bucket_of[j];
    std::vector<uint64_t>& g = got[(size_t)slot[(size_t)b]];
    const size_t local = r[j] - start[(size_t)b];
    std::nth_element(g.begin(), g.begin() + (std::ptrdiff_t)local, g.end());
    out[j] = from_order_key(g[local]);
  }
}

}  // namespace qv
