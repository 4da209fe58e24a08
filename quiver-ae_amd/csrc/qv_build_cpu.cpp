// qv_build_cpu.cpp -- CPU index construction in DiskANN's formats.
//
// DiskANN (deps/DiskANN, an empty submodule in the reference) is what the
// reference uses to build its indexes.  This file provides the same product
// from a clean description of the published algorithms:
//   * PQ: centre the data on its mean, split the dimensions into M contiguous
//     chunks, run Lloyd k-means (256 centres) per chunk, encode every point to
//     its nearest centre per chunk (DiskANN generate_pq_pivots / generate_pq_data).
//   * Graph: Vamana (Subramanya et al., NeurIPS 2019): insert points in a
//     random order; each point runs a greedy beam search of width L from the
//     medoid, RobustPrune(alpha, R) of the visited set gives its out-edges, and
//     every out-neighbour receives the reverse edge, pruned again when it
//     overflows R.  Optional first pass with alpha = 1.
// Adjacency lists are duplicate-free, which the search kernels require.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <mutex>
#include <numeric>
#include <vector>

#include <omp.h>

#include "qv_common.hpp"
#include "qv_mixture.hpp"

namespace qv {
namespace {

struct Base {
  const uint8_t* p;
  int dtype;
  int64_t n;
  int dim;
  float at(int64_t i, int j) const {
    if (dtype == QV_FLOAT) return reinterpret_cast<const float*>(p)[i * dim + j];
    if (dtype == QV_INT8) return (float)reinterpret_cast<const int8_t*>(p)[i * dim + j];
    return (float)p[i * dim + j];
  }
  // Squared L2 between two base points.
  float dist(int64_t a, int64_t b) const {
    if (dtype == QV_UINT8) {
      const uint8_t* x = p + a * dim;
      const uint8_t* y = p + b * dim;
      int32_t s = 0;
      for (int j = 0; j < dim; j++) {
        int32_t d = (int32_t)x[j] - (int32_t)y[j];
        s += d * d;
      }
      return (float)s;
    }
    if (dtype == QV_INT8) {
      const int8_t* x = reinterpret_cast<const int8_t*>(p) + a * dim;
      const int8_t* y = reinterpret_cast<const int8_t*>(p) + b * dim;
      int32_t s = 0;
      for (int j = 0; j < dim; j++) {
        int32_t d = (int32_t)x[j] - (int32_t)y[j];
        s += d * d;
      }
      return (float)s;
    }
    const float* x = reinterpret_cast<const float*>(p) + a * dim;
    const float* y = reinterpret_cast<const float*>(p) + b * dim;
    float s = 0.f;
    for (int j = 0; j < dim; j++) {
      float d = x[j] - y[j];
      s += d * d;
    }
    return s;
  }
  float dist_to(const float* q, int64_t b) const {
    float s = 0.f;
    for (int j = 0; j < dim; j++) {
      float d = q[j] - at(b, j);
      s += d * d;
    }
    return s;
  }
};

// ------------------------------------------------------------------ PQ ----
void train_pq(const Base& B, const qv_build_params& prm, PQTables& t) {
  const int d = B.dim, M = prm.num_chunks;
  if (M <= 0 || M > d) fail(QV_EINVAL, "num_chunks must be in [1, dim]");
  t.dim = d;
  t.num_chunks = M;
  t.num_pts = B.n;
  t.chunk_offsets.resize((size_t)M + 1);
  for (int i = 0; i <= M; i++) t.chunk_offsets[(size_t)i] = (int32_t)(((int64_t)i * d) / M);
  t.chunk_id.assign((size_t)d, 0);
  for (int i = 0; i < M; i++)
    for (int j = t.chunk_offsets[(size_t)i]; j < t.chunk_offsets[(size_t)i + 1]; j++) t.chunk_id[(size_t)j] = i;

  // Training sample: a seeded subset without replacement (partial shuffle).
  const int64_t ns = std::min<int64_t>(B.n, prm.pq_train_max > 0 ? prm.pq_train_max : 262144);
  std::vector<int64_t> sample((size_t)B.n);
  std::iota(sample.begin(), sample.end(), 0);
  for (int64_t i = 0; i < ns; i++) {
    int64_t j = i + (int64_t)(rng_u64(prm.seed, 11, (uint64_t)i) % (uint64_t)(B.n - i));
    std::swap(sample[(size_t)i], sample[(size_t)j]);
  }
  sample.resize((size_t)ns);

  // Mean of the sample (float64 accumulation).
  std::vector<double> acc((size_t)d, 0.0);
  for (int64_t s : sample)
    for (int j = 0; j < d; j++) acc[(size_t)j] += B.at(s, j);
  t.centroid.resize((size_t)d);
  for (int j = 0; j < d; j++) t.centroid[(size_t)j] = (float)(acc[(size_t)j] / (double)ns);

  t.pivots.assign((size_t)kNumPivots * d, 0.f);
  std::vector<float> X((size_t)ns * d);
  for (int64_t i = 0; i < ns; i++)
    for (int j = 0; j < d; j++) X[(size_t)i * d + j] = B.at(sample[(size_t)i], j) - t.centroid[(size_t)j];

  for (int m = 0; m < M; m++) {
    const int o = t.chunk_offsets[(size_t)m], w = t.chunk_offsets[(size_t)m + 1] - o;
    if (w == 0) continue;
    std::vector<float> C((size_t)kNumPivots * w);
    for (int c = 0; c < kNumPivots; c++) {
      int64_t pick = (int64_t)(rng_u64(prm.seed, 12 + (uint64_t)m, (uint64_t)c) % (uint64_t)ns);
      for (int j = 0; j < w; j++) C[(size_t)c * w + j] = X[(size_t)pick * d + o + j];
    }
    std::vector<int> assign((size_t)ns, 0);
    for (int it = 0; it < std::max(1, prm.kmeans_iters); it++) {
#pragma omp parallel for schedule(static) num_threads(prm.threads)
      for (int64_t i = 0; i < ns; i++) {
        const float* x = &X[(size_t)i * d + o];
        float best = INFINITY;
        int bi = 0;
        for (int c = 0; c < kNumPivots; c++) {
          float s = 0.f;
          for (int j = 0; j < w; j++) {
            float df = x[j] - C[(size_t)c * w + j];
            s += df * df;
          }
          if (s < best) { best = s; bi = c; }
        }
        assign[(size_t)i] = bi;
      }
      std::vector<double> sum((size_t)kNumPivots * w, 0.0);
      std::vector<int64_t> cnt((size_t)kNumPivots, 0);
      for (int64_t i = 0; i < ns; i++) {
        int c = assign[(size_t)i];
        cnt[(size_t)c]++;
        for (int j = 0; j < w; j++) sum[(size_t)c * w + j] += X[(size_t)i * d + o + j];
      }
      for (int c = 0; c < kNumPivots; c++) {
        if (cnt[(size_t)c] == 0) {  // re-seed an empty centre
          int64_t pick = (int64_t)(rng_u64(prm.seed, 400 + (uint64_t)m, (uint64_t)(it * 256 + c)) % (uint64_t)ns);
          for (int j = 0; j < w; j++) C[(size_t)c * w + j] = X[(size_t)pick * d + o + j];
        } else {
          for (int j = 0; j < w; j++) C[(size_t)c * w + j] = (float)(sum[(size_t)c * w + j] / (double)cnt[(size_t)c]);
        }
      }
    }
    for (int c = 0; c < kNumPivots; c++)
      for (int j = 0; j < w; j++) t.pivots[(size_t)c * d + o + j] = C[(size_t)c * w + j];
  }
  t.pivots_t.assign((size_t)d * kNumPivots, 0.f);
  for (int c = 0; c < kNumPivots; c++)
    for (int j = 0; j < d; j++) t.pivots_t[(size_t)j * kNumPivots + c] = t.pivots[(size_t)c * d + j];

  // Encode every point.
  t.codes.assign((size_t)B.n * M, 0);
#pragma omp parallel for schedule(static) num_threads(prm.threads)
  for (int64_t i = 0; i < B.n; i++) {
    std::vector<float> x((size_t)d);
    for (int j = 0; j < d; j++) x[(size_t)j] = B.at(i, j) - t.centroid[(size_t)j];
    for (int m = 0; m < M; m++) {
      const int o = t.chunk_offsets[(size_t)m], w = t.chunk_offsets[(size_t)m + 1] - o;
      float best = INFINITY;
      int bi = 0;
      for (int c = 0; c < kNumPivots; c++) {
        float s = 0.f;
        for (int j = 0; j < w; j++) {
          float df = x[(size_t)(o + j)] - t.pivots[(size_t)c * d + o + j];
          s += df * df;
        }
        if (s < best) { best = s; bi = c; }
      }
      t.codes[(size_t)i * M + m] = (uint8_t)bi;
    }
  }
}

// -------------------------------------------------------------- Vamana ----
struct Graph {
  int R;
  std::vector<uint32_t> adj;  // [n][R]
  std::vector<uint32_t> deg;  // [n]
  std::vector<std::mutex> locks;
  Graph(int64_t n, int r) : R(r), adj((size_t)n * r), deg((size_t)n, 0), locks((size_t)n) {}
};

struct Cand {
  float d;
  uint32_t id;
  bool operator<(const Cand& o) const { return d < o.d || (d == o.d && id < o.id); }
};

// Greedy beam search from `start` towards base point p; returns the expanded set.
void greedy_search(const Base& B, Graph& G, int64_t p, uint32_t start, int L,
                   std::vector<Cand>& visited, std::vector<uint32_t>& seen_stamp, uint32_t stamp) {
  std::vector<Cand> beam;
  std::vector<char> expanded;
  beam.push_back({B.dist(p, start), start});
  expanded.push_back(0);
  seen_stamp[start] = stamp;
  visited.clear();
  std::vector<uint32_t> nb;
  while (true) {
    int pick = -1;
    for (size_t i = 0; i < beam.size(); i++)
      if (!expanded[i]) { pick = (int)i; break; }
    if (pick < 0) break;
    expanded[(size_t)pick] = 1;
    const uint32_t v = beam[(size_t)pick].id;
    visited.push_back(beam[(size_t)pick]);
    {
      std::lock_guard<std::mutex> g(G.locks[v]);
      nb.assign(G.adj.begin() + (size_t)v * G.R, G.adj.begin() + (size_t)v * G.R + G.deg[v]);
    }
    for (uint32_t u : nb) {
      if (seen_stamp[u] == stamp) continue;
      seen_stamp[u] = stamp;
      Cand c{B.dist(p, u), u};
      if ((int)beam.size() >= L && !(c < beam.back())) continue;
      auto it = std::lower_bound(beam.begin(), beam.end(), c);
      size_t pos = (size_t)(it - beam.begin());
      beam.insert(it, c);
      expanded.insert(expanded.begin() + (ptrdiff_t)pos, 0);
      if ((int)beam.size() > L) {
        beam.pop_back();
        expanded.pop_back();
      }
    }
  }
}

// RobustPrune(p, C, alpha, R) with C sorted ascending by distance to p.
void robust_prune(const Base& B, int64_t p, std::vector<Cand>& C, float alpha, int R,
                  std::vector<uint32_t>& out) {
  out.clear();
  std::sort(C.begin(), C.end());
  C.erase(std::unique(C.begin(), C.end(), [](const Cand& a, const Cand& b) { return a.id == b.id; }),
          C.end());
  std::vector<char> dead(C.size(), 0);
  for (size_t i = 0; i < C.size() && (int)out.size() < R; i++) {
    if (dead[i] || (int64_t)C[i].id == p) continue;
    out.push_back(C[i].id);
    for (size_t j = i + 1; j < C.size(); j++) {
      if (dead[j]) continue;
      if (alpha * B.dist(C[i].id, C[j].id) <= C[j].d) dead[j] = 1;
    }
  }
}

void vamana_pass(const Base& B, Graph& G, uint32_t medoid, const qv_build_params& prm,
                 float alpha, const std::vector<int64_t>& order) {
  const int R = G.R;
  std::vector<std::vector<uint32_t>> stamps;
  int nt = prm.threads;
  stamps.resize((size_t)nt);
#pragma omp parallel num_threads(nt)
  {
    auto& st = stamps[(size_t)omp_get_thread_num()];
    st.assign((size_t)B.n, 0);
    uint32_t stamp = 0;
    std::vector<Cand> visited, cand;
    std::vector<uint32_t> pruned, tmp;
#pragma omp for schedule(dynamic, 64)
    for (int64_t oi = 0; oi < (int64_t)order.size(); oi++) {
      const int64_t p = order[(size_t)oi];
      if (++stamp == 0) {
        std::fill(st.begin(), st.end(), 0);
        stamp = 1;
      }
      greedy_search(B, G, p, medoid, prm.L, visited, st, stamp);
      cand = visited;
      {
        std::lock_guard<std::mutex> g(G.locks[(size_t)p]);
        for (uint32_t k = 0; k < G.deg[(size_t)p]; k++) {
          uint32_t u = G.adj[(size_t)p * R + k];
          cand.push_back({B.dist(p, u), u});
        }
      }
      robust_prune(B, p, cand, alpha, R, pruned);
      {
        std::lock_guard<std::mutex> g(G.locks[(size_t)p]);
        G.deg[(size_t)p] = (uint32_t)pruned.size();
        std::copy(pruned.begin(), pruned.end(), G.adj.begin() + (size_t)p * R);
      }
      for (uint32_t q : pruned) {
        std::lock_guard<std::mutex> g(G.locks[q]);
        uint32_t* aq = &G.adj[(size_t)q * R];
        uint32_t dq = G.deg[q];
        bool present = false;
        for (uint32_t k = 0; k < dq; k++) present |= (aq[k] == (uint32_t)p);
        if (present) continue;
        if ((int)dq < R) {
          aq[dq] = (uint32_t)p;
          G.deg[q] = dq + 1;
        } else {
          cand.clear();
          for (uint32_t k = 0; k < dq; k++) cand.push_back({B.dist(q, aq[k]), aq[k]});
          cand.push_back({B.dist(q, p), (uint32_t)p});
          robust_prune(B, q, cand, alpha, R, tmp);
          G.deg[q] = (uint32_t)tmp.size();
          std::copy(tmp.begin(), tmp.end(), aq);
        }
      }
    }
  }
}

}  // namespace

void build_index_cpu(const void* base, int dtype, int64_t n, int dim,
                     const qv_build_params& prm_in, const std::string& prefix) {
  qv_build_params prm = prm_in;
  if (prm.threads <= 0) prm.threads = omp_get_num_procs();
  if (n <= 1 || n > (int64_t)INT32_MAX) fail(QV_EINVAL, "n must be in [2, 2^31)");
  if (prm.R <= 0 || prm.R > kMaxDegree) fail(QV_EINVAL, "R must be in [1, 128]");
  if (prm.L < prm.R) fail(QV_EINVAL, "L must be >= R");
  Base B{static_cast<const uint8_t*>(base), dtype, n, dim};

  PQTables pq;
  train_pq(B, prm, pq);

  // Medoid: the point nearest to the mean of all points.
  std::vector<double> mean((size_t)dim, 0.0);
  for (int64_t i = 0; i < n; i++)
    for (int j = 0; j < dim; j++) mean[(size_t)j] += B.at(i, j);
  std::vector<float> meanf((size_t)dim);
  for (int j = 0; j < dim; j++) meanf[(size_t)j] = (float)(mean[(size_t)j] / (double)n);
  int64_t medoid = 0;
  float best = INFINITY;
  for (int64_t i = 0; i < n; i++) {
    float dd = B.dist_to(meanf.data(), i);
    if (dd < best) { best = dd; medoid = i; }
  }

  Graph G(n, prm.R);
  std::vector<int64_t> order((size_t)n);
  std::iota(order.begin(), order.end(), 0);
  for (int64_t i = n - 1; i > 0; i--) {
    int64_t j = (int64_t)(rng_u64(prm.seed, 21, (uint64_t)i) % (uint64_t)(i + 1));
    std::swap(order[(size_t)i], order[(size_t)j]);
  }
  if (prm.passes >= 2) vamana_pass(B, G, (uint32_t)medoid, prm, 1.0f, order);
  vamana_pass(B, G, (uint32_t)medoid, prm, prm.alpha, order);

  Layout lay;
  lay.data_type = dtype;
  lay.num_data = n;
  lay.num_dims = dim;
  lay.max_m0 = prm.R;
  lay.enter_point = medoid;
  lay.data_size = (int64_t)dim * elem_size(dtype);
  lay.node_size = lay.data_size + 4 + 4ll * prm.R;
  if (lay.node_size > kPageSize) fail(QV_EINVAL, "node record exceeds one 4 KB page");
  lay.nodes_per_page = kPageSize / lay.node_size;
  lay.num_pages = (n + lay.nodes_per_page - 1) / lay.nodes_per_page;
  write_diskann_index(prefix + "_disk.index", lay, base, G.adj, G.deg);
  write_pq_tables(prefix + "_pq_pivots.bin", prefix + "_pq_compressed.bin", pq);
}

// Navigation graph over sample rows (their base ids in ids): a Vamana graph
// of degree R <= 32 over the sample, start = the sample's medoid, written in
// the format NavGraph::init reads (nav_graph.cu:12-73).
void build_nav_cpu(const void* rows, const int32_t* ids, int64_t s, int dim, int dtype,
                   const qv_build_params& prm_in, const std::string& dir) {
  qv_build_params prm = prm_in;
  if (prm.threads <= 0) prm.threads = omp_get_num_procs();
  if (s <= 1 || s > (int64_t)INT32_MAX) fail(QV_EINVAL, "sample size must be in [2, 2^31)");
  if (prm.R <= 0 || prm.R > 32) fail(QV_EINVAL, "nav graph degree must be in [1, 32]");
  if (prm.L < prm.R) fail(QV_EINVAL, "L must be >= R");
  Base B{static_cast<const uint8_t*>(rows), dtype, s, dim};
  std::vector<double> mean((size_t)dim, 0.0);
  for (int64_t i = 0; i < s; i++)
    for (int j = 0; j < dim; j++) mean[(size_t)j] += B.at(i, j);
  std::vector<float> meanf((size_t)dim);
  for (int j = 0; j < dim; j++) meanf[(size_t)j] = (float)(mean[(size_t)j] / (double)s);
  int64_t medoid = 0;
  float best = INFINITY;
  for (int64_t i = 0; i < s; i++) {
    const float dd = B.dist_to(meanf.data(), i);
    if (dd < best) {
      best = dd;
      medoid = i;
    }
  }
  Graph G(s, prm.R);
  std::vector<int64_t> order((size_t)s);
  std::iota(order.begin(), order.end(), 0);
  for (int64_t i = s - 1; i > 0; i--) {
    const int64_t j = (int64_t)(rng_u64(prm.seed, 23, (uint64_t)i) % (uint64_t)(i + 1));
    std::swap(order[(size_t)i], order[(size_t)j]);
  }
  if (prm.passes >= 2) vamana_pass(B, G, (uint32_t)medoid, prm, 1.0f, order);
  vamana_pass(B, G, (uint32_t)medoid, prm, prm.alpha, order);

  NavGraphHost nav;
  nav.num_node = (int32_t)s;
  nav.dims = dim;
  nav.max_m = prm.R;
  nav.start = (int32_t)medoid;
  const size_t bytes = (size_t)s * (size_t)dim * (size_t)elem_size(dtype);
  nav.data.assign(static_cast<const uint8_t*>(rows), static_cast<const uint8_t*>(rows) + bytes);
  nav.graph.assign((size_t)s * prm.R, -1);
  for (int64_t v = 0; v < s; v++) {
    if (G.deg[(size_t)v] == 0) fail(QV_EINDEX, "nav graph node without neighbours (duplicate sample rows?)");
    for (uint32_t k = 0; k < G.deg[(size_t)v]; k++)
      nav.graph[(size_t)v * prm.R + k] = (int32_t)G.adj[(size_t)v * prm.R + k];
  }
  nav.mapping.assign(ids, ids + s);
  write_nav(dir, dtype, nav);
}

}  // namespace qv
