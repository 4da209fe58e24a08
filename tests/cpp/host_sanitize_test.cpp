// host_sanitize_test.cpp -- the host-only C++ of libquiver_hip (file formats,
// CPU index builder, C ABI helpers, synthetic data) and the CPU oracle, built
// with AddressSanitizer and UndefinedBehaviorSanitizer (g++/gcc only; no GPU
// code is compiled or run).  It builds small uint8 and float indexes and a nav
// graph, reads them back through the same readers the library uses, searches
// them with the oracle (plain, gpruning, pipe width 2, nav entry), drives
// the error paths with malformed files and arguments, and checks the search
// report's order statistics (qv_order_stats.hpp) against a full sort.  Any sanitizer report
// aborts the program (-fno-sanitize-recover=all); a failed check exits 1.
//
// usage: host_sanitize_test WORK_DIR
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <string>
#include <vector>

#include "qv_common.hpp"
#include "qv_oracle.h"
#include "qv_order_stats.hpp"
#include "quiver_hip.h"

namespace {

int g_failures = 0;

void expect(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAILED: %s (last error: %s)\n", what, qv_last_error());
    g_failures++;
  }
}

struct Built {
  qv_index_info info{};
  std::vector<uint8_t> pages;
  qv::PQTables pq;
  qvo_index ix{};
};

// Reads an index written by the CPU builder back through the library's readers
// and wraps it for the oracle.
bool load(const std::string& dir, const char* dtype, Built& b) {
  char index_file[4096], prefix[4096];
  if (qv_find_index_files(dir.c_str(), index_file, prefix, sizeof(index_file)) != QV_OK) return false;
  if (qv_read_layout(index_file, dtype, &b.info) != QV_OK) return false;
  b.pages.resize((size_t)b.info.num_pages * 4096);
  if (qv_read_index_pages(index_file, b.info.num_pages, b.pages.data()) != QV_OK) return false;
  qv::read_pq_tables(std::string(prefix) + "_pivots.bin", std::string(prefix) + "_compressed.bin", b.pq);
  b.ix.dtype = (int)b.info.data_type;
  b.ix.dim = (int)b.info.num_dims;
  b.ix.num_points = b.info.num_data;
  b.ix.max_m = (int)b.info.max_m0;
  b.ix.medoid = b.info.enter_point;
  b.ix.node_size = b.info.node_size;
  b.ix.nodes_per_page = b.info.nodes_per_page;
  b.ix.data_size = b.info.data_size;
  b.ix.pages = b.pages.data();
  b.ix.num_chunks = b.pq.num_chunks;
  b.ix.codes = b.pq.codes.data();
  b.ix.centroid = b.pq.centroid.data();
  b.ix.pivots_t = b.pq.pivots_t.data();
  b.ix.chunk_id = b.pq.chunk_id.data();
  return true;
}

// Oracle searches of queries against base; returns Recall@10 against brute force.
double search_recall(const Built& b, const std::vector<uint8_t>& base, int dtype, const std::vector<float>& q,
                     int nq, const qvo_search_params& p) {
  const int k = 10;
  std::vector<int32_t> ids((size_t)nq * k), found((size_t)nq), hops((size_t)nq), gt((size_t)nq * k);
  std::vector<float> dists((size_t)nq * k), gtd((size_t)nq * k);
  expect(qvo_search(&b.ix, q.data(), nq, &p, 2, ids.data(), dists.data(), found.data(), hops.data()) == QVO_OK,
         "oracle search");
  for (int32_t id : ids) expect(id >= -1 && id < b.info.num_data, "result id in range");
  for (int i = 0; i < nq; i++) expect(hops[(size_t)i] >= 1, "at least one hop");
  qvo_ground_truth(base.data(), dtype, b.info.num_data, (int)b.info.num_dims, q.data(), nq, k, 2, gt.data(),
                   gtd.data());
  return qvo_recall(ids.data(), gt.data(), nq, k, k);
}

std::vector<uint8_t> mixture(int dtype, int64_t first, int64_t rows, int dim, uint64_t seed) {
  qv_mixture m{};
  m.seed = seed;
  m.num_centers = 16;
  m.dim = dim;
  m.data_type = dtype;
  m.center_lo = 32.f;
  m.center_hi = 224.f;
  m.sigma = dtype == QV_FLOAT ? 1.f : 20.f;
  m.normalize = dtype == QV_FLOAT ? 1 : 0;
  std::vector<uint8_t> v((size_t)(rows * dim * (dtype == QV_FLOAT ? 4 : 1)));
  expect(qv_mixture_fill_host(&m, first, rows, v.data()) == QV_OK, "mixture");
  return v;
}

std::vector<float> as_float(const std::vector<uint8_t>& raw, int dtype) {
  if (dtype == QV_FLOAT) {
    std::vector<float> f(raw.size() / 4);
    std::memcpy(f.data(), raw.data(), raw.size());
    return f;
  }
  return std::vector<float>(raw.begin(), raw.end());
}

void truncate_copy(const std::string& from, const std::string& to, size_t keep) {
  std::ifstream in(from, std::ios::binary);
  std::vector<char> buf(keep);
  in.read(buf.data(), (std::streamsize)keep);
  std::ofstream(to, std::ios::binary).write(buf.data(), in.gcount());
}

}  // namespace

// select_ranks against std::sort: n from 1 to 100k; latencies spread and
// clustered, integer-valued with many ties, all equal, zeros, negatives and
// denormals; ranks at the report's percentiles, both ends and at random.
void check_order_stats() {
  uint64_t s = 0x0DDBA11;
  auto next = [&]() {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return s;
  };
  auto unit = [&]() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); };
  int cases = 0, bad = 0;
  for (size_t n : {(size_t)1, (size_t)2, (size_t)3, (size_t)17, (size_t)1000, (size_t)10000, (size_t)100000}) {
    for (int kind = 0; kind < 7; kind++) {
      std::vector<double> v(n);
      for (size_t i = 0; i < n; i++) {
        const double u = unit();
        switch (kind) {
          case 0: v[i] = 0.3 + 4.0 * u; break;                             // a batch's latencies
          case 1: v[i] = std::exp(8.0 * u - 4.0); break;                   // many binades
          case 2: v[i] = (double)(next() % 7); break;                      // few values, many ties
          case 3: v[i] = 1.25; break;                                      // all equal
          case 4: v[i] = u < 0.5 ? 0.0 : u; break;                         // zeros
          case 5: v[i] = 2.0 * u - 1.0; break;                             // negatives
          default: v[i] = (u < 0.3 ? 4.9e-324 * (double)(next() % 5) : u * 1e-300); break;  // denormals
        }
      }
      std::vector<double> sorted = v;
      std::sort(sorted.begin(), sorted.end());
      std::vector<size_t> r = {n / 2, (size_t)(0.9 * (double)n), (size_t)(0.99 * (double)n),
                               (size_t)(0.999 * (double)n), n - 1, 0, (size_t)(next() % n), (size_t)(next() % n)};
      for (size_t& x : r) x = std::min(x, n - 1);
      std::vector<double> out(r.size());
      const std::vector<double> before = v;
      qv::select_ranks(v.data(), n, r.data(), (int)r.size(), out.data());
      cases++;
      bool ok = v == before;
      for (size_t j = 0; j < r.size(); j++) ok = ok && out[j] == sorted[r[j]];
      if (!ok) {
        bad++;
        std::fprintf(stderr, "order statistics differ: n=%zu kind=%d\n", n, kind);
      }
    }
  }
  expect(bad == 0, "select_ranks equals the sorted order statistics");
  expect(cases == 49, "order statistics cases run");
}

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s WORK_DIR\n", argv[0]);
    return 2;
  }
  namespace fs = std::filesystem;
  const fs::path work = argv[1];
  fs::create_directories(work);

  for (int dtype : {QV_UINT8, QV_FLOAT}) {
    const int dim = dtype == QV_FLOAT ? 24 : 32, n = 3000, nq = 60;
    const char* dname = dtype == QV_FLOAT ? "float" : "uint8";
    const std::vector<uint8_t> base = mixture(dtype, 0, n, dim, 0xA5A5 + (uint64_t)dtype);
    const std::vector<float> q = as_float(mixture(dtype, 1 << 20, nq, dim, 0xA5A5 + (uint64_t)dtype), dtype);
    const fs::path dir = work / dname;
    fs::create_directories(dir);
    qv_build_params p;
    qv_build_params_default(&p);
    p.R = 24;
    p.L = 48;
    p.num_chunks = dim / 4;
    p.threads = 2;
    p.kmeans_iters = 4;
    expect(qv_build_index_cpu(base.data(), dtype, n, dim, &p, (dir / "ix").c_str()) == QV_OK, "CPU build");
    Built b;
    expect(load(dir.string(), dname, b), "read back");
    if (g_failures) return 1;
    expect(b.info.num_data == n && b.info.max_m0 == 24, "layout");

    qvo_search_params sp{};
    sp.topk = 10;
    sp.ef_search = 64;
    sp.pipe_width = 1;
    sp.early_exit = QVO_EXIT_NONE;
    sp.gpruning_warmup = 10;
    sp.gpruning_patience = 8;
    const double r1 = search_recall(b, base, dtype, q, nq, sp);
    expect(r1 > 0.5, "recall of the plain search");
    sp.early_exit = QVO_EXIT_GPRUNING;
    sp.pipe_width = 2;
    search_recall(b, base, dtype, q, nq, sp);

    // a nav graph over every 7th point, read back and used as the entry
    std::vector<int32_t> ids;
    std::vector<uint8_t> rows;
    const size_t esz = dtype == QV_FLOAT ? 4 : 1;
    for (int i = 0; i < n; i += 7) {
      ids.push_back(i);
      rows.insert(rows.end(), base.begin() + (size_t)i * dim * esz, base.begin() + (size_t)(i + 1) * dim * esz);
    }
    qv_build_params np = p;
    np.R = 12;
    np.L = 24;
    expect(qv_build_nav(rows.data(), ids.data(), (int64_t)ids.size(), dim, dtype, &np, (dir / "nav").c_str()) ==
               QV_OK,
           "nav build");
    qv::NavGraphHost nav;
    qv::read_nav((dir / "nav").string(), dtype, n, dim, nav);
    qvo_nav on{};
    on.dtype = dtype;
    on.dim = dim;
    on.num_node = nav.num_node;
    on.max_m = nav.max_m;
    on.start = nav.start;
    on.data = nav.data.data();
    on.graph = nav.graph.data();
    on.mapping = nav.mapping.data();
    sp.nav = &on;
    sp.pipe_width = 1;
    sp.early_exit = QVO_EXIT_NONE;
    expect(search_recall(b, base, dtype, q, nq, sp) > 0.5, "recall from the nav entry");
    sp.nav = nullptr;

    // malformed inputs: every reader must fail with a status, not read past its buffers
    char index_file[4096], prefix[4096];
    expect(qv_find_index_files(dir.c_str(), index_file, prefix, sizeof(index_file)) == QV_OK, "find files");
    const fs::path bad = work / "bad";
    fs::create_directories(bad);
    for (size_t keep : {(size_t)0, (size_t)17, (size_t)4096, (size_t)4096 + 100}) {
      truncate_copy(index_file, (bad / "t_disk.index").string(), keep);
      qv_index_info info{};
      const int rc = qv_read_layout((bad / "t_disk.index").c_str(), dname, &info);
      if (rc == QV_OK) {
        std::vector<uint8_t> pg((size_t)info.num_pages * 4096);
        expect(qv_read_index_pages((bad / "t_disk.index").c_str(), info.num_pages, pg.data()) != QV_OK,
               "truncated page image rejected");
      }
    }
    for (size_t keep : {(size_t)5, (size_t)4096, (size_t)4200}) {
      truncate_copy(std::string(prefix) + "_pivots.bin", (bad / "t_pq_pivots.bin").string(), keep);
      qv::PQTables t;
      bool threw = false;
      try {
        qv::read_pq_tables((bad / "t_pq_pivots.bin").string(), std::string(prefix) + "_compressed.bin", t);
      } catch (const qv::Error&) {
        threw = true;
      }
      expect(threw, "truncated pivot file rejected");
    }
  }

  qv_build_params p;
  qv_build_params_default(&p);
  p.R = 0;
  uint8_t tiny[64] = {};
  expect(qv_build_index_cpu(tiny, QV_UINT8, 8, 8, &p, (work / "x").c_str()) == QV_EINVAL, "R = 0 rejected");
  qv_build_params_default(&p);
  p.R = 129;
  p.L = 200;
  expect(qv_build_index_cpu(tiny, QV_UINT8, 8, 8, &p, (work / "x").c_str()) == QV_EINVAL, "R = 129 rejected");
  qv_index_info info{};
  expect(qv_read_layout((work / "missing_disk.index").c_str(), "uint8", &info) != QV_OK, "missing file");
  expect(qv_read_layout((work / "missing_disk.index").c_str(), "bogus", &info) != QV_OK, "bad type name");
  char a[8], b2[8];
  expect(qv_find_index_files(work.c_str(), a, b2, sizeof(a)) != QV_OK, "short path buffer or no index");

  check_order_stats();

  if (g_failures) {
    std::fprintf(stderr, "%d check(s) failed\n", g_failures);
    return 1;
  }
  std::printf("host sanitize test: all checks passed\n");
  return 0;
}
