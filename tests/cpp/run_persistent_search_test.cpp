// run_persistent_search_test.cpp -- drives qv_compat::run_persistent_search
// (the reference's argument list, src/quiver/search.cuh:45-66) the way
// bin/quiver_search.cu:290-307 calls run_persistent_search, from index files.
//
// The index is opened once through the C ABI only to obtain what the
// reference's caller holds in host memory (the heap page image, PQSearchData's
// tables with chunk_id per dimension), then closed; run_persistent_search then
// builds its own handle from those arrays.  Writes <out>_ids.bin,
// <out>_distances.bin and <out>_found.bin (int32 (count, width) headers).
//
// usage: run_persistent_search_test INDEX_DIR QUERIES.u8bin EF POLICY(0|2) OUT
//        [GT.ibin THRESHOLD CSV]
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

#include "qv_run_persistent_search.hpp"
#include "quiver_hip.h"

namespace {

template <class T>
std::vector<T> read_matrix(const std::string& path, int32_t& rows, int32_t& cols) {
  std::ifstream in(path, std::ios::binary);
  if (!in) throw std::runtime_error("cannot open " + path);
  in.read(reinterpret_cast<char*>(&rows), 4);
  in.read(reinterpret_cast<char*>(&cols), 4);
  std::vector<T> v((size_t)rows * (size_t)cols);
  in.read(reinterpret_cast<char*>(v.data()), (std::streamsize)(v.size() * sizeof(T)));
  if (!in) throw std::runtime_error("short file " + path);
  return v;
}

template <class T>
void write_matrix(const std::string& path, const T* data, int32_t rows, int32_t cols) {
  std::ofstream out(path, std::ios::binary);
  out.write(reinterpret_cast<const char*>(&rows), 4);
  out.write(reinterpret_cast<const char*>(&cols), 4);
  out.write(reinterpret_cast<const char*>(data), (std::streamsize)sizeof(T) * rows * cols);
}

void check(int rc) {
  if (rc != QV_OK) throw std::runtime_error(qv_last_error());
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 6 && argc != 9) {
    std::cerr << "usage: " << argv[0] << " INDEX_DIR QUERIES.u8bin EF POLICY OUT [GT THRESHOLD CSV]\n";
    return 2;
  }
  try {
    const std::string dir = argv[1];
    const int ef = std::atoi(argv[3]);
    const int policy = std::atoi(argv[4]);
    const std::string out = argv[5];
    const int topk = 10;

    // what the reference's caller holds: layout, heap image, PQ host tables
    qv_index* ix = nullptr;
    check(qv_index_open(dir.c_str(), "uint8", "heap", nullptr, 0, &ix));
    qv_index_info info{};
    check(qv_index_get_info(ix, &info));
    const int dim = (int)info.num_dims, M = info.num_chunks;
    std::vector<uint8_t> pages((size_t)info.num_pages * 4096), codes((size_t)info.num_data * M);
    std::vector<float> centroid((size_t)dim), pivots((size_t)256 * dim);
    std::vector<int32_t> offsets((size_t)M + 1);
    check(qv_index_copy_out(ix, pages.data(), codes.data(), centroid.data(), pivots.data(), offsets.data()));
    qv_index_close(ix);
    std::vector<int> chunk_id((size_t)dim);
    for (int m = 0; m < M; m++)
      for (int j = offsets[(size_t)m]; j < offsets[(size_t)m + 1]; j++) chunk_id[(size_t)j] = m;

    qv_compat::LayoutView layout;
    layout.num_dims = info.num_dims;
    layout.max_m0 = info.max_m0;
    layout.enter_point = info.enter_point;
    layout.data_size = info.data_size;
    layout.node_size = info.node_size;
    layout.num_pages = info.num_pages;
    layout.num_data = info.num_data;
    layout.nodes_per_page = info.nodes_per_page;
    // the heap loader's submit_direct, page by page
    qv_compat::PageReader read = [&](int64_t first, int64_t count, uint8_t* dst) {
      for (int64_t p = 0; p < count; p++)
        std::copy(pages.begin() + (first + p) * 4096, pages.begin() + (first + p + 1) * 4096, dst + p * 4096);
    };
    qv_compat::PQView pq;
    pq.dim = dim;
    pq.num_chunks = M;
    pq.num_pts = (int)info.num_data;
    pq.centroid = centroid.data();
    pq.pivots = pivots.data();
    pq.chunk_id = chunk_id.data();
    pq.compressed_data = codes.data();

    int32_t nq = 0, qd = 0;
    const std::vector<uint8_t> q8 = read_matrix<uint8_t>(argv[2], nq, qd);
    std::vector<float> qf(q8.begin(), q8.end());  // load_queries_as_float
    std::vector<int32_t> gt;
    qv_compat::StepRecallView sr;
    if (argc == 9) {
      int32_t gn = 0, gw = 0;
      gt = read_matrix<int32_t>(argv[6], gn, gw);
      sr.ground_truth = gt.data();
      sr.ground_truth_width = gw;
      sr.ground_truth_count = gn;
      sr.threshold = std::strtof(argv[7], nullptr);
      sr.csv_path = argv[8];
    }
    qv_compat::EarlyExitView ee;
    ee.policy = policy;  // quiver_search.cu:202-205: gpruning with warmup 10, patience 8
    ee.gpruning_warmup_steps = 10;
    ee.gpruning_patience = 8;
    std::vector<int> nns((size_t)nq * topk), found((size_t)nq);
    std::vector<float> dists((size_t)nq * topk);
    uint8_t starter[4096] = {};
    const qv_search_report rep = qv_compat::run_persistent_search(
        layout, QV_UINT8, /*pipe_w=*/1, /*thread_cnt=*/6, /*mini_batch=*/756, read, pq, nullptr,
        (int)info.enter_point, starter, qf.data(), nq, topk, ef, nns.data(), dists.data(), found.data(),
        /*queries_per_block=*/1, /*repeat=*/1, sr, ee);
    write_matrix(out + "_ids.bin", nns.data(), nq, topk);
    write_matrix(out + "_distances.bin", dists.data(), nq, topk);
    write_matrix(out + "_found.bin", found.data(), nq, 1);
    std::cout << "QPS: " << rep.qps << " queries=" << nq << std::endl;
  } catch (const std::exception& e) {
    std::cerr << e.what() << std::endl;
    return 1;
  }
  return 0;
}
