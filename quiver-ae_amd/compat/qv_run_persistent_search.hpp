// qv_run_persistent_search.hpp -- quiver::run_persistent_search's contract
// (src/quiver/search.cuh:45-66) on top of libquiver_hip's C ABI.
//
// The argument list is the reference's, in its order and meaning, with the
// reference's types replaced by plain views of what they hold, so that the
// mapping below is compiled and tested without the reference's headers:
//   shared::Layout                -> LayoutView (same fields, layout.hpp:7-19)
//   shared::DataType              -> int (UINT8 = 0, FLOAT = 1, INT8 = 2)
//   shared::IndexLoader           -> PageReader: copies image pages [first,
//                                    first + count) to dst, as submit_direct
//                                    does page by page (mem_loader.cpp:104-117)
//   shared::PQSearch              -> PQView: PQSearchData's host tables
//                                    (pq_search.hpp:13-29)
//   shared::NavGraph (nullable)   -> NavView (nav_graph.hpp), or nullptr
//   PerStepRecallOptions          -> StepRecallView (search.cuh:17-28)
//   EarlyExitOptions              -> EarlyExitView (search.cuh:30-44)
// quiver_hip_shim.cpp beside this file is the reference-side function that
// converts the real types and calls run_persistent_search below.
//
// Behaviour: a handle is built from the arrays (qv_index_from_memory; the
// reference's own init_device copies its tables to the GPU per call as well,
// pq_search.cu:116-177), the nav graph is set when given, the queries are
// searched with the reference's knobs (mini_batch = num_blocks, pipe width,
// queries per block), the handle is closed.  thread_cnt (poll threads) and
// starter (an unused page, search.cu:357-1361) have no counterpart; repeat
// only labels the report, as in the reference (search.cu:1184), because the
// caller has already repeated the query set (load_queries_as_float,
// data_io.hpp:94-104).  Errors throw std::runtime_error with the library's
// message (the reference throws for CUDA errors and exits for bad options).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <fstream>
#include <functional>
#include <iomanip>
#include <iostream>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>
#include <algorithm>

#include "quiver_hip.h"

namespace qv_compat {

struct LayoutView {
  int64_t num_dims = 0;
  int64_t max_m0 = 0;
  int64_t enter_point = 0;
  int64_t data_size = 0;
  int64_t node_size = 0;
  int64_t num_pages = 0;
  int64_t num_data = 0;
  int64_t nodes_per_page = 0;
};

// Copies pages [first, first + count) of the index image (page k = page k + 1
// of the disk index) to dst.
using PageReader = std::function<void(int64_t first, int64_t count, uint8_t* dst)>;

struct PQView {
  int dim = 0;
  int num_chunks = 0;
  int num_pts = 0;
  const float* centroid = nullptr;          // [dim]
  const float* pivots = nullptr;            // [256][dim]
  const int* chunk_id = nullptr;            // [dim]
  const uint8_t* compressed_data = nullptr;  // [num_pts][num_chunks]
};

struct NavView {
  const uint8_t* data = nullptr;  // [num_node][dim] elements
  const int* graph = nullptr;     // [num_node][max_m], -1 after a node's neighbours
  const int* mapping = nullptr;   // [num_node]
  int num_node = 0;
  int start = 0;
  int max_m = 0;
};

struct StepRecallView {
  const int* ground_truth = nullptr;
  int ground_truth_width = 0;
  int ground_truth_count = 0;
  float threshold = 0.9f;
  const char* csv_path = nullptr;
  bool enabled() const {  // PerStepRecallOptions::enabled (search.cuh:24-27)
    return ground_truth != nullptr && ground_truth_width > 0 && ground_truth_count > 0 && csv_path != nullptr;
  }
};

// EarlyExitPolicy (io_control.cuh:41-46): kDefault 0, kDarth 1, kGPruning 2, kDarthTrace 3.
struct EarlyExitView {
  int policy = 0;
  int gpruning_warmup_steps = 0;
  int gpruning_patience = 0;
};

namespace detail {

inline void check(int rc) {
  if (rc != QV_OK) throw std::runtime_error(qv_last_error());
}

struct Handle {
  qv_index* ix = nullptr;
  ~Handle() { qv_index_close(ix); }
};

// write_step_recall_csv (src/quiver/search.cu:100-153).
inline void write_step_recall_csv(const StepRecallView& sr, const std::vector<int32_t>& steps,
                                  const std::vector<int32_t>& hits, int topk) {
  std::ofstream out(sr.csv_path);
  if (!out.is_open()) throw std::runtime_error(std::string("Failed to open step recall CSV ") + sr.csv_path);
  out << "query_id,step,hits,recall,reached\n";
  std::vector<int32_t> reached;
  for (size_t q = 0; q < steps.size(); q++) {
    const bool ok = steps[q] >= 0;
    if (ok) reached.push_back(steps[q]);
    out << q << "," << steps[q] << "," << hits[q] << "," << std::fixed << std::setprecision(6)
        << (double)hits[q] / (double)topk << "," << (ok ? 1 : 0) << "\n";
  }
  std::sort(reached.begin(), reached.end());
  const int required = std::max(1, std::min(topk, (int)std::ceil(sr.threshold * (float)topk - 1e-6f)));
  std::cout << "[Quiver] Step recall CSV: " << sr.csv_path << "\n"
            << "[Quiver] Step recall reached=" << reached.size() << " unreached=" << steps.size() - reached.size()
            << " threshold=" << sr.threshold << " required_hits=" << required << std::endl;
  if (!reached.empty()) {
    auto pct = [&](double p) {
      size_t i = (size_t)((double)reached.size() * p / 100.0);
      return (double)reached[std::min(i, reached.size() - 1)];
    };
    std::cout << "[Quiver] Step recall steps p50=" << pct(50) << " p90=" << pct(90) << " p99=" << pct(99)
              << " max=" << reached.back() << std::endl;
  }
}

}  // namespace detail

// quiver::run_persistent_search with plain views; returns the run's report
// (QPS, latency percentiles) for the caller to print.
inline qv_search_report run_persistent_search(
    const LayoutView& layout, int data_type, int pipe_w, int /*thread_cnt*/, int mini_batch,
    const PageReader& pages, const PQView& pq, const NavView* nav, int enter_point, uint8_t* /*starter*/,
    const float* qdata, int num_queries, int topk, int ef_search, int* nns, float* distances, int* found_cnt,
    int queries_per_block = 1, int /*repeat*/ = 1, const StepRecallView& per_step_recall = {},
    const EarlyExitView& early_exit = {}, int device = 0) {
  if (early_exit.policy != 0 && early_exit.policy != 2)
    throw std::runtime_error("early-exit policy " + std::to_string(early_exit.policy) +
                             " (DARTH) is not supported; use gpruning or none");
  qv_index_info info{};
  info.num_data = layout.num_data;
  info.num_dims = layout.num_dims;
  info.max_m0 = layout.max_m0;
  info.enter_point = enter_point;  // the entry the caller passes (kernel_q1.cuh:199-206)
  info.data_size = layout.data_size;
  info.node_size = layout.node_size;
  info.num_pages = layout.num_pages;
  info.nodes_per_page = layout.nodes_per_page;
  info.data_type = data_type;
  if (pq.dim != layout.num_dims || pq.num_pts != layout.num_data)
    throw std::runtime_error("PQ tables do not match the layout");
  std::vector<uint8_t> image((size_t)layout.num_pages * 4096);
  const int64_t chunk = 16384;
  for (int64_t p = 0; p < layout.num_pages; p += chunk)
    pages(p, std::min(chunk, layout.num_pages - p), image.data() + p * 4096);
  detail::Handle h;
  detail::check(qv_index_from_memory(&info, image.data(), pq.centroid, pq.pivots, pq.chunk_id, pq.num_chunks,
                                     pq.compressed_data, device, &h.ix));
  std::vector<uint8_t>().swap(image);
  if (nav)
    detail::check(qv_index_set_nav(h.ix, nav->data, nav->graph, nav->mapping, nav->num_node, nav->max_m,
                                   nav->start));
  qv_search_opts o;
  qv_search_opts_default(&o);
  o.num_blocks = mini_batch;
  o.pipe_width = pipe_w;
  o.queries_per_block = queries_per_block;
  o.early_exit = early_exit.policy == 2 ? QV_EXIT_GPRUNING : QV_EXIT_NONE;
  o.gpruning_warmup = early_exit.gpruning_warmup_steps;
  o.gpruning_patience = early_exit.gpruning_patience;
  if (const char* e = std::getenv("QUIVER_PREFEED")) o.prefeed = std::atoi(e);
  if (const char* e = std::getenv("QUIVER_ADMIT_MIN_BATCH")) o.admit_min_batch = std::max(1, std::atoi(e));
  std::vector<int32_t> sr_step, sr_hits;
  if (per_step_recall.enabled()) {
    sr_step.resize((size_t)num_queries);
    sr_hits.resize((size_t)num_queries);
    o.step_recall_gt = per_step_recall.ground_truth;
    o.step_recall_gt_width = per_step_recall.ground_truth_width;
    o.step_recall_gt_count = per_step_recall.ground_truth_count;
    o.step_recall_threshold = per_step_recall.threshold;
    o.step_recall_step = sr_step.data();
    o.step_recall_hits = sr_hits.data();
  }
  qv_search_report rep{};
  detail::check(qv_search(h.ix, qdata, num_queries, (int32_t)layout.num_dims, topk, ef_search, &o, nns,
                          distances, found_cnt, &rep));
  if (per_step_recall.enabled()) detail::write_step_recall_csv(per_step_recall, sr_step, sr_hits, topk);
  return rep;
}

}  // namespace qv_compat
