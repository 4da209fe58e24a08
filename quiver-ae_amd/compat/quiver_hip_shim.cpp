// quiver_hip_shim.cpp -- quiver::run_persistent_search (src/quiver/search.cuh:45-66)
// for the reference's bin/ programs, served by libquiver_hip on an MI355X.
//
// Built inside the reference tree in place of src/quiver/search.cu, with the
// reference's src/ and this repository's include/ and quiver-ae_amd/compat/ on
// the include path, and linked with -lquiver_hip.  It only converts the
// reference's types into the views of qv_run_persistent_search.hpp, reading
// the page image through the loader's own submit_direct, and prints the run
// report lines the reference's format_run_report prints (run_report.hpp:96-140,
// which the AE parsers read; that header itself needs spdlog).
#include <cstdint>
#include <cstdio>
#include <iomanip>
#include <sstream>
#include <vector>

#include "quiver/search.cuh"
#include "qv_run_persistent_search.hpp"

namespace quiver {

void run_persistent_search(const shared::Layout& layout, shared::DataType data_type, int pipe_w,
                           int thread_cnt, int mini_batch, std::shared_ptr<shared::IndexLoader> loader,
                           shared::PQSearch* pq, shared::NavGraph* nav, int enter_point, uint8_t* starter,
                           const float* qdata, int num_queries, int topk, int ef_search, int* nns,
                           float* distances, int* found_cnt, int queries_per_block, int repeat,
                           const PerStepRecallOptions& per_step_recall, const EarlyExitOptions& early_exit) {
  qv_compat::LayoutView lv;
  lv.num_dims = layout.num_dims;
  lv.max_m0 = layout.max_m0;
  lv.enter_point = layout.enter_point;
  lv.data_size = layout.data_size;
  lv.node_size = layout.node_size;
  lv.num_pages = layout.num_pages;
  lv.num_data = layout.num_data;
  lv.nodes_per_page = layout.nodes_per_page;

  // The image through the loader interface: one direct request per page,
  // each complete when its status word holds the done value.
  qv_compat::PageReader read = [&](int64_t first, int64_t count, uint8_t* dst) {
    std::vector<int32_t> status((size_t)count, 0);
    std::vector<shared::DirectIoRequest> reqs;
    reqs.reserve((size_t)count);
    for (int64_t i = 0; i < count; i++)
      reqs.push_back({(int)(first + i), dst + i * shared::PAGE_SIZE, &status[(size_t)i], 1, nullptr});
    loader->submit_direct(reqs, 0);
    for (int64_t i = 0; i < count; i++)
      while (__atomic_load_n(&status[(size_t)i], __ATOMIC_ACQUIRE) != 1) {
      }
  };

  const shared::PQSearchData& d = pq->get_data();
  qv_compat::PQView pv;
  pv.dim = d.dim;
  pv.num_chunks = d.num_chunks;
  pv.num_pts = d.num_pts;
  pv.centroid = d.centroid;
  pv.pivots = d.pivots;
  pv.chunk_id = d.chunk_id;
  pv.compressed_data = d.compressed_data;

  qv_compat::NavView nv;
  if (nav) {
    nv.data = nav->data;
    nv.graph = nav->graph;
    nv.mapping = nav->mapping.data();
    nv.num_node = nav->num_node;
    nv.start = nav->start;
    nv.max_m = nav->max_m;
  }

  qv_compat::StepRecallView sv;
  sv.ground_truth = per_step_recall.ground_truth;
  sv.ground_truth_width = per_step_recall.ground_truth_width;
  sv.ground_truth_count = per_step_recall.ground_truth_count;
  sv.threshold = per_step_recall.threshold;
  sv.csv_path = per_step_recall.csv_path;

  qv_compat::EarlyExitView ev;
  ev.policy = static_cast<int>(early_exit.policy);
  ev.gpruning_warmup_steps = early_exit.gpruning_warmup_steps;
  ev.gpruning_patience = early_exit.gpruning_patience;

  const qv_search_report rep = qv_compat::run_persistent_search(
      lv, static_cast<int>(data_type), pipe_w, thread_cnt, mini_batch, read, pv, nav ? &nv : nullptr,
      enter_point, starter, qdata, num_queries, topk, ef_search, nns, distances, found_cnt, queries_per_block,
      repeat, sv, ev);

  static const char* const kTypes[] = {"uint8", "float", "int8"};
  std::ostringstream os;
  os << std::fixed;
  os << "========== Quiver Result ==========\n";
  os << "Query Params:\n  topk=" << topk << " ef_search=" << ef_search << " repeat=" << repeat
     << " data_type=" << kTypes[static_cast<int>(data_type) % 3] << "\n";
  os << "Runtime Params:\n  backend=libquiver_hip num_blocks=" << rep.num_blocks << " pipe_width=" << pipe_w
     << " queries_per_block=" << queries_per_block << " max_inflight=" << rep.max_inflight << "\n\n";
  os << "Performance:\n  QPS: " << std::setprecision(2) << rep.qps << "\n";
  os << "  QueryLatency(ms): avg=" << std::setprecision(3) << rep.lat_avg_ms << " p50=" << rep.lat_p50_ms
     << " p90=" << rep.lat_p90_ms << " p99=" << rep.lat_p99_ms << " p99.9=" << rep.lat_p999_ms
     << " max=" << rep.lat_max_ms << "\n";
  os << "===================================\n";
  std::printf("%s", os.str().c_str());
}

}  // namespace quiver
