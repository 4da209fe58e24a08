// qv_index_impl.hpp -- the opaque qv_index handle shared by the library's
// translation units (index open, search, GPU build).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "qv_common.hpp"

struct qv_index {
  int device = 0;
  qv::Layout lay;
  int M = 0;
  uint8_t* d_pages = nullptr;  // HBM, or pinned host memory when pages_in_host
  bool pages_in_host = false;
  uint8_t* d_codes = nullptr;
  float* d_centroid = nullptr;
  float* d_pivots_t = nullptr;
  int32_t* d_chunk_off = nullptr;
  // navigation graph (optional): vectors, [nodes][max_m] adjacency, base ids
  uint8_t* d_nav_data = nullptr;
  int32_t* d_nav_graph = nullptr;
  int32_t* d_nav_map = nullptr;
  int64_t nav_nodes = 0;
  int32_t nav_max_m = 0, nav_start = 0;
  // neighbour code table (optional): [n][max_m][M], node v's neighbours' code rows
  uint8_t* d_nbr_codes = nullptr;
  int64_t nbr_codes_bytes = 0;
  int64_t device_bytes = 0;
  int num_cus = 0;
  int lds_cu = 0;  // LDS bytes per CU
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  // search scratch (grown on demand, reused across calls)
  int64_t cap_q = 0;
  int cap_k = 0;
  float* d_queries = nullptr;
  int32_t* d_ids = nullptr;
  float* d_dists = nullptr;
  int32_t* d_found = nullptr;
  int32_t* d_hops = nullptr;
  int32_t* d_stopped = nullptr;
  int32_t* d_evals = nullptr;
  uint64_t* d_tstart = nullptr;
  uint64_t* d_tend = nullptr;
  int32_t* d_counters = nullptr;
  uint64_t* d_feed_mirror = nullptr;  // device copies of the feed word (search kernels' feed wait)
  uint32_t feed_epoch = 0;            // epoch of the last search that used them
  int32_t* h_ctrl = nullptr;   // [0] feed_count, [1] terminate (host-coherent)
  int32_t* h_ring = nullptr;   // [cap_q] completion ring (host-coherent)
  int32_t* h_stage = nullptr;  // pinned: counters [kStageHead], hops, stopped, evals [cap_q each]
  float* h_qstage = nullptr;   // pinned, coherent: a host-buffer call's queries [cap_q][d], read in place
  // pinned, coherent: a host-buffer call's results as the kernel writes them,
  // ids [cap_q][cap_k] int32, dists [cap_q][cap_k] float, found [cap_q] int32
  void* h_results = nullptr;
  std::vector<int32_t> last_hops;
  std::vector<double> last_lat_ms;  // per-query latency of the last search, query order
  // host copies of the PQ tables (for saving the index)
  std::vector<float> h_centroid, h_pivots;
  std::vector<int32_t> h_chunk_off;
  std::mutex mu;
};

namespace qv {

// Extra per-query outputs of a search: the expanded nodes in order with their
// exact distances (used by the graph builder).
struct SearchRecord {
  int32_t* ids = nullptr;    // [nq][cap]
  float* dists = nullptr;    // [nq][cap]
  int32_t cap = 0;
};

// Creates a handle around device buffers the caller allocated with hipMalloc
// (ownership moves to the handle) and host PQ tables; validates the graph.
// With pages_in_host the page image is pinned host memory from hipHostMalloc.
qv_index* make_index(int device, const Layout& lay, const PQTables& pq, uint8_t* d_pages,
                     uint8_t* d_codes, bool validate, bool pages_in_host = false);

void release_index(qv_index* ix);

// Loads the nav graph of dir (nav_index, nav_index.data, map.txt) to the device.
void load_nav(qv_index* ix, const std::string& dir);
// Checks a nav graph held in host memory and moves it to the handle's device.
void upload_nav(qv_index* ix, const NavGraphHost& nav);

// Builds (enable) or frees the neighbour code table on the handle's device.
void set_neighbour_codes(qv_index* ix, bool enable);

// Checks degree <= R, neighbour ids < n and duplicate-free lists on the device;
// throws QV_EINDEX on the first violation.
void validate_graph(qv_index* ix);

// Device-buffer search in whole-batch admission with optional record output.
void search_record(qv_index* ix, const float* d_queries, int64_t nq, int ef,
                   const SearchRecord& rec, int32_t* d_hops, int num_blocks);

}  // namespace qv
