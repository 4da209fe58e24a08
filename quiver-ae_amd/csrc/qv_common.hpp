// qv_common.hpp -- host-side types shared by the library translation units.
#pragma once

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "quiver_hip.h"

namespace qv {

constexpr int64_t kPageSize = 4096;   // shared::PAGE_SIZE (src/shared/io/loader.hpp:25)
constexpr int kNumPivots = 256;       // PQSearchData::num_pivots (pq_search.hpp:14)
constexpr int kMaxDegree = 128;       // two neighbour slots per wavefront lane
constexpr int kMaxBuildDegree = 128;  // the GPU builder: a list in two slots per lane
constexpr int kMaxEf = 2048;          // 32 beam positions per lane (per-query-LUT kernel)
constexpr int kMaxEfShared = 1024;    // 16 beam positions per lane (shared-pivot kernel)
constexpr int kMaxTopk = 1024;        // 64 in registers, the rest in LDS (per-query-LUT kernel)
constexpr int kMaxPipeWidth = 16;     // bin/common/cli_validation.hpp:9
constexpr int kMaxQueriesPerBlock = 8; // bin/common/cli_validation.hpp:10

// Error carrying a QV_* status; converted at the C ABI boundary.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

[[noreturn]] inline void fail(int code, const std::string& msg) { throw Error(code, msg); }

void set_last_error(const std::string& msg);

// shared::Layout (src/shared/common/layout.hpp:7-19) + element type.
struct Layout {
  int64_t num_dims = 0;
  int64_t max_m0 = 0;
  int64_t enter_point = 0;
  int64_t data_size = 0;
  int64_t node_size = 0;
  int64_t num_pages = 0;
  int64_t num_data = 0;
  int64_t nodes_per_page = 0;
  int data_type = QV_UINT8;
};

inline int64_t elem_size(int data_type) { return data_type == QV_FLOAT ? 4 : 1; }

// PQ tables as the reference holds them on the host (pq_search.hpp:13-29).
struct PQTables {
  int dim = 0;
  int num_chunks = 0;
  int64_t num_pts = 0;
  std::vector<float> centroid;      // [dim]
  std::vector<float> pivots;        // [256][dim]
  std::vector<float> pivots_t;      // [dim][256]
  std::vector<int32_t> chunk_id;    // [dim]
  std::vector<int32_t> chunk_offsets;  // [M+1], contiguous dimension ranges
  std::vector<uint8_t> codes;       // [num_pts][M]
};

// ---- formats (qv_formats.cpp) ----
int parse_data_type(const std::string& s);  // "uint8" | "float" | "float32" | "int8"
const char* data_type_name(int t);
Layout parse_diskann_metadata(const std::string& path, int data_type);
std::string find_index_file(const std::string& index_dir);
std::string find_pq_prefix(const std::string& index_dir);
void read_pq_tables(const std::string& pivots_file, const std::string& codes_file,
                    PQTables& out);
// Pages 1..num_pages of the disk index (the heap memory backend's image).
void read_index_pages(const std::string& path, int64_t num_pages, uint8_t* dst);

void write_diskann_index(const std::string& path, const Layout& lay,
                         const void* base, const std::vector<uint32_t>& adj,
                         const std::vector<uint32_t>& deg);
void write_index_image(const std::string& path, const Layout& lay, const uint8_t* pages);
void write_pq_tables(const std::string& pivots_file, const std::string& codes_file,
                     const PQTables& t);

// Navigation graph (shared::NavGraph, src/shared/index/nav_graph.hpp): a small
// in-memory graph over a sample of the base points, searched per query for the
// entry node.  graph is [num_node][max_m] with -1 after each node's degree;
// mapping[i] is the base id of nav node i.
struct NavGraphHost {
  int32_t num_node = 0;
  int32_t dims = 0;
  int32_t max_m = 0;
  int32_t start = 0;
  std::vector<uint8_t> data;     // [num_node][dims] elements of the base type
  std::vector<int32_t> graph;    // [num_node][max_m]
  std::vector<int32_t> mapping;  // [num_node]
};
// find_nav_dir (bin/common/index_discovery.hpp:105-115): index_dir itself when
// it holds nav_index, else index_dir/nav when that does, else "".
std::string find_nav_dir(const std::string& index_dir);
// NavGraph::init (src/shared/index/nav_graph.cu:12-73): nav_index,
// nav_index.data and map.txt of dir; validated against the base (ids, dims).
void read_nav(const std::string& dir, int data_type, int64_t base_n, int64_t dims, NavGraphHost& nav);
void write_nav(const std::string& dir, int data_type, const NavGraphHost& nav);
// The checks read_nav applies to its files, for a graph given in memory.
void check_nav(const NavGraphHost& nav, int64_t base_n, int64_t dims, int data_type);

// typed .bin with int32 (n, d) header (bin/common/data_io.hpp:29-51, 116-140)
template <class T>
std::vector<T> read_typed_bin(const std::string& path, int64_t& n, int64_t& d);
template <class T>
void write_typed_bin(const std::string& path, const T* data, int64_t n, int64_t d);

}  // namespace qv
