// qv_formats.cpp -- readers and writers of the on-disk formats the reference
// consumes: the DiskANN disk index (header page + 4 KB node pages), the PQ pivot
// table and code file, and the int32-headed .bin arrays.
#include <algorithm>
#include <cerrno>
#include <cstring>
#include <filesystem>
#include <fstream>

#include "qv_common.hpp"

namespace fs = std::filesystem;

namespace qv {

int parse_data_type(const std::string& s) {
  // bin/common/cli_shared.hpp:61-74 plus the Python spelling "float32"
  // (python/quiver/index.py:19-24).
  if (s == "uint8") return QV_UINT8;
  if (s == "float" || s == "float32") return QV_FLOAT;
  if (s == "int8") return QV_INT8;
  fail(QV_EINVAL, "Unsupported data type '" + s + "'. Expected one of: uint8, int8, float");
}

const char* data_type_name(int t) {
  switch (t) {
    case QV_UINT8: return "uint8";
    case QV_INT8: return "int8";
    case QV_FLOAT: return "float";
  }
  return "unknown";
}

// bin/common/metadata.hpp:15-72.  The element size of uint8 and int8 data is 1.
Layout parse_diskann_metadata(const std::string& path, int data_type) {
  std::ifstream in(path, std::ios::binary);
  if (!in.is_open()) fail(QV_EIO, "Failed to open file " + path);
  uint32_t nr = 0, nc = 0;
  uint64_t v[8] = {};
  in.read(reinterpret_cast<char*>(&nr), 4);
  in.read(reinterpret_cast<char*>(&nc), 4);
  in.read(reinterpret_cast<char*>(v), sizeof(v));
  if (!in) fail(QV_EIO, "Truncated DiskANN header in " + path);
  Layout lay;
  lay.data_type = data_type;
  const uint64_t esz = (uint64_t)elem_size(data_type);
  lay.num_data = (int64_t)v[0];
  lay.num_dims = (int64_t)v[1];
  lay.enter_point = (int64_t)v[2];
  const uint64_t max_node_len = v[3];
  lay.nodes_per_page = (int64_t)v[4];
  if (lay.num_data <= 0 || lay.num_dims <= 0 || lay.nodes_per_page <= 0 ||
      max_node_len <= v[1] * esz + 4 || max_node_len * v[4] > (uint64_t)kPageSize)
    fail(QV_EIO, "Malformed DiskANN header in " + path);
  lay.max_m0 = (int64_t)((max_node_len - v[1] * esz) / sizeof(uint32_t)) - 1;
  lay.num_pages = (lay.num_data + lay.nodes_per_page - 1) / lay.nodes_per_page;
  lay.node_size = (int64_t)max_node_len;
  lay.data_size = lay.num_dims * (int64_t)esz;
  if (lay.enter_point < 0 || lay.enter_point >= lay.num_data)
    fail(QV_EINDEX, "Medoid out of range in " + path);
  return lay;
}

static std::vector<std::string> suffix_matches(const std::string& dir,
                                               const std::string& suffix) {
  std::vector<std::string> out;
  for (const auto& e : fs::directory_iterator(dir)) {
    if (!fs::is_regular_file(e.path())) continue;
    const std::string name = e.path().filename().string();
    if (name.size() >= suffix.size() &&
        name.compare(name.size() - suffix.size(), suffix.size(), suffix) == 0)
      out.push_back(e.path().string());
  }
  std::sort(out.begin(), out.end());
  return out;
}

static std::string join(const std::vector<std::string>& v) {
  std::string s;
  for (size_t i = 0; i < v.size(); i++) s += (i ? ", " : "") + v[i];
  return s;
}

// bin/common/index_discovery.hpp:57-78
std::string find_index_file(const std::string& dir) {
  if (!fs::is_directory(dir))
    fail(QV_EIO, "--index-dir '" + dir + "' does not exist or is not a directory");
  auto m = suffix_matches(dir, "_disk.index");
  if (m.size() == 1) return m.front();
  if (m.size() > 1)
    fail(QV_EIO, "Multiple *_disk.index candidates found in " + dir + ": " + join(m));
  fs::path fb = fs::path(dir) / "disk.index";
  if (fs::exists(fb) && fs::is_regular_file(fb)) return fb.string();
  fail(QV_EIO, "No *_disk.index or disk.index found in " + dir);
}

// bin/common/index_discovery.hpp:80-103
std::string find_pq_prefix(const std::string& dir) {
  if (!fs::is_directory(dir))
    fail(QV_EIO, "--index-dir '" + dir + "' does not exist or is not a directory");
  auto m = suffix_matches(dir, "_pq_pivots.bin");
  if (m.size() == 1) return m.front().substr(0, m.front().size() - std::string("_pivots.bin").size());
  if (m.size() > 1)
    fail(QV_EIO, "Multiple *_pq_pivots.bin candidates found in " + dir + ": " + join(m));
  fs::path fb = fs::path(dir) / "pq";
  if (fs::exists(fb.string() + "_pivots.bin")) return fb.string();
  fail(QV_EIO, "No PQ pivot files found in " + dir);
}

// read_bin (src/shared/index/pq_search.cu:179-194): int32 rows, int32 cols, data.
template <class T>
static std::vector<T> read_bin_at(const std::string& path, size_t offset, int& nr, int& nc) {
  std::ifstream in(path, std::ios::binary);
  if (!in.is_open()) fail(QV_EIO, "Cannot open file: " + path);
  in.seekg((std::streamoff)offset, std::ios::beg);
  in.read(reinterpret_cast<char*>(&nr), 4);
  in.read(reinterpret_cast<char*>(&nc), 4);
  if (!in || nr < 0 || nc < 0) fail(QV_EIO, "Bad bin header in " + path);
  std::vector<T> data((size_t)nr * (size_t)nc);
  in.read(reinterpret_cast<char*>(data.data()), (std::streamsize)(sizeof(T) * data.size()));
  if (!in) fail(QV_EIO, "Truncated bin section in " + path);
  return data;
}

// PQSearch::read_data (src/shared/index/pq_search.cu:62-114).
void read_pq_tables(const std::string& pivots_file, const std::string& codes_file,
                    PQTables& t) {
  int nr = 0, nc = 0;
  t.codes = read_bin_at<uint8_t>(codes_file, 0, nr, nc);
  t.num_pts = nr;
  t.num_chunks = nc;
  auto offs = read_bin_at<uint64_t>(pivots_file, 0, nr, nc);
  if (!((nr == 4 || nr == 5) && nc == 1)) fail(QV_EIO, "Bad PQ metadata table in " + pivots_file);
  const int chunk_index = nr == 5 ? 3 : 2;
  t.pivots = read_bin_at<float>(pivots_file, offs[0], nr, nc);
  if (nr != kNumPivots) fail(QV_EIO, "PQ pivots must have 256 rows in " + pivots_file);
  t.dim = nc;
  t.pivots_t.assign((size_t)t.dim * kNumPivots, 0.f);
  for (int i = 0; i < kNumPivots; i++)
    for (int j = 0; j < t.dim; j++) t.pivots_t[(size_t)j * kNumPivots + i] = t.pivots[(size_t)i * t.dim + j];
  t.centroid = read_bin_at<float>(pivots_file, offs[1], nr, nc);
  if (nr != t.dim || nc != 1) fail(QV_EIO, "PQ centroid shape mismatch in " + pivots_file);
  auto co = read_bin_at<int32_t>(pivots_file, offs[chunk_index], nr, nc);
  if (nr != t.num_chunks + 1 || nc != 1) fail(QV_EIO, "PQ chunk offsets shape mismatch in " + pivots_file);
  // chunk_id[j] = i for j in [co[i], co[i+1]) (pq_search.cu:103-109).  Every
  // dimension must belong to a chunk; the reference would index LUT row -1.
  if (co[0] != 0 || co[t.num_chunks] != t.dim)
    fail(QV_EIO, "PQ chunk offsets must cover [0, dim) in " + pivots_file);
  t.chunk_id.assign((size_t)t.dim, -1);
  for (int i = 0; i < t.num_chunks; i++) {
    if (co[i + 1] < co[i]) fail(QV_EIO, "PQ chunk offsets must be non-decreasing in " + pivots_file);
    for (int j = co[i]; j < co[i + 1]; j++) t.chunk_id[(size_t)j] = i;
  }
  t.chunk_offsets = co;
}

// MemLoaderSync::load_heap (src/shared/io/mem_loader.cpp:28-44): pages
// 1..num_pages (page 0 is the header) in order.
void read_index_pages(const std::string& path, int64_t num_pages, uint8_t* dst) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) fail(QV_EIO, "Failed to open Mem Index: " + path);
  if (std::fseek(f, kPageSize, SEEK_SET) != 0) {
    std::fclose(f);
    fail(QV_EIO, "Failed to seek Mem Index: " + path);
  }
  int64_t got = (int64_t)std::fread(dst, kPageSize, (size_t)num_pages, f);
  std::fclose(f);
  if (got != num_pages)
    fail(QV_EIO, "Mem Index Load FAILED: " + std::to_string(got) + " pages read from " + path);
}

// Writer for the same layout: header page (save_bin of nine u64 metadata
// values: nnodes, ndims, medoid, max_node_len, nnodes_per_sector, frozen count,
// frozen id, reorder flag, file size) followed by node pages with records
// [vector | u32 degree | u32 neighbours[R]].
void write_diskann_index(const std::string& path, const Layout& lay, const void* base,
                         const std::vector<uint32_t>& adj, const std::vector<uint32_t>& deg) {
  std::ofstream out(path, std::ios::binary | std::ios::trunc);
  if (!out.is_open()) fail(QV_EIO, "Failed to open " + path + " for writing");
  const int64_t R = lay.max_m0;
  const int64_t file_size = (lay.num_pages + 1) * kPageSize;
  std::vector<uint8_t> page((size_t)kPageSize, 0);
  uint32_t hdr[2] = {9, 1};
  uint64_t meta[9] = {(uint64_t)lay.num_data, (uint64_t)lay.num_dims, (uint64_t)lay.enter_point,
                      (uint64_t)lay.node_size, (uint64_t)lay.nodes_per_page, 0, 0, 0,
                      (uint64_t)file_size};
  std::memcpy(page.data(), hdr, sizeof(hdr));
  std::memcpy(page.data() + sizeof(hdr), meta, sizeof(meta));
  out.write(reinterpret_cast<const char*>(page.data()), kPageSize);
  const uint8_t* b = static_cast<const uint8_t*>(base);
  for (int64_t p = 0; p < lay.num_pages; p++) {
    std::fill(page.begin(), page.end(), 0);
    for (int64_t k = 0; k < lay.nodes_per_page; k++) {
      const int64_t v = p * lay.nodes_per_page + k;
      if (v >= lay.num_data) break;
      uint8_t* rec = page.data() + k * lay.node_size;
      std::memcpy(rec, b + v * lay.data_size, (size_t)lay.data_size);
      uint32_t* nb = reinterpret_cast<uint32_t*>(rec + lay.data_size);
      nb[0] = deg[(size_t)v];
      std::memcpy(nb + 1, adj.data() + (size_t)v * R, sizeof(uint32_t) * deg[(size_t)v]);
    }
    out.write(reinterpret_cast<const char*>(page.data()), kPageSize);
  }
  if (!out) fail(QV_EIO, "Failed writing " + path);
}

// Header page followed by an existing page image (pages 1..num_pages).
void write_index_image(const std::string& path, const Layout& lay, const uint8_t* pages) {
  std::ofstream out(path, std::ios::binary | std::ios::trunc);
  if (!out.is_open()) fail(QV_EIO, "Failed to open " + path + " for writing");
  std::vector<uint8_t> page((size_t)kPageSize, 0);
  uint32_t hdr[2] = {9, 1};
  uint64_t meta[9] = {(uint64_t)lay.num_data, (uint64_t)lay.num_dims, (uint64_t)lay.enter_point,
                      (uint64_t)lay.node_size, (uint64_t)lay.nodes_per_page, 0, 0, 0,
                      (uint64_t)((lay.num_pages + 1) * kPageSize)};
  std::memcpy(page.data(), hdr, sizeof(hdr));
  std::memcpy(page.data() + sizeof(hdr), meta, sizeof(meta));
  out.write(reinterpret_cast<const char*>(page.data()), kPageSize);
  out.write(reinterpret_cast<const char*>(pages), (std::streamsize)(lay.num_pages * kPageSize));
  if (!out) fail(QV_EIO, "Failed writing " + path);
}

// DiskANN pivot file: a 4 KB metadata block holding four u64 offsets
// (pivots, centroid, chunk offsets, end), then the three bin sections.
void write_pq_tables(const std::string& pivots_file, const std::string& codes_file,
                     const PQTables& t) {
  {
    std::ofstream out(pivots_file, std::ios::binary | std::ios::trunc);
    if (!out.is_open()) fail(QV_EIO, "Failed to open " + pivots_file + " for writing");
    const uint64_t o0 = 4096;
    const uint64_t o1 = o0 + 8 + 4ull * kNumPivots * (uint64_t)t.dim;
    const uint64_t o2 = o1 + 8 + 4ull * (uint64_t)t.dim;
    const uint64_t o3 = o2 + 8 + 4ull * (uint64_t)(t.num_chunks + 1);
    std::vector<uint8_t> meta(4096, 0);
    int32_t h[2] = {4, 1};
    uint64_t offs[4] = {o0, o1, o2, o3};
    std::memcpy(meta.data(), h, 8);
    std::memcpy(meta.data() + 8, offs, sizeof(offs));
    out.write(reinterpret_cast<const char*>(meta.data()), (std::streamsize)meta.size());
    int32_t hp[2] = {kNumPivots, t.dim};
    out.write(reinterpret_cast<const char*>(hp), 8);
    out.write(reinterpret_cast<const char*>(t.pivots.data()), (std::streamsize)(4 * t.pivots.size()));
    int32_t hc[2] = {t.dim, 1};
    out.write(reinterpret_cast<const char*>(hc), 8);
    out.write(reinterpret_cast<const char*>(t.centroid.data()), (std::streamsize)(4 * t.centroid.size()));
    int32_t ho[2] = {t.num_chunks + 1, 1};
    out.write(reinterpret_cast<const char*>(ho), 8);
    out.write(reinterpret_cast<const char*>(t.chunk_offsets.data()), 4 * (std::streamsize)(t.num_chunks + 1));
    if (!out) fail(QV_EIO, "Failed writing " + pivots_file);
  }
  write_typed_bin<uint8_t>(codes_file, t.codes.data(), t.num_pts, t.num_chunks);
}

// ---- navigation graph ------------------------------------------------------

std::string find_nav_dir(const std::string& index_dir) {
  if (fs::exists(fs::path(index_dir) / "nav_index")) return index_dir;
  if (fs::exists(fs::path(index_dir) / "nav" / "nav_index")) return (fs::path(index_dir) / "nav").string();
  return "";
}

// nav_index: the DiskANN in-memory graph file -- u64 file size, u32 max
// degree, u32 start, u64 frozen-point count, then per node u32 degree and the
// neighbour ids (NavGraph::init reads the header as six ints, nav_graph.cu:47-53).
// nav_index.data: i32 num_node, i32 dims, then the vectors.  map.txt: num_node
// whitespace-separated base ids.
void read_nav(const std::string& dir, int data_type, int64_t base_n, int64_t dims, NavGraphHost& nav) {
  const std::string data_file = dir + "/nav_index.data", index_file = dir + "/nav_index",
                    map_file = dir + "/map.txt";
  std::ifstream fd(data_file, std::ios::binary);
  if (!fd) fail(QV_EIO, "Failed to open data file: " + data_file);
  int32_t hdr[2] = {0, 0};
  fd.read(reinterpret_cast<char*>(hdr), sizeof(hdr));
  if (!fd || hdr[0] <= 0 || hdr[1] <= 0) fail(QV_EIO, "bad nav data header: " + data_file);
  nav.num_node = hdr[0];
  nav.dims = hdr[1];
  if (nav.dims != dims)
    fail(QV_EINDEX, "nav graph has " + std::to_string(nav.dims) + " dims, the index " + std::to_string(dims));
  const size_t bytes = (size_t)nav.num_node * (size_t)nav.dims * (size_t)elem_size(data_type);
  nav.data.resize(bytes);
  fd.read(reinterpret_cast<char*>(nav.data.data()), (std::streamsize)bytes);
  if (!fd) fail(QV_EIO, "short nav data file: " + data_file);

  std::ifstream fm(map_file);
  if (!fm) fail(QV_EIO, "Failed to open map file: " + map_file);
  nav.mapping.resize((size_t)nav.num_node);
  for (int32_t i = 0; i < nav.num_node; i++) {
    long long x = -1;
    if (!(fm >> x)) fail(QV_EIO, "Failed to read map entry " + std::to_string(i) + " from " + map_file);
    if (x < 0 || x >= base_n) fail(QV_EINDEX, "nav map entry out of range: " + std::to_string(x));
    nav.mapping[(size_t)i] = (int32_t)x;
  }

  std::ifstream fi(index_file, std::ios::binary);
  if (!fi) fail(QV_EIO, "Failed to open index file: " + index_file);
  uint64_t fsize = 0, frozen = 0;
  uint32_t max_m = 0, start = 0;
  fi.read(reinterpret_cast<char*>(&fsize), 8);
  fi.read(reinterpret_cast<char*>(&max_m), 4);
  fi.read(reinterpret_cast<char*>(&start), 4);
  fi.read(reinterpret_cast<char*>(&frozen), 8);
  if (!fi) fail(QV_EIO, "short nav index header: " + index_file);
  if (max_m == 0 || max_m > 32) fail(QV_EINDEX, "nav graph max degree must be in [1, 32]");  // nav_graph.cu:58
  if (start >= (uint32_t)nav.num_node) fail(QV_EINDEX, "nav start out of range");
  nav.max_m = (int32_t)max_m;
  nav.start = (int32_t)start;
  nav.graph.assign((size_t)nav.num_node * max_m, -1);
  for (int32_t i = 0; i < nav.num_node; i++) {
    uint32_t d = 0;
    fi.read(reinterpret_cast<char*>(&d), 4);
    if (!fi || d == 0 || d > max_m) fail(QV_EINDEX, "nav node " + std::to_string(i) + " has a bad degree");
    fi.read(reinterpret_cast<char*>(&nav.graph[(size_t)i * max_m]), 4 * (std::streamsize)d);
    if (!fi) fail(QV_EIO, "short nav index file: " + index_file);
    for (uint32_t j = 0; j < d; j++) {
      const int32_t v = nav.graph[(size_t)i * max_m + j];
      if (v < 0 || v >= nav.num_node) fail(QV_EINDEX, "nav neighbour id out of range");
    }
  }
}

void check_nav(const NavGraphHost& nav, int64_t base_n, int64_t dims, int data_type) {
  if (nav.num_node <= 0) fail(QV_EINDEX, "nav graph has no nodes");
  if (nav.dims != dims)
    fail(QV_EINDEX, "nav graph has " + std::to_string(nav.dims) + " dims, the index " + std::to_string(dims));
  if (nav.max_m < 1 || nav.max_m > 32) fail(QV_EINDEX, "nav graph max degree must be in [1, 32]");  // nav_graph.cu:58
  if (nav.start < 0 || nav.start >= nav.num_node) fail(QV_EINDEX, "nav start out of range");
  if (nav.data.size() != (size_t)nav.num_node * (size_t)dims * (size_t)elem_size(data_type))
    fail(QV_EINDEX, "nav data size does not match num_node x dims");
  if (nav.mapping.size() != (size_t)nav.num_node || nav.graph.size() != (size_t)nav.num_node * nav.max_m)
    fail(QV_EINDEX, "nav map or graph size does not match num_node");
  for (int32_t x : nav.mapping)
    if (x < 0 || x >= base_n) fail(QV_EINDEX, "nav map entry out of range: " + std::to_string(x));
  for (int32_t v : nav.graph)
    if (v < -1 || v >= nav.num_node) fail(QV_EINDEX, "nav neighbour id out of range");
}

void write_nav(const std::string& dir, int data_type, const NavGraphHost& nav) {
  fs::create_directories(dir);
  {
    std::ofstream f(dir + "/nav_index.data", std::ios::binary);
    const int32_t hdr[2] = {nav.num_node, nav.dims};
    f.write(reinterpret_cast<const char*>(hdr), sizeof(hdr));
    f.write(reinterpret_cast<const char*>(nav.data.data()),
            (std::streamsize)((size_t)nav.num_node * nav.dims * elem_size(data_type)));
    if (!f) fail(QV_EIO, "cannot write " + dir + "/nav_index.data");
  }
  {
    std::ofstream f(dir + "/map.txt");
    for (int32_t i = 0; i < nav.num_node; i++) f << nav.mapping[(size_t)i] << "\n";
    if (!f) fail(QV_EIO, "cannot write " + dir + "/map.txt");
  }
  std::vector<uint32_t> body;
  for (int32_t i = 0; i < nav.num_node; i++) {
    uint32_t d = 0;
    while (d < (uint32_t)nav.max_m && nav.graph[(size_t)i * nav.max_m + d] >= 0) d++;
    body.push_back(d);
    for (uint32_t j = 0; j < d; j++) body.push_back((uint32_t)nav.graph[(size_t)i * nav.max_m + j]);
  }
  std::ofstream f(dir + "/nav_index", std::ios::binary);
  const uint64_t fsize = 24 + 4 * (uint64_t)body.size(), frozen = 0;
  const uint32_t max_m = (uint32_t)nav.max_m, start = (uint32_t)nav.start;
  f.write(reinterpret_cast<const char*>(&fsize), 8);
  f.write(reinterpret_cast<const char*>(&max_m), 4);
  f.write(reinterpret_cast<const char*>(&start), 4);
  f.write(reinterpret_cast<const char*>(&frozen), 8);
  f.write(reinterpret_cast<const char*>(body.data()), (std::streamsize)(4 * body.size()));
  if (!f) fail(QV_EIO, "cannot write " + dir + "/nav_index");
}

template <class T>
std::vector<T> read_typed_bin(const std::string& path, int64_t& n, int64_t& d) {
  int nr = 0, nc = 0;
  auto v = read_bin_at<T>(path, 0, nr, nc);
  n = nr;
  d = nc;
  return v;
}

// write_typed_bin (bin/common/data_io.hpp:116-140)
template <class T>
void write_typed_bin(const std::string& path, const T* data, int64_t n, int64_t d) {
  if (n > INT32_MAX || d > INT32_MAX) fail(QV_EINVAL, "Binary dimensions exceed int32 range");
  std::ofstream out(path, std::ios::binary | std::ios::trunc);
  if (!out.is_open()) fail(QV_EIO, "Failed to open binary result file " + path);
  int32_t h[2] = {(int32_t)n, (int32_t)d};
  out.write(reinterpret_cast<const char*>(h), 8);
  out.write(reinterpret_cast<const char*>(data), (std::streamsize)(sizeof(T) * (size_t)n * (size_t)d));
  if (!out) fail(QV_EIO, "Failed to write binary result file " + path);
}

template std::vector<float> read_typed_bin<float>(const std::string&, int64_t&, int64_t&);
template std::vector<uint8_t> read_typed_bin<uint8_t>(const std::string&, int64_t&, int64_t&);
template std::vector<int8_t> read_typed_bin<int8_t>(const std::string&, int64_t&, int64_t&);
template std::vector<int32_t> read_typed_bin<int32_t>(const std::string&, int64_t&, int64_t&);
template void write_typed_bin<float>(const std::string&, const float*, int64_t, int64_t);
template void write_typed_bin<uint8_t>(const std::string&, const uint8_t*, int64_t, int64_t);
template void write_typed_bin<int8_t>(const std::string&, const int8_t*, int64_t, int64_t);
template void write_typed_bin<int32_t>(const std::string&, const int32_t*, int64_t, int64_t);

}  // namespace qv
