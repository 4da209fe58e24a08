// qv_search.hip -- persistent beam-search kernel for CDNA4 and its host driver.
//
// Reference path (ruc-system/quiver-ae): persistent_search_kernel
// (src/quiver/kernel_core/kernel_q1.cuh:20-757) driven by run_persistent_search
// (src/quiver/search.cu:357-1361).  Differences by design:
//   * one 64-lane wavefront per query, in one of two kernels: search_kernel
//     (one-wave workgroups, the query's fp32 LUT in LDS) or search_kernel_sp
//     (one workgroup of up to 16 waves per CU sharing the PQ pivots in LDS,
//     each LUT entry recomputed where it is read); query and beam live in LDS;
//     neighbour lists, vectors and PQ codes are read straight from HBM (no CPU
//     poll threads, no 4 KB page copies), and the next node's record is
//     requested while the current hop finishes;
//   * the merge is built by rank: "is this neighbour already in the beam" is
//     answered by the neighbour's own rank in the sorted LDS beam (a beam
//     entry of the same id has the same key), and the few new candidates are
//     scattered into LDS in place, instead of merge-path rounds with block
//     barriers;
//   * a device work queue (atomic ticket) gated by a host-written feed count,
//     completion published to a host ring so per-query latency is exact.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <tuple>
#include <mutex>
#include <numeric>
#include <thread>
#include <vector>

#include "qv_common.hpp"
#include "qv_device.hpp"
#include "qv_hip_util.hpp"
#include "qv_index_impl.hpp"
#include "qv_order_stats.hpp"

using namespace qv;
using namespace qv::dev;

#include "qv_search_kernels.hpp"

using namespace qv::sk;

namespace {

// Graph check run once at open: degree <= R, neighbour ids < n, no duplicate id
// inside one adjacency list (the reference's merge-path sort assumes distinct
// keys, kernel_helpers.cuh:300-329).  One wave per node; with R > 64 lane l
// also holds slot l + 64, and each id is compared with every later one.
__global__ __launch_bounds__(256) void validate_kernel(const uint8_t* pages, int64_t n,
                                                       int64_t npp, int64_t node_size,
                                                       int64_t data_size, int R,
                                                       int32_t* err, int64_t* first_bad) {
  const int lane = lane_id();
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x / kWave);
  for (int64_t v = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave; v < n;
       v += waves) {
    const int64_t page = v / npp;
    const uint8_t* rec = pages + page * 4096 + (v - page * npp) * node_size;
    const uint32_t* r32 = reinterpret_cast<const uint32_t*>(rec + data_size);
    const uint32_t deg = (uint32_t)__builtin_amdgcn_readfirstlane((int)r32[0]);
    int32_t bits = 0;
    if (deg > (uint32_t)R) bits |= 1;
    const uint32_t lim = deg < (uint32_t)R ? deg : (uint32_t)R;
    const bool has = (uint32_t)lane < lim;
    const uint32_t nb = has ? r32[1 + lane] : 0u;
    if (has && (int64_t)nb >= n) bits |= 2;
    if (R <= kWave) {
      uint64_t key = has ? (uint64_t)nb : ((1ull << 32) + (uint64_t)lane);
      key = wave_sort_desc(key);
      const uint64_t up = ((uint64_t)lane_up1_u32((uint32_t)(key >> 32)) << 32) | lane_up1_u32((uint32_t)key);
      if (lane > 0 && up == key) bits |= 4;
    } else {
      const bool has2 = (uint32_t)(lane + kWave) < lim;
      const uint32_t nb2 = has2 ? r32[1 + kWave + lane] : 0u;
      if (has2 && (int64_t)nb2 >= n) bits |= 2;
      for (uint32_t j = 0; j < lim; j++) {
        const uint32_t b = j < (uint32_t)kWave ? read_lane_u32(nb, (int)j) : read_lane_u32(nb2, (int)j - kWave);
        if ((has && (uint32_t)lane > j && nb == b) || (has2 && (uint32_t)(lane + kWave) > j && nb2 == b)) bits |= 4;
      }
    }
    const uint64_t any = __ballot(bits != 0);
    if (any) {
      int32_t all = bits;
      for (int off = 32; off > 0; off >>= 1) all |= __shfl_xor(all, off);
      if (lane == 0) {
        atomicOr(err, all);
        atomicMin(reinterpret_cast<unsigned long long*>(first_bad), (unsigned long long)v);
      }
    }
  }
}

// Neighbour code table: row (v, j) of [n][R][M] is the code row of node v's
// neighbour j, zero past v's degree.  One thread per row, 16 bytes at a time.
__global__ __launch_bounds__(256) void neighbour_codes_kernel(const uint8_t* pages, int64_t n, int64_t npp,
                                                              int64_t node_size, int64_t data_size, int R,
                                                              const uint8_t* codes, int M, uint8_t* out) {
  const int64_t rows = n * R;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = r / R;
    const int j = (int)(r - v * R);
    const int64_t page = v / npp;
    const uint32_t* r32 =
        reinterpret_cast<const uint32_t*>(pages + page * 4096 + (v - page * npp) * node_size + data_size);
    const uint32_t deg = r32[0];
    uint4* dst = reinterpret_cast<uint4*>(out + r * M);
    if ((uint32_t)j < deg) {
      const uint4* src = reinterpret_cast<const uint4*>(codes + (int64_t)r32[1 + j] * M);
      for (int t = 0; t < M / 16; t++) dst[t] = src[t];
    } else {
      for (int t = 0; t < M / 16; t++) dst[t] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
}

// Kernels of this translation unit: one neighbour per lane (R <= 64) and up
// to 7 beam positions per lane (ef <= 448); the others come from
// qv_search_r128.hip and qv_search_deep.hip.
template <class T, int Q>
KernelFn pick_mc(int M) {
  if (M == 32) return search_kernel<T, Q, 32, 1>;
  if (M == 48) return search_kernel<T, Q, 48, 1>;
  return search_kernel<T, Q, 0, 1>;
}

template <class T>
KernelFn pick_q(int Q, int M) {
  if (Q == 1) return pick_mc<T, 1>(M);
  if (Q == 2) return pick_mc<T, 2>(M);
  if (Q == 4) return pick_mc<T, 4>(M);
  return pick_mc<T, 7>(M);
}

KernelFn pick_kernel(int dtype, int Q, int M, int npl) {
  KernelFn k = nullptr;
  if (npl > 1)
    k = pick_kernel_r128(dtype, Q, M);
  else if (Q > 7)
    k = pick_kernel_deep(dtype, Q, M);
  else if (dtype == QV_UINT8)
    k = pick_q<uint8_t>(Q, M);
  else if (dtype == QV_INT8)
    k = pick_q<int8_t>(Q, M);
  else
    k = pick_q<float>(Q, M);
  if (!k) fail(QV_EUNSUPPORTED, "no search kernel for this degree and ef");
  return k;
}

// Shared-pivot kernels: M = 32 chunks of 4 dimensions, M = 48 chunks of 2.
template <class T, int MC, int SC>
KernelFn pick_sp_q(int Q) {
  switch (Q) {
    case 1: return search_kernel_sp<T, 1, MC, SC, 1>;
    case 2: return search_kernel_sp<T, 2, MC, SC, 1>;
    case 3: return search_kernel_sp<T, 3, MC, SC, 1>;
    case 4: return search_kernel_sp<T, 4, MC, SC, 1>;
    case 5: return search_kernel_sp<T, 5, MC, SC, 1>;
    case 6: return search_kernel_sp<T, 6, MC, SC, 1>;
    default: return search_kernel_sp<T, 7, MC, SC, 1>;
  }
}

template <class T>
KernelFn pick_sp_t(int Q, int M) {
  return M == 32 ? pick_sp_q<T, 32, 4>(Q) : pick_sp_q<T, 48, 2>(Q);
}

KernelFn pick_kernel_sp(int dtype, int Q, int M, int npl) {
  KernelFn k = nullptr;
  if (npl > 1)
    k = pick_kernel_sp_r128(dtype, Q, M);
  else if (Q > 7)
    k = pick_kernel_sp_deep(dtype, Q, M);
  else if (dtype == QV_UINT8)
    k = pick_sp_t<uint8_t>(Q, M);
  else if (dtype == QV_INT8)
    k = pick_sp_t<int8_t>(Q, M);
  else
    k = pick_sp_t<float>(Q, M);
  if (!k) fail(QV_EUNSUPPORTED, "no shared-pivot kernel for this degree and ef");
  return k;
}

// Beam positions per lane for ef (beam capacity 64 Q >= ef; kMaxEf = 2048 = 64 * 32).
// The per-query-LUT kernel comes in Q = 1, 2, 4, 7, 10, 16 and 32 (its 32 KB LUT,
// not the beam, sets how many queries a CU holds up to Q = 16); the shared-pivot
// kernel stops at ef = 1024 (kMaxEfShared) and comes in
// every Q from 1 to 7, then 10 and 16 (its LDS beam holds ef rounded up to 8
// entries, and that decides how many queries a CU holds: at d = 128, 16 up to
// ef = 192, then 15 at 208, 13 at 240, 12 at 256, 11 at 288, 10 at 320, 9 at
// 384, 8 at 448, 7 at 512 and 3 at 1024).
int beam_chunks(int ef) {
  return ef <= 64 ? 1 : (ef <= 128 ? 2 : (ef <= 256 ? 4 : (ef <= 448 ? 7 : (ef <= 640 ? 10 : (ef <= 1024 ? 16 : kXlQ)))));
}
int beam_chunks_sp(int ef) {
  const int q = (std::max(ef, 1) + kWave - 1) / kWave;
  return q <= 7 ? q : (q <= 10 ? 10 : 16);
}

// Neighbour slots per lane for an index of max degree R.
int slots_per_lane(int64_t R) { return R <= kWave ? 1 : 2; }

// A search launch: kernel, workgroup size (waves = queries per workgroup),
// dynamic LDS and the query slots (waves) one CU holds.
struct LaunchPlan {
  KernelFn kern = nullptr;
  int waves = 1;
  int lds = 0;
  int slots_per_cu = 0;
  int variant = QV_KERNEL_LUT;
  int lds_shared = 0;  // LDS of the workgroup beside its waves' (the shared pivots)
  int lds_wave = 0;    // LDS per wave (query)
};

// Grid of a launch holding `slots` query slots.  A shared-pivot workgroup
// that a full device would give lp.waves waves gets fewer when the slots do
// not fill every CU, so the queries spread over all CUs instead of packing
// into the first ones.
struct LaunchShape {
  int grid, waves, lds;
};
LaunchShape shape_launch(const LaunchPlan& lp, int64_t slots, int num_cus) {
  LaunchShape sh;
  sh.waves = lp.waves;
  if (lp.variant == QV_KERNEL_SHARED_PIVOTS)
    sh.waves = (int)std::max<int64_t>(1, std::min<int64_t>(lp.waves, (slots + num_cus - 1) / num_cus));
  sh.grid = (int)((slots + sh.waves - 1) / sh.waves);
  sh.lds = lp.variant == QV_KERNEL_SHARED_PIVOTS ? lp.lds_shared + sh.waves * lp.lds_wave : lp.lds;
  return sh;
}

// ---- scratch of the allocation-free search entry point (qv_search_noalloc) --
// One fixed array per device, held from module load to process end:
//   [0, 256)                     dispatch counters (ticket, done, error bits)
//   [256, +4 kNoAllocMaxQueries) per-query hop counts
//   [.., +4 kNoAllocMaxQueries)  per-query ADC evaluation counts
//   [.., +4 kNoAllocMaxQueries)  per-query early-exit flags
//   [.., +4 kMaxTailWorkgroups)  ended waves per workgroup (shared-pivot tail mode)
// Host code never uses the symbol's name as an address: each device's copy is
// looked up once with hipGetSymbolAddress.
constexpr int64_t kNoAllocBytes = QV_NOALLOC_SCRATCH_BYTES;
constexpr int64_t kNoAllocMaxQueries = QV_NOALLOC_MAX_QUERIES;
constexpr int64_t kNoAllocHopsOff = 256;
constexpr int64_t kNoAllocEvalsOff = kNoAllocHopsOff + 4 * kNoAllocMaxQueries;
constexpr int64_t kNoAllocStoppedOff = kNoAllocEvalsOff + 4 * kNoAllocMaxQueries;
constexpr int64_t kNoAllocWgDoneOff = kNoAllocStoppedOff + 4 * kNoAllocMaxQueries;
static_assert(kNoAllocWgDoneOff + 4 * kMaxTailWorkgroups <= kNoAllocBytes, "scratch holds every count");
__device__ __align__(256) uint8_t scratch[kNoAllocBytes];

// Zero fill by vector stores: the allocation-free entry point calls no
// memset of any kind.
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int64_t words) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// totals[0] += sum of hops, totals[1] += sum of evals, totals[2] += early
// exits (64-bit).
__global__ __launch_bounds__(256) void sum_counts_kernel(const int32_t* hops, const int32_t* evals,
                                                         const int32_t* stopped, int64_t n,
                                                         unsigned long long* totals) {
  unsigned long long h = 0, e = 0, s = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    h += (unsigned long long)hops[i];
    e += (unsigned long long)evals[i];
    s += (unsigned long long)stopped[i];
  }
  for (int off = 32; off > 0; off >>= 1) {
    h += shfl_xor64(h, off);
    e += shfl_xor64(e, off);
    s += shfl_xor64(s, off);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&totals[0], h);
    atomicAdd(&totals[1], e);
    atomicAdd(&totals[2], s);
  }
}

}  // namespace

// ============================================================== host side ===

namespace qv {

static void free_scratch(qv_index* ix) {
  hipFree(ix->d_queries);
  hipFree(ix->d_ids);
  hipFree(ix->d_dists);
  hipFree(ix->d_found);
  hipFree(ix->d_hops);
  hipFree(ix->d_stopped);
  hipFree(ix->d_evals);
  hipFree(ix->d_tstart);
  hipFree(ix->d_tend);
  hipHostFree(ix->h_ring);
  hipHostFree(ix->h_stage);
  hipHostFree(ix->h_qstage);
  hipHostFree(ix->h_results);
  ix->d_queries = nullptr;
  ix->d_ids = ix->d_found = ix->d_hops = ix->d_stopped = ix->d_evals = nullptr;
  ix->d_dists = nullptr;
  ix->d_tstart = ix->d_tend = nullptr;
  ix->h_ring = nullptr;
  ix->h_stage = nullptr;
  ix->h_qstage = nullptr;
  ix->h_results = nullptr;
  ix->cap_q = 0;
  ix->cap_k = 0;
}

static void ensure_scratch(qv_index* ix, int64_t nq, int k) {
  if (!ix->d_counters) {
    // 64 bytes of launch counters, then the shared-pivot kernel's count of
    // ended waves per workgroup (tail mode)
    HIP_OK(hipMalloc(&ix->d_counters, 64 + 4 * kMaxTailWorkgroups));
    HIP_OK(hipHostMalloc(reinterpret_cast<void**>(&ix->h_ctrl), 64, hipHostMallocCoherent));
  }
  if (!ix->d_feed_mirror) {
    HIP_OK(hipMalloc(&ix->d_feed_mirror, kFeedMirrorBytes));
    HIP_OK(hipMemset(ix->d_feed_mirror, 0, kFeedMirrorBytes));
    HIP_OK(hipDeviceSynchronize());
    ix->feed_epoch = 0;
  }
  if (nq <= ix->cap_q && k <= ix->cap_k) return;
  free_scratch(ix);
  const int64_t cq = std::max<int64_t>(nq, 1024);
  const int ck = std::max(k, 16);
  const int d = (int)ix->lay.num_dims;
  HIP_OK(hipMalloc(&ix->d_queries, sizeof(float) * (size_t)cq * d));
  HIP_OK(hipMalloc(&ix->d_ids, sizeof(int32_t) * (size_t)cq * ck));
  HIP_OK(hipMalloc(&ix->d_dists, sizeof(float) * (size_t)cq * ck));
  HIP_OK(hipMalloc(&ix->d_found, sizeof(int32_t) * (size_t)cq));
  HIP_OK(hipMalloc(&ix->d_hops, sizeof(int32_t) * (size_t)cq));
  HIP_OK(hipMalloc(&ix->d_stopped, sizeof(int32_t) * (size_t)cq));
  HIP_OK(hipMalloc(&ix->d_evals, sizeof(int32_t) * (size_t)cq));
  HIP_OK(hipMalloc(&ix->d_tstart, sizeof(uint64_t) * (size_t)cq));
  HIP_OK(hipMalloc(&ix->d_tend, sizeof(uint64_t) * (size_t)cq));
  HIP_OK(hipHostMalloc(reinterpret_cast<void**>(&ix->h_ring), sizeof(int32_t) * (size_t)cq,
                       hipHostMallocCoherent));
  // coherent: the search kernel writes the per-query hop, stop and evaluation
  // counts straight into it
  HIP_OK(hipHostMalloc(reinterpret_cast<void**>(&ix->h_stage), sizeof(int32_t) * (size_t)(kStageHead + 3 * cq),
                       hipHostMallocCoherent));
  // coherent (not cached by the GPU): a host-buffer call copies its queries
  // here while the kernel already runs, and the kernel reads them in place
  HIP_OK(hipHostMalloc(reinterpret_cast<void**>(&ix->h_qstage), sizeof(float) * (size_t)cq * d,
                       hipHostMallocCoherent));
  // coherent: a host-buffer call's kernel writes its results here, and the
  // host copies them out once the launch has ended (one host memcpy instead of
  // a device-to-pageable copy through the runtime's bounce buffers)
  HIP_OK(hipHostMalloc(&ix->h_results, sizeof(int32_t) * (size_t)cq * (2 * (size_t)ck + 1), hipHostMallocCoherent));
  ix->cap_q = cq;
  ix->cap_k = ck;
}

void release_index(qv_index* ix) {
  if (!ix) return;
  hipSetDevice(ix->device);
  free_scratch(ix);
  hipFree(ix->d_counters);
  hipFree(ix->d_feed_mirror);
  hipHostFree(ix->h_ctrl);
  hipFree(ix->d_nav_data);
  hipFree(ix->d_nav_graph);
  hipFree(ix->d_nav_map);
  hipFree(ix->d_nbr_codes);
  if (ix->pages_in_host)
    hipHostFree(ix->d_pages);
  else
    hipFree(ix->d_pages);
  hipFree(ix->d_codes);
  hipFree(ix->d_centroid);
  hipFree(ix->d_pivots_t);
  hipFree(ix->d_chunk_off);
  if (ix->ev0) hipEventDestroy(ix->ev0);
  if (ix->ev1) hipEventDestroy(ix->ev1);
  if (ix->stream) hipStreamDestroy(ix->stream);
  delete ix;
}

// Source of the page image: the file read with stdio (heap backend,
// mem_loader.cpp:28-44) or mapped read-only (mmap backend, mem_loader.cpp:46-85,
// including its size check).  Either way the pages are copied once, at open,
// to where the kernel reads them.
class PageSource {
 public:
  PageSource(const std::string& path, int64_t num_pages, bool use_mmap) : path_(path) {
    if (!use_mmap) {
      f_ = std::fopen(path.c_str(), "rb");
      if (!f_) fail(QV_EIO, "Failed to open Mem Index: " + path);
      if (std::fseek(f_, kPageSize, SEEK_SET) != 0) fail(QV_EIO, "Failed to seek Mem Index: " + path);
      return;
    }
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) fail(QV_EIO, "Failed to open mmap Mem Index " + path + ": " + std::strerror(errno));
    struct stat st {};
    if (::fstat(fd_, &st) != 0) fail(QV_EIO, "Failed to stat mmap Mem Index " + path + ": " + std::strerror(errno));
    const int64_t required = (num_pages + 1) * kPageSize;
    if ((int64_t)st.st_size < required)
      fail(QV_EIO, "mmap Mem Index " + path + " is too small: size=" + std::to_string((long long)st.st_size) +
                       " required=" + std::to_string((long long)required));
    len_ = (size_t)st.st_size;
    void* m = ::mmap(nullptr, len_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (m == MAP_FAILED) fail(QV_EIO, "Failed to mmap Mem Index " + path + ": " + std::strerror(errno));
    map_ = static_cast<uint8_t*>(m);
    ::madvise(map_, len_, MADV_SEQUENTIAL);
  }
  ~PageSource() {
    if (f_) std::fclose(f_);
    if (map_) ::munmap(map_, len_);
    if (fd_ >= 0) ::close(fd_);
  }
  // Copies pages [p, p + cnt) of the image (file page p + 1) to host memory dst.
  void read(int64_t p, int64_t cnt, uint8_t* dst) {
    if (map_) {
      std::memcpy(dst, map_ + (p + 1) * kPageSize, (size_t)(cnt * kPageSize));
      return;
    }
    const int64_t got = (int64_t)std::fread(dst, kPageSize, (size_t)cnt, f_);
    if (got != cnt)
      fail(QV_EIO, "Mem Index Load FAILED: " + std::to_string(p + got) + " pages read from " + path_);
  }

 private:
  std::string path_;
  FILE* f_ = nullptr;
  int fd_ = -1;
  uint8_t* map_ = nullptr;
  size_t len_ = 0;
};

// Copies the page image to HBM through a pinned staging buffer, or straight
// into dst when dst is pinned host memory.
static void upload_index_pages(PageSource& src, int64_t num_pages, uint8_t* dst, bool dst_in_host) {
  const int64_t chunk_pages = 16384;  // 64 MB
  if (dst_in_host) {
    for (int64_t p = 0; p < num_pages; p += chunk_pages)
      src.read(p, std::min(chunk_pages, num_pages - p), dst + p * kPageSize);
    return;
  }
  uint8_t* stage = nullptr;
  HIP_OK(hipHostMalloc(reinterpret_cast<void**>(&stage), (size_t)(chunk_pages * kPageSize),
                       hipHostMallocDefault));
  std::unique_ptr<uint8_t, void (*)(uint8_t*)> guard(stage, [](uint8_t* p) { hipHostFree(p); });
  for (int64_t p = 0; p < num_pages; p += chunk_pages) {
    const int64_t cnt = std::min(chunk_pages, num_pages - p);
    src.read(p, cnt, stage);
    HIP_OK(hipMemcpy(dst + p * kPageSize, stage, (size_t)(cnt * kPageSize), hipMemcpyHostToDevice));
  }
}

void validate_graph(qv_index* ix) {
  int32_t* d_err = nullptr;
  int64_t* d_bad = nullptr;
  HIP_OK(hipMalloc(&d_err, sizeof(int32_t)));
  HIP_OK(hipMalloc(&d_bad, sizeof(int64_t)));
  HIP_OK(hipMemsetAsync(d_err, 0, sizeof(int32_t), ix->stream));
  HIP_OK(hipMemsetAsync(d_bad, 0x7f, sizeof(int64_t), ix->stream));
  const Layout& L = ix->lay;
  const int blocks = (int)std::min<int64_t>((L.num_data + 3) / 4, 65536);
  hipLaunchKernelGGL(validate_kernel, dim3(blocks), dim3(256), 0, ix->stream, ix->d_pages,
                     L.num_data, L.nodes_per_page, L.node_size, L.data_size, (int)L.max_m0,
                     d_err, d_bad);
  HIP_OK(hipGetLastError());
  HIP_OK(hipStreamSynchronize(ix->stream));
  int32_t err = 0;
  int64_t bad = 0;
  HIP_OK(hipMemcpy(&err, d_err, sizeof(err), hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(&bad, d_bad, sizeof(bad), hipMemcpyDeviceToHost));
  hipFree(d_err);
  hipFree(d_bad);
  if (err) {
    std::string what;
    if (err & 1) what += " degree>R";
    if (err & 2) what += " neighbour-id>=n";
    if (err & 4) what += " duplicate-neighbour";
    fail(QV_EINDEX, "invalid graph (first bad node " + std::to_string(bad) + "):" + what);
  }
}

qv_index* open_index(const std::string& index_dir, const std::string& dtype_s,
                     const std::string& backend, const std::string& mem_file, int device, int placement) {
  const int dtype = parse_data_type(dtype_s);
  if (backend != "heap" && backend != "mmap")
    fail(QV_EINVAL, "Unsupported --memory-backend '" + backend + "'. Expected one of: heap, mmap");
  if (placement != QV_GRAPH_HBM && placement != QV_GRAPH_HOST)
    fail(QV_EINVAL, "graph placement must be QV_GRAPH_HBM or QV_GRAPH_HOST");
  const std::string index_file = find_index_file(index_dir);
  const std::string pages_file = mem_file.empty() ? index_file : mem_file;
  const std::string prefix = find_pq_prefix(index_dir);
  Layout lay = parse_diskann_metadata(index_file, dtype);
  PQTables pq;
  read_pq_tables(prefix + "_pivots.bin", prefix + "_compressed.bin", pq);
  if (pq.dim != lay.num_dims)
    fail(QV_EIO, "PQ dimension " + std::to_string(pq.dim) + " != index dimension " +
                     std::to_string(lay.num_dims));
  if (pq.num_pts != lay.num_data)
    fail(QV_EIO, "PQ point count " + std::to_string(pq.num_pts) + " != index point count " +
                     std::to_string(lay.num_data));
  if (lay.max_m0 > kMaxDegree || lay.max_m0 < 1)
    fail(QV_EUNSUPPORTED, "max degree " + std::to_string(lay.max_m0) + " outside [1, 128]");
  if ((lay.data_size & 3) || (lay.node_size & 3))
    fail(QV_EUNSUPPORTED, "node records must be 4-byte aligned");
  if (lay.num_data > INT32_MAX) fail(QV_EUNSUPPORTED, "more than 2^31-1 points");
  PageSource src(pages_file, lay.num_pages, backend == "mmap");

  int ndev = 0;
  HIP_OK(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev) fail(QV_EINVAL, "device " + std::to_string(device) + " not present");
  HIP_OK(hipSetDevice(device));
  const size_t page_bytes = (size_t)(lay.num_pages * kPageSize);
  const size_t code_bytes = (size_t)lay.num_data * (size_t)pq.num_chunks;
  const bool in_host = placement == QV_GRAPH_HOST;
  uint8_t* d_pages = nullptr;
  uint8_t* d_codes = nullptr;
  if (in_host) {
    // Pinned, device-mapped host memory, cached by the GPU (written once here,
    // before any kernel reads it, and never again).
    HIP_OK(hipHostMalloc(reinterpret_cast<void**>(&d_pages), page_bytes, hipHostMallocNonCoherent));
  } else {
    HIP_OK(hipMalloc(&d_pages, page_bytes));
  }
  std::unique_ptr<uint8_t, void (*)(uint8_t*)> pg(
      d_pages, in_host ? +[](uint8_t* p) { (void)hipHostFree(p); } : +[](uint8_t* p) { (void)hipFree(p); });
  HIP_OK(hipMalloc(&d_codes, std::max<size_t>(code_bytes, 64)));
  std::unique_ptr<uint8_t, void (*)(uint8_t*)> cg(d_codes, [](uint8_t* p) { (void)hipFree(p); });
  upload_index_pages(src, lay.num_pages, d_pages, in_host);
  HIP_OK(hipMemcpy(d_codes, pq.codes.data(), code_bytes, hipMemcpyHostToDevice));
  pg.release();
  cg.release();
  std::unique_ptr<qv_index, void (*)(qv_index*)> ix(
      make_index(device, lay, pq, d_pages, d_codes, true, in_host), release_index);
  const std::string nav_dir = find_nav_dir(index_dir);  // search_setup.hpp:96-106
  if (!nav_dir.empty()) load_nav(ix.get(), nav_dir);
  return ix.release();
}

// A handle from an index the caller already holds in host memory: the
// Layout, the heap image of the pages (page k = page k + 1 of the disk index,
// MemLoaderSync::load_heap, mem_loader.cpp:28-44) and PQSearchData's host
// tables (pq_search.hpp:13-29; chunk_id per dimension, contiguous chunks).
// Checked as open_index checks files; everything is copied to HBM.
qv_index* index_from_memory(const qv_index_info& li, const uint8_t* pages, const float* centroid,
                            const float* pivots, const int32_t* chunk_id, int num_chunks, const uint8_t* codes,
                            int device) {
  if (!pages || !centroid || !pivots || !chunk_id || !codes) fail(QV_EINVAL, "null argument");
  Layout lay;
  lay.data_type = li.data_type;
  if (lay.data_type != QV_UINT8 && lay.data_type != QV_FLOAT && lay.data_type != QV_INT8)
    fail(QV_EINVAL, "data type must be QV_UINT8, QV_FLOAT or QV_INT8");
  lay.num_data = li.num_data;
  lay.num_dims = li.num_dims;
  lay.max_m0 = li.max_m0;
  lay.enter_point = li.enter_point;
  lay.data_size = li.data_size;
  lay.node_size = li.node_size;
  lay.num_pages = li.num_pages;
  lay.nodes_per_page = li.nodes_per_page;
  if (lay.num_data <= 0 || lay.num_data > INT32_MAX) fail(QV_EUNSUPPORTED, "num_data must be in [1, 2^31-1]");
  if (lay.num_dims <= 0 || lay.data_size != lay.num_dims * elem_size(lay.data_type))
    fail(QV_EINDEX, "data_size must be num_dims x the element size");
  if (lay.max_m0 > kMaxDegree || lay.max_m0 < 1)
    fail(QV_EUNSUPPORTED, "max degree " + std::to_string(lay.max_m0) + " outside [1, 128]");
  if (lay.node_size != lay.data_size + 4 + 4 * lay.max_m0)
    fail(QV_EINDEX, "node_size must be data_size + 4 + 4 max_m0");
  if ((lay.data_size & 3) || (lay.node_size & 3)) fail(QV_EUNSUPPORTED, "node records must be 4-byte aligned");
  if (lay.nodes_per_page != kPageSize / lay.node_size || lay.nodes_per_page < 1)
    fail(QV_EINDEX, "nodes_per_page must be 4096 / node_size");
  if (lay.num_pages < (lay.num_data + lay.nodes_per_page - 1) / lay.nodes_per_page)
    fail(QV_EINDEX, "num_pages too small for num_data records");
  if (lay.enter_point < 0 || lay.enter_point >= lay.num_data) fail(QV_EINDEX, "enter_point out of range");
  const int dim = (int)lay.num_dims;
  if (num_chunks < 1 || num_chunks > dim) fail(QV_EINVAL, "num_chunks must be in [1, dim]");
  PQTables pq;
  pq.dim = dim;
  pq.num_chunks = num_chunks;
  pq.num_pts = lay.num_data;
  pq.centroid.assign(centroid, centroid + dim);
  pq.pivots.assign(pivots, pivots + (size_t)kNumPivots * dim);
  pq.pivots_t.assign((size_t)dim * kNumPivots, 0.f);
  for (int c = 0; c < kNumPivots; c++)
    for (int j = 0; j < dim; j++) pq.pivots_t[(size_t)j * kNumPivots + c] = pq.pivots[(size_t)c * dim + j];
  pq.chunk_id.assign(chunk_id, chunk_id + dim);
  pq.chunk_offsets.assign((size_t)num_chunks + 1, 0);
  for (int j = 0; j < dim; j++) {
    const int m = chunk_id[j];
    if (m < 0 || m >= num_chunks || (j > 0 && m < chunk_id[j - 1]))
      fail(QV_EINDEX, "chunk_id must be non-decreasing in [0, num_chunks): PQ chunks are contiguous");
    pq.chunk_offsets[(size_t)m + 1]++;
  }
  for (int m = 0; m < num_chunks; m++) pq.chunk_offsets[(size_t)m + 1] += pq.chunk_offsets[(size_t)m];

  int ndev = 0;
  HIP_OK(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev) fail(QV_EINVAL, "device " + std::to_string(device) + " not present");
  HIP_OK(hipSetDevice(device));
  const size_t page_bytes = (size_t)(lay.num_pages * kPageSize);
  const size_t code_bytes = (size_t)lay.num_data * (size_t)num_chunks;
  uint8_t* d_pages = nullptr;
  uint8_t* d_codes = nullptr;
  HIP_OK(hipMalloc(&d_pages, page_bytes));
  std::unique_ptr<uint8_t, void (*)(uint8_t*)> pg(d_pages, [](uint8_t* p) { (void)hipFree(p); });
  HIP_OK(hipMalloc(&d_codes, std::max<size_t>(code_bytes, 64)));
  std::unique_ptr<uint8_t, void (*)(uint8_t*)> cg(d_codes, [](uint8_t* p) { (void)hipFree(p); });
  HIP_OK(hipMemcpy(d_pages, pages, page_bytes, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_codes, codes, code_bytes, hipMemcpyHostToDevice));
  pg.release();
  cg.release();
  return make_index(device, lay, pq, d_pages, d_codes, true, false);
}

// NavGraph::init + copy_to_dev (nav_graph.cu:12-73) into this handle's device.
void set_neighbour_codes(qv_index* ix, bool enable) {
  HIP_OK(hipSetDevice(ix->device));
  if (!enable) {
    if (ix->d_nbr_codes) {
      HIP_OK(hipStreamSynchronize(ix->stream));
      hipFree(ix->d_nbr_codes);
      ix->device_bytes -= ix->nbr_codes_bytes;
    }
    ix->d_nbr_codes = nullptr;
    ix->nbr_codes_bytes = 0;
    return;
  }
  if (ix->d_nbr_codes) return;
  const Layout& L = ix->lay;
  // Only the 32- and 48-chunk hops read code rows from the table (kRows);
  // any other M would hold its bytes and change nothing.
  if (ix->M != 32 && ix->M != 48) fail(QV_EUNSUPPORTED, "the neighbour code table needs M = 32 or 48");
  if (L.max_m0 > kWave) fail(QV_EUNSUPPORTED, "the neighbour code table needs R <= 64");
  const int64_t bytes = L.num_data * L.max_m0 * ix->M;
  size_t free_b = 0, total_b = 0;
  HIP_OK(hipMemGetInfo(&free_b, &total_b));
  if ((int64_t)free_b < bytes + (int64_t)(1ll << 30))
    fail(QV_ENOMEM, "the neighbour code table needs " + std::to_string(bytes >> 20) + " MiB, " +
                        std::to_string(free_b >> 20) + " MiB free");
  uint8_t* d = nullptr;
  HIP_OK(hipMalloc(&d, (size_t)bytes));
  hipLaunchKernelGGL(neighbour_codes_kernel, dim3(65536), dim3(256), 0, ix->stream, ix->d_pages, L.num_data,
                     L.nodes_per_page, L.node_size, L.data_size, (int)L.max_m0, ix->d_codes, ix->M, d);
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    const hipError_t s2 = hipStreamSynchronize(ix->stream);
    if (s2 == hipSuccess) {
      ix->d_nbr_codes = d;
      ix->nbr_codes_bytes = bytes;
      ix->device_bytes += bytes;
      return;
    }
    hipFree(d);
    fail(QV_EHIP, std::string("neighbour_codes_kernel: ") + hipGetErrorString(s2));
  }
  hipFree(d);
  fail(QV_EHIP, std::string("neighbour_codes_kernel: ") + hipGetErrorString(e));
}

void load_nav(qv_index* ix, const std::string& dir) {
  NavGraphHost nav;
  read_nav(dir, ix->lay.data_type, ix->lay.num_data, ix->lay.num_dims, nav);
  upload_nav(ix, nav);
}

// A nav graph already in host memory (checked like read_nav's files) to the
// handle's device, replacing any previous one.
void upload_nav(qv_index* ix, const NavGraphHost& nav) {
  check_nav(nav, ix->lay.num_data, ix->lay.num_dims, ix->lay.data_type);
  HIP_OK(hipSetDevice(ix->device));
  uint8_t* dd = nullptr;
  int32_t *dg = nullptr, *dm = nullptr;
  HIP_OK(hipMalloc(&dd, nav.data.size()));
  HIP_OK(hipMalloc(&dg, sizeof(int32_t) * nav.graph.size()));
  HIP_OK(hipMalloc(&dm, sizeof(int32_t) * nav.mapping.size()));
  HIP_OK(hipMemcpy(dd, nav.data.data(), nav.data.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dg, nav.graph.data(), sizeof(int32_t) * nav.graph.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dm, nav.mapping.data(), sizeof(int32_t) * nav.mapping.size(), hipMemcpyHostToDevice));
  hipFree(ix->d_nav_data);
  hipFree(ix->d_nav_graph);
  hipFree(ix->d_nav_map);
  ix->d_nav_data = dd;
  ix->d_nav_graph = dg;
  ix->d_nav_map = dm;
  ix->nav_nodes = nav.num_node;
  ix->nav_max_m = nav.max_m;
  ix->nav_start = nav.start;
}

qv_index* make_index(int device, const Layout& lay, const PQTables& pq, uint8_t* d_pages,
                     uint8_t* d_codes, bool validate, bool pages_in_host) {
  std::unique_ptr<qv_index, void (*)(qv_index*)> ix(new qv_index(), release_index);
  ix->device = device;
  ix->lay = lay;
  ix->M = pq.num_chunks;
  ix->d_pages = d_pages;
  ix->pages_in_host = pages_in_host;
  ix->d_codes = d_codes;
  HIP_OK(hipSetDevice(device));
  hipDeviceProp_t prop;
  HIP_OK(hipGetDeviceProperties(&prop, device));
  ix->num_cus = prop.multiProcessorCount;
  HIP_OK(hipDeviceGetAttribute(&ix->lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, device));
  HIP_OK(hipStreamCreateWithFlags(&ix->stream, hipStreamNonBlocking));
  HIP_OK(hipEventCreate(&ix->ev0));
  HIP_OK(hipEventCreate(&ix->ev1));
  HIP_OK(hipMalloc(&ix->d_centroid, sizeof(float) * pq.centroid.size()));
  HIP_OK(hipMalloc(&ix->d_pivots_t, sizeof(float) * pq.pivots_t.size()));
  HIP_OK(hipMalloc(&ix->d_chunk_off, sizeof(int32_t) * pq.chunk_offsets.size()));
  ix->device_bytes = (int64_t)((pages_in_host ? 0 : lay.num_pages * kPageSize) + lay.num_data * pq.num_chunks +
                               4 * (int64_t)(pq.centroid.size() + pq.pivots_t.size()));
  HIP_OK(hipMemcpy(ix->d_centroid, pq.centroid.data(), sizeof(float) * pq.centroid.size(),
                   hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(ix->d_pivots_t, pq.pivots_t.data(), sizeof(float) * pq.pivots_t.size(),
                   hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(ix->d_chunk_off, pq.chunk_offsets.data(),
                   sizeof(int32_t) * pq.chunk_offsets.size(), hipMemcpyHostToDevice));
  ix->h_centroid = pq.centroid;
  ix->h_pivots = pq.pivots;
  ix->h_chunk_off = pq.chunk_offsets;
  if (validate) validate_graph(ix.get());
  return ix.release();
}

// Resident workgroups of kernel k per CU at `waves` waves and `lds` bytes on
// `device` (the current one).  The first query of a kernel on a device also
// lets it take up to lds_cu bytes of dynamic LDS; answers are cached, since a
// search asks for its plan on every call.
static int occupancy(int device, int lds_cu, KernelFn k, int waves, int lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, const void*, int, int>, int> cache;
  const void* f = reinterpret_cast<const void*>(k);
  std::lock_guard<std::mutex> lk(mu);
  const auto key = std::make_tuple(device, f, waves, lds);
  const auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  const auto any = cache.lower_bound(std::make_tuple(device, f, INT32_MIN, INT32_MIN));
  if (any == cache.end() || std::get<0>(any->first) != device || std::get<1>(any->first) != f) {
    HIP_OK(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, std::max(lds_cu, 65536)));
    // The ADC addresses the per-query LUT or the shared pivot table at LDS
    // address 0: the search kernels keep all their LDS dynamic, so the area
    // starts there.
    hipFuncAttributes fa{};
    HIP_OK(hipFuncGetAttributes(&fa, f));
    if (fa.sharedSizeBytes != 0) fail(QV_EHIP, "search kernel has static LDS; the LUT or pivot table must start at 0");
  }
  int nb = 0;
  HIP_OK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, kWave * waves, (size_t)lds));
  cache.emplace(key, nb);
  return nb;
}

// The per-query-LUT kernel (one wave per workgroup, as many per CU as the LDS
// holds), or the shared-pivot kernel when the index has chunks of 4 dims
// (M = 32) or 2 dims (M = 48), one workgroup of more waves fits a CU and more
// than the LUT kernel's resident slots would be busy (`need`: queries the
// call can have in flight).  A query alone runs faster with its own LUT (a
// table read per code byte instead of a recompute); the shared pivots pay
// when twice the queries per CU keep twice the random rows in flight.
// `want` (QV_KERNEL_*) forces one; a forced shared-pivot plan the index or the
// CU cannot take is QV_EUNSUPPORTED.  A top-k above 64 runs on the
// per-query-LUT kernel only (entries past 64 in its LDS).
LaunchPlan launch_plan(qv_index* ix, int ef, int want, int64_t need, int topk) {
  if (want != QV_KERNEL_AUTO && want != QV_KERNEL_LUT && want != QV_KERNEL_SHARED_PIVOTS)
    fail(QV_EINVAL, "search kernel must be QV_KERNEL_AUTO, QV_KERNEL_LUT or QV_KERNEL_SHARED_PIVOTS");
  const bool wide = topk > kRegTopk;
  const int P = wide ? wide_beam_chunks(ef) : beam_chunks(ef);
  const int M = ix->M, d = (int)ix->lay.num_dims;
  LaunchPlan lut;
  const int npl = slots_per_lane(ix->lay.max_m0);
  lut.kern = P == kXlQ ? pick_kernel_xl(ix->lay.data_type, M, npl, wide)
                       : (wide ? pick_kernel_wide(ix->lay.data_type, P, M, npl)
                               : pick_kernel(ix->lay.data_type, P, M, npl));
  if (!lut.kern) fail(QV_EUNSUPPORTED, "no search kernel for this top-k, degree and ef");
  lut.waves = 1;
  lut.lds = lds_plan(M, d, P, true, ef, topk).total;
  lut.slots_per_cu = occupancy(ix->device, ix->lds_cu, lut.kern, 1, lut.lds);
  if (want == QV_KERNEL_LUT) return lut;
  const bool forced = want == QV_KERNEL_SHARED_PIVOTS;
  if (wide) {
    if (forced)
      fail(QV_EUNSUPPORTED, "the shared-pivot kernel keeps at most 64 results per query; topk=" +
                                std::to_string(topk) + " runs on the per-query-LUT kernel");
    return lut;
  }
  if (ef > kMaxEfShared) {
    if (forced)
      fail(QV_EUNSUPPORTED, "the shared-pivot kernel holds beams of at most 1024; ef_search=" + std::to_string(ef) +
                                " runs on the per-query-LUT kernel");
    return lut;
  }
  if (!forced && lut.slots_per_cu > 0 && need <= (int64_t)lut.slots_per_cu * ix->num_cus) return lut;
  const int sc = M == 32 ? 4 : (M == 48 ? 2 : 0);
  bool uniform = sc > 0 && d == M * sc && (int)ix->h_chunk_off.size() == M + 1;
  for (int m = 0; uniform && m <= M; m++) uniform = ix->h_chunk_off[(size_t)m] == m * sc;
  if (!uniform) {
    if (forced) fail(QV_EUNSUPPORTED, "the shared-pivot kernel needs PQ chunks of 4 dims (M = 32) or 2 dims (M = 48)");
    return lut;
  }
  const int lds_cu = ix->lds_cu;
  const int Psp = beam_chunks_sp(ef);
  const int per_wave = lds_plan(M, d, Psp, false, ef, topk).total;
  const int waves = std::min(sp_max_waves(Psp, slots_per_lane(ix->lay.max_m0)), (lds_cu - piv_bytes(d)) / per_wave);
  if (!forced && waves <= lut.slots_per_cu) return lut;
  LaunchPlan sp;
  sp.kern = pick_kernel_sp(ix->lay.data_type, Psp, M, slots_per_lane(ix->lay.max_m0));
  sp.waves = waves;
  sp.lds = piv_bytes(d) + waves * per_wave;
  sp.lds_shared = piv_bytes(d);
  sp.lds_wave = per_wave;
  sp.variant = QV_KERNEL_SHARED_PIVOTS;
  if (waves < 1 || occupancy(ix->device, ix->lds_cu, sp.kern, waves, sp.lds) < 1) {
    if (forced) fail(QV_EUNSUPPORTED, "the shared-pivot kernel does not fit on a compute unit");
    return lut;
  }
  sp.slots_per_cu = waves;
  return sp;
}

int slots_per_cu(qv_index* ix, int ef) { return launch_plan(ix, ef, QV_KERNEL_AUTO, INT64_MAX, 10).slots_per_cu; }

// page = floor(v / npp) as (v * m) >> k with k = 32 + ceil(log2 npp) and
// m = ceil(2^k / npp): the error term v (m npp - 2^k) / (npp 2^k) stays below
// 1 / (2 npp) for v < 2^31, so the quotient is exact for every node id.
static void set_page_divisor(SearchArgs& a, int64_t npp) {
  if (npp < 1 || npp > 4096) fail(QV_EINDEX, "nodes per page out of range");
  int l = 0;
  while ((int64_t(1) << l) < npp) ++l;
  const int k = 32 + l;
  a.npp_magic = ((uint64_t(1) << k) + (uint64_t)npp - 1) / (uint64_t)npp;
  a.npp_shift = k;
  for (uint64_t v : {uint64_t(0), uint64_t(npp - 1), uint64_t(npp), uint64_t(INT32_MAX - 1), uint64_t(INT32_MAX)})
    if (((v * a.npp_magic) >> k) != v / (uint64_t)npp) fail(QV_EINDEX, "page divisor check failed");
}

static SearchArgs base_args(qv_index* ix) {
  const Layout& L = ix->lay;
  SearchArgs a{};
  a.pages = ix->d_pages;
  a.codes = ix->d_codes;
  a.centroid = ix->d_centroid;
  a.pivots_t = ix->d_pivots_t;
  a.chunk_off = ix->d_chunk_off;
  a.num_points = L.num_data;
  a.nodes_per_page = L.nodes_per_page;
  set_page_divisor(a, L.nodes_per_page);
  a.node_size = L.node_size;
  a.data_size = L.data_size;
  a.dim = (int32_t)L.num_dims;
  a.num_chunks = ix->M;
  a.max_m = (int32_t)L.max_m0;
  a.medoid = (int32_t)L.enter_point;
  a.nav_data = ix->d_nav_data;
  a.nav_graph = ix->d_nav_graph;
  a.nav_map = ix->d_nav_map;
  a.nav_nodes = ix->nav_nodes;
  a.nav_max_m = ix->nav_max_m;
  a.nav_start = ix->nav_start;
  a.nbr_codes = ix->d_nbr_codes;
  return a;
}

// Whole-batch search over device queries that records every expanded node and
// its exact distance (the greedy-search step of graph construction).
void search_record(qv_index* ix, const float* d_queries, int64_t nq, int ef, const SearchRecord& rec,
                   int32_t* d_hops, int num_blocks) {
  std::lock_guard<std::mutex> lk(ix->mu);
  if (nq <= 0 || nq > INT32_MAX - 1) fail(QV_EINVAL, "number of queries out of range: " + std::to_string(nq));
  if (ef <= 0 || ef > kMaxEf) fail(QV_EINVAL, "ef_search must be in [1, 2048]");
  HIP_OK(hipSetDevice(ix->device));
  ensure_scratch(ix, nq, 1);
  const LaunchPlan lp =
      launch_plan(ix, ef, QV_KERNEL_AUTO, num_blocks > 0 ? std::min<int64_t>(nq, num_blocks) : nq, 1);
  if (lp.slots_per_cu <= 0) fail(QV_EUNSUPPORTED, "search kernel does not fit on a compute unit");
  int nb = num_blocks > 0 ? num_blocks : lp.slots_per_cu * ix->num_cus;
  nb = (int)std::min<int64_t>(std::min<int64_t>(nb, nq), (int64_t)lp.slots_per_cu * ix->num_cus);
  const LaunchShape ls = shape_launch(lp, nb, ix->num_cus);
  const int grid = ls.grid;
  SearchArgs a = base_args(ix);
  a.queries = d_queries;
  a.nq = (int32_t)nq;
  a.topk = 1;
  a.ef = ef;
  a.pipe_w = 1;
  a.early_exit = QV_EXIT_NONE;
  a.warmup = 0;
  a.patience = 0;
  a.out_ids = ix->d_ids;
  a.out_dists = ix->d_dists;
  a.out_found = nullptr;
  a.out_hops = d_hops;
  a.out_stopped = nullptr;
  a.out_evals = nullptr;
  a.t_start = nullptr;
  a.t_end = nullptr;
  a.counters = ix->d_counters;
  a.feed_count = nullptr;
  a.terminate = nullptr;
  a.ring = nullptr;
  a.spin_limit_ticks = (uint64_t)(60.0 * 1e8);
  a.rec_ids = rec.ids;
  a.rec_dists = rec.dists;
  a.rec_cap = rec.cap;
  HIP_OK(hipMemsetAsync(ix->d_counters, 0, 64, ix->stream));
  hipLaunchKernelGGL(lp.kern, dim3(grid), dim3(kWave * ls.waves), (size_t)ls.lds, ix->stream, a);
  HIP_OK(hipGetLastError());
  HIP_OK(hipStreamSynchronize(ix->stream));
  int32_t counters[4] = {0, 0, 0, 0};
  HIP_OK(hipMemcpy(counters, ix->d_counters, sizeof(counters), hipMemcpyDeviceToHost));
  if (counters[1] != nq)
    fail(QV_EHIP, "record search finished " + std::to_string(counters[1]) + " of " + std::to_string(nq) + " queries");
}

// Ranks of P50 / P90 / P99 / P99.9 / max in n ascending latencies, as the
// reference indexes its sorted buffer (search.cu:1141-1145): n 50 / 100,
// n 90 / 100 and n 99 / 100 in integers, floor(n 0.999) in double, n - 1.
static void percentile_ranks(size_t n, size_t r[5]) {
  r[0] = n * 50 / 100;
  r[1] = n * 90 / 100;
  r[2] = n * 99 / 100;
  r[3] = std::min(n - 1, (size_t)((double)n * 0.999));
  r[4] = n - 1;
}

void search(qv_index* ix, const float* queries, int64_t nq, int dim, int topk, int ef,
            const qv_search_opts& o, int32_t* ids, float* dists, int32_t* found,
            qv_search_report* rep) {
  std::lock_guard<std::mutex> lk(ix->mu);
  const Layout& L = ix->lay;
  if (nq <= 0 || nq > INT32_MAX - 1) fail(QV_EINVAL, "number of queries must be in [1, 2^31-2]");
  if (dim != L.num_dims)
    fail(QV_EINVAL, "Query dimension mismatch: queries have " + std::to_string(dim) +
                        " dims, but the index expects " + std::to_string(L.num_dims));
  if (topk <= 0 || topk > kMaxTopk) fail(QV_EINVAL, "topk must be in [1, 1024]");
  if (ef <= 0 || ef > kMaxEf) fail(QV_EINVAL, "ef_search must be in [1, 2048]");
  if (o.pipe_width < 1 || o.pipe_width > kMaxPipeWidth) fail(QV_EINVAL, "--pipe-width must be in [1, 16]");
  if (o.queries_per_block < 1 || o.queries_per_block > kMaxQueriesPerBlock)
    fail(QV_EINVAL, "--queries-per-block must be in [1, 8]");
  if (o.early_exit != QV_EXIT_NONE && o.early_exit != QV_EXIT_GPRUNING)
    fail(QV_EINVAL, "early exit policy must be none or gpruning");
  if (o.num_blocks < 0) fail(QV_EINVAL, "--num-blocks must be positive");
  const bool step_recall = o.step_recall_gt != nullptr;
  if (step_recall) {  // search.cu:492-505
    if (o.queries_per_block != 1 || o.pipe_width != 1)
      fail(QV_EINVAL, "Per-step recall currently supports only queries_per_block=1 and pipe_width=1");
    if (o.step_recall_gt_count < 1 || o.step_recall_gt_width < 1)
      fail(QV_EINVAL, "per-step recall needs a non-empty ground truth");
    if (topk > o.step_recall_gt_width)
      fail(QV_EINVAL, "Per-step recall topk=" + std::to_string(topk) + " exceeds ground truth width=" +
                          std::to_string(o.step_recall_gt_width));
    if (!(o.step_recall_threshold > 0.0f && o.step_recall_threshold <= 1.0f))
      fail(QV_EINVAL, "Per-step recall threshold must be in (0, 1], got " + std::to_string(o.step_recall_threshold));
    if (o.step_recall_gt_width > 4 * kWave)
      fail(QV_EUNSUPPORTED, "per-step recall ground truth wider than 256 ids");
  }

  const bool open_loop = o.arrival_qps > 0.0;
  if (open_loop) {
    if (o.admission != QV_ADMIT_STREAMING)
      fail(QV_EINVAL, "open-loop arrival (arrival_qps > 0) needs QV_ADMIT_STREAMING admission");
    if (o.arrival_batch < 1) fail(QV_EINVAL, "arrival_batch must be at least 1");
    if (step_recall) fail(QV_EINVAL, "open-loop arrival does not take per-step recall");
    if (!(o.arrival_qps < 1e12) || (double)nq / o.arrival_qps > 3600.0)
      fail(QV_EINVAL, "open-loop arrival must offer its queries within an hour");
  }

  HIP_OK(hipSetDevice(ix->device));
  ensure_scratch(ix, nq, topk);
  const int64_t requested = o.num_blocks > 0 ? (int64_t)o.num_blocks * o.queries_per_block : INT64_MAX;
  // Queries the call can have in flight.  Open loop: by Little's law, the
  // offered rate times a nominal 1.5 ms in the system, plus one arrival.
  int64_t need = std::min<int64_t>(nq, requested);
  if (open_loop) need = std::min<int64_t>(need, (int64_t)std::ceil(o.arrival_qps * 1.5e-3) + o.arrival_batch);
  const LaunchPlan lp = launch_plan(ix, ef, o.kernel, need, topk);
  const int spc = lp.slots_per_cu;
  if (spc <= 0) fail(QV_EUNSUPPORTED, "search kernel does not fit on a compute unit");
  // Query slots (search.cu:393-399): num_blocks x queries_per_block.  Each slot
  // is a one-wave workgroup, so the reference's Q-interleave -- a block
  // switching between its slots while one waits on memory -- is the CU's own
  // wave interleaving here.  Slots beyond what the device holds resident would
  // only wait for a free CU, and slots beyond the number of queries would find
  // no ticket, so the grid stops at both; the admission window keeps the
  // requested slot count.
  const int64_t slots = (int64_t)(o.num_blocks > 0 ? o.num_blocks : spc * ix->num_cus) * o.queries_per_block;
  const int64_t launched = std::min<int64_t>(std::min<int64_t>(slots, (int64_t)spc * ix->num_cus), nq);
  const LaunchShape ls = shape_launch(lp, launched, ix->num_cus);
  const int grid = ls.grid;
  const int num_blocks = grid * ls.waves;  // query slots (waves) launched
  if (o.admission != QV_ADMIT_STREAMING && o.admission != QV_ADMIT_BATCH && o.admission != QV_ADMIT_STATIC)
    fail(QV_EINVAL, "admission must be QV_ADMIT_STREAMING, QV_ADMIT_BATCH or QV_ADMIT_STATIC");
  // Open loop: every arrival is admitted on its clock, however many queries
  // are still in flight.
  const int max_inflight = open_loop ? (int)nq
                                     : (int)std::min<int64_t>(
                                           nq, o.admission == QV_ADMIT_STATIC ? slots : slots + std::max(0, o.prefeed));

  // Host queries under host-fed admission are not uploaded ahead of the
  // launch: the host copies them into the pinned, GPU-uncached staging buffer
  // a chunk at a time while the kernel already runs, feeds each query once
  // its chunk is there, and the kernel reads every query in place, once (its
  // 4 d bytes, read at system scope).  Only the first chunk's copy precedes
  // the first feed.
  const bool stage_q = !o.device_buffers && (o.admission == QV_ADMIT_STREAMING || o.admission == QV_ADMIT_STATIC);
  float* dev_qstage = nullptr;
  if (stage_q) HIP_OK(hipHostGetDevicePointer(reinterpret_cast<void**>(&dev_qstage), ix->h_qstage, 0));
  const float* d_q = o.device_buffers ? queries : (stage_q ? dev_qstage : ix->d_queries);
  // Host buffers: the kernel writes ids, distances and found counts straight
  // into pinned host memory (h_results), laid out [nq][topk] as the caller's.
  int32_t* d_ids = o.device_buffers ? ids : ix->d_ids;
  float* d_dists = o.device_buffers ? dists : ix->d_dists;
  int32_t* d_found = (o.device_buffers && found) ? found : ix->d_found;
  int32_t* const h_ids = static_cast<int32_t*>(ix->h_results);
  float* const h_dists = reinterpret_cast<float*>(h_ids + (size_t)ix->cap_q * ix->cap_k);
  int32_t* const h_found = h_ids + (size_t)ix->cap_q * ix->cap_k * 2;
  if (!o.device_buffers) {
    int32_t* dev_res = nullptr;
    HIP_OK(hipHostGetDevicePointer(reinterpret_cast<void**>(&dev_res), ix->h_results, 0));
    d_ids = dev_res;
    d_dists = reinterpret_cast<float*>(dev_res + (size_t)ix->cap_q * ix->cap_k);
    d_found = dev_res + (size_t)ix->cap_q * ix->cap_k * 2;
  }

  // Shared-pivot launches count the ended waves of each workgroup, so that a
  // workgroup's last wave can take the pivot table over for its own LUT.
  // Only with two waves or more per workgroup: the others' end then says that
  // every ticket is out, so the last wave gets no further query.
  const bool tail = lp.variant == QV_KERNEL_SHARED_PIVOTS && grid <= kMaxTailWorkgroups && ls.waves > 1;
  HIP_OK(hipMemsetAsync(ix->d_counters, 0, 64 + (tail ? 4 * (size_t)grid : 0), ix->stream));
  // Static batches (StaticDispatch, search.cu:1703-1796): sequential batches of
  // num_blocks x queries_per_block queries, each admitted once the previous
  // one has completed; served by the same persistent launch, the host gating
  // admission, instead of one launch per batch.
  const bool static_batches = o.admission == QV_ADMIT_STATIC;
  const bool streaming = o.admission == QV_ADMIT_STREAMING || static_batches;  // the host feeds tickets
  volatile int32_t* feed = ix->h_ctrl;
  volatile int32_t* term = ix->h_ctrl + 1;
  *feed = streaming ? 0 : (int32_t)nq;
  *term = 0;
  std::memset(ix->h_ring, 0, sizeof(int32_t) * (size_t)nq);
  std::atomic_thread_fence(std::memory_order_seq_cst);

  int32_t* dev_ctrl = nullptr;
  int32_t* dev_ring = nullptr;
  HIP_OK(hipHostGetDevicePointer(reinterpret_cast<void**>(&dev_ctrl), ix->h_ctrl, 0));
  HIP_OK(hipHostGetDevicePointer(reinterpret_cast<void**>(&dev_ring), ix->h_ring, 0));

  SearchArgs a = base_args(ix);
  a.queries = d_q;
  a.nq = (int32_t)nq;
  a.topk = topk;
  a.ef = ef;
  a.pipe_w = o.pipe_width;
  a.early_exit = o.early_exit;
  if (o.skip_nav) a.nav_data = nullptr;  // --skip-nav (quiver_search.cu:241-246)
  a.warmup = o.gpruning_warmup;
  a.patience = o.gpruning_patience;
  a.out_ids = d_ids;
  a.out_dists = d_dists;
  a.out_found = d_found;
  // per-query counts into the pinned staging buffer (no copies after the launch)
  {
    int32_t* dev_stage = nullptr;
    HIP_OK(hipHostGetDevicePointer(reinterpret_cast<void**>(&dev_stage), ix->h_stage, 0));
    a.out_hops = dev_stage + kStageHead;
    a.out_stopped = dev_stage + kStageHead + ix->cap_q;
    a.out_evals = dev_stage + kStageHead + 2 * (size_t)ix->cap_q;
  }
  a.t_start = ix->d_tstart;
  a.t_end = ix->d_tend;
  a.counters = ix->d_counters;
  a.wg_done = tail ? ix->d_counters + 16 : nullptr;
  a.feed_count = dev_ctrl;
  a.terminate = dev_ctrl + 1;
  a.ring = dev_ring;
  // A new epoch per search makes the mirror words of earlier searches read as
  // 0 without a clear; at the end of the epochs the words are cleared once.
  if (ix->feed_epoch == UINT32_MAX) {
    HIP_OK(hipMemsetAsync(ix->d_feed_mirror, 0, kFeedMirrorBytes, ix->stream));
    ix->feed_epoch = 0;
  }
  a.feed_mirror = ix->d_feed_mirror;
  a.feed_epoch = ++ix->feed_epoch;
  // Feed waits end on their own after this long even if the host never
  // admits more work, so a lost host thread cannot leave the kernel spinning
  // (open loop: the arrivals' own span on top).
  const double spin_s =
      (o.timeout_s > 0 ? o.timeout_s + 5.0 : 60.0) + (open_loop ? (double)nq / o.arrival_qps : 0.0);
  a.spin_limit_ticks = (uint64_t)(spin_s * 1e8);
  a.rec_ids = nullptr;
  a.rec_dists = nullptr;
  a.rec_cap = 0;
  // per-step recall: ground truth and per-query outputs on the device for this call
  struct DevFree {
    void operator()(void* p) const { (void)hipFree(p); }
  };
  std::unique_ptr<int32_t, DevFree> sr_gt, sr_out;
  if (step_recall) {
    const size_t gt_elems = (size_t)o.step_recall_gt_count * (size_t)o.step_recall_gt_width;
    int32_t* p = nullptr;
    HIP_OK(hipMalloc(&p, sizeof(int32_t) * gt_elems));
    sr_gt.reset(p);
    HIP_OK(hipMemcpy(p, o.step_recall_gt, sizeof(int32_t) * gt_elems, hipMemcpyHostToDevice));
    HIP_OK(hipMalloc(&p, sizeof(int32_t) * 2 * (size_t)nq));
    sr_out.reset(p);
    a.sr_gt = sr_gt.get();
    a.sr_width = o.step_recall_gt_width;
    a.sr_count = o.step_recall_gt_count;
    // required_hits_for_threshold (search.cu:100-102), in the reference's float arithmetic
    a.sr_required = std::max(1, std::min(topk, (int)std::ceil(o.step_recall_threshold * (float)topk - 1e-6f)));
    a.sr_step = sr_out.get();
    a.sr_hits = sr_out.get() + nq;
  }

  using clock = std::chrono::steady_clock;
  // The clock starts before the queries leave host memory and before the
  // launch: the reference takes t0 ahead of H2D_initial and stamps the whole
  // initial window with it (search.cu:865-877).  Without staging the upload
  // and the launch share the stream, so the kernel starts once its queries
  // are in HBM.
  const auto t0 = clock::now();
  if (!o.device_buffers && !stage_q)
    HIP_OK(hipMemcpyAsync(ix->d_queries, queries, sizeof(float) * (size_t)nq * dim, hipMemcpyHostToDevice,
                          ix->stream));
  HIP_OK(hipEventRecord(ix->ev0, ix->stream));
  hipLaunchKernelGGL(lp.kern, dim3(grid), dim3(kWave * ls.waves), (size_t)ls.lds, ix->stream, a);
  HIP_OK(hipGetLastError());
  HIP_OK(hipEventRecord(ix->ev1, ix->stream));
  // The launch counters follow the kernel into pinned memory on its stream, so
  // they are there once the stream is idle (no round trip after the wait).
  int32_t* const st_counters = ix->h_stage;
  HIP_OK(hipMemcpyAsync(st_counters, ix->d_counters, 5 * sizeof(int32_t), hipMemcpyDeviceToHost, ix->stream));

  const bool has_deadline = o.timeout_s > 0;
  const auto deadline = t0 + std::chrono::duration_cast<clock::duration>(
                                 std::chrono::duration<double>(has_deadline ? o.timeout_s : 0.0));
  bool timed_out = false;
  std::vector<double> lat_ms;
  if (streaming) {
    // Host admission loop (search.cu:983-1051): keep at most max_inflight
    // admitted-but-unfinished queries; stamp each completion from the ring.
    std::vector<clock::time_point> admit((size_t)nq);
    lat_ms.assign((size_t)nq, 0.0);
    const int64_t stride = static_batches ? std::min<int64_t>(nq, slots) : 0;
    // Open loop: arrival j brings queries [j B, (j + 1) B) at t0 + j B / rate,
    // and each query's latency runs from its arrival's scheduled time, so a
    // late admission by the host counts against the search.
    const int64_t arr_b = open_loop ? o.arrival_batch : 1;
    const double arr_gap = open_loop ? (double)arr_b / o.arrival_qps : 0.0;
    auto arrival_time = [&](int64_t j) {
      return t0 + std::chrono::duration_cast<clock::duration>(std::chrono::duration<double>((double)j * arr_gap));
    };
    // Staged queries [0, staged): copied into h_qstage, each copy ordered
    // (full fence, which also orders streaming stores) before the feed word
    // that admits them.
    int64_t staged = stage_q ? 0 : nq;
    auto stage_to = [&](int64_t upto) {
      upto = std::min<int64_t>(upto, nq);
      if (upto <= staged) return;
      std::memcpy(ix->h_qstage + (size_t)staged * dim, queries + (size_t)staged * dim,
                  sizeof(float) * (size_t)(upto - staged) * dim);
      std::atomic_thread_fence(std::memory_order_seq_cst);
      staged = upto;
    };
    constexpr int64_t kStageChunk = 256;  // queries per copy (128 KB at d = 128)
    int64_t fed = static_batches ? stride : (open_loop ? std::min<int64_t>(nq, arr_b) : max_inflight);
    int64_t batch_begin = 0;  // static batches: the batch in flight is [batch_begin, fed)
    auto batch_t = t0;
    // a static batch's queries all take its wall time as their latency (search.cu:1783-1788)
    auto close_batch = [&](clock::time_point now) {
      const double ms = std::chrono::duration<double, std::milli>(now - batch_t).count();
      for (int64_t i = batch_begin; i < fed; i++) lat_ms[(size_t)i] = ms;
    };
    for (int64_t i = 0; i < fed; i++) admit[(size_t)i] = t0;
    // the initial window, a chunk at a time when staging
    for (int64_t f = stage_q ? 0 : fed; f < fed;) {
      f = std::min<int64_t>(fed, f + kStageChunk);
      stage_to(f);
      __atomic_store_n(ix->h_ctrl, (int32_t)f, __ATOMIC_RELEASE);
    }
    __atomic_store_n(ix->h_ctrl, (int32_t)fed, __ATOMIC_RELEASE);
    int64_t done = 0;
    const int min_batch = std::max(1, o.admit_min_batch);
    while (done < nq) {
      bool progressed = false;
      // copy ahead of the feeds while the kernel runs
      if (staged < nq) {
        stage_to(staged + kStageChunk);
        progressed = true;
      }
      while (done < nq) {
        const int32_t e = __atomic_load_n(ix->h_ring + done, __ATOMIC_ACQUIRE);
        if (e == 0) break;
        const auto now = clock::now();
        lat_ms[(size_t)(e - 1)] = std::chrono::duration<double, std::milli>(now - admit[(size_t)(e - 1)]).count();
        done++;
        progressed = true;
      }
      const int64_t target = std::min<int64_t>(nq, done + max_inflight);
      if (open_loop) {
        if (fed < nq) {
          const auto now = clock::now();
          int64_t to = fed;
          while (to < nq && arrival_time(to / arr_b) <= now) {
            const int64_t end = std::min<int64_t>(nq, to + arr_b);
            const auto at = arrival_time(to / arr_b);
            for (int64_t i = to; i < end; i++) admit[(size_t)i] = at;
            to = end;
          }
          if (to > fed) {
            stage_to(to);
            fed = to;
            __atomic_store_n(ix->h_ctrl, (int32_t)fed, __ATOMIC_RELEASE);
            progressed = true;
          }
        }
      } else if (static_batches) {
        if (done == fed && fed < nq) {
          const auto now = clock::now();
          close_batch(now);
          batch_begin = fed;
          fed = std::min<int64_t>(nq, fed + stride);
          batch_t = now;
          for (int64_t i = batch_begin; i < fed; i++) admit[(size_t)i] = now;
          stage_to(fed);
          __atomic_store_n(ix->h_ctrl, (int32_t)fed, __ATOMIC_RELEASE);
        }
      } else if (target > fed && (target - fed >= min_batch || target == nq || fed - done == 0)) {
        const auto now = clock::now();
        for (int64_t i = fed; i < target; i++) admit[(size_t)i] = now;
        stage_to(target);
        fed = target;
        __atomic_store_n(ix->h_ctrl, (int32_t)fed, __ATOMIC_RELEASE);
      }
      if (!progressed) {
        if (has_deadline && clock::now() > deadline) {
          timed_out = true;
          break;
        }
        if (hipStreamQuery(ix->stream) == hipSuccess) {
          // The kernel has ended: every completion it published is visible
          // now, including those written after the empty read above.
          const auto now = clock::now();
          while (done < nq) {
            const int32_t e = __atomic_load_n(ix->h_ring + done, __ATOMIC_ACQUIRE);
            if (e == 0) break;
            lat_ms[(size_t)(e - 1)] = std::chrono::duration<double, std::milli>(now - admit[(size_t)(e - 1)]).count();
            done++;
          }
          if (done < nq) break;  // it ended early (error path): nothing more will arrive
        }
      }
    }
    if (static_batches && done == nq) close_batch(clock::now());
  }
  // Wait for the kernel, honouring the deadline.
  while (true) {
    hipError_t st = hipStreamQuery(ix->stream);
    if (st == hipSuccess) break;
    if (st != hipErrorNotReady) HIP_OK(st);
    if (has_deadline && !timed_out && clock::now() > deadline) timed_out = true;
    if (timed_out) __atomic_store_n(ix->h_ctrl + 1, 1, __ATOMIC_RELEASE);
    // Streaming: every completion is in, the launch is draining its last
    // waves; a short sleep request is rounded up to tens of microseconds, so
    // the host keeps polling instead.
    if (streaming)
      std::this_thread::yield();
    else
      std::this_thread::sleep_for(std::chrono::microseconds(50));
  }
  // The stream is idle: the kernel's writes to pinned memory (results, counts)
  // and the counters' copy behind it are all visible.
  HIP_OK(hipStreamSynchronize(ix->stream));
  if (!o.device_buffers) {
    std::memcpy(ids, h_ids, sizeof(int32_t) * (size_t)nq * topk);
    std::memcpy(dists, h_dists, sizeof(float) * (size_t)nq * topk);
    if (found) std::memcpy(found, h_found, sizeof(int32_t) * (size_t)nq);
  }
  const auto t1 = clock::now();

  // The kernel wrote the hop counts, stop flags and evaluation counts into the
  // pinned staging buffer directly.
  int32_t* const st_hops = ix->h_stage + kStageHead;
  int32_t* const st_stopped = st_hops + ix->cap_q;
  int32_t* const st_evals = st_stopped + ix->cap_q;
  int32_t counters[5];
  std::memcpy(counters, st_counters, sizeof(counters));
  if (counters[2] & kErrSpinTimeout) fail(QV_ETIMEDOUT, "search kernel watchdog: feed wait exceeded its limit");
  if (timed_out || counters[1] < nq) {
    char buf[96];
    std::snprintf(buf, sizeof(buf), "quiver_search exceeded the %g second timeout", o.timeout_s);
    fail(QV_ETIMEDOUT, buf);
  }
  ix->last_hops.assign(st_hops, st_hops + nq);
  if (step_recall) {
    if (o.step_recall_step)
      HIP_OK(hipMemcpy(o.step_recall_step, a.sr_step, sizeof(int32_t) * (size_t)nq, hipMemcpyDeviceToHost));
    if (o.step_recall_hits)
      HIP_OK(hipMemcpy(o.step_recall_hits, a.sr_hits, sizeof(int32_t) * (size_t)nq, hipMemcpyDeviceToHost));
  }
  if (!streaming) {
    // every query admitted at launch: latency = its completion tick - the first start tick
    std::vector<uint64_t> ts((size_t)nq), te((size_t)nq);
    HIP_OK(hipMemcpy(ts.data(), ix->d_tstart, sizeof(uint64_t) * (size_t)nq, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(te.data(), ix->d_tend, sizeof(uint64_t) * (size_t)nq, hipMemcpyDeviceToHost));
    const uint64_t t_first = *std::min_element(ts.begin(), ts.end());
    lat_ms.resize((size_t)nq);
    for (int64_t i = 0; i < nq; i++) lat_ms[(size_t)i] = (double)(te[(size_t)i] - t_first) * 1e-5;
  }
  ix->last_lat_ms = lat_ms;

  if (rep) {
    std::memset(rep, 0, sizeof(*rep));
    const double secs = std::chrono::duration<double>(t1 - t0).count();
    rep->search_time_s = secs;
    rep->qps = (double)nq / secs;
    float kms = 0.f;
    HIP_OK(hipEventElapsedTime(&kms, ix->ev0, ix->ev1));
    rep->kernel_ms = kms;
    rep->num_blocks = num_blocks;
    rep->max_inflight = max_inflight;
    rep->kernel = lp.variant;
    rep->early_stopped = (int32_t)std::accumulate(st_stopped, st_stopped + nq, 0);
    double hop_sum = 0;
    for (int32_t h : ix->last_hops) hop_sum += h;
    rep->avg_hops = hop_sum / (double)nq;
    rep->total_hops = hop_sum;
    double ev_sum = 0;
    for (int64_t i = 0; i < nq; i++) ev_sum += st_evals[i];
    rep->total_evals = ev_sum;
    rep->tail_queries = counters[4];
    rep->lat_avg_ms = std::accumulate(lat_ms.begin(), lat_ms.end(), 0.0) / (double)nq;
    // Order statistics by radix selection (a full sort of 10k latencies costs
    // about half a millisecond of host time per search, successive
    // nth_element passes 0.07-0.10 ms).
    size_t ranks[5];
    percentile_ranks(lat_ms.size(), ranks);
    double vals[5];
    select_ranks(lat_ms.data(), lat_ms.size(), ranks, 5, vals);
    rep->lat_p50_ms = vals[0];
    rep->lat_p90_ms = vals[1];
    rep->lat_p99_ms = vals[2];
    rep->lat_p999_ms = vals[3];
    rep->lat_max_ms = vals[4];
  }
}

// ---- allocation-free search -------------------------------------------------
// Per device: the address of its copy of `scratch` (hipGetSymbolAddress, once,
// with the device current).
struct NoAllocDevice {
  std::mutex mu;  // one array per device: calls on one GPU are serialised by it
  uint8_t* ptr = nullptr;
};
static std::mutex g_noalloc_lookup_mu;  // guards only the one-time address lookups
static NoAllocDevice g_noalloc[64];

// The device's entry with its array's address looked up (the device must be
// current).
static NoAllocDevice& noalloc_device(int device) {
  if (device < 0 || device >= 64) fail(QV_EINVAL, "device out of range");
  NoAllocDevice& nd = g_noalloc[device];
  std::lock_guard<std::mutex> lk(g_noalloc_lookup_mu);
  if (!nd.ptr) {
    void* p = nullptr;
    HIP_OK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) fail(QV_EHIP, "hipGetSymbolAddress returned no address for the search scratch");
    nd.ptr = static_cast<uint8_t*>(p);
  }
  return nd;
}

static void zero_words(uint8_t* p, int64_t bytes, hipStream_t s) {
  const int64_t words = bytes / 4;
  const int blocks = (int)std::min<int64_t>((words + 255) / 256, 4096);
  hipLaunchKernelGGL(zero_words_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<uint32_t*>(p), words);
  HIP_OK(hipGetLastError());
}

// qv_search with every query admitted at launch, device buffers only, and its
// scratch taken from the fixed per-device array: no device or pinned-host
// allocation, no memset.
void search_noalloc(qv_index* ix, const float* d_queries, int64_t nq, int dim, int topk, int ef,
                    const qv_search_opts& o, int32_t* d_ids, float* d_dists, int32_t* d_found,
                    qv_search_report* rep) {
  std::lock_guard<std::mutex> lk(ix->mu);
  const Layout& L = ix->lay;
  if (nq <= 0 || nq > kNoAllocMaxQueries)
    fail(QV_EINVAL, "qv_search_noalloc takes 1 to " + std::to_string(kNoAllocMaxQueries) +
                        " queries per call (its fixed scratch holds their counts); got " + std::to_string(nq));
  if (dim != L.num_dims)
    fail(QV_EINVAL, "Query dimension mismatch: queries have " + std::to_string(dim) +
                        " dims, but the index expects " + std::to_string(L.num_dims));
  if (topk <= 0 || topk > kMaxTopk) fail(QV_EINVAL, "topk must be in [1, 1024]");
  if (ef <= 0 || ef > kMaxEf) fail(QV_EINVAL, "ef_search must be in [1, 2048]");
  if (o.pipe_width < 1 || o.pipe_width > kMaxPipeWidth) fail(QV_EINVAL, "--pipe-width must be in [1, 16]");
  if (o.queries_per_block < 1 || o.queries_per_block > kMaxQueriesPerBlock)
    fail(QV_EINVAL, "--queries-per-block must be in [1, 8]");
  if (o.early_exit != QV_EXIT_NONE && o.early_exit != QV_EXIT_GPRUNING)
    fail(QV_EINVAL, "early exit policy must be none or gpruning");
  if (o.num_blocks < 0) fail(QV_EINVAL, "--num-blocks must be positive");
  if (o.timeout_s != 0.0) fail(QV_EINVAL, "qv_search_noalloc has no deadline (timeout_s must be 0)");
  if (o.step_recall_gt) fail(QV_EINVAL, "qv_search_noalloc does not take per-step recall");
  if (!d_queries || !d_ids || !d_dists) fail(QV_EINVAL, "null argument");

  HIP_OK(hipSetDevice(ix->device));
  NoAllocDevice& nd = noalloc_device(ix->device);
  std::lock_guard<std::mutex> dlk(nd.mu);  // calls on one GPU share its array
  uint8_t* const base = nd.ptr;
  const int64_t requested = o.num_blocks > 0 ? (int64_t)o.num_blocks * o.queries_per_block : INT64_MAX;
  const LaunchPlan lp = launch_plan(ix, ef, o.kernel, std::min<int64_t>(nq, requested), topk);
  if (lp.slots_per_cu <= 0) fail(QV_EUNSUPPORTED, "search kernel does not fit on a compute unit");
  const int64_t slots = (int64_t)(o.num_blocks > 0 ? o.num_blocks : lp.slots_per_cu * ix->num_cus) * o.queries_per_block;
  const int64_t launched = std::min<int64_t>(std::min<int64_t>(slots, (int64_t)lp.slots_per_cu * ix->num_cus), nq);
  const LaunchShape ls = shape_launch(lp, launched, ix->num_cus);

  int32_t* const counters = reinterpret_cast<int32_t*>(base);
  int32_t* const hops = reinterpret_cast<int32_t*>(base + kNoAllocHopsOff);
  int32_t* const evals = reinterpret_cast<int32_t*>(base + kNoAllocEvalsOff);
  int32_t* const stopped = reinterpret_cast<int32_t*>(base + kNoAllocStoppedOff);
  zero_words(base, kNoAllocHopsOff, ix->stream);  // counters and the 64-bit totals
  // tail mode as in search(): workgroups of two waves or more
  const bool tail = lp.variant == QV_KERNEL_SHARED_PIVOTS && ls.grid <= kMaxTailWorkgroups && ls.waves > 1;
  int32_t* const wg_done = reinterpret_cast<int32_t*>(base + kNoAllocWgDoneOff);
  if (tail) zero_words(base + kNoAllocWgDoneOff, 4 * (int64_t)ls.grid, ix->stream);

  SearchArgs a = base_args(ix);
  a.queries = d_queries;
  a.nq = (int32_t)nq;
  a.topk = topk;
  a.ef = ef;
  a.pipe_w = o.pipe_width;
  a.early_exit = o.early_exit;
  if (o.skip_nav) a.nav_data = nullptr;
  a.warmup = o.gpruning_warmup;
  a.patience = o.gpruning_patience;
  a.out_ids = d_ids;
  a.out_dists = d_dists;
  a.out_found = d_found;
  a.out_hops = hops;
  a.out_stopped = stopped;
  a.out_evals = evals;
  a.t_start = nullptr;
  a.t_end = nullptr;
  a.counters = counters;
  a.wg_done = tail ? wg_done : nullptr;
  a.feed_count = nullptr;  // every query admitted at launch
  a.terminate = nullptr;
  a.ring = nullptr;
  a.spin_limit_ticks = 0;
  a.rec_ids = nullptr;
  a.rec_dists = nullptr;
  a.rec_cap = 0;

  const auto t0 = std::chrono::steady_clock::now();
  HIP_OK(hipEventRecord(ix->ev0, ix->stream));
  hipLaunchKernelGGL(lp.kern, dim3(ls.grid), dim3(kWave * ls.waves), (size_t)ls.lds, ix->stream, a);
  HIP_OK(hipGetLastError());
  HIP_OK(hipEventRecord(ix->ev1, ix->stream));
  unsigned long long* const totals = reinterpret_cast<unsigned long long*>(base + 64);
  hipLaunchKernelGGL(sum_counts_kernel, dim3((unsigned)std::min<int64_t>((nq + 255) / 256, 1024)), dim3(256), 0,
                     ix->stream, hops, evals, stopped, nq, totals);
  HIP_OK(hipGetLastError());
  HIP_OK(hipStreamSynchronize(ix->stream));
  const auto t1 = std::chrono::steady_clock::now();
  int32_t c[5] = {0, 0, 0, 0, 0};
  unsigned long long tot[3] = {0, 0, 0};
  HIP_OK(hipMemcpy(c, counters, sizeof(c), hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(tot, totals, sizeof(tot), hipMemcpyDeviceToHost));
  if (c[1] != nq)
    fail(QV_EHIP, "search kernel finished " + std::to_string(c[1]) + " of " + std::to_string(nq) + " queries");
  if (rep) {
    std::memset(rep, 0, sizeof(*rep));
    rep->search_time_s = std::chrono::duration<double>(t1 - t0).count();
    rep->qps = (double)nq / rep->search_time_s;
    float kms = 0.f;
    HIP_OK(hipEventElapsedTime(&kms, ix->ev0, ix->ev1));
    rep->kernel_ms = kms;
    rep->num_blocks = ls.grid * ls.waves;
    rep->max_inflight = (int32_t)nq;
    rep->kernel = lp.variant;
    rep->total_hops = (double)tot[0];
    rep->total_evals = (double)tot[1];
    rep->avg_hops = (double)tot[0] / (double)nq;
    rep->early_stopped = (int32_t)tot[2];
    rep->tail_queries = c[4];
  }
}

}  // namespace qv

// ================================================================ C ABI ====

extern "C" {

void qv_search_opts_default(qv_search_opts* o) {
  if (!o) return;
  std::memset(o, 0, sizeof(*o));
  o->num_blocks = 0;
  o->queries_per_block = 1;
  o->pipe_width = 1;
  o->early_exit = QV_EXIT_GPRUNING;
  o->gpruning_warmup = 10;
  o->gpruning_patience = 8;
  o->prefeed = 0;
  o->admit_min_batch = 32;
  o->admission = QV_ADMIT_STREAMING;
  o->device_buffers = 0;
  o->timeout_s = 0.0;
  o->skip_nav = 0;
  o->kernel = QV_KERNEL_AUTO;
  o->step_recall_gt = nullptr;
  o->step_recall_threshold = 0.9f;
  o->arrival_qps = 0.0;
  o->arrival_batch = 1;
}

int qv_index_open(const char* index_dir, const char* data_type, const char* memory_backend,
                  const char* memory_index_file, int device, qv_index** out) {
  return qv::guard([&] {
    if (!index_dir || !data_type || !out) qv::fail(QV_EINVAL, "null argument");
    *out = nullptr;
    *out = qv::open_index(index_dir, data_type, memory_backend ? memory_backend : "heap",
                          memory_index_file ? memory_index_file : "", device, QV_GRAPH_HBM);
  });
}

int qv_index_open_ex(const char* index_dir, const char* data_type, const char* memory_backend,
                     const char* memory_index_file, int device, int32_t graph_placement, qv_index** out) {
  return qv::guard([&] {
    if (!index_dir || !data_type || !out) qv::fail(QV_EINVAL, "null argument");
    *out = nullptr;
    *out = qv::open_index(index_dir, data_type, memory_backend ? memory_backend : "heap",
                          memory_index_file ? memory_index_file : "", device, graph_placement);
  });
}

int qv_index_place_graph(qv_index* ix, int32_t graph_placement) {
  return qv::guard([&] {
    if (!ix) qv::fail(QV_EINVAL, "null argument");
    if (graph_placement != QV_GRAPH_HBM && graph_placement != QV_GRAPH_HOST)
      qv::fail(QV_EINVAL, "graph placement must be QV_GRAPH_HBM or QV_GRAPH_HOST");
    std::lock_guard<std::mutex> lk(ix->mu);
    const bool to_host = graph_placement == QV_GRAPH_HOST;
    if (to_host == ix->pages_in_host) return;
    HIP_OK(hipSetDevice(ix->device));
    const size_t bytes = (size_t)(ix->lay.num_pages * qv::kPageSize);
    uint8_t* p = nullptr;
    if (to_host)
      HIP_OK(hipHostMalloc(reinterpret_cast<void**>(&p), bytes, hipHostMallocNonCoherent));
    else
      HIP_OK(hipMalloc(&p, bytes));
    const hipError_t e = hipMemcpy(p, ix->d_pages, bytes, hipMemcpyDefault);
    if (e != hipSuccess) {
      if (to_host)
        hipHostFree(p);
      else
        hipFree(p);
      HIP_OK(e);
    }
    if (ix->pages_in_host)
      hipHostFree(ix->d_pages);
    else
      hipFree(ix->d_pages);
    ix->d_pages = p;
    ix->pages_in_host = to_host;
    ix->device_bytes += to_host ? -(int64_t)bytes : (int64_t)bytes;
  });
}

int qv_index_from_memory(const qv_index_info* layout, const uint8_t* pages, const float* centroid,
                         const float* pivots, const int32_t* chunk_id, int32_t num_chunks, const uint8_t* codes,
                         int device, qv_index** out) {
  return qv::guard([&] {
    if (!layout || !out) qv::fail(QV_EINVAL, "null argument");
    *out = nullptr;
    *out = qv::index_from_memory(*layout, pages, centroid, pivots, chunk_id, num_chunks, codes, device);
  });
}

int qv_index_set_nav(qv_index* ix, const void* data, const int32_t* graph, const int32_t* mapping,
                     int64_t num_node, int32_t max_m, int32_t start) {
  return qv::guard([&] {
    if (!ix || !data || !graph || !mapping) qv::fail(QV_EINVAL, "null argument");
    if (num_node <= 0 || num_node > INT32_MAX) qv::fail(QV_EINVAL, "num_node out of range");
    if (max_m < 1 || max_m > 32) qv::fail(QV_EINDEX, "nav graph max degree must be in [1, 32]");
    std::lock_guard<std::mutex> lk(ix->mu);
    qv::NavGraphHost nav;
    nav.num_node = (int32_t)num_node;
    nav.dims = (int32_t)ix->lay.num_dims;
    nav.max_m = max_m;
    nav.start = start;
    const size_t bytes = (size_t)num_node * (size_t)ix->lay.data_size;
    nav.data.assign(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + bytes);
    nav.graph.assign(graph, graph + (size_t)num_node * (size_t)max_m);
    nav.mapping.assign(mapping, mapping + num_node);
    qv::upload_nav(ix, nav);
  });
}

int qv_index_neighbour_codes(qv_index* ix, int32_t enable) {
  return qv::guard([&] {
    if (!ix) qv::fail(QV_EINVAL, "null index");
    std::lock_guard<std::mutex> lk(ix->mu);
    qv::set_neighbour_codes(ix, enable != 0);
  });
}

int qv_index_load_nav(qv_index* ix, const char* nav_dir) {
  return qv::guard([&] {
    if (!ix || !nav_dir) qv::fail(QV_EINVAL, "null argument");
    std::lock_guard<std::mutex> lk(ix->mu);
    qv::load_nav(ix, nav_dir);
  });
}

int qv_index_get_info(const qv_index* ix, qv_index_info* info) {
  return qv::guard([&] {
    if (!ix || !info) qv::fail(QV_EINVAL, "null argument");
    const Layout& L = ix->lay;
    info->num_data = L.num_data;
    info->num_dims = L.num_dims;
    info->max_m0 = L.max_m0;
    info->enter_point = L.enter_point;
    info->data_size = L.data_size;
    info->node_size = L.node_size;
    info->num_pages = L.num_pages;
    info->nodes_per_page = L.nodes_per_page;
    info->data_type = L.data_type;
    info->num_chunks = ix->M;
    info->device = ix->device;
    HIP_OK(hipSetDevice(ix->device));
    info->slots_per_cu = qv::slots_per_cu(const_cast<qv_index*>(ix), 64);
    info->device_bytes = ix->device_bytes;
    info->nav_nodes = ix->nav_nodes;
    info->nav_max_m = ix->nav_max_m;
  });
}

void qv_index_close(qv_index* ix) { qv::release_index(ix); }

int qv_search(qv_index* ix, const float* queries, int64_t nq, int32_t dim, int32_t topk,
              int32_t ef, const qv_search_opts* opts, int32_t* ids, float* dists,
              int32_t* found, qv_search_report* rep) {
  return qv::guard([&] {
    if (!ix || !queries || !ids || !dists) qv::fail(QV_EINVAL, "null argument");
    qv_search_opts o;
    qv_search_opts_default(&o);
    if (opts) o = *opts;
    qv::search(ix, queries, nq, dim, topk, ef, o, ids, dists, found, rep);
  });
}

int qv_search_noalloc(qv_index* ix, const float* d_queries, int64_t nq, int32_t dim, int32_t topk,
                      int32_t ef, const qv_search_opts* opts, int32_t* d_ids, float* d_dists,
                      int32_t* d_found, qv_search_report* rep) {
  return qv::guard([&] {
    if (!ix) qv::fail(QV_EINVAL, "null argument");
    qv_search_opts o;
    qv_search_opts_default(&o);
    if (opts) o = *opts;
    qv::search_noalloc(ix, d_queries, nq, dim, topk, ef, o, d_ids, d_dists, d_found, rep);
  });
}

int qv_index_save(const qv_index* ix, const char* out_prefix) {
  return qv::guard([&] {
    if (!ix || !out_prefix) qv::fail(QV_EINVAL, "null argument");
    const Layout& L = ix->lay;
    HIP_OK(hipSetDevice(ix->device));
    std::vector<uint8_t> pages((size_t)(L.num_pages * kPageSize));
    HIP_OK(hipMemcpy(pages.data(), ix->d_pages, pages.size(), hipMemcpyDefault));
    const std::string pre = out_prefix;
    qv::write_index_image(pre + "_disk.index", L, pages.data());
    qv::PQTables t;
    t.dim = (int)L.num_dims;
    t.num_chunks = ix->M;
    t.num_pts = L.num_data;
    t.centroid = ix->h_centroid;
    t.pivots = ix->h_pivots;
    t.chunk_offsets = ix->h_chunk_off;
    t.codes.resize((size_t)L.num_data * ix->M);
    HIP_OK(hipMemcpy(t.codes.data(), ix->d_codes, t.codes.size(), hipMemcpyDeviceToHost));
    qv::write_pq_tables(pre + "_pq_pivots.bin", pre + "_pq_compressed.bin", t);
  });
}

int qv_index_copy_out(const qv_index* ix, uint8_t* pages, uint8_t* codes, float* centroid,
                      float* pivots, int32_t* chunk_offsets) {
  return qv::guard([&] {
    if (!ix) qv::fail(QV_EINVAL, "null index");
    const Layout& L = ix->lay;
    HIP_OK(hipSetDevice(ix->device));
    if (pages) HIP_OK(hipMemcpy(pages, ix->d_pages, (size_t)(L.num_pages * kPageSize), hipMemcpyDefault));
    if (codes) HIP_OK(hipMemcpy(codes, ix->d_codes, (size_t)L.num_data * ix->M, hipMemcpyDeviceToHost));
    if (centroid) std::memcpy(centroid, ix->h_centroid.data(), sizeof(float) * ix->h_centroid.size());
    if (pivots) std::memcpy(pivots, ix->h_pivots.data(), sizeof(float) * ix->h_pivots.size());
    if (chunk_offsets)
      std::memcpy(chunk_offsets, ix->h_chunk_off.data(), sizeof(int32_t) * ix->h_chunk_off.size());
  });
}

int qv_last_hops(const qv_index* ix, int32_t* hops, int64_t nq) {
  return qv::guard([&] {
    if (!ix || !hops) qv::fail(QV_EINVAL, "null argument");
    if ((size_t)nq > ix->last_hops.size()) qv::fail(QV_EINVAL, "nq exceeds the last search");
    std::memcpy(hops, ix->last_hops.data(), sizeof(int32_t) * (size_t)nq);
  });
}

int qv_last_latencies(const qv_index* ix, double* ms, int64_t nq) {
  return qv::guard([&] {
    if (!ix || !ms) qv::fail(QV_EINVAL, "null argument");
    if (nq < 0 || (size_t)nq > ix->last_lat_ms.size()) qv::fail(QV_EINVAL, "nq exceeds the last search");
    std::memcpy(ms, ix->last_lat_ms.data(), sizeof(double) * (size_t)nq);
  });
}

int qv_lut_build(qv_index* ix, const float* d_queries, int64_t nq, float* d_luts, float* d_q_used) {
  return qv::guard([&] {
    if (!ix) qv::fail(QV_EINVAL, "null index");
    int rc = qv_lut_build_raw(ix->d_centroid, ix->d_pivots_t, ix->d_chunk_off, (int32_t)ix->lay.num_dims,
                              ix->M, d_queries, nq, d_luts, d_q_used, ix->device);
    if (rc != QV_OK) qv::fail(rc, qv_last_error());
  });
}

}  // extern "C"
