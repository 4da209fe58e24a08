// qv_build_gpu.hip -- index construction on the GPU, and brute-force ground truth.
//
// DiskANN's builder is absent from the reference checkout (deps/DiskANN is an
// empty submodule), so the 10M-100M point configurations are built here, on the
// device, in the same formats the reference reads.  Algorithms:
//   * PQ: data centred on the sample mean, M contiguous chunks, Lloyd k-means
//     with 256 centres per chunk (nearest-centre assignment on the GPU, centre
//     update on the host in float64), then every point encoded on the GPU.
//   * Medoid: the point nearest to the mean of all points.
//   * Graph: Vamana with batched insertion (batch sizes double up to a cap).  For
//     each batch the persistent search kernel runs a beam search of width L for
//     every inserted point and records the expanded nodes; a wave per point then
//     applies RobustPrune(alpha, R) to expanded nodes plus current neighbours;
//     reverse edges are sorted by target (rocPRIM radix sort) and a wave per
//     target merges them, pruning again when the list would exceed R.
// Every step is deterministic for a given seed.
#include <cstring>

#include <rocprim/device/device_radix_sort.hpp>

#include <algorithm>
#include <type_traits>
#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <numeric>
#include <vector>

#include "qv_common.hpp"
#include "qv_device.hpp"
#include "qv_hip_util.hpp"
#include "qv_index_impl.hpp"
#include "qv_mixture.hpp"

using namespace qv;
using namespace qv::dev;

namespace {

struct GLayout {
  uint8_t* pages;
  int64_t n;
  int64_t npp;
  int64_t node_size;
  int64_t data_size;
  int32_t dim;
  int32_t R;
};

__device__ __forceinline__ uint8_t* node_rec(const GLayout& L, int64_t v) {
  const int64_t page = v / L.npp;
  return L.pages + page * 4096 + (v - page * L.npp) * L.node_size;
}

template <class T>
__global__ void gather_rows_f32(const T* __restrict__ base, int dim, const int32_t* __restrict__ ids,
                                int64_t count, float* __restrict__ out) {
  const int64_t total = count * dim;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / dim;
    const int j = (int)(e - r * dim);
    out[e] = (float)base[(int64_t)ids[r] * dim + j];
  }
}

// Nearest centre of chunk blockIdx.y for rows[i] (or row i when rows is null).
// Centres are pivots [256][dim]; the chunk's 256 sub-vectors are staged in LDS.
template <class T, class OUT>
__global__ __launch_bounds__(256) void pq_assign_kernel(const T* __restrict__ base, int dim,
                                                        const int32_t* __restrict__ rows, int64_t nrows,
                                                        const float* __restrict__ centroid,
                                                        const int32_t* __restrict__ chunk_off, int M,
                                                        const float* __restrict__ pivots, OUT* __restrict__ out) {
  extern __shared__ __align__(16) float cen[];
  const int m = blockIdx.y;
  const int o = chunk_off[m], w = chunk_off[m + 1] - o;
  for (int i = threadIdx.x; i < 256 * w; i += blockDim.x) cen[i] = pivots[(i / w) * dim + o + (i % w)];
  __syncthreads();
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < nrows;
       r += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = rows ? (int64_t)rows[r] : r;
    float x[16];
    for (int j = 0; j < w && j < 16; j++) x[j] = (float)base[row * dim + o + j] - centroid[o + j];
    float best = __int_as_float(0x7f800000);
    int bi = 0;
    for (int c = 0; c < 256; c++) {
      float s = 0.f;
      for (int j = 0; j < w; j++) {
        const float d = x[j] - cen[c * w + j];
        s = __fmaf_rn(d, d, s);
      }
      if (s < best) {
        best = s;
        bi = c;
      }
    }
    out[r * M + m] = (OUT)bi;
  }
}

template <class T>
__global__ void mean_partial_kernel(const T* __restrict__ base, int64_t n, int dim, int64_t rows_per_block,
                                    double* __restrict__ partial) {
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = min(n, r0 + rows_per_block);
  for (int j = threadIdx.x; j < dim; j += blockDim.x) {
    double s = 0.0;
    for (int64_t r = r0; r < r1; r++) s += (double)base[r * dim + j];
    partial[(int64_t)blockIdx.x * dim + j] = s;
  }
}

template <class T>
__global__ void nearest_kernel(const T* __restrict__ base, int64_t n, int dim, const float* __restrict__ target,
                               unsigned long long* __restrict__ best) {
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int j = 0; j < dim; j++) {
      const float d = (float)base[r * dim + j] - target[j];
      s = __fmaf_rn(d, d, s);
    }
    atomicMin(best, ((unsigned long long)__float_as_uint(s) << 32) | (unsigned long long)r);
  }
}

// Node records: vector bytes, degree 0.
template <class T>
__global__ void init_pages_kernel(GLayout L, const T* __restrict__ base) {
  const int64_t ds4 = L.data_size / 4;
  const int64_t total = L.n * (ds4 + 1);
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = e / (ds4 + 1);
    const int64_t w = e - v * (ds4 + 1);
    uint32_t* rec = reinterpret_cast<uint32_t*>(node_rec(L, v));
    rec[w] = w < ds4 ? reinterpret_cast<const uint32_t*>(base + v * L.dim)[w] : 0u;
  }
}

// ---- wave RobustPrune ------------------------------------------------------

constexpr int kSlots = 8;            // candidate slots per lane (512 keys)
constexpr int kMaxCand = kSlots * kWave;

template <int P>
__device__ __forceinline__ void wave_sort_asc_full(uint64_t (&b)[P]) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 2; k <= P * kWave; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= kWave) {
        const int js = j / kWave;
#pragma unroll
        for (int s = 0; s < P; s++) {
          const int t = s ^ js;
          if (t > s) {
            const bool up = ((s * kWave) & k) == 0;
            const uint64_t lo = umin64(b[s], b[t]), hi = umax64(b[s], b[t]);
            b[s] = up ? lo : hi;
            b[t] = up ? hi : lo;
          }
        }
      } else {
#pragma unroll
        for (int s = 0; s < P; s++) {
          const uint64_t other = shfl_xor64(b[s], j);
          const bool up = ((s * kWave + lane) & k) == 0;
          const bool lower = (lane & j) == 0;
          b[s] = (lower == up) ? umin64(b[s], other) : umax64(b[s], other);
        }
      }
    }
  }
}

template <class T>
__device__ __forceinline__ int32_t vec_norm(const uint32_t* a, int ds4) {
  if constexpr (sizeof(T) == 4) {
    return 0;
  } else if constexpr (std::is_signed<T>::value) {
    int32_t acc = 0;
    for (int w = 0; w < ds4; w++) acc = __builtin_amdgcn_sdot4((int)a[w], (int)a[w], acc, false);
    return acc;
  } else {
    uint32_t acc = 0;
    for (int w = 0; w < ds4; w++) acc = __builtin_amdgcn_udot4(a[w], a[w], acc, false);
    return (int32_t)acc;
  }
}

struct PruneArgs {
  GLayout L;
  int mode;                  // 0: forward (search record), 1: reverse (marked segments), 2: flush
  const int32_t* centers;    // modes 0 and 2: node ids
  int64_t num_centers;
  const int32_t* rec_ids;    // forward: [num_centers][rec_cap]
  const int32_t* hops;       // forward: [num_centers]
  int rec_cap;
  const uint64_t* pairs;     // reverse: sorted (target << 32 | source)
  const int32_t* heads;      // reverse: segment starts
  const int32_t* marks;      // reverse: indexes into heads of the segments to prune
  int64_t num_pairs;
  uint32_t* pend;            // [n][P] pending reverse edges (the slack beyond R)
  int32_t* pcnt;             // [n] pending count
  int P;
  float alpha;
  int cmax;                  // candidate capacity after dedupe
  int stride;                // LDS row stride in dwords: a multiple of 4, stride / 4 odd, >= the row
  int G;                     // lanes that fetch one row together (power of two, >= 4)
};

// LDS of one prune wave: keys [cmax] u64, norms [cmax] i32, the centre row and
// cmax candidate rows at `stride` dwords (16-byte aligned), then the output list.
// The candidate rows double as the fetch phase's (id, distance) table.
struct PruneLds {
  int norms_off, cvec_off, vecs_off, outl_off, total;
};
__host__ __device__ inline PruneLds prune_lds_plan(int cmax, int stride, int R) {
  PruneLds p;
  p.norms_off = 8 * cmax;
  p.cvec_off = (12 * cmax + 15) & ~15;
  p.vecs_off = p.cvec_off + 4 * stride;
  const int vec_bytes = 4 * cmax * stride > 8 * kMaxCand ? 4 * cmax * stride : 8 * kMaxCand;
  p.outl_off = p.vecs_off + vec_bytes;
  p.total = p.outl_off + 4 * R;
  return p;
}

// Partial squared distance between the centre words c and row words x (8-bit
// data: x.x - 2 c.x, the centre's norm added once per row; float: (c - x)^2).
template <class T>
struct RowAcc {
  using type = typename std::conditional<sizeof(T) == 4, float, int32_t>::type;
  __device__ static __forceinline__ type add(type acc, uint32_t c, uint32_t x) {
    if constexpr (sizeof(T) == 4) {
      const float d = __uint_as_float(c) - __uint_as_float(x);
      return __fmaf_rn(d, d, acc);
    } else if constexpr (std::is_signed<T>::value) {
      return acc + __builtin_amdgcn_sdot4((int)x, (int)x, 0, false) - 2 * __builtin_amdgcn_sdot4((int)c, (int)x, 0, false);
    } else {
      return acc + (int32_t)__builtin_amdgcn_udot4(x, x, 0u, false) -
             2 * (int32_t)__builtin_amdgcn_udot4(c, x, 0u, false);
    }
  }
  __device__ static __forceinline__ type norm_add(type acc, uint32_t x) {
    if constexpr (sizeof(T) == 4) return acc;
    else if constexpr (std::is_signed<T>::value) return acc + __builtin_amdgcn_sdot4((int)x, (int)x, 0, false);
    else return acc + (int32_t)__builtin_amdgcn_udot4(x, x, 0u, false);
  }
};

template <class V>
__device__ __forceinline__ V group_sum(V v, int G) {
  for (int off = G >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Squared distance of two LDS rows read 16 bytes at a time (q4 pieces; words
// past the row are zero in both).  Float: the same dimension order as a
// sequential loop; 8-bit data: exact integers from the dot product and norms.
template <class T>
__device__ __forceinline__ float lds_row_dist(const uint32_t* a, const uint32_t* b, int q4, int32_t na, int32_t nb) {
  const uint4* a4 = reinterpret_cast<const uint4*>(a);
  const uint4* b4 = reinterpret_cast<const uint4*>(b);
  if constexpr (sizeof(T) == 4) {
    float s = 0.f;
    for (int q = 0; q < q4; q++) {
      const uint4 x = a4[q], y = b4[q];
      float d = __uint_as_float(x.x) - __uint_as_float(y.x);
      s = __fmaf_rn(d, d, s);
      d = __uint_as_float(x.y) - __uint_as_float(y.y);
      s = __fmaf_rn(d, d, s);
      d = __uint_as_float(x.z) - __uint_as_float(y.z);
      s = __fmaf_rn(d, d, s);
      d = __uint_as_float(x.w) - __uint_as_float(y.w);
      s = __fmaf_rn(d, d, s);
    }
    return s;
  } else if constexpr (std::is_signed<T>::value) {
    int32_t acc = 0;
    for (int q = 0; q < q4; q++) {
      const uint4 x = a4[q], y = b4[q];
      acc = __builtin_amdgcn_sdot4((int)x.x, (int)y.x, acc, false);
      acc = __builtin_amdgcn_sdot4((int)x.y, (int)y.y, acc, false);
      acc = __builtin_amdgcn_sdot4((int)x.z, (int)y.z, acc, false);
      acc = __builtin_amdgcn_sdot4((int)x.w, (int)y.w, acc, false);
    }
    return (float)(na + nb - 2 * acc);
  } else {
    uint32_t acc = 0;
    for (int q = 0; q < q4; q++) {
      const uint4 x = a4[q], y = b4[q];
      acc = __builtin_amdgcn_udot4(x.x, y.x, acc, false);
      acc = __builtin_amdgcn_udot4(x.y, y.y, acc, false);
      acc = __builtin_amdgcn_udot4(x.z, y.z, acc, false);
      acc = __builtin_amdgcn_udot4(x.w, y.w, acc, false);
    }
    return (float)((int64_t)na + (int64_t)nb - 2 * (int64_t)acc);
  }
}

// LDS areas of a prune wave.
struct PruneSmem {
  uint64_t* keys;
  int32_t* norms;
  uint32_t* cvec;
  uint32_t* vecs;
  uint32_t* outl;
};

// Prune of one centre over its C0 candidates (cand(i) -> node id, or -1 to
// skip): exact distances from the centre, sort by (distance, id), dedupe, then
// the list is the candidates themselves when they fit in R, else
// RobustPrune(alpha, R) over them.  SL slots of 64 lanes hold the sort
// (C0 <= 64 SL).  The centre's pending edges are cleared: the caller put them
// among the candidates.
// Candidate rows are fetched cooperatively: G lanes per row, lane p of a row
// reading words p, p + G, ... (a contiguous G-word run per load instruction),
// 64 / G rows per instruction and two instructions' rows in flight, so the
// fetch costs a few memory round trips per centre instead of one per word.
template <class T, int SL, class F>
__device__ __forceinline__ void prune_one(const PruneArgs& a, const PruneSmem& m, int64_t center, int C0, F cand) {
  using Acc = RowAcc<T>;
  using AccT = typename Acc::type;
  const GLayout& L = a.L;
  const int lane = lane_id();
  const int ds4 = (int)(L.data_size / 4);
  const int S = a.stride;
  const int w4 = (ds4 + 3) & ~3;  // row words read by lds_row_dist (zero past ds4)
  const int G = a.G, rpr = kWave / G, p = lane & (G - 1), sub = lane / G;
  const int kk = (ds4 + G - 1) / G;  // words per lane per row
  uint32_t* cand_id = m.vecs;            // fetch phase: [kMaxCand] ids (~0u: none)
  uint32_t* cand_d = m.vecs + kMaxCand;  // fetch phase: [kMaxCand] distance bits
  uint32_t* crec = reinterpret_cast<uint32_t*>(node_rec(L, center));
  uint32_t* cnb = crec + ds4;
  const int32_t cnorm = vec_norm<T>(m.cvec, ds4);

  // ---- distances centre -> candidates, rows fetched by groups of G lanes
  for (int r0 = 0; r0 < C0; r0 += 2 * rpr) {
    const int i0 = r0 + sub, i1 = r0 + rpr + sub;
    const int64_t id0 = i0 < C0 ? cand(i0) : -1;
    const int64_t id1 = i1 < C0 ? cand(i1) : -1;
    const uint32_t* x0 = reinterpret_cast<const uint32_t*>(node_rec(L, id0 >= 0 ? id0 : center));
    const uint32_t* x1 = reinterpret_cast<const uint32_t*>(node_rec(L, id1 >= 0 ? id1 : center));
    AccT s0 = 0, s1 = 0;
    for (int k0 = 0; k0 < kk; k0 += 4) {
      uint32_t v0[4], v1[4], cw[4];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int w = p + G * (k0 + t);
        const bool ok = k0 + t < kk && w < ds4;
        v0[t] = ok ? x0[w] : 0u;
        v1[t] = ok ? x1[w] : 0u;
        cw[t] = ok ? m.cvec[w] : 0u;
      }
#pragma unroll
      for (int t = 0; t < 4; t++) {
        s0 = Acc::add(s0, cw[t], v0[t]);
        s1 = Acc::add(s1, cw[t], v1[t]);
      }
    }
    s0 = group_sum(s0, G);
    s1 = group_sum(s1, G);
    if (p == 0) {
      float d0, d1;
      if constexpr (sizeof(T) == 4) {
        d0 = s0;
        d1 = s1;
      } else {
        d0 = (float)(cnorm + s0);
        d1 = (float)(cnorm + s1);
      }
      if (i0 < C0) {
        cand_id[i0] = id0 >= 0 ? (uint32_t)id0 : ~0u;
        cand_d[i0] = __float_as_uint(d0);
      }
      if (i1 < C0) {
        cand_id[i1] = id1 >= 0 ? (uint32_t)id1 : ~0u;
        cand_d[i1] = __float_as_uint(d1);
      }
    }
  }
  __syncthreads();
  uint64_t b[SL];
#pragma unroll
  for (int s = 0; s < SL; s++) {
    const int i = s * kWave + lane;
    uint64_t key = kPadKey;
    if (i < C0) {
      const uint32_t id = cand_id[i];
      if (id != ~0u) key = ((uint64_t)cand_d[i] << 32) | (uint64_t)id;
    }
    b[s] = key;
  }
  __syncthreads();  // the fetch table is overwritten by the rows below
  wave_sort_asc_full<SL>(b);
  // dedupe (equal ids are adjacent: equal distance) and compact into LDS
  int C = 0;
  uint32_t prev = 0xffffffffu;
  bool prev_valid = false;
#pragma unroll
  for (int s = 0; s < SL; s++) {
    const uint32_t id = (uint32_t)b[s];
    uint32_t pid = (uint32_t)__shfl_up((int)id, 1);
    bool pvalid = __shfl_up((int)(b[s] != kPadKey), 1) != 0;
    if (lane == 0) {
      pid = prev;
      pvalid = prev_valid;
    }
    const bool keep = b[s] != kPadKey && !(pvalid && pid == id);
    const uint64_t km = __ballot(keep);
    const int pos = C + __popcll(km & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
    if (keep && pos < a.cmax) m.keys[pos] = b[s];
    C += __popcll(km);
    prev = (uint32_t)__shfl((int)id, kWave - 1);
    prev_valid = __shfl((int)(b[s] != kPadKey), kWave - 1) != 0;
  }
  C = min(C, a.cmax);
  __syncthreads();

  int out_n = 0;
  if (C <= L.R) {
    for (int i = lane; i < C; i += kWave) cnb[1 + i] = (uint32_t)m.keys[i];
    out_n = C;
  } else {
    // stage the candidate rows (and their norms) in LDS, fetched as above
    for (int r0 = 0; r0 < C; r0 += 2 * rpr) {
      const int i0 = r0 + sub, i1 = r0 + rpr + sub;
      const int64_t id0 = i0 < C ? (int64_t)(uint32_t)m.keys[i0] : center;
      const int64_t id1 = i1 < C ? (int64_t)(uint32_t)m.keys[i1] : center;
      const uint32_t* x0 = reinterpret_cast<const uint32_t*>(node_rec(L, id0));
      const uint32_t* x1 = reinterpret_cast<const uint32_t*>(node_rec(L, id1));
      AccT n0 = 0, n1 = 0;
      for (int k0 = 0; k0 < kk; k0 += 4) {
        uint32_t v0[4], v1[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int w = p + G * (k0 + t);
          const bool ok = k0 + t < kk && w < ds4;
          v0[t] = ok ? x0[w] : 0u;
          v1[t] = ok ? x1[w] : 0u;
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int w = p + G * (k0 + t);
          if (k0 + t < kk && w < w4) {
            if (i0 < C) m.vecs[i0 * S + w] = v0[t];
            if (i1 < C) m.vecs[i1 * S + w] = v1[t];
          }
          n0 = Acc::norm_add(n0, v0[t]);
          n1 = Acc::norm_add(n1, v1[t]);
        }
      }
      if constexpr (sizeof(T) != 4) {
        n0 = group_sum(n0, G);
        n1 = group_sum(n1, G);
        if (p == 0) {
          if (i0 < C) m.norms[i0] = n0;
          if (i1 < C) m.norms[i1] = n1;
        }
      }
    }
    __syncthreads();
    uint32_t alive = 0;
#pragma unroll
    for (int s = 0; s < SL; s++)
      if (s * kWave + lane < C) alive |= 1u << s;
    const int q4 = w4 / 4;
    for (int i = 0; i < C && out_n < L.R; i++) {
      const uint32_t owner = (uint32_t)__shfl((int)alive, i & (kWave - 1));
      if (!((owner >> (i >> 6)) & 1u)) continue;
      if (lane == 0) m.outl[out_n] = (uint32_t)m.keys[i];
      out_n++;
      const uint32_t* vi = m.vecs + i * S;
      const int32_t ni = sizeof(T) == 4 ? 0 : m.norms[i];
#pragma unroll
      for (int s = 0; s < SL; s++) {
        const int j = s * kWave + lane;
        if (j > i && j < C && ((alive >> s) & 1u)) {
          const float dij = lds_row_dist<T>(vi, m.vecs + j * S, q4, ni, sizeof(T) == 4 ? 0 : m.norms[j]);
          const float dpj = __uint_as_float((uint32_t)(m.keys[j] >> 32));
          if (a.alpha * dij <= dpj) alive &= ~(1u << s);
        }
      }
    }
    __syncthreads();
    for (int i = lane; i < out_n; i += kWave) cnb[1 + i] = m.outl[i];
  }
  if (lane == 0) {
    cnb[0] = (uint32_t)out_n;
    a.pcnt[center] = 0;
  }
  __syncthreads();
}

// One wave per centre: forward prunes (mode 0: the nodes expanded by the
// centre's build search, then its current list and pending edges), reverse
// prunes of marked segments (mode 1: current list, pending edges, then the
// segment's incoming sources) and the flush of pending edges (mode 2: list and
// pending).  The sort width follows the candidate count.
template <class T>
__global__ __launch_bounds__(64) void prune_kernel(PruneArgs a) {
  extern __shared__ __align__(16) char smem[];
  const GLayout& L = a.L;
  const int lane = lane_id();
  const int ds4 = (int)(L.data_size / 4);
  const PruneLds pl = prune_lds_plan(a.cmax, a.stride, L.R);
  PruneSmem m;
  m.keys = reinterpret_cast<uint64_t*>(smem);
  m.norms = reinterpret_cast<int32_t*>(smem + pl.norms_off);
  m.cvec = reinterpret_cast<uint32_t*>(smem + pl.cvec_off);
  m.vecs = reinterpret_cast<uint32_t*>(smem + pl.vecs_off);
  m.outl = reinterpret_cast<uint32_t*>(smem + pl.outl_off);
  for (int64_t ci = blockIdx.x; ci < a.num_centers; ci += gridDim.x) {
    int64_t center;
    int64_t seg_begin = 0, seg_end = 0;
    if (a.mode != 1) {
      center = a.centers[ci];
    } else {
      seg_begin = a.heads[a.marks[ci]];
      center = (int64_t)(a.pairs[seg_begin] >> 32);
      // pairs are sorted by target, so the segment is the run of pairs whose
      // target matches: advance by whole waves, then to the first miss
      seg_end = seg_begin;
      while (true) {
        const int64_t q = seg_end + lane;
        const bool same = q < a.num_pairs && (int64_t)(a.pairs[q] >> 32) == center;
        const uint64_t mk = __ballot(same);
        if (mk == ~0ull) {
          seg_end += kWave;
          continue;
        }
        seg_end += __ffsll((long long)~mk) - 1;
        break;
      }
    }
    uint32_t* crec = reinterpret_cast<uint32_t*>(node_rec(L, center));
    for (int w = lane; w < a.stride; w += kWave) m.cvec[w] = w < ds4 ? crec[w] : 0u;
    const uint32_t* cnb = crec + ds4;
    const int cdeg = (int)cnb[0];
    const int pc = a.pcnt[center];
    const uint32_t* pend = a.pend + center * a.P;
    // candidate i: [lead candidates][current list][pending][trailing sources]
    int lead = 0, tail = 0;
    if (a.mode == 0) lead = min(a.hops[ci], a.rec_cap);
    if (a.mode == 1) tail = (int)min<int64_t>(seg_end - seg_begin, kMaxCand - L.R - a.P);
    const int C0 = min(lead + cdeg + pc + tail, kMaxCand);
    auto cand = [&](int i) -> int64_t {
      int64_t id;
      if (i < lead) id = (int64_t)a.rec_ids[ci * a.rec_cap + i];
      else if (i < lead + cdeg) id = (int64_t)cnb[1 + (i - lead)];
      else if (i < lead + cdeg + pc) id = (int64_t)pend[i - lead - cdeg];
      else id = (int64_t)(uint32_t)a.pairs[seg_begin + (i - lead - cdeg - pc)];
      return id == center ? -1 : id;
    };
    __syncthreads();
    if (C0 <= 2 * kWave) prune_one<T, 2>(a, m, center, C0, cand);
    else if (C0 <= 4 * kWave) prune_one<T, 4>(a, m, center, C0, cand);
    else prune_one<T, kSlots>(a, m, center, C0, cand);
  }
}

// Reverse edges of a batch, one wave per target (a run of sorted pairs):
// sources already among the target's list or pending edges are dropped; the
// rest are appended to the list while it has room, then to the pending edges
// (up to P, DiskANN's graph slack: a list may hold 1.3 R before it is pruned);
// a target whose new edges fit neither is marked for a reverse prune.
__global__ __launch_bounds__(64) void reverse_insert_kernel(GLayout L, const uint64_t* __restrict__ pairs,
                                                            const int32_t* __restrict__ heads, int64_t nheads,
                                                            int64_t npairs, uint32_t* __restrict__ pend,
                                                            int32_t* __restrict__ pcnt, int P,
                                                            int32_t* __restrict__ marks,
                                                            unsigned int* __restrict__ nmarks) {
  const int lane = lane_id();
  for (int64_t hi = blockIdx.x; hi < nheads; hi += gridDim.x) {
    const int64_t b = heads[hi];
    const uint32_t t = (uint32_t)(pairs[b] >> 32);
    uint32_t* nb = reinterpret_cast<uint32_t*>(node_rec(L, t) + L.data_size);
    const int cdeg = (int)nb[0];
    const int pc = pcnt[t];
    // the list, two slots per lane (R <= 128), and the pending edges (P <= 64)
    const uint32_t mine0 = lane < cdeg ? nb[1 + lane] : ~0u;
    const uint32_t mine1 = lane + kWave < cdeg ? nb[1 + kWave + lane] : ~0u;
    const uint32_t pmine = lane < pc ? pend[(int64_t)t * P + lane] : ~0u;
    const int c0 = min(cdeg, kWave);
    // new sources, counted over the whole run, 64 pairs at a time
    auto fresh = [&](int64_t q, uint32_t& src) -> bool {
      if (q >= npairs || (uint32_t)(pairs[q] >> 32) != t) return false;
      src = (uint32_t)pairs[q];
      bool dup = false;
      for (int k = 0; k < c0; k++) dup |= src == (uint32_t)__builtin_amdgcn_readlane((int)mine0, k);
      for (int k = kWave; k < cdeg; k++) dup |= src == (uint32_t)__builtin_amdgcn_readlane((int)mine1, k - kWave);
      for (int k = 0; k < pc; k++) dup |= src == (uint32_t)__builtin_amdgcn_readlane((int)pmine, k);
      return !dup;
    };
    int u = 0;
    int64_t q0 = b;
    while (true) {
      uint32_t src = 0;
      const bool in_run = q0 + lane < npairs && (uint32_t)(pairs[q0 + lane] >> 32) == t;
      const bool f = in_run && fresh(q0 + lane, src);
      u += __popcll(__ballot(f));
      if (__ballot(in_run) != ~0ull) break;
      q0 += kWave;
    }
    const int room = L.R - cdeg;
    if (u > room + (P - pc)) {
      if (lane == 0) marks[atomicAdd(nmarks, 1u)] = (int32_t)hi;
      continue;
    }
    if (u == 0) continue;
    int placed = 0;
    q0 = b;
    while (true) {
      uint32_t src = 0;
      const bool in_run = q0 + lane < npairs && (uint32_t)(pairs[q0 + lane] >> 32) == t;
      const bool f = in_run && fresh(q0 + lane, src);
      const uint64_t fm = __ballot(f);
      if (f) {
        const int r = placed + __popcll(fm & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
        if (r < room) nb[1 + cdeg + r] = src;
        else pend[(int64_t)t * P + pc + (r - room)] = src;
      }
      placed += __popcll(fm);
      if (__ballot(in_run) != ~0ull) break;
      q0 += kWave;
    }
    if (lane == 0) {
      const int to_list = min(u, room);
      nb[0] = (uint32_t)(cdeg + to_list);
      pcnt[t] = pc + (u - to_list);
    }
  }
}

// Nodes with pending edges, for the flush at the end of a pass.
__global__ void pending_nodes_kernel(const int32_t* __restrict__ pcnt, int64_t n, int32_t* __restrict__ out,
                                     unsigned int* __restrict__ count) {
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < n; v += (int64_t)gridDim.x * blockDim.x)
    if (pcnt[v] > 0) out[atomicAdd(count, 1u)] = (int32_t)v;
}

// Reverse-edge pairs (target << 32 | source) of every new list of the batch.
__global__ void emit_pairs_kernel(GLayout L, const int32_t* __restrict__ centers, int64_t nc,
                                  uint64_t* __restrict__ pairs, unsigned long long* __restrict__ count) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < nc * L.R;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t ci = e / L.R;
    const int j = (int)(e - ci * L.R);
    const int64_t p = centers[ci];
    const uint32_t* nb = reinterpret_cast<const uint32_t*>(node_rec(L, p) + L.data_size);
    uint64_t key = kPadKey;
    if (j < (int)nb[0]) {
      key = ((uint64_t)nb[1 + j] << 32) | (uint64_t)(uint32_t)p;
      atomicAdd(count, 1ull);
    }
    pairs[e] = key;
  }
}

__global__ void heads_kernel(const uint64_t* __restrict__ pairs, int64_t n, int32_t* __restrict__ heads,
                             unsigned int* __restrict__ nheads) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (i == 0 || (pairs[i] >> 32) != (pairs[i - 1] >> 32)) heads[atomicAdd(nheads, 1u)] = (int32_t)i;
  }
}

// ---- brute-force ground truth ----------------------------------------------

constexpr int kGtQ = 8;

__device__ __forceinline__ void gt_offer(uint64_t& tk, int k, uint64_t key) {
  uint64_t cand = __ballot(key < (((uint64_t)(uint32_t)__shfl((int)(uint32_t)(tk >> 32), k - 1) << 32) |
                                  (uint32_t)__shfl((int)(uint32_t)tk, k - 1)));
  while (cand) {
    const int l = __ffsll((long long)cand) - 1;
    cand &= cand - 1;
    const uint64_t ck = ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(key >> 32), l) << 32) |
                        (uint32_t)__shfl((int)(uint32_t)key, l);
    const uint64_t th = ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(tk >> 32), k - 1) << 32) |
                        (uint32_t)__shfl((int)(uint32_t)tk, k - 1);
    if (ck < th) {
      const int lane = lane_id();
      const int pos = __popcll(__ballot(lane < k && tk < ck));
      const uint64_t prev = ((uint64_t)(uint32_t)__shfl_up((int)(uint32_t)(tk >> 32), 1) << 32) |
                            (uint32_t)__shfl_up((int)(uint32_t)tk, 1);
      if (lane < k) {
        if (lane == pos) tk = ck;
        else if (lane > pos) tk = prev;
      }
    }
  }
}

// Block (query group, base slice): 4 waves stream the slice, each lane one base
// row at a time, distances to kGtQ queries in fp32 (exact for 8-bit data).
template <class T>
__global__ __launch_bounds__(256) void gt_kernel(const T* __restrict__ base, int64_t n, int dim,
                                                 const float* __restrict__ queries, int64_t nq, int k,
                                                 int64_t slice, int S, uint64_t* __restrict__ part) {
  extern __shared__ __align__(16) char smem[];
  float* q = reinterpret_cast<float*>(smem);
  uint64_t* xk = reinterpret_cast<uint64_t*>(q + kGtQ * dim);
  const int64_t q0 = (int64_t)blockIdx.x * kGtQ;
  const int s = blockIdx.y;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  for (int i = tid; i < kGtQ * dim; i += 256) {
    const int64_t qi = q0 + i / dim;
    q[i] = qi < nq ? queries[qi * dim + (i % dim)] : 0.f;
  }
  __syncthreads();
  uint64_t tk[kGtQ];
#pragma unroll
  for (int t = 0; t < kGtQ; t++) tk[t] = kPadKey;
  const int64_t r0 = (int64_t)s * slice, r1 = min(n, r0 + slice);
  for (int64_t rb = r0 + wave * kWave; rb < r1; rb += 4 * kWave) {
    const int64_t r = rb + lane;
    float acc[kGtQ];
#pragma unroll
    for (int t = 0; t < kGtQ; t++) acc[t] = 0.f;
    if (r < r1) {
      // rows are read a dword at a time (dim * sizeof(T) is a multiple of 4)
      constexpr int per = 4 / (int)sizeof(T);
      const uint32_t* x32 = reinterpret_cast<const uint32_t*>(base + r * dim);
      for (int w = 0; w < dim / per; w++) {
        const uint32_t word = x32[w];
#pragma unroll
        for (int e = 0; e < per; e++) {
          float xv;
          if constexpr (sizeof(T) == 4) xv = __uint_as_float(word);
          else if constexpr (std::is_signed<T>::value) xv = (float)(int8_t)(word >> (8 * e));
          else xv = (float)((word >> (8 * e)) & 0xffu);
          const int j = w * per + e;
#pragma unroll
          for (int t = 0; t < kGtQ; t++) {
            const float d = q[t * dim + j] - xv;
            acc[t] = __fmaf_rn(d, d, acc[t]);
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kGtQ; t++) {
      const uint64_t key = r < r1 ? (((uint64_t)__float_as_uint(acc[t]) << 32) | (uint64_t)r) : kPadKey;
      gt_offer(tk[t], k, key);
    }
  }
#pragma unroll
  for (int t = 0; t < kGtQ; t++) {
    xk[(t * 4 + wave) * kWave + lane] = tk[t];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < kGtQ; t++) {
      uint64_t m = tk[t];
      for (int w = 1; w < 4; w++) gt_offer(m, k, lane < k ? xk[(t * 4 + w) * kWave + lane] : kPadKey);
      const int64_t qi = q0 + t;
      if (qi < nq && lane < k) part[(qi * S + s) * k + lane] = m;
    }
  }
}

__global__ void gt_final_kernel(const uint64_t* __restrict__ part, int64_t nq, int S, int k,
                                int32_t* __restrict__ ids, float* __restrict__ dists) {
  const int lane = lane_id();
  for (int64_t qi = blockIdx.x; qi < nq; qi += gridDim.x) {
    uint64_t tk = kPadKey;
    for (int s = 0; s < S; s++) gt_offer(tk, k, lane < k ? part[(qi * S + s) * k + lane] : kPadKey);
    if (lane < k) {
      ids[qi * k + lane] = tk == kPadKey ? -1 : (int32_t)(uint32_t)tk;
      dists[qi * k + lane] = tk == kPadKey ? __int_as_float(0x7f800000) : __uint_as_float((uint32_t)(tk >> 32));
    }
  }
}

// Ground truth for 8-bit data with integer dot products: each lane owns one
// query (its elements packed four to a register, zero past dim <= 128), tiles
// of kGtTile consecutive base rows are staged in LDS with coalesced loads
// (rows of kGtStride words: nine 16-byte pieces, an odd count, so the row-per-
// thread norm pass is conflict-free) and every lane compares its query with
// each staged row: d = |q|^2 + |x|^2 - 2 q.x, exact in int32 and in fp32
// (< 2^24), so keys (d, id) -- and the top-k with ties to the smaller id --
// equal the floating-point kernel's.
constexpr int kGtTile = 256;
constexpr int kGtWords = 32;
constexpr int kGtStride = 36;
constexpr int kGtMaxK = 16;

template <class T>
__device__ __forceinline__ uint32_t dot4(uint32_t a, uint32_t b, uint32_t acc) {
  if constexpr (std::is_signed<T>::value)
    return (uint32_t)__builtin_amdgcn_sdot4((int)a, (int)b, (int)acc, false);
  else
    return __builtin_amdgcn_udot4(a, b, acc, false);
}

template <class T>
__global__ __launch_bounds__(256) void gt_int_kernel(const T* __restrict__ base, int64_t n, int dim,
                                                     const float* __restrict__ queries, int64_t nq, int k,
                                                     int64_t slice, int S, uint64_t* __restrict__ part) {
  __shared__ __align__(16) uint32_t rows[kGtTile * kGtStride];
  __shared__ int32_t norms[kGtTile];
  const int tid = threadIdx.x;
  const int64_t qi = (int64_t)blockIdx.x * 256 + tid;
  const int s = blockIdx.y;
  const int d4 = dim / 4;
  uint32_t qw[kGtWords];
#pragma unroll
  for (int w = 0; w < kGtWords; w++) {
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int j = 4 * w + e;
      const int v = qi < nq && j < dim ? (int)queries[qi * dim + j] : 0;
      packed |= ((uint32_t)v & 0xffu) << (8 * e);
    }
    qw[w] = packed;
  }
  uint32_t qn = 0;
#pragma unroll
  for (int w = 0; w < kGtWords; w++) qn = dot4<T>(qw[w], qw[w], qn);
  for (int i = tid; i < kGtTile * kGtStride; i += 256) rows[i] = 0u;  // pads stay zero
  uint64_t tk[kGtMaxK];
#pragma unroll
  for (int i = 0; i < kGtMaxK; i++) tk[i] = kPadKey;
  uint64_t thr = kPadKey;
  const int64_t r0 = (int64_t)s * slice, r1 = min(n, r0 + slice);
  __syncthreads();
  for (int64_t t0 = r0; t0 < r1; t0 += kGtTile) {
    const int here = (int)min<int64_t>(kGtTile, r1 - t0);
    const uint8_t* src = reinterpret_cast<const uint8_t*>(base + t0 * dim);
    if ((d4 & 3) == 0) {
      const int pr = d4 / 4;  // 16-byte pieces per row
      const uint4* s4 = reinterpret_cast<const uint4*>(src);
      for (int u = tid; u < here * pr; u += 256) {
        const int r = u / pr, c = u - r * pr;
        *reinterpret_cast<uint4*>(rows + r * kGtStride + 4 * c) = s4[u];
      }
    } else {
      const uint32_t* s1 = reinterpret_cast<const uint32_t*>(src);
      for (int u = tid; u < here * d4; u += 256) {
        const int r = u / d4, c = u - r * d4;
        rows[r * kGtStride + c] = s1[u];
      }
    }
    __syncthreads();
    if (tid < here) {
      const uint4* rp = reinterpret_cast<const uint4*>(rows + tid * kGtStride);
      uint32_t nn = 0;
#pragma unroll
      for (int pc = 0; pc < kGtWords / 4; pc++) {
        const uint4 x = rp[pc];
        nn = dot4<T>(x.x, x.x, nn);
        nn = dot4<T>(x.y, x.y, nn);
        nn = dot4<T>(x.z, x.z, nn);
        nn = dot4<T>(x.w, x.w, nn);
      }
      norms[tid] = (int32_t)nn;
    }
    __syncthreads();
    for (int r = 0; r < here; r++) {
      const uint4* rp = reinterpret_cast<const uint4*>(rows + r * kGtStride);
      uint32_t acc = 0;
#pragma unroll
      for (int pc = 0; pc < kGtWords / 4; pc++) {
        const uint4 x = rp[pc];
        acc = dot4<T>(qw[4 * pc + 0], x.x, acc);
        acc = dot4<T>(qw[4 * pc + 1], x.y, acc);
        acc = dot4<T>(qw[4 * pc + 2], x.z, acc);
        acc = dot4<T>(qw[4 * pc + 3], x.w, acc);
      }
      const int32_t d = (int32_t)qn + norms[r] - 2 * (int32_t)acc;
      const uint64_t key = ((uint64_t)__float_as_uint((float)d) << 32) | (uint64_t)(t0 + r);
      if (key < thr) {
#pragma unroll
        for (int i = kGtMaxK - 1; i > 0; i--) {
          const uint64_t lo = tk[i - 1], cur = tk[i];
          tk[i] = key < lo ? lo : (key < cur ? key : cur);
        }
        tk[0] = key < tk[0] ? key : tk[0];
        uint64_t t = tk[0];
#pragma unroll
        for (int i = 1; i < kGtMaxK; i++) t = i == k - 1 ? tk[i] : t;
        thr = t;
      }
    }
    __syncthreads();
  }
  if (qi < nq) {
#pragma unroll
    for (int i = 0; i < kGtMaxK; i++)
      if (i < k) part[(qi * S + s) * k + i] = tk[i];
  }
}

// Sets *bad when a query element is not an integer of the element type's range
// (then the 8-bit kernel does not apply).
template <class T>
__global__ void gt_query_check(const float* __restrict__ q, int64_t count, int32_t* __restrict__ bad) {
  const float lo = std::is_signed<T>::value ? -128.f : 0.f, hi = std::is_signed<T>::value ? 127.f : 255.f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
    const float v = q[i];
    if (!(v >= lo && v <= hi && v == rintf(v))) *bad = 1;
  }
}

int grid_of(int64_t work, int block) {
  return (int)std::max<int64_t>(1, std::min<int64_t>((work + block - 1) / block, 1 << 20));
}

template <class T>
void ground_truth_t(const T* d_base, int64_t n, int dim, const float* d_q, int64_t nq, int k, int32_t* d_ids,
                    float* d_dists, hipStream_t st) {
  if constexpr (sizeof(T) == 1) {
    if (dim <= 4 * kGtWords && dim % 4 == 0 && k <= kGtMaxK) {
      int32_t* d_bad = nullptr;
      HIP_OK(hipMallocAsync(reinterpret_cast<void**>(&d_bad), sizeof(int32_t), st));
      HIP_OK(hipMemsetAsync(d_bad, 0, sizeof(int32_t), st));
      hipLaunchKernelGGL(gt_query_check<T>, dim3((unsigned)grid_of(nq * dim, 256)), dim3(256), 0, st, d_q, nq * dim,
                         d_bad);
      HIP_OK(hipGetLastError());
      int32_t bad = 0;
      HIP_OK(hipMemcpyAsync(&bad, d_bad, sizeof(bad), hipMemcpyDeviceToHost, st));
      HIP_OK(hipStreamSynchronize(st));
      HIP_OK(hipFreeAsync(d_bad, st));
      if (!bad) {
        const int64_t groups = (nq + 255) / 256;
        const int64_t tiles = (n + kGtTile - 1) / kGtTile;
        const int S = (int)std::max<int64_t>(1, std::min<int64_t>({256, tiles, (2048 + groups - 1) / groups}));
        const int64_t slice = (tiles + S - 1) / S * kGtTile;
        uint64_t* part = nullptr;
        HIP_OK(hipMallocAsync(reinterpret_cast<void**>(&part), sizeof(uint64_t) * (size_t)(nq * S * k), st));
        hipLaunchKernelGGL(gt_int_kernel<T>, dim3((unsigned)groups, (unsigned)S), dim3(256), 0, st, d_base, n, dim,
                           d_q, nq, k, slice, S, part);
        HIP_OK(hipGetLastError());
        hipLaunchKernelGGL(gt_final_kernel, dim3((unsigned)std::min<int64_t>(nq, 65536)), dim3(64), 0, st, part, nq,
                           S, k, d_ids, d_dists);
        HIP_OK(hipGetLastError());
        HIP_OK(hipFreeAsync(part, st));
        HIP_OK(hipStreamSynchronize(st));
        return;
      }
    }
  }
  const int S = (int)std::max<int64_t>(1, std::min<int64_t>(64, 4096 / std::max<int64_t>(1, (nq + kGtQ - 1) / kGtQ)));
  const int64_t slice = (n + S - 1) / S;
  uint64_t* part = nullptr;
  HIP_OK(hipMallocAsync(reinterpret_cast<void**>(&part), sizeof(uint64_t) * (size_t)(nq * S * k), st));
  const size_t lds = (size_t)kGtQ * dim * 4 + (size_t)kGtQ * 4 * kWave * 8;
  hipLaunchKernelGGL(gt_kernel<T>, dim3((unsigned)((nq + kGtQ - 1) / kGtQ), (unsigned)S), dim3(256), lds, st,
                     d_base, n, dim, d_q, nq, k, slice, S, part);
  HIP_OK(hipGetLastError());
  hipLaunchKernelGGL(gt_final_kernel, dim3((unsigned)std::min<int64_t>(nq, 65536)), dim3(64), 0, st, part, nq, S,
                     k, d_ids, d_dists);
  HIP_OK(hipGetLastError());
  HIP_OK(hipFreeAsync(part, st));
  HIP_OK(hipStreamSynchronize(st));
}

// ---- host driver ------------------------------------------------------------

template <class T>
void train_pq_gpu(const T* d_base, int64_t n, int dim, const qv_build_params& prm, PQTables& t, hipStream_t st) {
  const int M = prm.num_chunks;
  if (M <= 0 || M > dim) fail(QV_EINVAL, "num_chunks must be in [1, dim]");
  t.dim = dim;
  t.num_chunks = M;
  t.num_pts = n;
  t.chunk_offsets.resize((size_t)M + 1);
  for (int i = 0; i <= M; i++) t.chunk_offsets[(size_t)i] = (int32_t)(((int64_t)i * dim) / M);
  for (int i = 0; i < M; i++)
    if (t.chunk_offsets[(size_t)i + 1] - t.chunk_offsets[(size_t)i] > 16)
      fail(QV_EUNSUPPORTED, "PQ chunks wider than 16 dimensions");
  t.chunk_id.assign((size_t)dim, 0);
  for (int i = 0; i < M; i++)
    for (int j = t.chunk_offsets[(size_t)i]; j < t.chunk_offsets[(size_t)i + 1]; j++) t.chunk_id[(size_t)j] = i;

  const int64_t ns = std::min<int64_t>(n, prm.pq_train_max > 0 ? prm.pq_train_max : 262144);
  std::vector<int32_t> rows((size_t)ns);
  for (int64_t i = 0; i < ns; i++) rows[(size_t)i] = (int32_t)((i * n) / ns);
  int32_t* d_rows = nullptr;
  HIP_OK(hipMalloc(&d_rows, sizeof(int32_t) * (size_t)ns));
  HIP_OK(hipMemcpy(d_rows, rows.data(), sizeof(int32_t) * (size_t)ns, hipMemcpyHostToDevice));
  std::vector<float> xs((size_t)ns * dim);
  {
    float* d_xs = nullptr;
    HIP_OK(hipMalloc(&d_xs, sizeof(float) * xs.size()));
    hipLaunchKernelGGL(gather_rows_f32<T>, dim3((unsigned)grid_of(ns * dim, 256)), dim3(256), 0, st, d_base, dim,
                       d_rows, ns, d_xs);
    HIP_OK(hipGetLastError());
    HIP_OK(hipMemcpyAsync(xs.data(), d_xs, sizeof(float) * xs.size(), hipMemcpyDeviceToHost, st));
    HIP_OK(hipStreamSynchronize(st));
    (void)hipFree(d_xs);
  }
  std::vector<double> acc((size_t)dim, 0.0);
  for (int64_t i = 0; i < ns; i++)
    for (int j = 0; j < dim; j++) acc[(size_t)j] += (double)xs[(size_t)i * dim + j];
  t.centroid.resize((size_t)dim);
  for (int j = 0; j < dim; j++) t.centroid[(size_t)j] = (float)(acc[(size_t)j] / (double)ns);

  t.pivots.assign((size_t)kNumPivots * dim, 0.f);
  for (int m = 0; m < M; m++) {
    const int o = t.chunk_offsets[(size_t)m], w = t.chunk_offsets[(size_t)m + 1] - o;
    for (int c = 0; c < kNumPivots; c++) {
      const int64_t pick = (int64_t)(rng_u64(prm.seed, 12 + (uint64_t)m, (uint64_t)c) % (uint64_t)ns);
      for (int j = 0; j < w; j++)
        t.pivots[(size_t)c * dim + o + j] = (float)xs[(size_t)pick * dim + o + j] - t.centroid[(size_t)(o + j)];
    }
  }
  int32_t *d_off = nullptr, *d_assign = nullptr;
  float *d_cent = nullptr, *d_piv = nullptr;
  HIP_OK(hipMalloc(&d_off, sizeof(int32_t) * (size_t)(M + 1)));
  HIP_OK(hipMalloc(&d_assign, sizeof(int32_t) * (size_t)ns * M));
  HIP_OK(hipMalloc(&d_cent, sizeof(float) * (size_t)dim));
  HIP_OK(hipMalloc(&d_piv, sizeof(float) * t.pivots.size()));
  HIP_OK(hipMemcpy(d_off, t.chunk_offsets.data(), sizeof(int32_t) * (size_t)(M + 1), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_cent, t.centroid.data(), sizeof(float) * (size_t)dim, hipMemcpyHostToDevice));
  std::vector<int32_t> assign((size_t)ns * M);
  const int maxw = (dim + M - 1) / M;
  const size_t lds = 256 * (size_t)maxw * 4;
  const int gx = grid_of(ns, 256);
  for (int it = 0; it < std::max(1, prm.kmeans_iters); it++) {
    HIP_OK(hipMemcpy(d_piv, t.pivots.data(), sizeof(float) * t.pivots.size(), hipMemcpyHostToDevice));
    hipLaunchKernelGGL((pq_assign_kernel<T, int32_t>), dim3((unsigned)std::min(gx, 4096), (unsigned)M), dim3(256),
                       lds, st, d_base, dim, d_rows, ns, d_cent, d_off, M, d_piv, d_assign);
    HIP_OK(hipGetLastError());
    HIP_OK(hipMemcpyAsync(assign.data(), d_assign, sizeof(int32_t) * assign.size(), hipMemcpyDeviceToHost, st));
    HIP_OK(hipStreamSynchronize(st));
    std::vector<double> sum((size_t)kNumPivots * dim, 0.0);
    std::vector<int64_t> cnt((size_t)kNumPivots * M, 0);
    for (int64_t i = 0; i < ns; i++) {
      for (int m = 0; m < M; m++) {
        const int c = assign[(size_t)i * M + m];
        cnt[(size_t)c * M + m]++;
        for (int j = t.chunk_offsets[(size_t)m]; j < t.chunk_offsets[(size_t)m + 1]; j++)
          sum[(size_t)c * dim + j] += (double)xs[(size_t)i * dim + j] - (double)t.centroid[(size_t)j];
      }
    }
    for (int m = 0; m < M; m++) {
      for (int c = 0; c < kNumPivots; c++) {
        const int64_t k = cnt[(size_t)c * M + m];
        for (int j = t.chunk_offsets[(size_t)m]; j < t.chunk_offsets[(size_t)m + 1]; j++) {
          if (k == 0) {
            const int64_t pick = (int64_t)(rng_u64(prm.seed, 400 + (uint64_t)m, (uint64_t)(it * 256 + c)) % (uint64_t)ns);
            t.pivots[(size_t)c * dim + j] = (float)xs[(size_t)pick * dim + j] - t.centroid[(size_t)j];
          } else {
            t.pivots[(size_t)c * dim + j] = (float)(sum[(size_t)c * dim + j] / (double)k);
          }
        }
      }
    }
  }
  HIP_OK(hipMemcpy(d_piv, t.pivots.data(), sizeof(float) * t.pivots.size(), hipMemcpyHostToDevice));
  uint8_t* d_codes = nullptr;
  HIP_OK(hipMalloc(&d_codes, (size_t)n * M));
  hipLaunchKernelGGL((pq_assign_kernel<T, uint8_t>), dim3((unsigned)std::min(grid_of(n, 256), 16384), (unsigned)M),
                     dim3(256), lds, st, d_base, dim, nullptr, n, d_cent, d_off, M, d_piv, d_codes);
  HIP_OK(hipGetLastError());
  t.codes.resize((size_t)n * M);
  HIP_OK(hipMemcpyAsync(t.codes.data(), d_codes, (size_t)n * M, hipMemcpyDeviceToHost, st));
  HIP_OK(hipStreamSynchronize(st));
  hipFree(d_codes);
  hipFree(d_rows);
  hipFree(d_off);
  hipFree(d_assign);
  hipFree(d_cent);
  hipFree(d_piv);
  t.pivots_t.assign((size_t)dim * kNumPivots, 0.f);
  for (int c = 0; c < kNumPivots; c++)
    for (int j = 0; j < dim; j++) t.pivots_t[(size_t)j * kNumPivots + c] = t.pivots[(size_t)c * dim + j];
}

template <class T>
int64_t medoid_gpu(const T* d_base, int64_t n, int dim, hipStream_t st) {
  const int64_t rpb = 4096;
  const int64_t nblk = (n + rpb - 1) / rpb;
  double* d_part = nullptr;
  HIP_OK(hipMalloc(&d_part, sizeof(double) * (size_t)(nblk * dim)));
  hipLaunchKernelGGL(mean_partial_kernel<T>, dim3((unsigned)nblk), dim3(128), 0, st, d_base, n, dim, rpb, d_part);
  HIP_OK(hipGetLastError());
  std::vector<double> part((size_t)(nblk * dim));
  HIP_OK(hipMemcpyAsync(part.data(), d_part, sizeof(double) * part.size(), hipMemcpyDeviceToHost, st));
  HIP_OK(hipStreamSynchronize(st));
  hipFree(d_part);
  std::vector<float> mean((size_t)dim);
  for (int j = 0; j < dim; j++) {
    double s = 0.0;
    for (int64_t b = 0; b < nblk; b++) s += part[(size_t)(b * dim + j)];
    mean[(size_t)j] = (float)(s / (double)n);
  }
  float* d_mean = nullptr;
  unsigned long long* d_best = nullptr;
  HIP_OK(hipMalloc(&d_mean, sizeof(float) * (size_t)dim));
  HIP_OK(hipMalloc(&d_best, sizeof(unsigned long long)));
  HIP_OK(hipMemcpy(d_mean, mean.data(), sizeof(float) * (size_t)dim, hipMemcpyHostToDevice));
  HIP_OK(hipMemsetAsync(d_best, 0xff, sizeof(unsigned long long), st));
  hipLaunchKernelGGL(nearest_kernel<T>, dim3((unsigned)grid_of(n, 256)), dim3(256), 0, st, d_base, n, dim, d_mean,
                     d_best);
  HIP_OK(hipGetLastError());
  unsigned long long best = 0;
  HIP_OK(hipMemcpyAsync(&best, d_best, sizeof(best), hipMemcpyDeviceToHost, st));
  HIP_OK(hipStreamSynchronize(st));
  hipFree(d_mean);
  hipFree(d_best);
  return (int64_t)(best & 0xffffffffull);
}

struct DevBuf {
  void* p = nullptr;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  template <class U>
  U* as() const {
    return static_cast<U*>(p);
  }
};

template <class T>
qv_index* build_gpu_t(const T* d_base, int dtype, int64_t n, int dim, const qv_build_params& prm, int device) {
  hipStream_t st;
  HIP_OK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  std::unique_ptr<std::remove_pointer<hipStream_t>::type, void (*)(hipStream_t)> sg(
      st, [](hipStream_t s) { (void)hipStreamDestroy(s); });
  const auto t_start = std::chrono::steady_clock::now();

  PQTables pq;
  train_pq_gpu<T>(d_base, n, dim, prm, pq, st);
  const int64_t medoid = medoid_gpu<T>(d_base, n, dim, st);

  Layout lay;
  lay.data_type = dtype;
  lay.num_data = n;
  lay.num_dims = dim;
  lay.max_m0 = prm.R;
  lay.enter_point = medoid;
  lay.data_size = (int64_t)dim * (int64_t)sizeof(T);
  lay.node_size = lay.data_size + 4 + 4ll * prm.R;
  if (lay.node_size > kPageSize) fail(QV_EINVAL, "node record exceeds one 4 KB page");
  if (lay.data_size % 4) fail(QV_EUNSUPPORTED, "vector bytes must be a multiple of 4");
  lay.nodes_per_page = kPageSize / lay.node_size;
  lay.num_pages = (n + lay.nodes_per_page - 1) / lay.nodes_per_page;

  uint8_t* d_pages = nullptr;
  uint8_t* d_codes = nullptr;
  HIP_OK(hipMalloc(&d_pages, (size_t)(lay.num_pages * kPageSize)));
  HIP_OK(hipMalloc(&d_codes, std::max<size_t>((size_t)n * pq.num_chunks, 64)));
  HIP_OK(hipMemsetAsync(d_pages, 0, (size_t)(lay.num_pages * kPageSize), st));
  HIP_OK(hipMemcpy(d_codes, pq.codes.data(), (size_t)n * pq.num_chunks, hipMemcpyHostToDevice));
  GLayout G{d_pages, n, lay.nodes_per_page, lay.node_size, lay.data_size, dim, prm.R};
  hipLaunchKernelGGL(init_pages_kernel<T>, dim3((unsigned)grid_of(n * (lay.data_size / 4 + 1), 256)), dim3(256), 0,
                     st, G, d_base);
  HIP_OK(hipGetLastError());
  HIP_OK(hipStreamSynchronize(st));
  std::unique_ptr<qv_index, void (*)(qv_index*)> ix(make_index(device, lay, pq, d_pages, d_codes, false),
                                                     release_index);

  // insertion order: seeded Fisher-Yates
  std::vector<int32_t> order((size_t)n);
  std::iota(order.begin(), order.end(), 0);
  for (int64_t i = n - 1; i > 0; i--) {
    const int64_t j = (int64_t)(rng_u64(prm.seed, 21, (uint64_t)i) % (uint64_t)(i + 1));
    std::swap(order[(size_t)i], order[(size_t)j]);
  }
  const int64_t max_batch = std::max<int64_t>(1024, std::min<int64_t>(262144, n / 40));
  const int rec_cap = 256;
  DevBuf d_order, d_q, d_rec, d_recd, d_hops, d_pairs, d_sorted, d_heads, d_cnt, d_tmp;
  HIP_OK(hipMalloc(&d_order.p, sizeof(int32_t) * (size_t)n));
  HIP_OK(hipMemcpy(d_order.p, order.data(), sizeof(int32_t) * (size_t)n, hipMemcpyHostToDevice));
  HIP_OK(hipMalloc(&d_q.p, sizeof(float) * (size_t)(max_batch * dim)));
  HIP_OK(hipMalloc(&d_rec.p, sizeof(int32_t) * (size_t)(max_batch * rec_cap)));
  HIP_OK(hipMalloc(&d_recd.p, sizeof(float) * (size_t)(max_batch * rec_cap)));
  HIP_OK(hipMalloc(&d_hops.p, sizeof(int32_t) * (size_t)max_batch));
  HIP_OK(hipMalloc(&d_pairs.p, sizeof(uint64_t) * (size_t)(max_batch * prm.R)));
  HIP_OK(hipMalloc(&d_sorted.p, sizeof(uint64_t) * (size_t)(max_batch * prm.R)));
  HIP_OK(hipMalloc(&d_heads.p, sizeof(int32_t) * (size_t)(max_batch * prm.R)));
  HIP_OK(hipMalloc(&d_cnt.p, 64));
  // graph slack (DiskANN's GRAPH_SLACK_FACTOR 1.3): up to P reverse edges per
  // node wait beside its record's R slots until a prune folds them in
  const int P = (int)std::ceil(0.3 * prm.R);
  DevBuf d_pend, d_pcnt, d_marks, d_flush;
  HIP_OK(hipMalloc(&d_pend.p, sizeof(uint32_t) * (size_t)n * (size_t)P));
  HIP_OK(hipMalloc(&d_pcnt.p, sizeof(int32_t) * (size_t)n));
  HIP_OK(hipMemsetAsync(d_pcnt.p, 0, sizeof(int32_t) * (size_t)n, st));
  HIP_OK(hipMalloc(&d_marks.p, sizeof(int32_t) * (size_t)(max_batch * prm.R)));
  HIP_OK(hipMalloc(&d_flush.p, sizeof(int32_t) * (size_t)n));
  size_t tmp_bytes = 0;
  HIP_OK(rocprim::radix_sort_keys(nullptr, tmp_bytes, d_pairs.as<uint64_t>(), d_sorted.as<uint64_t>(),
                                  (size_t)(max_batch * prm.R), 0, 64, st));
  HIP_OK(hipMalloc(&d_tmp.p, tmp_bytes));

  // Prune wave geometry: rows of `stride` dwords (16-byte pieces, an odd
  // number of them, so 16 lanes reading 16 different rows hit distinct banks),
  // G lanes per cooperative row fetch, and the largest candidate capacity
  // that keeps 4 waves per CU (2 for long rows).
  const int ds4 = (int)(lay.data_size / 4);
  int stride4 = (ds4 + 3) / 4;
  if (stride4 % 2 == 0) stride4++;
  const int stride = 4 * stride4;
  int fetch_lanes = 4;
  while (fetch_lanes < 64 && fetch_lanes * 4 < ds4) fetch_lanes *= 2;
  int lds_cu = 0;
  HIP_OK(hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, device));
  auto waves_at = [&](int c) {
    const int bytes = (prune_lds_plan(c, stride, prm.R).total + 1023) & ~1023;
    return lds_cu / bytes;
  };
  int cmax = 256;
  while (cmax > 192 && waves_at(cmax) < 4) cmax -= 8;
  if (waves_at(cmax) < 4) {
    cmax = 256;
    while (cmax > 64 && waves_at(cmax) < 2) cmax -= 8;
  }
  const size_t prune_lds = (size_t)prune_lds_plan(cmax, stride, prm.R).total;
  HIP_OK(hipFuncSetAttribute(reinterpret_cast<const void*>(prune_kernel<T>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)prune_lds));

  const int passes = std::max(1, std::min(2, prm.passes));
  // QV_BUILD_PROGRESS=1: a progress line on stderr at most every 10 s (long builds)
  const bool progress = std::getenv("QV_BUILD_PROGRESS") != nullptr;
  auto last_note = std::chrono::steady_clock::now();
  for (int pass = 0; pass < passes; pass++) {
    const float alpha = (passes == 2 && pass == 0) ? 1.0f : prm.alpha;
    int64_t done = 0, bsz = 1;
    while (done < n) {
      const int64_t nb = std::min(n - done, pass == 0 ? std::min(bsz, max_batch) : max_batch);
      const int32_t* ids = d_order.as<int32_t>() + done;
      hipLaunchKernelGGL(gather_rows_f32<T>, dim3((unsigned)grid_of(nb * dim, 256)), dim3(256), 0, st, d_base, dim,
                         ids, nb, d_q.as<float>());
      HIP_OK(hipGetLastError());
      HIP_OK(hipStreamSynchronize(st));
      SearchRecord rec;
      rec.ids = d_rec.as<int32_t>();
      rec.dists = d_recd.as<float>();
      rec.cap = rec_cap;
      search_record(ix.get(), d_q.as<float>(), nb, std::min(prm.L, kMaxEfShared), rec, d_hops.as<int32_t>(), 0);

      PruneArgs pa{};
      pa.L = G;
      pa.mode = 0;
      pa.centers = ids;
      pa.num_centers = nb;
      pa.rec_ids = d_rec.as<int32_t>();
      pa.hops = d_hops.as<int32_t>();
      pa.rec_cap = rec_cap;
      pa.pend = d_pend.as<uint32_t>();
      pa.pcnt = d_pcnt.as<int32_t>();
      pa.P = P;
      pa.alpha = alpha;
      pa.cmax = cmax;
      pa.stride = stride;
      pa.G = fetch_lanes;
      hipLaunchKernelGGL(prune_kernel<T>, dim3((unsigned)std::min<int64_t>(nb, 65536)), dim3(64), prune_lds, st, pa);
      HIP_OK(hipGetLastError());

      HIP_OK(hipMemsetAsync(d_cnt.p, 0, 64, st));
      const int64_t np = nb * prm.R;
      hipLaunchKernelGGL(emit_pairs_kernel, dim3((unsigned)grid_of(np, 256)), dim3(256), 0, st, G, ids, nb,
                         d_pairs.as<uint64_t>(), d_cnt.as<unsigned long long>());
      HIP_OK(hipGetLastError());
      HIP_OK(rocprim::radix_sort_keys(d_tmp.p, tmp_bytes, d_pairs.as<uint64_t>(), d_sorted.as<uint64_t>(),
                                      (size_t)np, 0, 64, st));
      unsigned long long nvalid = 0;
      HIP_OK(hipMemcpyAsync(&nvalid, d_cnt.p, sizeof(nvalid), hipMemcpyDeviceToHost, st));
      HIP_OK(hipStreamSynchronize(st));
      if (nvalid > 0) {
        unsigned int* d_nh = reinterpret_cast<unsigned int*>(d_cnt.as<char>() + 32);
        unsigned int* d_nm = reinterpret_cast<unsigned int*>(d_cnt.as<char>() + 40);
        HIP_OK(hipMemsetAsync(d_nh, 0, 16, st));
        hipLaunchKernelGGL(heads_kernel, dim3((unsigned)grid_of((int64_t)nvalid, 256)), dim3(256), 0, st,
                           d_sorted.as<uint64_t>(), (int64_t)nvalid, d_heads.as<int32_t>(), d_nh);
        HIP_OK(hipGetLastError());
        unsigned int nheads = 0;
        HIP_OK(hipMemcpyAsync(&nheads, d_nh, 4, hipMemcpyDeviceToHost, st));
        HIP_OK(hipStreamSynchronize(st));
        // append reverse edges where the list or its slack has room; mark the rest
        hipLaunchKernelGGL(reverse_insert_kernel, dim3((unsigned)std::min<unsigned>(nheads, 65536u)), dim3(64), 0,
                           st, G, d_sorted.as<uint64_t>(), d_heads.as<int32_t>(), (int64_t)nheads,
                           (int64_t)nvalid, d_pend.as<uint32_t>(), d_pcnt.as<int32_t>(), P,
                           d_marks.as<int32_t>(), d_nm);
        HIP_OK(hipGetLastError());
        unsigned int nmarks = 0;
        HIP_OK(hipMemcpyAsync(&nmarks, d_nm, 4, hipMemcpyDeviceToHost, st));
        HIP_OK(hipStreamSynchronize(st));
        if (nmarks > 0) {
          PruneArgs ra = pa;
          ra.mode = 1;
          ra.centers = nullptr;
          ra.num_centers = nmarks;
          ra.pairs = d_sorted.as<uint64_t>();
          ra.heads = d_heads.as<int32_t>();
          ra.marks = d_marks.as<int32_t>();
          ra.num_pairs = (int64_t)nvalid;
          hipLaunchKernelGGL(prune_kernel<T>, dim3((unsigned)std::min<unsigned>(nmarks, 65536u)), dim3(64),
                             prune_lds, st, ra);
          HIP_OK(hipGetLastError());
          HIP_OK(hipStreamSynchronize(st));
        }
      }
      done += nb;
      bsz = std::min<int64_t>(bsz * 2, max_batch);  // capped: no overflow on long builds
      if (progress && std::chrono::steady_clock::now() - last_note > std::chrono::seconds(10)) {
        last_note = std::chrono::steady_clock::now();
        std::fprintf(stderr, "[qv build] pass %d/%d: %lld of %lld points inserted\n", pass + 1, passes,
                     (long long)done, (long long)n);
        std::fflush(stderr);
      }
    }
    // end of the pass: fold every node's pending edges into its list (DiskANN's
    // final prune of lists longer than R)
    unsigned int* d_nf = reinterpret_cast<unsigned int*>(d_cnt.as<char>() + 48);
    HIP_OK(hipMemsetAsync(d_nf, 0, 4, st));
    hipLaunchKernelGGL(pending_nodes_kernel, dim3((unsigned)grid_of(n, 256)), dim3(256), 0, st,
                       d_pcnt.as<int32_t>(), n, d_flush.as<int32_t>(), d_nf);
    HIP_OK(hipGetLastError());
    unsigned int nflush = 0;
    HIP_OK(hipMemcpyAsync(&nflush, d_nf, 4, hipMemcpyDeviceToHost, st));
    HIP_OK(hipStreamSynchronize(st));
    if (nflush > 0) {
      PruneArgs fa{};
      fa.L = G;
      fa.mode = 2;
      fa.centers = d_flush.as<int32_t>();
      fa.num_centers = nflush;
      fa.pend = d_pend.as<uint32_t>();
      fa.pcnt = d_pcnt.as<int32_t>();
      fa.P = P;
      fa.alpha = alpha;
      fa.cmax = cmax;
      fa.stride = stride;
      fa.G = fetch_lanes;
      hipLaunchKernelGGL(prune_kernel<T>, dim3((unsigned)std::min<unsigned>(nflush, 65536u)), dim3(64), prune_lds,
                         st, fa);
      HIP_OK(hipGetLastError());
      HIP_OK(hipStreamSynchronize(st));
    }
  }
  (void)t_start;
  return ix.release();
}

}  // namespace

extern "C" {

int qv_build_index_gpu(const void* d_base, int32_t data_type, int64_t n, int32_t dim,
                       const qv_build_params* params, int device, qv_index** out) {
  return qv::guard([&] {
    if (!d_base || !out || dim <= 0) qv::fail(QV_EINVAL, "bad argument");
    *out = nullptr;
    if (n <= 1 || n > (int64_t)INT32_MAX - 64) qv::fail(QV_EINVAL, "n must be in [2, 2^31 - 64)");
    qv_build_params p;
    qv_build_params_default(&p);
    if (params) p = *params;
    if (p.R <= 0 || p.R > kMaxBuildDegree) qv::fail(QV_EINVAL, "R must be in [1, 128]");
    if (p.L < p.R) qv::fail(QV_EINVAL, "L must be >= R");
    HIP_OK(hipSetDevice(device));
    if (data_type == QV_UINT8)
      *out = build_gpu_t<uint8_t>(static_cast<const uint8_t*>(d_base), data_type, n, dim, p, device);
    else if (data_type == QV_INT8)
      *out = build_gpu_t<int8_t>(static_cast<const int8_t*>(d_base), data_type, n, dim, p, device);
    else if (data_type == QV_FLOAT)
      *out = build_gpu_t<float>(static_cast<const float*>(d_base), data_type, n, dim, p, device);
    else
      qv::fail(QV_EINVAL, "bad data type");
    qv::validate_graph(*out);
  });
}

int qv_ground_truth(const void* d_base, int32_t data_type, int64_t n, int32_t dim, const float* d_queries,
                    int64_t nq, int32_t k, int32_t* d_ids, float* d_dists, int device) {
  return qv::guard([&] {
    if (!d_base || !d_queries || !d_ids || !d_dists) qv::fail(QV_EINVAL, "null argument");
    if (k <= 0 || k > 64 || n <= 0 || n > INT32_MAX || nq <= 0 || dim <= 0) qv::fail(QV_EINVAL, "bad shape");
    if ((dim * (data_type == QV_FLOAT ? 4 : 1)) % 4) qv::fail(QV_EUNSUPPORTED, "row bytes must be a multiple of 4");
    HIP_OK(hipSetDevice(device));
    hipStream_t st;
    HIP_OK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    if (data_type == QV_UINT8)
      ground_truth_t<uint8_t>(static_cast<const uint8_t*>(d_base), n, dim, d_queries, nq, k, d_ids, d_dists, st);
    else if (data_type == QV_INT8)
      ground_truth_t<int8_t>(static_cast<const int8_t*>(d_base), n, dim, d_queries, nq, k, d_ids, d_dists, st);
    else
      ground_truth_t<float>(static_cast<const float*>(d_base), n, dim, d_queries, nq, k, d_ids, d_dists, st);
    HIP_OK(hipStreamDestroy(st));
  });
}

}  // extern "C"
