// qv_adc.hip -- LUT build and ADC gather-sum + top-k kernels in isolation, and
// the counter-based synthetic-data fills.
//
// The ADC kernel is the fused gather-sum of persistent_merge_data
// (src/quiver/kernel_core/kernel_helpers.cuh:271-287) detached from graph
// traversal: each workgroup owns one query, stages its 32-48 KB LUT in LDS once,
// and four waves stream 64 code rows per step (one row per lane, 16-byte
// vector loads), summing each row in the reference's sequential order.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "qv_common.hpp"
#include "qv_device.hpp"
#include "qv_hip_util.hpp"
#include "qv_mixture.hpp"

using namespace qv;
using namespace qv::dev;

namespace {

// One 64-lane workgroup per query; the LUT is accumulated in registers and
// written to HBM.  Same arithmetic as the search kernel's LDS build.
__global__ __launch_bounds__(64) void lut_kernel(const float* __restrict__ centroid,
                                                 const float* __restrict__ pivots_t,
                                                 const int32_t* __restrict__ chunk_off, int dim,
                                                 int M, const float* __restrict__ queries,
                                                 float* __restrict__ luts, float* __restrict__ q_used) {
  extern __shared__ __align__(16) char smem[];
  float* qc = reinterpret_cast<float*>(smem);
  const int64_t q = blockIdx.x;
  const int lane = lane_id();
  for (int i = lane; i < dim; i += kWave) {
    const float c = queries[q * dim + i] - centroid[i];
    qc[i] = c;
    if (q_used) q_used[q * dim + i] = c + centroid[i];
  }
  __syncthreads();
  build_lut_lds(qc, pivots_t, chunk_off, M, luts + q * (int64_t)M * kPivots);
}

constexpr int kAdcWaves = 8;   // waves per query workgroup, sharing one LDS LUT

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint64_t bench_key(float d, uint32_t s) {
  return ((uint64_t)__float_as_uint(d) << 32) | s;
}

// Inserts key k into the ascending top-k held by lanes [0, k).
__device__ __forceinline__ void topk_key_insert(uint64_t& tk, int k, uint64_t key) {
  const int lane = lane_id();
  const int pos = __popcll(__ballot(lane < k && tk < key));
  const uint64_t prev = ((uint64_t)(uint32_t)__shfl_up((int)(uint32_t)(tk >> 32), 1) << 32) |
                        (uint32_t)__shfl_up((int)(uint32_t)tk, 1);
  if (lane < k) {
    if (lane == pos) tk = key;
    else if (lane > pos) tk = prev;
  }
}

__device__ __forceinline__ uint64_t lane_bcast64(uint64_t v, int l) {
  return ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(v >> 32), l) << 32) | (uint32_t)__shfl((int)(uint32_t)v, l);
}

__device__ __forceinline__ void topk_offer(uint64_t& tk, int k, uint64_t key) {
  uint64_t cand = __ballot(key < lane_bcast64(tk, k - 1));
  while (cand) {
    const int l = __ffsll((long long)cand) - 1;
    cand &= cand - 1;
    const uint64_t ck = lane_bcast64(key, l);
    if (ck < lane_bcast64(tk, k - 1)) topk_key_insert(tk, k, ck);
  }
}

// Ids of one step: lane l owns positions s0 + PER*l .. s0 + PER*l + PER-1 (-1 past the end).
template <int PER>
__device__ __forceinline__ i32x4 load_ids(const int32_t* __restrict__ qids, int64_t per_q, int64_t s0,
                                          bool vec_ok) {
  const int64_t s = s0 + (int64_t)lane_id() * PER;
  i32x4 r = {-1, -1, -1, -1};
  if (vec_ok && s + PER <= per_q) {
    if constexpr (PER == 4) {
      r = *reinterpret_cast<const i32x4*>(qids + s);
    } else {
      const int2 v = *reinterpret_cast<const int2*>(qids + s);
      r[0] = v.x;
      r[1] = v.y;
    }
  } else {
    for (int u = 0; u < PER; u++)
      if (s + u < per_q) r[u] = qids[s + u];
  }
  return r;
}

template <int MC, int PER>
struct Rows {
  u32x4 v[PER][MC / 16];
};

// Code rows of one step.  32-byte rows are fetched by lane pairs: in each load
// instruction the even lane reads the first and the odd lane the second half of
// the same row, so every row is one 32-byte access of one instruction (random
// rows cost one cache-line access each instead of two); a DPP swap inside the
// pair then gives each lane its own full row.  Other widths load whole rows per
// lane.  Rows outside [0, last_row] are never read: padding lanes load row 0.
template <int MC, int PER>
__device__ __forceinline__ void load_rows(Rows<MC, PER>& rw, const uint8_t* __restrict__ codes, const i32x4& id,
                                          int64_t last_row) {
  if constexpr (MC == 32) {
    const bool odd = lane_id() & 1;
#pragma unroll
    for (int u = 0; u < PER; u++) {
      const int32_t row = (int32_t)min((int64_t)(id[u] < 0 ? 0 : id[u]), last_row);
      const int32_t prow = __builtin_amdgcn_update_dpp(0, row, 0xB1, 0xF, 0xF, false);  // partner lane's row
      const int64_t re = odd ? prow : row;  // the even lane's row
      const int64_t ro = odd ? row : prow;  // the odd lane's row
      const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes + re * 32) + (odd ? 1 : 0));
      const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes + ro * 32) + (odd ? 1 : 0));
      u32x4 sa, sb;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        sa[c] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a[c], 0xB1, 0xF, 0xF, false);
        sb[c] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)b[c], 0xB1, 0xF, 0xF, false);
      }
      rw.v[u][0] = odd ? sb : a;
      rw.v[u][1] = odd ? b : sa;
    }
  } else {
#pragma unroll
    for (int u = 0; u < PER; u++) {
      const int64_t row = min((int64_t)(id[u] < 0 ? 0 : id[u]), last_row);
      const u32x4* r = reinterpret_cast<const u32x4*>(codes + row * MC);
#pragma unroll
      for (int t = 0; t < MC / 16; t++) rw.v[u][t] = __builtin_nontemporal_load(r + t);
    }
  }
}

// Sequential fp32 ADC of a code row held in registers (kernel_helpers.cuh:280-285).
template <int MC>
__device__ __forceinline__ float adc_regs(const u32x4 (&w)[MC / 16], const float* __restrict__ lut) {
  float dist = 0.f;
#pragma unroll
  for (int j = 0; j < MC; j++) {
    const uint32_t word = w[j >> 4][(j >> 2) & 3];
    dist += lut[j * kPivots + (int)((word >> ((j & 3) * 8)) & 0xffu)];
  }
  return dist;
}

// One workgroup per query.  Code rows of the next step are requested before the
// current step is summed, so every wave keeps two steps of row loads in flight.
template <int MC, int PER>
__global__ __launch_bounds__(kAdcWaves * 64) void adc_bench_kernel(
    const float* __restrict__ luts, int M, const uint8_t* __restrict__ codes,
    int64_t num_codes, const int32_t* __restrict__ ids, int64_t per_q, int k, int32_t* __restrict__ out_ids,
    float* __restrict__ out_dists, double* __restrict__ dist_sums) {
  extern __shared__ __align__(16) char smem[];
  float* lut = reinterpret_cast<float*>(smem);
  uint64_t* xk = reinterpret_cast<uint64_t*>(smem + (size_t)M * kPivots * 4);
  double* xs = reinterpret_cast<double*>(xk + kAdcWaves * kWave);
  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;

  const float4* src = reinterpret_cast<const float4*>(luts + q * (int64_t)M * kPivots);
  float4* dst = reinterpret_cast<float4*>(lut);
  for (int i = tid; i < M * kPivots / 4; i += kAdcWaves * kWave) dst[i] = src[i];
  __syncthreads();

  const int32_t* qids = ids + q * per_q;
  constexpr int kAdcStep = kWave * PER;
  const bool vec_ok = (per_q % PER) == 0;
  uint64_t tk = kPadKey;
  double sum = 0.0;
  const int64_t steps = (per_q + kAdcStep - 1) / kAdcStep;
  if constexpr (MC > 0 && MC % 16 == 0) {
    int64_t st = wave;
    i32x4 id_cur = {-1, -1, -1, -1};
    Rows<MC, PER> cur;
    if (st < steps) {
      id_cur = load_ids<PER>(qids, per_q, st * kAdcStep, vec_ok);
      load_rows<MC, PER>(cur, codes, id_cur, num_codes - 1);
    }
    for (; st < steps; st += kAdcWaves) {
      const int64_t nx = st + kAdcWaves;
      i32x4 id_nxt = {-1, -1, -1, -1};
      Rows<MC, PER> nxt;
      if (nx < steps) {
        id_nxt = load_ids<PER>(qids, per_q, nx * kAdcStep, vec_ok);
        load_rows<MC, PER>(nxt, codes, id_nxt, num_codes - 1);
      }
#pragma unroll
      for (int u = 0; u < PER; u++) {
        uint64_t key = kPadKey;
        if (id_cur[u] >= 0) {
          const float d = adc_regs<MC>(cur.v[u], lut);
          sum += (double)d;
          key = bench_key(d, (uint32_t)(st * kAdcStep + lane * PER + u));
        }
        topk_offer(tk, k, key);
      }
      id_cur = id_nxt;
      cur = nxt;
    }
  } else {
    for (int64_t st = wave; st < steps; st += kAdcWaves) {
      const i32x4 id = load_ids<PER>(qids, per_q, st * kAdcStep, vec_ok);
#pragma unroll
      for (int u = 0; u < PER; u++) {
        uint64_t key = kPadKey;
        if (id[u] >= 0) {
          const float d = adc_row<0>(codes + min((int64_t)id[u], num_codes - 1) * M, lut, M);
          sum += (double)d;
          key = bench_key(d, (uint32_t)(st * kAdcStep + lane * PER + u));
        }
        topk_offer(tk, k, key);
      }
    }
  }
  xk[wave * kWave + lane] = lane < k ? tk : kPadKey;
  xs[tid] = sum;
  __syncthreads();
  if (wave == 0) {
    for (int w = 1; w < kAdcWaves; w++) topk_offer(tk, k, xk[w * kWave + lane]);
    if (lane < k) {
      const bool ok = tk != kPadKey;
      const uint32_t s = (uint32_t)tk;
      out_ids[q * k + lane] = ok ? qids[s] : -1;
      out_dists[q * k + lane] = ok ? key_dist(tk) : __int_as_float(0x7f800000);
    }
    if (dist_sums && lane == 0) {
      double t = 0.0;
      for (int i = 0; i < kAdcWaves * kWave; i++) t += xs[i];
      dist_sums[q] = t;
    }
  }
}

// Random 32-byte row gather with nothing else: lane pairs read the two halves
// of row ids[i] in one instruction, as the ADC kernel does, and XOR-fold them
// into one word per workgroup.  Its row rate is the ceiling of the ADC gather.
__global__ __launch_bounds__(256) void gather_kernel(const uint8_t* __restrict__ rows, int64_t last_row,
                                                     const int32_t* __restrict__ ids, int64_t n,
                                                     uint32_t* __restrict__ fold) {
  __shared__ uint32_t part[4];
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t i = t >> 1;
  uint32_t x = 0;
  if (i < n) {
    const int64_t row = min((int64_t)max(ids[i], 0), last_row);
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rows + row * 32) + (t & 1));
    x = a[0] ^ a[1] ^ a[2] ^ a[3];
  }
  for (int off = 32; off > 0; off >>= 1) x ^= (uint32_t)__shfl_xor((int)x, off);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) fold[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// The same gather for rows of ROW bytes (ROW / 16 lanes per row, one 16-byte
// piece each): row = id >> shift, clamped to the table, so one id array
// addresses uniformly random rows of any width over one table.  Comparing
// widths at the same row count separates a per-row cost from a per-byte one.
template <int ROW>
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint8_t* __restrict__ rows, int64_t last_row,
                                                          const int32_t* __restrict__ ids, int64_t n, int shift,
                                                          uint32_t* __restrict__ fold) {
  constexpr int kLanes = ROW / 16;
  __shared__ uint32_t part[4];
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t i = t / kLanes;
  uint32_t x = 0;
  if (i < n) {
    const int64_t row = min((int64_t)(max(ids[i], 0) >> shift), last_row);
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rows + row * ROW) + (t % kLanes));
    x = a[0] ^ a[1] ^ a[2] ^ a[3];
  }
  for (int off = 32; off > 0; off >>= 1) x ^= (uint32_t)__shfl_xor((int)x, off);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) fold[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// Streaming read of nwords 16-byte words (grid-stride, four loads in flight
// per thread), XOR-folded into one word per workgroup: the device's sequential
// read bandwidth, the measured counterpart of the nominal HBM peak.
// Random row gather of a configurable shape, for the access-rate matrix: rows
// of ROW bytes (ROW / 16 lanes per row, 16 bytes each), PER rows requested per
// lane group before any is used, nontemporal (NT) or default loads.  Row id i
// is (ids[i] * row_mul) >> 32: ids uniform over [0, id_range) land uniformly
// in the table's rows when row_mul = floor(rows * 2^32 / id_range).  The grid
// is persistent (as many workgroups as are resident); each wave XOR-folds
// what it read into fold[0].
template <int ROW, int PER, bool NT>
__global__ __launch_bounds__(256) void gather_sweep_kernel(const uint8_t* __restrict__ table, uint64_t row_mul,
                                                           uint64_t last_row, const int32_t* __restrict__ ids,
                                                           int64_t n, uint32_t* __restrict__ fold) {
  constexpr int kLanes = ROW / 16;
  constexpr int kGroups = 256 / kLanes;  // rows per workgroup per request round
  const int g = (int)threadIdx.x / kLanes, part = (int)threadIdx.x % kLanes;
  const int64_t rounds_stride = (int64_t)gridDim.x * kGroups;
  uint32_t x = 0;
  for (int64_t base = (int64_t)blockIdx.x * kGroups + g; base < n; base += rounds_stride * PER) {
    u32x4 v[PER];
#pragma unroll
    for (int p = 0; p < PER; p++) {
      const int64_t i = min(base + p * rounds_stride, n - 1);
      const uint64_t row = min(((uint64_t)(uint32_t)ids[i] * row_mul) >> 32, last_row);
      const u32x4* ptr = reinterpret_cast<const u32x4*>(table + row * ROW) + part;
      v[p] = NT ? __builtin_nontemporal_load(ptr) : *ptr;
    }
#pragma unroll
    for (int p = 0; p < PER; p++)
      if (base + p * rounds_stride < n) x ^= v[p][0] ^ v[p][1] ^ v[p][2] ^ v[p][3];
  }
  for (int off = 32; off > 0; off >>= 1) x ^= (uint32_t)__shfl_xor((int)x, off);
  if ((threadIdx.x & 63) == 0) atomicXor(fold, x);
}

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src, int64_t nwords,
                                                          uint32_t* __restrict__ fold) {
  __shared__ uint32_t part[4];
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t w = (int64_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t x = 0;
  for (; w + 3 * stride < nwords; w += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(src + w);
    const u32x4 b = __builtin_nontemporal_load(src + w + stride);
    const u32x4 c = __builtin_nontemporal_load(src + w + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(src + w + 3 * stride);
    x ^= (a[0] ^ a[1] ^ a[2] ^ a[3]) ^ (b[0] ^ b[1] ^ b[2] ^ b[3]) ^ (c[0] ^ c[1] ^ c[2] ^ c[3]) ^
         (d[0] ^ d[1] ^ d[2] ^ d[3]);
  }
  for (; w < nwords; w += stride) {
    const u32x4 a = __builtin_nontemporal_load(src + w);
    x ^= a[0] ^ a[1] ^ a[2] ^ a[3];
  }
  for (int off = 32; off > 0; off >>= 1) x ^= (uint32_t)__shfl_xor((int)x, off);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) fold[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// Device-to-device copy of 16-byte words (grid-stride); also the reference
// kernel of known traffic against which HBM byte counters are scaled.
__global__ __launch_bounds__(256) void copy_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                   int64_t nwords) {
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < nwords;
       w += (int64_t)gridDim.x * blockDim.x)
    dst[w] = src[w];
}

__global__ void fill_bytes_kernel(uint8_t* dst, int64_t nbytes, uint64_t seed) {
  const int64_t nw = (nbytes + 7) / 8;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < nw;
       w += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t h = rng_u64(seed, kStreamBytes, (uint64_t)w);
    if (w * 8 + 8 <= nbytes) {
      reinterpret_cast<uint64_t*>(dst)[w] = h;
    } else {
      for (int b = 0; w * 8 + b < nbytes; b++) dst[w * 8 + b] = (uint8_t)(h >> (8 * b));
    }
  }
}

__global__ void fill_ids_kernel(int32_t* dst, int64_t count, uint32_t num_codes, uint64_t seed) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = (int32_t)rng_below(rng_u64(seed, kStreamIds, (uint64_t)i), num_codes);
}

__global__ void mixture_u8_kernel(qv_mixture m, int64_t first, int64_t rows, uint8_t* dst) {
  const int64_t total = rows * m.dim;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / m.dim;
    const int32_t j = (int32_t)(e - r * m.dim);
    dst[e] = mixture_u8(m.seed, m.num_centers, m.dim, m.center_lo, m.center_hi, m.sigma, first + r, j);
  }
}

__global__ void mixture_f32_kernel(qv_mixture m, int64_t first, int64_t rows, float* dst) {
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows;
       r += (int64_t)gridDim.x * blockDim.x) {
    float* row = dst + r * m.dim;
    double ss = 0.0;
    for (int j = 0; j < m.dim; j++) {
      const float v = mixture_f32_raw(m.seed, m.num_centers, m.dim, m.sigma, first + r, j);
      row[j] = v;
      const double dv = (double)v;
      ss = ss + dv * dv;
    }
    if (m.normalize) {
      const double inv = 1.0 / sqrt(ss);
      for (int j = 0; j < m.dim; j++) row[j] = (float)((double)row[j] * inv);
    }
  }
}

int grid_for(int64_t work, int block) {
  const int64_t g = (work + block - 1) / block;
  return (int)std::max<int64_t>(1, std::min<int64_t>(g, 1 << 20));
}

}  // namespace

extern "C" {

int qv_lut_build_raw(const float* d_centroid, const float* d_pivots_t, const int32_t* d_chunk_offsets,
                     int32_t dim, int32_t num_chunks, const float* d_queries, int64_t nq,
                     float* d_luts, float* d_q_used, int device) {
  return qv::guard([&] {
    if (!d_centroid || !d_pivots_t || !d_chunk_offsets || !d_queries || !d_luts)
      qv::fail(QV_EINVAL, "null argument");
    if (dim <= 0 || num_chunks <= 0 || nq <= 0 || nq > INT32_MAX) qv::fail(QV_EINVAL, "bad shape");
    HIP_OK(hipSetDevice(device));
    hipLaunchKernelGGL(lut_kernel, dim3((unsigned)nq), dim3(64), (size_t)dim * 4, 0, d_centroid,
                       d_pivots_t, d_chunk_offsets, dim, num_chunks, d_queries, d_luts, d_q_used);
    HIP_OK(hipGetLastError());
    HIP_OK(hipDeviceSynchronize());
  });
}

int qv_adc_bench(const float* d_luts, int32_t M, const uint8_t* d_codes, int64_t num_codes,
                 const int32_t* d_ids, int64_t nq, int64_t ids_per_query, int32_t topk,
                 int32_t* d_out_ids, float* d_out_dists, double* d_dist_sums, int device,
                 float* elapsed_ms) {
  return qv::guard([&] {
    if (!d_luts || !d_codes || !d_ids || !d_out_ids || !d_out_dists) qv::fail(QV_EINVAL, "null argument");
    if (M <= 0 || M > 128 || num_codes <= 0 || nq <= 0 || nq > INT32_MAX || ids_per_query <= 0 ||
        ids_per_query > UINT32_MAX)
      qv::fail(QV_EINVAL, "bad shape");
    if (topk <= 0 || topk > 64) qv::fail(QV_EINVAL, "topk must be in [1, 64]");
    HIP_OK(hipSetDevice(device));
    const size_t lds = (size_t)M * kPivots * 4 + kAdcWaves * kWave * 8 + kAdcWaves * kWave * 8;
    if (reinterpret_cast<uintptr_t>(d_ids) & 15) qv::fail(QV_EINVAL, "ids must be 16-byte aligned");
    // ids per lane per step: 2 keeps two steps of code rows in flight within
    // 64 VGPRs (8 waves per SIMD); 4 doubles the rows per step at 5 waves per SIMD
    int per = 2;
    if (const char* e = std::getenv("QV_ADC_IDS_PER_LANE")) per = std::atoi(e) == 4 ? 4 : 2;
    void (*k)(const float*, int, const uint8_t*, int64_t, const int32_t*, int64_t, int, int32_t*, float*,
              double*) =
        M == 32 ? (per == 4 ? adc_bench_kernel<32, 4> : adc_bench_kernel<32, 2>)
                : (M == 48 ? (per == 4 ? adc_bench_kernel<48, 4> : adc_bench_kernel<48, 2>)
                           : adc_bench_kernel<0, 2>);
    if (lds > 65536)
      HIP_OK(hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    HIP_OK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(k, dim3((unsigned)nq), dim3(kAdcWaves * 64), lds, 0, d_luts, M, d_codes, num_codes, d_ids,
                       ids_per_query, topk, d_out_ids, d_out_dists, d_dist_sums);
    HIP_OK(hipGetLastError());
    HIP_OK(hipEventRecord(e1, 0));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (elapsed_ms) *elapsed_ms = ms;
  });
}

int qv_gather_bench(const uint8_t* d_rows, int64_t num_rows, const int32_t* d_ids, int64_t n, uint32_t* d_fold,
                    int device, float* elapsed_ms) {
  return qv::guard([&] {
    if (!d_rows || !d_ids || !d_fold || num_rows <= 0 || n <= 0 || n > ((int64_t)1 << 36))
      qv::fail(QV_EINVAL, "bad argument");
    if ((reinterpret_cast<uintptr_t>(d_rows) & 15) != 0) qv::fail(QV_EINVAL, "rows must be 16-byte aligned");
    HIP_OK(hipSetDevice(device));
    const int64_t blocks = (2 * n + 255) / 256;
    if (blocks > INT32_MAX) qv::fail(QV_EINVAL, "too many rows");
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    HIP_OK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(gather_kernel, dim3((unsigned)blocks), dim3(256), 0, 0, d_rows, num_rows - 1, d_ids, n, d_fold);
    HIP_OK(hipGetLastError());
    HIP_OK(hipEventRecord(e1, 0));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (elapsed_ms) *elapsed_ms = ms;
  });
}

int qv_gather_sweep_bench(const uint8_t* d_table, int64_t table_rows, int32_t row_bytes, const int32_t* d_ids,
                          int64_t n, int64_t id_range, int32_t rows_in_flight, int32_t waves_per_cu,
                          int32_t nontemporal, uint32_t* d_fold, int device, float* elapsed_ms,
                          int32_t* waves_launched) {
  return qv::guard([&] {
    if (!d_table || !d_ids || !d_fold || n <= 0 || n > ((int64_t)1 << 34) || table_rows < 1 ||
        table_rows >= ((int64_t)1 << 32) || id_range < 1 || id_range > ((int64_t)1 << 32))
      qv::fail(QV_EINVAL, "bad argument");
    if (row_bytes != 32 && row_bytes != 64 && row_bytes != 128 && row_bytes != 256)
      qv::fail(QV_EINVAL, "row_bytes must be 32, 64, 128 or 256");
    if (rows_in_flight != 1 && rows_in_flight != 2 && rows_in_flight != 4)
      qv::fail(QV_EINVAL, "rows_in_flight must be 1, 2 or 4");
    if (waves_per_cu != 8 && waves_per_cu != 16 && waves_per_cu != 32)
      qv::fail(QV_EINVAL, "waves_per_cu must be 8, 16 or 32");
    if ((reinterpret_cast<uintptr_t>(d_table) & 15) != 0) qv::fail(QV_EINVAL, "table must be 16-byte aligned");
    // row = (id * row_mul) >> 32 < table_rows for every id < id_range
    const uint64_t row_mul = (uint64_t)(((unsigned __int128)table_rows << 32) / (unsigned __int128)id_range);
    if (row_mul == 0) qv::fail(QV_EINVAL, "table has fewer rows than the id range can spread over");
    HIP_OK(hipSetDevice(device));
    hipDeviceProp_t prop;
    HIP_OK(hipGetDeviceProperties(&prop, device));
    int lds_cu = 0;
    HIP_OK(hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, device));
    // waves per CU set through LDS: four-wave workgroups, waves_per_cu / 4 of
    // them fit a CU's LDS
    const int wgs = waves_per_cu / 4;
    const size_t lds = (size_t)(lds_cu / wgs) & ~(size_t)255;
    using Kern = void (*)(const uint8_t*, uint64_t, uint64_t, const int32_t*, int64_t, uint32_t*);
    Kern kern = nullptr;
    auto pick = [&](auto rowc, auto perc) {
      constexpr int R = decltype(rowc)::value, P = decltype(perc)::value;
      kern = nontemporal ? gather_sweep_kernel<R, P, true> : gather_sweep_kernel<R, P, false>;
    };
    auto by_per = [&](auto rowc) {
      if (rows_in_flight == 1) pick(rowc, std::integral_constant<int, 1>{});
      else if (rows_in_flight == 2) pick(rowc, std::integral_constant<int, 2>{});
      else pick(rowc, std::integral_constant<int, 4>{});
    };
    if (row_bytes == 32) by_per(std::integral_constant<int, 32>{});
    else if (row_bytes == 64) by_per(std::integral_constant<int, 64>{});
    else if (row_bytes == 128) by_per(std::integral_constant<int, 128>{});
    else by_per(std::integral_constant<int, 256>{});
    HIP_OK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)lds));
    int per_cu = 0;
    HIP_OK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern), 256, lds));
    if (per_cu < 1) qv::fail(QV_EHIP, "gather sweep kernel does not fit on a compute unit");
    per_cu = std::min(per_cu, wgs);
    const int grid = per_cu * prop.multiProcessorCount;
    if (waves_launched) *waves_launched = grid * 4;
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    HIP_OK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, 0, d_table, row_mul, (uint64_t)(table_rows - 1), d_ids, n,
                       d_fold);
    HIP_OK(hipGetLastError());
    HIP_OK(hipEventRecord(e1, 0));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (elapsed_ms) *elapsed_ms = ms;
  });
}

int qv_gather_rows_bench(const uint8_t* d_table, int64_t table_bytes, int32_t row_bytes, const int32_t* d_ids,
                         int64_t n, int32_t id_shift, uint32_t* d_fold, int device, float* elapsed_ms) {
  return qv::guard([&] {
    if (!d_table || !d_ids || !d_fold || n <= 0 || n > ((int64_t)1 << 34) || id_shift < 0 || id_shift > 30)
      qv::fail(QV_EINVAL, "bad argument");
    if (row_bytes != 32 && row_bytes != 64 && row_bytes != 128 && row_bytes != 256)
      qv::fail(QV_EINVAL, "row_bytes must be 32, 64, 128 or 256");
    if ((reinterpret_cast<uintptr_t>(d_table) & 15) != 0) qv::fail(QV_EINVAL, "table must be 16-byte aligned");
    const int64_t num_rows = table_bytes / row_bytes;
    if (num_rows < 1) qv::fail(QV_EINVAL, "table smaller than one row");
    HIP_OK(hipSetDevice(device));
    const int64_t blocks = (n * (row_bytes / 16) + 255) / 256;
    if (blocks > INT32_MAX) qv::fail(QV_EINVAL, "too many rows");
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    HIP_OK(hipEventRecord(e0, 0));
    auto launch = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, 0, d_table, num_rows - 1, d_ids, n, id_shift,
                         d_fold);
    };
    if (row_bytes == 32) launch(gather_rows_kernel<32>);
    else if (row_bytes == 64) launch(gather_rows_kernel<64>);
    else if (row_bytes == 128) launch(gather_rows_kernel<128>);
    else launch(gather_rows_kernel<256>);
    HIP_OK(hipGetLastError());
    HIP_OK(hipEventRecord(e1, 0));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (elapsed_ms) *elapsed_ms = ms;
  });
}

int qv_stream_read_bench(const uint8_t* d_src, int64_t nbytes, uint32_t* d_fold, int device, float* elapsed_ms) {
  return qv::guard([&] {
    if (!d_src || !d_fold || nbytes < 16 || (nbytes & 15) != 0) qv::fail(QV_EINVAL, "bad argument");
    if ((reinterpret_cast<uintptr_t>(d_src) & 15) != 0) qv::fail(QV_EINVAL, "source must be 16-byte aligned");
    HIP_OK(hipSetDevice(device));
    const int64_t nwords = nbytes / 16;
    const int64_t blocks = std::min<int64_t>(QV_STREAM_READ_BLOCKS, (nwords + 255) / 256);
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    HIP_OK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(256), 0, 0,
                       reinterpret_cast<const u32x4*>(d_src), nwords, d_fold);
    HIP_OK(hipGetLastError());
    HIP_OK(hipEventRecord(e1, 0));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (elapsed_ms) *elapsed_ms = ms;
  });
}

int qv_fill_uniform_bytes(uint8_t* d_dst, int64_t nbytes, uint64_t seed, int device) {
  return qv::guard([&] {
    if (!d_dst || nbytes < 0) qv::fail(QV_EINVAL, "bad argument");
    HIP_OK(hipSetDevice(device));
    hipLaunchKernelGGL(fill_bytes_kernel, dim3(grid_for((nbytes + 7) / 8, 256)), dim3(256), 0, 0, d_dst,
                       nbytes, seed);
    HIP_OK(hipGetLastError());
    HIP_OK(hipDeviceSynchronize());
  });
}

int qv_fill_uniform_ids(int32_t* d_dst, int64_t count, int64_t num_codes, uint64_t seed, int device) {
  return qv::guard([&] {
    if (!d_dst || count < 0 || num_codes <= 0 || num_codes > INT32_MAX) qv::fail(QV_EINVAL, "bad argument");
    HIP_OK(hipSetDevice(device));
    hipLaunchKernelGGL(fill_ids_kernel, dim3(grid_for(count, 256)), dim3(256), 0, 0, d_dst, count,
                       (uint32_t)num_codes, seed);
    HIP_OK(hipGetLastError());
    HIP_OK(hipDeviceSynchronize());
  });
}

int qv_mixture_fill_device(const qv_mixture* m, int64_t first_row, int64_t rows, void* d_dst, int device) {
  return qv::guard([&] {
    if (!m || !d_dst || rows < 0 || m->dim <= 0 || m->num_centers <= 0) qv::fail(QV_EINVAL, "bad argument");
    HIP_OK(hipSetDevice(device));
    if (m->data_type == QV_UINT8) {
      hipLaunchKernelGGL(mixture_u8_kernel, dim3(grid_for(rows * m->dim, 256)), dim3(256), 0, 0, *m,
                         first_row, rows, static_cast<uint8_t*>(d_dst));
    } else if (m->data_type == QV_FLOAT) {
      hipLaunchKernelGGL(mixture_f32_kernel, dim3(grid_for(rows, 128)), dim3(128), 0, 0, *m, first_row,
                         rows, static_cast<float*>(d_dst));
    } else {
      qv::fail(QV_EINVAL, "mixture data_type must be uint8 or float");
    }
    HIP_OK(hipGetLastError());
    HIP_OK(hipDeviceSynchronize());
  });
}

int qv_device_info(int device, char* name, int32_t name_len, int32_t* num_cus, int64_t* total_mem) {
  return qv::guard([&] {
    int n = 0;
    HIP_OK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) qv::fail(QV_EINVAL, "device not present");
    hipDeviceProp_t p;
    HIP_OK(hipGetDeviceProperties(&p, device));
    if (name && name_len > 0) {
      std::strncpy(name, p.gcnArchName, (size_t)name_len - 1);
      name[name_len - 1] = 0;
    }
    if (num_cus) *num_cus = p.multiProcessorCount;
    if (total_mem) *total_mem = (int64_t)p.totalGlobalMem;
  });
}

int qv_device_mem_info(int device, int64_t* free_bytes, int64_t* total_bytes) {
  return qv::guard([&] {
    int n = 0;
    HIP_OK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) qv::fail(QV_EINVAL, "device not present");
    HIP_OK(hipSetDevice(device));
    size_t f = 0, t = 0;
    HIP_OK(hipMemGetInfo(&f, &t));
    if (free_bytes) *free_bytes = (int64_t)f;
    if (total_bytes) *total_bytes = (int64_t)t;
  });
}

int qv_device_count(int32_t* count) {
  return qv::guard([&] {
    if (!count) qv::fail(QV_EINVAL, "null argument");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = (e == hipSuccess) ? n : 0;
  });
}

int qv_dev_alloc(int device, int64_t bytes, void** out) {
  return qv::guard([&] {
    if (!out || bytes <= 0) qv::fail(QV_EINVAL, "bad argument");
    HIP_OK(hipSetDevice(device));
    *out = nullptr;
    HIP_OK(hipMalloc(out, (size_t)bytes));
  });
}

int qv_dev_free(void* ptr) {
  return qv::guard([&] { HIP_OK(hipFree(ptr)); });
}

int qv_dev_copy(void* dst, const void* src, int64_t bytes, int32_t kind) {
  return qv::guard([&] {
    if (bytes < 0 || (bytes > 0 && (!dst || !src))) qv::fail(QV_EINVAL, "bad argument");
    if (bytes == 0) return;
    hipPointerAttribute_t da{}, sa{};
    if (kind == 2 && ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) | (uintptr_t)bytes) & 15) == 0 &&
        hipPointerGetAttributes(&da, dst) == hipSuccess && hipPointerGetAttributes(&sa, src) == hipSuccess &&
        da.type == hipMemoryTypeDevice && sa.type == hipMemoryTypeDevice && da.device == sa.device) {
      // device to device on one GPU, 16-byte aligned: one copy kernel
      HIP_OK(hipSetDevice(da.device));
      const int64_t nwords = bytes / 16;
      const int64_t blocks = std::min<int64_t>((nwords + 255) / 256, 8192);
      hipLaunchKernelGGL(copy_kernel, dim3((unsigned)blocks), dim3(256), 0, 0, reinterpret_cast<uint4*>(dst),
                         reinterpret_cast<const uint4*>(src), nwords);
      HIP_OK(hipGetLastError());
      HIP_OK(hipDeviceSynchronize());
      return;
    }
    const hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice
                                      : (kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice);
    HIP_OK(hipMemcpy(dst, src, (size_t)bytes, k));
  });
}

int qv_dev_clear(void* ptr, int64_t bytes) {
  return qv::guard([&] {
    if (bytes < 0 || (bytes > 0 && !ptr)) qv::fail(QV_EINVAL, "bad argument");
    if (bytes == 0) return;
    HIP_OK(hipMemset(ptr, 0, (size_t)bytes));
    HIP_OK(hipDeviceSynchronize());
  });
}

}  // extern "C"
