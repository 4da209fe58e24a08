// qv_adc.hip -- LUT build and ADC gather-sum + top-k kernels in isolation, and
// the counter-based synthetic-data fills.
//
// The ADC kernel is the fused gather-sum of persistent_merge_data
// (src/quiver/kernel_core/kernel_helpers.cuh:271-287) detached from graph
// traversal: each workgroup owns one query, stages its 32-48 KB LUT in LDS once,
// and four waves stream 64 code rows per step (one row per lane, 16-byte
// vector loads), summing each row in the reference's sequential order.
#include <cmath>
#include <cstring>

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

constexpr int kAdcWaves = 4;
constexpr int kAdcUnroll = 4;

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

template <int MC>
__global__ __launch_bounds__(kAdcWaves * 64) void adc_bench_kernel(
    const float* __restrict__ luts, int M, const uint8_t* __restrict__ codes,
    const int32_t* __restrict__ ids, int64_t per_q, int k, int32_t* __restrict__ out_ids,
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
  uint64_t tk = kPadKey;
  double sum = 0.0;
  const int64_t steps = (per_q + kWave - 1) / kWave;
  for (int64_t h0 = (int64_t)wave * kAdcUnroll; h0 < steps; h0 += kAdcWaves * kAdcUnroll) {
    int32_t id[kAdcUnroll];
#pragma unroll
    for (int u = 0; u < kAdcUnroll; u++) {
      const int64_t s = (h0 + u) * kWave + lane;
      id[u] = (h0 + u < steps && s < per_q) ? qids[s] : -1;
    }
    float d[kAdcUnroll];
#pragma unroll
    for (int u = 0; u < kAdcUnroll; u++)
      d[u] = id[u] >= 0 ? adc_row<MC>(codes + (int64_t)id[u] * M, lut, M) : 0.f;
#pragma unroll
    for (int u = 0; u < kAdcUnroll; u++) {
      const int64_t s = (h0 + u) * kWave + lane;
      uint64_t key = kPadKey;
      if (id[u] >= 0) {
        key = bench_key(d[u], (uint32_t)s);
        sum += (double)d[u];
      }
      if (h0 + u < steps) topk_offer(tk, k, key);
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
    (void)num_codes;  // ids are trusted to be < num_codes (the fill guarantees it)
    HIP_OK(hipSetDevice(device));
    const size_t lds = (size_t)M * kPivots * 4 + kAdcWaves * kWave * 8 + kAdcWaves * kWave * 8;
    void (*k)(const float*, int, const uint8_t*, const int32_t*, int64_t, int, int32_t*, float*, double*) =
        M == 32 ? adc_bench_kernel<32> : (M == 48 ? adc_bench_kernel<48> : adc_bench_kernel<0>);
    if (lds > 65536)
      HIP_OK(hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    HIP_OK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(k, dim3((unsigned)nq), dim3(kAdcWaves * 64), lds, 0, d_luts, M, d_codes, d_ids,
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
