// qv_device.hpp -- wave64 building blocks of the CDNA4 search path.
//
// One query is served by one 64-lane wavefront.  Lane l owns neighbour l of the
// node being expanded (R <= 64): its ADC gather-sum, its beam-membership test and
// its key.  The per-query LUT lives in LDS for the whole query; the beam lives in
// LDS and, chunk-major, in registers.
//
// Candidate keys are 64-bit: (fp32 bits of the PQ distance) << 32 |
// (id & 0x7fffffff) << 1 | (unvisited ? 1 : 0).  Distances are sums of squares,
// hence non-negative, so unsigned key order is the reference's (dist, id) order
// (pair_less, src/quiver/kernel_core/kernel_helpers.cuh:106-114), with a visited
// copy of an id ordered before an unvisited copy -- the position the reference's
// merge gives the beam's own entry (kernel_helpers.cuh:331-335).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace qv {
namespace dev {

constexpr int kWave = 64;
constexpr uint64_t kPadKey = ~0ull;
constexpr int kPivots = 256;

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ uint64_t make_key(float dist, uint32_t id, bool visited) {
  return ((uint64_t)__float_as_uint(dist) << 32) | ((uint64_t)(id & 0x7fffffffu) << 1) |
         (visited ? 0ull : 1ull);
}
__device__ __forceinline__ uint32_t key_id(uint64_t k) { return ((uint32_t)k) >> 1; }
__device__ __forceinline__ bool key_unvisited(uint64_t k) { return (k & 1ull) != 0; }
__device__ __forceinline__ float key_dist(uint64_t k) { return __uint_as_float((uint32_t)(k >> 32)); }

// Sentinel of an empty neighbour slot: (+inf, 0xffffffff - lane), as the
// reference pads lanes >= degree (kernel_helpers.cuh:273-277).
__device__ __forceinline__ uint64_t sentinel_key(int lane) {
  return make_key(__int_as_float(0x7f800000), 0xffffffffu - (uint32_t)lane, false);
}

// ---- wave64 exchange primitives ------------------------------------------
// DPP controls (GFX9): quad_perm [1,0,3,2] = 0xB1 (xor 1), [2,3,0,1] = 0x4E
// (xor 2), row_ror:8 = 0x128 (xor 8 inside a 16-lane row), wave_shr:1 = 0x138.
// ds_swizzle bit mode (and 0x1F, xor m) for xor 4 / 16 inside 32 lanes;
// ds_bpermute for xor 32.  Uniform-lane reads use v_readlane.
template <int M>
__device__ __forceinline__ uint32_t xor_lane32(uint32_t v, int lane) {
  if constexpr (M == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
  } else if constexpr (M == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
  } else if constexpr (M == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);
  } else if constexpr (M == 4 || M == 16) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x1F | (M << 10));
  } else {
    return (uint32_t)__builtin_amdgcn_ds_bpermute((lane ^ M) << 2, (int)v);
  }
}

template <int M>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v, int lane) {
  const uint32_t lo = xor_lane32<M>((uint32_t)v, lane);
  const uint32_t hi = xor_lane32<M>((uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

// Value of lane i-1 (lane 0 keeps its own value).
__device__ __forceinline__ uint32_t lane_up1_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x138, 0xF, 0xF, false);
}
__device__ __forceinline__ float lane_up1_f32(float v) { return __uint_as_float(lane_up1_u32(__float_as_uint(v))); }

// Value held by lane l (l wave-uniform).
__device__ __forceinline__ uint32_t read_lane_u32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ int32_t read_lane_i32(int32_t v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float read_lane_f32(float v, int l) {
  return __uint_as_float(read_lane_u32(__float_as_uint(v), l));
}
__device__ __forceinline__ uint64_t read_lane_u64(uint64_t v, int l) {
  return ((uint64_t)read_lane_u32((uint32_t)(v >> 32), l) << 32) | read_lane_u32((uint32_t)v, l);
}

// Element i of a query.  The queries of a host-buffer call sit in pinned
// host memory that the host fills while the kernel runs, so they are read at
// system scope (relaxed: coherent with the host's writes, no cache holding an
// older copy, no fence); each element is read once per query.
__device__ __forceinline__ float query_elem(const float* q, int i) {
  return __uint_as_float(__hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<float*>(q)) + i, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_SYSTEM));
}

// LDS byte address of a pointer into the dynamic LDS area, and the 8-byte
// word at byte address min(a, lim) + 8 OFF: one v_min against a wave-uniform
// bound, the offset in the instruction (min(x + k, t) = min(x, t - k) + k).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
template <int OFF>
__device__ __forceinline__ uint64_t lds_u64_min(uint32_t a, uint32_t lim) {
  const uint32_t m = min(a, lim);
  return ((const __attribute__((address_space(3))) uint64_t*)(uintptr_t)m)[OFF];
}

// Sum of v over the lanes below this one: an inclusive scan within each row of
// 16 lanes (DPP row_shr 1, 2, 4, 8; lanes shifted in from outside the row
// read 0), then lane 15 of rows 0 and 2 added to rows 1 and 3 (row_bcast:15)
// and lane 31 to rows 2 and 3 (row_bcast:31); rows a broadcast does not
// write keep the 0 given as the old value.
__device__ __forceinline__ uint32_t wave_excl_sum(uint32_t v) {
  int x = (int)v;
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
  return (uint32_t)x - v;
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = (uint32_t)__shfl_xor((int)lo, m);
  hi = (uint32_t)__shfl_xor((int)hi, m);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t umin64(uint64_t a, uint64_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a < b ? b : a; }

// Lane id the compiler cannot treat as loop-invariant: comparisons derived
// from it are recomputed where they are used instead of being hoisted into
// dozens of live 64-bit lane masks (which spill scalar registers).
__device__ __forceinline__ int opaque_lane() {
  int lane = lane_id();
  asm volatile("" : "+v"(lane));
  return lane;
}

// Compare-exchange of one bitonic stage (partner lane ^ J) for an ascending
// block when `up`.  Partners 16 and 32 apart are exchanged with the CDNA4
// permlane swaps, which hand both lanes of a pair the keys (A, B) of the lane
// with bit J clear and the lane with bit J set; the other distances use DPP or
// swizzle through xor_lane64.
template <int J>
__device__ __forceinline__ uint64_t cx_stage(uint64_t key, int lane, bool up) {
  if constexpr (J == 16 || J == 32) {
    const uint32_t lo = (uint32_t)key, hi = (uint32_t)(key >> 32);
    uint32_t alo, blo, ahi, bhi;
    if constexpr (J == 16) {
      const auto pl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
      const auto ph = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
      alo = pl[0]; blo = pl[1]; ahi = ph[0]; bhi = ph[1];
    } else {
      const auto pl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
      const auto ph = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
      alo = pl[0]; blo = pl[1]; ahi = ph[0]; bhi = ph[1];
    }
    const uint64_t A = ((uint64_t)ahi << 32) | alo;
    const uint64_t B = ((uint64_t)bhi << 32) | blo;
    const bool want_min = ((lane & J) == 0) == up;
    return ((A < B) == want_min) ? A : B;
  } else {
    const uint64_t other = xor_lane64<J>(key, lane);
    const bool lower = (lane & J) == 0;
    return (lower == up) ? umin64(key, other) : umax64(key, other);
  }
}

// Bitonic sort of one key per lane, descending across the wave (keys distinct).
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t key) {
  const int lane = opaque_lane();
#define QV_STAGE(K, J) key = cx_stage<J>(key, lane, (lane & (K)) != 0)
  QV_STAGE(2, 1);
  QV_STAGE(4, 2); QV_STAGE(4, 1);
  QV_STAGE(8, 4); QV_STAGE(8, 2); QV_STAGE(8, 1);
  QV_STAGE(16, 8); QV_STAGE(16, 4); QV_STAGE(16, 2); QV_STAGE(16, 1);
  QV_STAGE(32, 16); QV_STAGE(32, 8); QV_STAGE(32, 4); QV_STAGE(32, 2); QV_STAGE(32, 1);
  QV_STAGE(64, 32); QV_STAGE(64, 16); QV_STAGE(64, 8); QV_STAGE(64, 4); QV_STAGE(64, 2); QV_STAGE(64, 1);
#undef QV_STAGE
  return key;
}

// Minimum of one 64-bit value per lane, returned to every lane (uniform).
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t x) {
  const int lane = opaque_lane();
  x = umin64(x, xor_lane64<1>(x, lane));
  x = umin64(x, xor_lane64<2>(x, lane));
  x = umin64(x, xor_lane64<4>(x, lane));
  x = umin64(x, xor_lane64<8>(x, lane));
  const uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
  const auto pl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const auto ph = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  x = umin64(((uint64_t)ph[0] << 32) | pl[0], ((uint64_t)ph[1] << 32) | pl[1]);
  const uint32_t lo2 = (uint32_t)x, hi2 = (uint32_t)(x >> 32);
  const auto ql = __builtin_amdgcn_permlane32_swap(lo2, lo2, false, false);
  const auto qh = __builtin_amdgcn_permlane32_swap(hi2, hi2, false, false);
  // read back from lane 0 so the compiler sees a wave-uniform value
  return read_lane_u64(umin64(((uint64_t)qh[0] << 32) | ql[0], ((uint64_t)qh[1] << 32) | ql[1]), 0);
}

// Minimum of one 32-bit value per lane, returned to every lane (uniform):
// DPP steps inside each 16-lane row (quad_perm swaps, then rotations by 4 and
// 8), then the permlane swaps across rows; VALU only, no LDS.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  x = min(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, true));   // quad_perm [1,0,3,2]
  x = min(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, true));   // quad_perm [2,3,0,1]
  x = min(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x124, 0xF, 0xF, true));  // row_ror:4
  x = min(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xF, 0xF, true));  // row_ror:8
  const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = min(p[0], p[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return read_lane_u32(min(q[0], q[1]), 0);
}

// The smallest key among the lanes where `valid` holds (at least one), and a
// lane holding it (*at).  Keys order by their distance word first, so the
// minimum distance word and one ballot usually settle it; only equal distance
// words in two or more valid lanes take the full 64-bit minimum.
__device__ __forceinline__ uint64_t wave_min_key(uint64_t key, bool valid, int* at) {
  const uint32_t hi = (uint32_t)(key >> 32);
  const uint32_t m = wave_min_u32(valid ? hi : 0xffffffffu);
  const uint64_t b = __ballot(valid && hi == m);
  if ((b & (b - 1)) == 0) {
    *at = __ffsll((long long)b) - 1;
    return read_lane_u64(key, *at);
  }
  const uint64_t kv = wave_min_u64(valid ? key : ~0ull);
  *at = __ffsll((long long)__ballot(valid && key == kv)) - 1;
  return kv;
}

// Per-query LUT in LDS: PQSearchData::init_query (src/shared/index/
// pq_device.cuh:9-36).  Chunks are contiguous dimension ranges, so each
// (chunk, pivot) cell accumulates its dimensions in ascending order, exactly as
// the reference's i-ordered loop does; the fused multiply-add matches nvcc's
// contraction of `dist_vec[..] += dist * dist`.  Lane l owns pivots 4l..4l+3.
__device__ __forceinline__ void build_lut_lds(const float* __restrict__ qc_lds,
                                              const float* __restrict__ pivots_t,
                                              const int32_t* __restrict__ chunk_off,
                                              int num_chunks, float* __restrict__ lut) {
  const int lane = lane_id();
  for (int m = 0; m < num_chunks; m++) {
    const int o0 = chunk_off[m], o1 = chunk_off[m + 1];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int i = o0; i < o1; i++) {
      const float qi = qc_lds[i];
      const float4 p = reinterpret_cast<const float4*>(pivots_t + (size_t)i * kPivots)[lane];
      float d0 = qi - p.x, d1 = qi - p.y, d2 = qi - p.z, d3 = qi - p.w;
      acc.x = __fmaf_rn(d0, d0, acc.x);
      acc.y = __fmaf_rn(d1, d1, acc.y);
      acc.z = __fmaf_rn(d2, d2, acc.z);
      acc.w = __fmaf_rn(d3, d3, acc.w);
    }
    reinterpret_cast<float4*>(lut + m * kPivots)[lane] = acc;
  }
}

// Code row of MC bytes (MC % 16 == 0) held as MC/4 words.
template <int MC>
struct CodeRow {
  uint32_t w[MC / 4 > 0 ? MC / 4 : 1];
};

// Code row `row` (of MC bytes, MC % 16 == 0) of the table `codes` into this
// lane's registers.  Each lane loads its own row: in the latency-bound search a
// row waits for one load of its own only.
template <int MC>
__device__ __forceinline__ void adc_load(CodeRow<MC>& cr, const uint8_t* __restrict__ codes, uint32_t row) {
  const uint4* r4 = reinterpret_cast<const uint4*>(codes + (int64_t)row * MC);
#pragma unroll
  for (int t = 0; t < MC / 16; t++) {
    const uint4 v = r4[t];
    cr.w[4 * t + 0] = v.x;
    cr.w[4 * t + 1] = v.y;
    cr.w[4 * t + 2] = v.z;
    cr.w[4 * t + 3] = v.w;
  }
}

// A raw buffer descriptor for the `bytes` bytes at p, a wave-uniform
// address: loads through it take the base in scalar registers and a 32-bit
// offset per lane, so no 64-bit vector address is formed or held while they
// are in flight, and a load past `bytes` returns zero.  Word 3 is the gfx9
// raw-buffer data format (32-bit).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_at(const void* p, int bytes = 0x7fffffff) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// A code row of MC bytes at byte off of the buffer r.
template <int MC>
__device__ __forceinline__ void adc_load(CodeRow<MC>& cr, __amdgpu_buffer_rsrc_t r, uint32_t off) {
#pragma unroll
  for (int t = 0; t < MC / 16; t++) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(off + 16u * t), 0, 0);
    cr.w[4 * t + 0] = v.x;
    cr.w[4 * t + 1] = v.y;
    cr.w[4 * t + 2] = v.z;
    cr.w[4 * t + 3] = v.w;
  }
}

// The same from a row address (a row of the neighbour-code table).
template <int MC>
__device__ __forceinline__ void adc_load(CodeRow<MC>& cr, const uint8_t* __restrict__ row) {
  const uint4* r4 = reinterpret_cast<const uint4*>(row);
#pragma unroll
  for (int t = 0; t < MC / 16; t++) {
    const uint4 v = r4[t];
    cr.w[4 * t + 0] = v.x;
    cr.w[4 * t + 1] = v.y;
    cr.w[4 * t + 2] = v.z;
    cr.w[4 * t + 3] = v.w;
  }
}

template <int MC>
__device__ __forceinline__ float adc_sum(const CodeRow<MC>& cr, const float* __restrict__ lut) {
  float dist = 0.f;
#pragma unroll
  for (int j = 0; j < MC; j++) dist += lut[j * kPivots + (int)((cr.w[j >> 2] >> ((j & 3) * 8)) & 0xffu)];
  return dist;
}

// adc_sum for a LUT at LDS address 0 (the first bytes of the dynamic LDS
// area, with no static LDS before it): entry (m, c) is at byte
// 4 (STRIDE m + c) (STRIDE = 256: a packed table), so its address is one
// shift of the code byte (an SDWA source selects the byte) and the chunk's
// 4 STRIDE m is the instruction's offset.
template <int MC, int STRIDE = kPivots>
__device__ __forceinline__ float adc_sum_at0(const CodeRow<MC>& cr) {
  typedef const __attribute__((address_space(3))) float lds_f32;
  float dist = 0.f;
#pragma unroll
  for (int j = 0; j < MC; j++) {
    const uint32_t c = (cr.w[j >> 2] >> ((j & 3) * 8)) & 0xffu;
    dist += ((lds_f32*)(uintptr_t)(c << 2))[j * STRIDE];
  }
  return dist;
}

// A compile-time flag as an argument (for generic lambdas).
template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

typedef float qv_float4 __attribute__((ext_vector_type(4)));
typedef float qv_float2 __attribute__((ext_vector_type(2)));

// Query elements of the shared-pivot ADC, held in registers for the whole
// query: lane l holds q'[16 j + (l & 15)] in qd[j], so each 16-lane row of the
// wave holds the whole query.  DPP row_newbcast:i gives every lane of a row
// the value of the row's lane i, so dimension t is row_newbcast:(t & 15) of
// qd[t >> 4], read by the subtract that uses it (v_sub_f32_dpp): the query
// operand costs no LDS read and no instruction.  A group of four chunks reads
// one qd register (16 dims at SC = 4, 8 at SC = 2).

// Pivot reads of one group of four chunks (M0 .. M0 + 3, whose codes are the
// bytes of the code word w) for adc_recompute<MC, 4>, in one block so that
// the group costs one LDS round trip: per chunk, an SDWA shift (the source
// operand selects the byte) makes the address 16 c of the pivot entry (its 4
// dims contiguous, 16 bytes), which one ds_read_b128 reads at 4096 m + 16 c
// from the pivot table at LDS address 0.  The 16-bit instruction offset
// reaches chunks below 16; above, the address gets 65536 added first.  The
// block ends with its own wait, since the compiler does not count these
// reads.  dep is not read: it orders the block after the previous group's
// arithmetic, so a group's operands are the only ones held at a time.
template <int M0>
__device__ __forceinline__ void adc_group_reads(uint32_t w, float dep, qv_float4 (&pc)[4]) {
  static_assert(M0 % 4 == 0 && M0 + 3 < 32, "32 chunks of 4 KB");
  uint32_t a0, a1, a2, a3;
  if constexpr (M0 < 16) {
  asm volatile(
      "v_lshlrev_b32_sdwa %[a0], 4, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n\t"
      "v_lshlrev_b32_sdwa %[a1], 4, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n\t"
      "v_lshlrev_b32_sdwa %[a2], 4, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n\t"
      "v_lshlrev_b32_sdwa %[a3], 4, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3\n\t"
      "ds_read_b128 %[p0], %[a0] offset:%[o0]\n\t"
      "ds_read_b128 %[p1], %[a1] offset:%[o1]\n\t"
      "ds_read_b128 %[p2], %[a2] offset:%[o2]\n\t"
      "ds_read_b128 %[p3], %[a3] offset:%[o3]\n\t"
      "s_waitcnt lgkmcnt(0)"
      : [a0] "=&v"(a0), [a1] "=&v"(a1), [a2] "=&v"(a2), [a3] "=&v"(a3), [p0] "=&v"(pc[0]), [p1] "=&v"(pc[1]),
        [p2] "=&v"(pc[2]), [p3] "=&v"(pc[3])
      : [w] "v"(w), [dep] "v"(dep), [o0] "i"(4096 * M0), [o1] "i"(4096 * (M0 + 1)), [o2] "i"(4096 * (M0 + 2)),
        [o3] "i"(4096 * (M0 + 3)));
  } else {
  asm volatile(
      "v_lshlrev_b32_sdwa %[a0], 4, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n\t"
      "v_lshlrev_b32_sdwa %[a1], 4, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n\t"
      "v_lshlrev_b32_sdwa %[a2], 4, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n\t"
      "v_lshlrev_b32_sdwa %[a3], 4, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3\n\t"
      "v_add_u32 %[a0], 0x10000, %[a0]\n\t"
      "v_add_u32 %[a1], 0x10000, %[a1]\n\t"
      "v_add_u32 %[a2], 0x10000, %[a2]\n\t"
      "v_add_u32 %[a3], 0x10000, %[a3]\n\t"
      "ds_read_b128 %[p0], %[a0] offset:%[o0]\n\t"
      "ds_read_b128 %[p1], %[a1] offset:%[o1]\n\t"
      "ds_read_b128 %[p2], %[a2] offset:%[o2]\n\t"
      "ds_read_b128 %[p3], %[a3] offset:%[o3]\n\t"
      "s_waitcnt lgkmcnt(0)"
      : [a0] "=&v"(a0), [a1] "=&v"(a1), [a2] "=&v"(a2), [a3] "=&v"(a3), [p0] "=&v"(pc[0]), [p1] "=&v"(pc[1]),
        [p2] "=&v"(pc[2]), [p3] "=&v"(pc[3])
      : [w] "v"(w), [dep] "v"(dep), [o0] "i"(4096 * M0 - 65536), [o1] "i"(4096 * (M0 + 1) - 65536),
        [o2] "i"(4096 * (M0 + 2) - 65536), [o3] "i"(4096 * (M0 + 3) - 65536));
  }
}

// The arithmetic of one group of four chunks of 4 dims: per chunk, in its
// dims' order, d_k = q'_t - P[c][t] (q'_t by DPP from q, row lane t & 15),
// acc = d_0 * d_0 (the fused chain's first step from 0: fma(d, d, 0) rounds
// d * d once, as the multiply does), acc = fma(d_k, d_k, acc) for k = 1..3,
// then dist += acc -- the LUT build's entry and the table ADC's sum, bit for
// bit.  The block starts with s_nop 1: a DPP read needs two wait states after
// a VALU write of its source, and the compiler does not look inside it.
__device__ __forceinline__ float adc_math4(const qv_float4 (&pc)[4], float q, float dist) {
  float t0, t1, t2, t3, acc;
#define QV_CHUNK4(P, L0, L1, L2, L3)                                                          \
  "v_sub_f32_dpp %[t0], %[q], %[" P "x] row_newbcast:" L0 " row_mask:0xf bank_mask:0xf\n\t"  \
  "v_sub_f32_dpp %[t1], %[q], %[" P "y] row_newbcast:" L1 " row_mask:0xf bank_mask:0xf\n\t"  \
  "v_sub_f32_dpp %[t2], %[q], %[" P "z] row_newbcast:" L2 " row_mask:0xf bank_mask:0xf\n\t"  \
  "v_sub_f32_dpp %[t3], %[q], %[" P "w] row_newbcast:" L3 " row_mask:0xf bank_mask:0xf\n\t"  \
  "v_mul_f32 %[acc], %[t0], %[t0]\n\t"                                                     \
  "v_fmac_f32 %[acc], %[t1], %[t1]\n\t"                                                    \
  "v_fmac_f32 %[acc], %[t2], %[t2]\n\t"                                                    \
  "v_fmac_f32 %[acc], %[t3], %[t3]\n\t"                                                    \
  "v_add_f32 %[dist], %[dist], %[acc]\n\t"
  asm volatile("s_nop 1\n\t"
               QV_CHUNK4("p0", "0", "1", "2", "3")
               QV_CHUNK4("p1", "4", "5", "6", "7")
               QV_CHUNK4("p2", "8", "9", "10", "11")
               QV_CHUNK4("p3", "12", "13", "14", "15")
               : [dist] "+v"(dist), [t0] "=&v"(t0), [t1] "=&v"(t1), [t2] "=&v"(t2), [t3] "=&v"(t3),
                 [acc] "=&v"(acc)
               : [q] "v"(q), [p0x] "v"(pc[0].x), [p0y] "v"(pc[0].y), [p0z] "v"(pc[0].z), [p0w] "v"(pc[0].w),
                 [p1x] "v"(pc[1].x), [p1y] "v"(pc[1].y), [p1z] "v"(pc[1].z), [p1w] "v"(pc[1].w),
                 [p2x] "v"(pc[2].x), [p2y] "v"(pc[2].y), [p2z] "v"(pc[2].z), [p2w] "v"(pc[2].w),
                 [p3x] "v"(pc[3].x), [p3y] "v"(pc[3].y), [p3z] "v"(pc[3].z), [p3w] "v"(pc[3].w));
#undef QV_CHUNK4
  return dist;
}

// Groups G .. MC/4 - 1 of adc_recompute<MC, 4>: dist += LUT[m][c_m] in chunk
// order; group G's 16 dims are qd[G].
template <int G, int MC, int NQ>
__device__ __forceinline__ float adc_groups(const uint32_t* w, const float (&qd)[NQ], float dist) {
  if constexpr (4 * G >= MC) {
    return dist;
  } else {
    qv_float4 pc[4];
    adc_group_reads<4 * G>(w[G], dist, pc);
    dist = adc_math4(pc, qd[G], dist);
    return adc_groups<G + 1, MC, NQ>(w, qd, dist);
  }
}

// The same for adc_recompute<MC, 2> (M0 + 3 < 48): the pivot entry of chunk m
// (8 bytes at 2048 m + 8 c) is one ds_read_b64 from the address 8 c when its
// offset fits the instruction's 16 bits (m < 32), else one ds_read2st64_b64
// reading it twice (offsets 4 m in 512-byte units).
template <int M0>
__device__ __forceinline__ void adc_group_reads2(uint32_t w, float dep, qv_float2 (&pc)[4]) {
  static_assert(M0 % 4 == 0 && M0 + 3 < 48, "chunks of two dimensions, M <= 48");
  uint32_t a0, a1, a2, a3;
  if constexpr (M0 < 32) {
    asm volatile(
        "v_lshlrev_b32_sdwa %[a0], 3, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n\t"
        "v_lshlrev_b32_sdwa %[a1], 3, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n\t"
        "v_lshlrev_b32_sdwa %[a2], 3, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n\t"
        "v_lshlrev_b32_sdwa %[a3], 3, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3\n\t"
        "ds_read_b64 %[p0], %[a0] offset:%[o0]\n\t"
        "ds_read_b64 %[p1], %[a1] offset:%[o1]\n\t"
        "ds_read_b64 %[p2], %[a2] offset:%[o2]\n\t"
        "ds_read_b64 %[p3], %[a3] offset:%[o3]\n\t"
        "s_waitcnt lgkmcnt(0)"
        : [a0] "=&v"(a0), [a1] "=&v"(a1), [a2] "=&v"(a2), [a3] "=&v"(a3), [p0] "=&v"(pc[0]), [p1] "=&v"(pc[1]),
          [p2] "=&v"(pc[2]), [p3] "=&v"(pc[3])
        : [w] "v"(w), [dep] "v"(dep), [o0] "i"(2048 * M0), [o1] "i"(2048 * (M0 + 1)),
          [o2] "i"(2048 * (M0 + 2)), [o3] "i"(2048 * (M0 + 3)));
  } else {
    qv_float4 t0, t1, t2, t3;
    asm volatile(
        "v_lshlrev_b32_sdwa %[a0], 3, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n\t"
        "v_lshlrev_b32_sdwa %[a1], 3, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n\t"
        "v_lshlrev_b32_sdwa %[a2], 3, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n\t"
        "v_lshlrev_b32_sdwa %[a3], 3, %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3\n\t"
        "ds_read2st64_b64 %[p0], %[a0] offset0:%[o0] offset1:%[o0]\n\t"
        "ds_read2st64_b64 %[p1], %[a1] offset0:%[o1] offset1:%[o1]\n\t"
        "ds_read2st64_b64 %[p2], %[a2] offset0:%[o2] offset1:%[o2]\n\t"
        "ds_read2st64_b64 %[p3], %[a3] offset0:%[o3] offset1:%[o3]\n\t"
        "s_waitcnt lgkmcnt(0)"
        : [a0] "=&v"(a0), [a1] "=&v"(a1), [a2] "=&v"(a2), [a3] "=&v"(a3), [p0] "=&v"(t0), [p1] "=&v"(t1),
          [p2] "=&v"(t2), [p3] "=&v"(t3)
        : [w] "v"(w), [dep] "v"(dep), [o0] "i"(4 * M0), [o1] "i"(4 * (M0 + 1)), [o2] "i"(4 * (M0 + 2)),
          [o3] "i"(4 * (M0 + 3)));
    pc[0] = t0.xy;
    pc[1] = t1.xy;
    pc[2] = t2.xy;
    pc[3] = t3.xy;
  }
}

// adc_math4 for four chunks of 2 dims, whose 8 dims are row lanes B .. B + 7
// of q.
template <int B>
__device__ __forceinline__ float adc_math2(const qv_float2 (&pc)[4], float q, float dist) {
  static_assert(B == 0 || B == 8, "half a row");
  float t0, t1, acc;
#define QV_CHUNK2(P, L0, L1)                                                                   \
  "v_sub_f32_dpp %[t0], %[q], %[" P "x] row_newbcast:%[" L0 "] row_mask:0xf bank_mask:0xf\n\t" \
  "v_sub_f32_dpp %[t1], %[q], %[" P "y] row_newbcast:%[" L1 "] row_mask:0xf bank_mask:0xf\n\t" \
  "v_mul_f32 %[acc], %[t0], %[t0]\n\t"                                                      \
  "v_fmac_f32 %[acc], %[t1], %[t1]\n\t"                                                     \
  "v_add_f32 %[dist], %[dist], %[acc]\n\t"
  asm volatile("s_nop 1\n\t"
               QV_CHUNK2("p0", "l0", "l1")
               QV_CHUNK2("p1", "l2", "l3")
               QV_CHUNK2("p2", "l4", "l5")
               QV_CHUNK2("p3", "l6", "l7")
               : [dist] "+v"(dist), [t0] "=&v"(t0), [t1] "=&v"(t1), [acc] "=&v"(acc)
               : [q] "v"(q), [p0x] "v"(pc[0].x), [p0y] "v"(pc[0].y), [p1x] "v"(pc[1].x), [p1y] "v"(pc[1].y),
                 [p2x] "v"(pc[2].x), [p2y] "v"(pc[2].y), [p3x] "v"(pc[3].x), [p3y] "v"(pc[3].y), [l0] "i"(B),
                 [l1] "i"(B + 1), [l2] "i"(B + 2), [l3] "i"(B + 3), [l4] "i"(B + 4), [l5] "i"(B + 5),
                 [l6] "i"(B + 6), [l7] "i"(B + 7));
#undef QV_CHUNK2
  return dist;
}

// Groups G .. MC/4 - 1 of adc_recompute<MC, 2>; group G's 8 dims are row
// lanes 8 (G & 1) .. 8 (G & 1) + 7 of qd[G / 2].
template <int G, int MC, int NQ>
__device__ __forceinline__ float adc_groups2(const uint32_t* w, const float (&qd)[NQ], float dist) {
  if constexpr (4 * G >= MC) {
    return dist;
  } else {
    qv_float2 pc[4];
    adc_group_reads2<4 * G>(w[G], dist, pc);
    dist = adc_math2<8 * (G & 1)>(pc, qd[G / 2], dist);
    return adc_groups2<G + 1, MC, NQ>(w, qd, dist);
  }
}

// LDS float index of pivot dimension i for code c in the shared pivot table
// of adc_recompute<MC, SC>:
//  SC = 4: entry (m, c) at float (m * 256 + c) * 4, its 4 dims contiguous
//          (one ds_read_b128 in adc_group_reads);
//  SC = 2: entry (m, c) at float (m * 256 + c) * 2 (adc_group_reads2).
template <int SC>
__host__ __device__ __forceinline__ int piv_index(int i, int c) {
  const int m = i / SC, j = i % SC;
  if constexpr (SC == 4)
    return m * 1024 + c * 4 + j;
  else
    return (m * 256 + c) * SC + j;
}

// The same ADC with every LUT entry recomputed from the pivots instead of
// read from a per-query table: LUT[m][c] is the fused chain
// acc = fma(q'_i - P[c][i], q'_i - P[c][i], acc) over the SC dims i of chunk m
// from acc = 0 (the LUT build's own order), then dist += LUT[m][c] in chunk
// order, so the result is the table ADC's bit for bit.  The pivots sit in LDS
// at address 0 as piv_index<SC> places them (shared by the waves of a
// workgroup); qd holds q' as adc_math4 / adc_math2 read it (load_query_dpp).
template <int MC, int SC, int NQ>
__device__ __forceinline__ float adc_recompute(const CodeRow<MC>& cr, const float (&qd)[NQ]) {
  static_assert(MC % 4 == 0, "chunks in groups of four");
  static_assert(16 * NQ >= MC * SC, "every dimension in the query registers");
  if constexpr (SC == 4) {
    return adc_groups<0, MC, NQ>(cr.w, qd, 0.f);
  } else {
    static_assert(SC == 2, "chunks of 2 or 4 dimensions");
    return adc_groups2<0, MC, NQ>(cr.w, qd, 0.f);
  }
}

// q' (LDS, dim elements) into the registers adc_math4 / adc_math2 read: lane l takes
// element 16 j + (l & 15) into qd[j] (0 past dim).
template <int NQ>
__device__ __forceinline__ void load_query_dpp(const float* __restrict__ qc_lds, int dim, int lane,
                                               float (&qd)[NQ]) {
#pragma unroll
  for (int j = 0; j < NQ; j++) {
    const int i = 16 * j + (lane & 15);
    const float v = qc_lds[min(i, dim - 1)];
    qd[j] = i < dim ? v : 0.f;
  }
}

// Sequential fp32 ADC of one code row against an LDS LUT
// (kernel_helpers.cuh:280-285): dist = 0; dist += LUT[j][code_j] for j = 0..M-1.
template <int MC>
__device__ __forceinline__ float adc_row(const uint8_t* __restrict__ row,
                                         const float* __restrict__ lut, int M) {
  float dist = 0.f;
  if constexpr (MC > 0 && MC % 16 == 0) {
    const uint4* r4 = reinterpret_cast<const uint4*>(row);
    uint32_t w[MC / 4];
#pragma unroll
    for (int t = 0; t < MC / 16; t++) {
      const uint4 v = r4[t];
      w[4 * t + 0] = v.x;
      w[4 * t + 1] = v.y;
      w[4 * t + 2] = v.z;
      w[4 * t + 3] = v.w;
    }
#pragma unroll
    for (int j = 0; j < MC; j++) {
      uint32_t c = (w[j >> 2] >> ((j & 3) * 8)) & 0xffu;
      dist += lut[j * kPivots + (int)c];
    }
  } else {
    (void)MC;
    if ((M & 3) == 0) {
      const uint32_t* r = reinterpret_cast<const uint32_t*>(row);
      for (int t = 0; t < M / 4; t++) {
        uint32_t w = r[t];
#pragma unroll
        for (int b = 0; b < 4; b++) dist += lut[(4 * t + b) * kPivots + (int)((w >> (8 * b)) & 0xffu)];
      }
    } else {
      for (int j = 0; j < M; j++) dist += lut[j * kPivots + (int)row[j]];
    }
  }
  return dist;
}

template <class T>
__device__ __forceinline__ float elem_to_float(const uint8_t* rec, int i) {
  return (float)reinterpret_cast<const T*>(rec)[i];
}

// Elements lane + 32k (k < kVecPre) of a node vector, requested into registers
// by every lane with the index clamped into the vector (values of lanes >= 32
// and of indexes >= dim are never used), so that no load sits behind a branch
// and the loads stay in flight together with the neighbour list.
constexpr int kVecPre = 4;

template <class T>
__device__ __forceinline__ uint32_t elem_raw(const uint8_t* rec, int i) {
  if constexpr (sizeof(T) == 4) return reinterpret_cast<const uint32_t*>(rec)[i];
  else return (uint32_t)rec[i];
}

template <class T>
__device__ __forceinline__ float raw_to_float(uint32_t r) {
  if constexpr (sizeof(T) == 4) return __uint_as_float(r);
  else return (float)(T)(uint8_t)r;
}

template <class T, class R>
__device__ __forceinline__ void load_vec_pre(const uint8_t* __restrict__ rec, int dim, int lane,
                                             R (&x)[kVecPre]) {
#pragma unroll
  for (int k = 0; k < kVecPre; k++) x[k] = (R)elem_raw<T>(rec, min((lane & 31) + 32 * k, dim - 1));
}

// load_vec_pre for a dim KD known at compile time (a multiple of 32 up to
// 32 kVecPre): element (lane & 31) + 32 k for each k with 32 k < KD, at the
// lane's loop-invariant byte offset off = (lane & 31) sizeof(T) plus an
// immediate, so a request costs no address arithmetic.
template <class T, int KD, class R>
__device__ __forceinline__ void load_vec_pre_fixed(const uint8_t* __restrict__ rec, uint32_t off,
                                                   R (&x)[kVecPre]) {
  static_assert(KD % 32 == 0 && KD <= 32 * kVecPre, "whole 32-element rows");
#pragma unroll
  for (int k = 0; k < kVecPre; k++) x[k] = 32 * k < KD ? (R)elem_raw<T>(rec + off, 32 * k) : (R)0;
}

// load_vec_pre_fixed from the buffer r (a record), off = (lane & 31) sizeof(T).
template <class T, int KD, class R>
__device__ __forceinline__ void load_vec_pre_buf(__amdgpu_buffer_rsrc_t r, uint32_t off, R (&x)[kVecPre]) {
  static_assert(KD % 32 == 0 && KD <= 32 * kVecPre, "whole 32-element rows");
#pragma unroll
  for (int k = 0; k < kVecPre; k++) {
    const int o = (int)(off + 32u * k * (uint32_t)sizeof(T));
    if (32 * k >= KD)
      x[k] = (R)0;
    else if constexpr (sizeof(T) == 1)
      x[k] = (R)__builtin_amdgcn_raw_buffer_load_b8(r, o, 0, 0);
    else
      x[k] = (R)__builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0);
  }
}

// load_vec_pre from the buffer r (a record) for a dim known only at run time:
// the lane's byte offsets off[k] of elements min((lane & 31) + 32 k, dim - 1),
// computed once per query, so a request costs no address arithmetic.
template <class T, class R>
__device__ __forceinline__ void load_vec_pre_offs(__amdgpu_buffer_rsrc_t r, const uint32_t (&off)[kVecPre],
                                                  R (&x)[kVecPre]) {
#pragma unroll
  for (int k = 0; k < kVecPre; k++) {
    if constexpr (sizeof(T) == 1)
      x[k] = (R)__builtin_amdgcn_raw_buffer_load_b8(r, (int)off[k], 0, 0);
    else
      x[k] = (R)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off[k], 0, 0);
  }
}

// Query elements lane + 32k (k < kVecPre) of the first 32 lanes, kept in
// registers for the whole query (0 past dim).
__device__ __forceinline__ void load_query_pre(const float* __restrict__ qu_lds, int dim, int lane,
                                               float (&qv)[kVecPre]) {
#pragma unroll
  for (int k = 0; k < kVecPre; k++) {
    const int i = (lane & 31) + 32 * k;
    const float v = qu_lds[min(i, dim - 1)];
    qv[k] = i < dim ? v : 0.f;
  }
}

// The wave reduction of the exact distance over the lanes' sums (lanes < 32
// hold them): an exchange of lanes 16 apart inside each 32-lane half, then
// four row shifts, leave their total in lane 0 in exact_l2_ref's order.
__device__ __forceinline__ float exact_reduce(float val, int lane) {
  val += __uint_as_float(xor_lane32<16>(__float_as_uint(val), lane));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x108, 0xF, 0xF, false));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x104, 0xF, 0xF, false));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x102, 0xF, 0xF, false));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x101, 0xF, 0xF, false));
  return read_lane_f32(val, 0);
}

// exact_l2_ref with the first kVecPre elements of each lane taken from x and
// the matching query elements from qv.  Elements past dim contribute
// fma(0, 0, val) = val, so the sum is the reference's bit for bit.  Split in
// two: the lane's sum over its first kVecPre elements (exact_lane_pre), then
// the rest of its elements and the wave reduction (exact_l2_rest).
template <class T, class R>
__device__ __forceinline__ float exact_lane_pre(const R (&x)[kVecPre], const float (&qv)[kVecPre], int dim,
                                                int lane) {
  float val = 0.f;
  const bool lo = lane < 32;
#pragma unroll
  for (int k = 0; k < kVecPre; k++) {
    const int i = lane + 32 * k;
    const float diff = lo && i < dim ? qv[k] - raw_to_float<T>(x[k]) : 0.f;
    val = __fmaf_rn(diff, diff, val);
  }
  return val;
}

template <class T>
__device__ __forceinline__ float exact_l2_rest(float val, const uint8_t* __restrict__ rec,
                                               const float* __restrict__ qu_lds, int dim, int lane) {
  if (lane < 32) {
    for (int i = lane + 32 * kVecPre; i < dim; i += 32) {
      const float diff = qu_lds[i] - elem_to_float<T>(rec, i);
      val = __fmaf_rn(diff, diff, val);
    }
  }
  return exact_reduce(val, lane);
}

// exact_lane_pre for a dim KD known at compile time (a multiple of 32 up to
// 32 kVecPre): lanes < 32 accumulate the same chain as exact_lane_pre
// without its per-element tests (terms past KD would add fma(0, 0, val) =
// val), and lanes >= 32 compute values that no step of exact_reduce carries
// into lanes < 32 (the exchange stays inside 32-lane halves, the row shifts
// inside 16-lane rows), so lane 0 ends with the same sum bit for bit.
template <class T, int KD, class R>
__device__ __forceinline__ float exact_lane_fixed(const R (&x)[kVecPre], const float (&qv)[kVecPre]) {
  static_assert(KD % 32 == 0 && KD <= 32 * kVecPre, "whole 32-element rows");
  float val = 0.f;
#pragma unroll
  for (int k = 0; k < kVecPre; k++) {
    if (32 * k < KD) {
      const float diff = qv[k] - raw_to_float<T>(x[k]);
      val = __fmaf_rn(diff, diff, val);
    }
  }
  return val;
}

// Stable top-k insert (retset_push_topk_le32, kernel_helpers.cuh:65-104,
// generalised to k <= 64): lane i < k holds entry i; the value goes after every
// entry <= value; the caller applies the fc < k || value < D[k-1] guard.
__device__ __forceinline__ void topk_insert(float& td, int32_t& ti, int& fc, int k,
                                            float value, int32_t id) {
  const int lane = opaque_lane();
  uint64_t le = __ballot(lane < fc && td <= value);
  int pos = __popcll(le);
  int ns = fc < k ? fc + 1 : k;
  float pd = lane_up1_f32(td);
  int32_t pi = (int32_t)lane_up1_u32((uint32_t)ti);
  if (lane < ns) {
    if (lane == pos) {
      td = value;
      ti = id;
    } else if (lane > pos) {
      td = pd;
      ti = pi;
    }
  }
  fc = ns;
}

// ---- navigation-graph entry: inkernel_nav_entry (src/quiver/kernel_core/inkernel_nav.cuh:61-200)
// A greedy search over the small nav graph with a 32-slot queue: slots [0, 4)
// hold the best four, slots [4, 32) the neighbours of the last expanded node.
// The reference runs it with one 32-lane warp for the queue and four warps for
// the distances; here lanes 0..31 hold the slots and the two wave halves
// compute two neighbour distances at a time.
constexpr int kNavL = 4;
constexpr int kNavR = 28;
constexpr int kNavChunk = 7;  // neighbours per warp in the reference (28 over 4 warps)

// square_sum_32 (src/shared/common/gpu_primitives.cuh:26-44) of the float query
// q against vector x, per wave half: sub-lane s accumulates dimensions s, s+32,
// ... with a fused multiply-add, then the shuffle-down tree; the sum is valid
// at sub-lane 0 of each half.
template <class T>
__device__ __forceinline__ float nav_dist32(const float* __restrict__ q, const uint8_t* __restrict__ x, int dims,
                                            int lane) {
  float val = 0.f;
  for (int i = lane & 31; i < dims; i += 32) {
    const float diff = q[i] - elem_to_float<T>(x, i);
    val = __fmaf_rn(diff, diff, val);
  }
  val += __uint_as_float(xor_lane32<16>(__float_as_uint(val), lane));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x108, 0xF, 0xF, false));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x104, 0xF, 0xF, false));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x102, 0xF, 0xF, false));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x101, 0xF, 0xF, false));
  return val;
}

// The same sum with the query's elements of this sub-lane in registers (qn[k] =
// q[s + 32 k], 0 past dims) and the vector's elements already loaded (xr[k],
// any value past dims): for dims <= 32 kNavPre.  Elements past dims add
// fma(0, 0, val) = val, so the sum is nav_dist32's bit for bit.
constexpr int kNavPre = 4;
template <class T>
__device__ __forceinline__ float nav_dist32_pre(const float (&qn)[kNavPre], const uint32_t (&xr)[kNavPre],
                                                int dims, int lane) {
  float val = 0.f;
#pragma unroll
  for (int k = 0; k < kNavPre; k++) {
    const int i = (lane & 31) + 32 * k;
    const float diff = i < dims ? qn[k] - raw_to_float<T>(xr[k]) : 0.f;
    val = __fmaf_rn(diff, diff, val);
  }
  val += __uint_as_float(xor_lane32<16>(__float_as_uint(val), lane));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x108, 0xF, 0xF, false));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x104, 0xF, 0xF, false));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x102, 0xF, 0xF, false));
  val += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(val), 0x101, 0xF, 0xF, false));
  return val;
}

// Returns the mapped base id of the best nav node for query q (raw, before the
// LUT's centring).  graph is [num_node][max_m] with -1 after the degree;
// indexes past the end of graph read as -1.  With fewer than four distinct
// nodes in the queue, the last selection round swaps an empty slot into slot 0
// (all candidates +inf, the argmin stays at lane 0, and +inf != d); the
// reference then reads nav_mapping[0x7fffffff].  Here that case returns
// `fallback` (the medoid).
template <class T>
__device__ __forceinline__ int32_t nav_entry(const float* __restrict__ q, const uint8_t* __restrict__ data,
                             const int32_t* __restrict__ graph, const int32_t* __restrict__ mapping,
                             int64_t num_node, int dims, int max_m, int start, int32_t fallback) {
  const int lane = opaque_lane();
  const int half = lane >> 5;
  const int64_t row = (int64_t)dims * (int64_t)sizeof(T);
  const int64_t glen = num_node * (int64_t)max_m;
  // slot registers (lanes 0..31); unused slots carry id 0xffffffff (visited) and +inf
  uint32_t pid = 0xffffffffu;
  float pdist = __int_as_float(0x7f800000);
  {
    const float d0 = read_lane_f32(nav_dist32<T>(q, data + (int64_t)start * row, dims, lane), 0);
    if (lane == 0) {
      pid = (uint32_t)start;
      pdist = d0;
    }
  }
  // the query elements of this sub-lane, for the short-vector path
  const bool pre = dims <= 32 * kNavPre;
  float qn[kNavPre];
#pragma unroll
  for (int k = 0; k < kNavPre; k++) {
    const int i = (lane & 31) + 32 * k;
    qn[k] = query_elem(q, min(i, dims - 1));
  }
  int idx = 0;
  while (idx != -1) {
    const int u = (int)(read_lane_u32(pid, idx) & 0x7fffffffu);
    if (lane == idx) pid |= 0x80000000u;
    // Distance phase: neighbour i fills slot kNavL + i; in each 7-neighbour
    // chunk (one warp of the reference) the first -1 ends the chunk, and the
    // slots it leaves keep their values.
    const int64_t e0 = (int64_t)max_m * u;
    if (pre) {
      // The 28 reads of the row in one load (lane i reads entry i), then every
      // pair's vector elements requested before the first distance is summed.
      const int32_t gv = lane < kNavR && e0 + lane < glen ? graph[e0 + lane] : -1;
      const uint64_t neg = __ballot(lane < kNavR && gv == -1);
      uint32_t okm = 0;  // neighbour i counts iff no -1 precedes it in its chunk
#pragma unroll
      for (int c = 0; c < kNavR / kNavChunk; c++) {
        const uint32_t cm = (uint32_t)(neg >> (kNavChunk * c)) & ((1u << kNavChunk) - 1u);
        const int first = cm ? __ffs((int)cm) - 1 : kNavChunk;
        okm |= ((1u << first) - 1u) << (kNavChunk * c);
      }
      // Pairs in batches of kNavBatch: every pair of a batch has its vector
      // elements requested before the first of them is summed.
      constexpr int kNavBatch = 7;
#pragma unroll
      for (int b = 0; b < kNavR / 2; b += kNavBatch) {
        uint32_t xr[kNavBatch][kNavPre];
#pragma unroll
        for (int jj = 0; jj < kNavBatch; jj++) {
          const int j = b + jj;
          if (j >= kNavR / 2) break;
          // half h of the wave takes neighbour 2 j + h (node 0 when it does not count)
          const int32_t v0 = (okm >> (2 * j)) & 1u ? read_lane_i32(gv, 2 * j) : 0;
          const int32_t v1 = (okm >> (2 * j + 1)) & 1u ? read_lane_i32(gv, 2 * j + 1) : 0;
          load_vec_pre<T>(data + (int64_t)(half ? v1 : v0) * row, dims, lane, xr[jj]);
        }
#pragma unroll
        for (int jj = 0; jj < kNavBatch; jj++) {
          const int j = b + jj;
          if (j >= kNavR / 2) break;
          const int i0 = 2 * j, i1 = 2 * j + 1;
          const bool ok0 = (okm >> i0) & 1u, ok1 = (okm >> i1) & 1u;
          if (!ok0 && !ok1) continue;
          const float dh = nav_dist32_pre<T>(qn, xr[jj], dims, lane);
          const float d0 = read_lane_f32(dh, 0), d1 = read_lane_f32(dh, 32);
          if (ok0 && lane == kNavL + i0) {
            pid = (uint32_t)read_lane_i32(gv, i0);
            pdist = d0;
          }
          if (ok1 && lane == kNavL + i1) {
            pid = (uint32_t)read_lane_i32(gv, i1);
            pdist = d1;
          }
        }
      }
    }
    uint32_t broken = 0;  // chunks that met a -1
    for (int j = 0; !pre && j < kNavR / 2; j++) {
      const int i0 = 2 * j, i1 = 2 * j + 1;
      const int32_t v0 = e0 + i0 < glen ? graph[e0 + i0] : -1;
      const int32_t v1 = e0 + i1 < glen ? graph[e0 + i1] : -1;
      bool ok0 = false, ok1 = false;
      if (!(broken >> (i0 / kNavChunk) & 1u)) {
        if (v0 == -1) broken |= 1u << (i0 / kNavChunk);
        else ok0 = true;
      }
      if (!(broken >> (i1 / kNavChunk) & 1u)) {
        if (v1 == -1) broken |= 1u << (i1 / kNavChunk);
        else ok1 = true;
      }
      if (!ok0 && !ok1) continue;
      const int32_t vh = half ? (ok1 ? v1 : 0) : (ok0 ? v0 : 0);
      const float dh = nav_dist32<T>(q, data + (int64_t)vh * row, dims, lane);
      const float d0 = read_lane_f32(dh, 0), d1 = read_lane_f32(dh, 32);
      if (ok0 && lane == kNavL + i0) {
        pid = (uint32_t)v0;
        pdist = d0;
      }
      if (ok1 && lane == kNavL + i1) {
        pid = (uint32_t)v1;
        pdist = d1;
      }
    }
    // Selection phase: promote the four smallest to slots 0..3.
#pragma unroll
    for (int i = 0; i < kNavL; i++) {
      // Slots below i are final.  A slot at or above i holding the id selected
      // last round is a duplicate: its visited bit joins that slot
      // (pq_id[i-1] |= pq_id[lane]) and it drops out with +inf.
      bool dup = false;
      if (i != 0) {
        const uint32_t prev = read_lane_u32(pid, i - 1);
        dup = lane >= i && lane < 32 && ((pid ^ prev) & 0x7fffffffu) == 0;
        const uint64_t visited_dups = __ballot(dup && (pid & 0x80000000u));
        if (lane == i - 1 && visited_dups) pid |= 0x80000000u;
        if (dup) pdist = __int_as_float(0x7f800000);
      }
      float dist = (lane < 32 && lane >= i && !dup) ? pdist : __int_as_float(0x7f800000);
      int pos = lane;
      // 32-lane shuffle-down argmin, strict <, result at lane 0
      {
        float od = __uint_as_float(xor_lane32<16>(__float_as_uint(dist), lane));
        int op = (int)xor_lane32<16>((uint32_t)pos, lane);
        if (od < dist) { dist = od; pos = op; }
#define QV_NAV_STEP(CTRL)                                                                               \
  od = __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(dist), CTRL, 0xF, 0xF, false)); \
  op = __builtin_amdgcn_update_dpp(0, pos, CTRL, 0xF, 0xF, false);                                      \
  if (od < dist) { dist = od; pos = op; }
        QV_NAV_STEP(0x108)
        QV_NAV_STEP(0x104)
        QV_NAV_STEP(0x102)
        QV_NAV_STEP(0x101)
#undef QV_NAV_STEP
      }
      const int p0 = read_lane_i32(pos, 0);
      if (i != p0) {
        const float t = read_lane_f32(pdist, i), y = read_lane_f32(pdist, p0);
        if (t != y) {
          const uint32_t mi = read_lane_u32(pid, i), mp = read_lane_u32(pid, p0);
          if (lane == i) { pdist = y; pid = mp; }
          if (lane == p0) { pdist = t; pid = mi; }
        }
      }
    }
    const uint64_t unv = __ballot(lane < 32 && !(pid & 0x80000000u));
    const int x = unv ? __ffsll((long long)unv) - 1 : 32;
    idx = x < kNavL ? x : -1;
  }
  const uint32_t best = read_lane_u32(pid, 0) & 0x7fffffffu;
  return best < (uint64_t)num_node ? mapping[best] : fallback;
}

// Wall clock at 100 MHz (s_memrealtime).
__device__ __forceinline__ uint64_t wall_ticks() { return wall_clock64(); }

}  // namespace dev
}  // namespace qv
