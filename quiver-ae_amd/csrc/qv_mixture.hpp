// qv_mixture.hpp -- counter-based synthetic data shared by the host and the
// device generators.  Every value depends only on (seed, stream, counter), so a
// row can be produced anywhere, in any order, with identical bits: all
// arithmetic is integer or exactly representable float, and the translation
// units that include this file are built with -ffp-contract=off.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define QV_HD __host__ __device__ inline
#else
#define QV_HD inline
#endif

namespace qv {

// SplitMix64 output function (Steele, Lea, Flood 2014).
QV_HD uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

QV_HD uint64_t rng_u64(uint64_t seed, uint64_t stream, uint64_t counter) {
  return mix64(mix64(seed + stream * 0xD1B54A32D192ED03ull) ^ counter);
}

// Uniform in [0, 1) with 24 bits: exact in float.
QV_HD float rng_unit24(uint64_t h) { return (float)(h >> 40) * (1.0f / 16777216.0f); }

// Irwin-Hall(12) standard normal deviate from twelve 16-bit uniforms taken from
// three hashes.  With u_k = (x_k + 0.5) / 65536, sum(u_k) - 6 equals
// (S - 393210) / 65536 for the integer S = sum(x_k): exact in float.
QV_HD float rng_normal(uint64_t seed, uint64_t stream, uint64_t counter) {
  int32_t s = 0;
  for (int w = 0; w < 3; w++) {
    uint64_t h = rng_u64(seed, stream, counter * 3ull + (uint64_t)w);
    s += (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
         (int32_t)((h >> 32) & 0xffff) + (int32_t)(h >> 48);
  }
  return (float)(s - 393210) * (1.0f / 65536.0f);
}

// Index in [0, n) from the high 32 bits (multiply-shift, n < 2^32).
QV_HD uint32_t rng_below(uint64_t h, uint32_t n) {
  return (uint32_t)(((h >> 32) * (uint64_t)n) >> 32);
}

enum : uint64_t { kStreamCenter = 1, kStreamAssign = 2, kStreamNoise = 3, kStreamBytes = 4, kStreamIds = 5 };

// uint8 element j of row i: clip(rint(c_k[j] + sigma * z), 0, 255) with
// c_k[j] = lo + (hi - lo) * u.
QV_HD uint8_t mixture_u8(uint64_t seed, int32_t num_centers, int32_t dim, float lo,
                         float hi, float sigma, int64_t i, int32_t j) {
  uint32_t k = rng_below(rng_u64(seed, kStreamAssign, (uint64_t)i), (uint32_t)num_centers);
  float u = rng_unit24(rng_u64(seed, kStreamCenter, (uint64_t)k * (uint64_t)dim + (uint64_t)j));
  float span = hi - lo;
  float c = span * u;
  c = c + lo;
  float z = rng_normal(seed, kStreamNoise, (uint64_t)i * (uint64_t)dim + (uint64_t)j);
  float n = sigma * z;
  float v = c + n;
  v = __builtin_rintf(v);
  v = v < 0.f ? 0.f : (v > 255.f ? 255.f : v);
  return (uint8_t)v;
}

// float element j of row i before normalisation: c_k[j] + sigma * z with c ~ N(0,1).
QV_HD float mixture_f32_raw(uint64_t seed, int32_t num_centers, int32_t dim, float sigma,
                            int64_t i, int32_t j) {
  uint32_t k = rng_below(rng_u64(seed, kStreamAssign, (uint64_t)i), (uint32_t)num_centers);
  float c = rng_normal(seed, kStreamCenter, (uint64_t)k * (uint64_t)dim + (uint64_t)j);
  float z = rng_normal(seed, kStreamNoise, (uint64_t)i * (uint64_t)dim + (uint64_t)j);
  float n = sigma * z;
  return c + n;
}

}  // namespace qv
