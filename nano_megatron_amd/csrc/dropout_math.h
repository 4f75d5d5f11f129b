// Counter-based dropout masks.
//
// Element idx of the stream keyed by `seed` is kept iff keep_bits(seed, idx)
// >= threshold, with keep_bits the 32-bit half (idx & 1: 0 low, 1 high) of
// SplitMix64's output for counter idx >> 1.  SplitMix64 is the generator of
// Steele, Lea and Flood ("Fast splittable pseudorandom number generators",
// OOPSLA 2014) in the form of Vigna's public-domain splitmix64.c: state +=
// 0x9E3779B97F4A7C15, then two xor-shift-multiply rounds and a final
// xor-shift; output k (k = 1, 2, ...) of a generator seeded with s is
// splitmix64(s, k - 1) below.  The mask is a pure function of (seed, idx), so
// the forward, the recompute of an activation checkpoint and the backward all
// regenerate it without storing it.
#pragma once

#include <stdint.h>

#include <hip/hip_runtime.h>

namespace nmb {

__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t seed, uint64_t counter) {
  uint64_t z = seed + (counter + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ uint32_t keep_bits(uint64_t seed, uint64_t idx) {
  const uint64_t z = splitmix64(seed, idx >> 1);
  return (idx & 1) ? static_cast<uint32_t>(z >> 32) : static_cast<uint32_t>(z);
}

// threshold = floor(p * 2^32) (keep probability 1 - threshold / 2^32) and the
// kept entries' factor 1 / (1 - p); threshold 0 keeps everything.
struct DropoutParams {
  uint64_t seed;
  uint32_t threshold;
  float scale;
};

// host side: p in [0, 1)
inline DropoutParams make_dropout(double p, uint64_t seed) {
  DropoutParams d{};
  d.seed = seed;
  d.threshold = static_cast<uint32_t>(p * 4294967296.0);
  d.scale = static_cast<float>(1.0 / (1.0 - p));
  return d;
}

// the factor of attention-probability element idx: scale if kept, else 0
__device__ __forceinline__ float drop_factor(const DropoutParams& d, uint64_t idx) {
  if (d.threshold == 0) return d.scale;
  return keep_bits(d.seed, idx) >= d.threshold ? d.scale : 0.f;
}

}  // namespace nmb
