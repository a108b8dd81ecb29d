// Row and column sampling draws (subsample, colsample_by{tree,level,node}).
//
// The reference forwards these keys to the trainer unchanged
// (native/class_native_training.cuh:30-31, :63).  Upstream draws them from a
// global generator whose stream cannot be reproduced here, so this build fixes
// its own counter-based draws: every draw is a pure function of (seed, stream,
// a, b, index), so any kernel, on any launch order, and the CPU restatement
// derive the same sample.
//
//   mix64(z)        the SplitMix64 output function (Steele, Lea & Flood 2014):
//                   z += 0x9E3779B97F4A7C15; two xor-shift-multiply rounds;
//                   a final xor-shift.
//   prefix(s,t,a,b) = mix64(mix64(mix64(s ^ (t << 56)) ^ a) ^ b)
//   draw(p, c)      = upper 32 bits of mix64(p ^ c)
//
// Rows (stream 1, a = round, b = output << 32): row r is kept iff
// draw(prefix, r) < floor(subsample * 2^32); a dropped row's gradient pair is
// zero for that tree.  Columns: stages tree (stream 2, b = output << 32), level
// (stream 3, b = output << 32 | depth) and node (stream 4, b = output << 32 |
// node id), each with a = round.  A stage keeps the n = max(1, floor(fraction
// * m)) of its m candidate features with the smallest keys, key(f) = the draw
// with its low fbits bits replaced by f (fbits: bits of n_features - 1), so
// keys are distinct; the level stage chooses among the tree stage's features
// and the node stage among the level stage's.
#pragma once

#include <cstdint>

namespace dp {

__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

enum : uint64_t { kRowStream = 1, kTreeStream = 2, kLevelStream = 3, kNodeStream = 4 };

__host__ __device__ inline uint64_t sample_prefix(uint64_t seed, uint64_t stream, uint64_t a,
                                                  uint64_t b) {
  return mix64(mix64(mix64(seed ^ (stream << 56)) ^ a) ^ b);
}

__host__ __device__ inline uint32_t sample_draw(uint64_t prefix, uint64_t index) {
  return uint32_t(mix64(prefix ^ index) >> 32);
}

// Bits that hold a feature index below n_features.
__host__ __device__ inline int feature_bits(int32_t n_features) {
  int b = 0;
  while (b < 31 && (int64_t(1) << b) < int64_t(n_features)) ++b;
  return b;
}

__host__ __device__ inline uint32_t feature_key(uint64_t prefix, int32_t f, int fbits) {
  const uint32_t low = fbits >= 32 ? 0xffffffffu : ((1u << fbits) - 1u);
  return (sample_draw(prefix, uint64_t(f)) & ~low) | uint32_t(f);
}

// Features a stage keeps out of m candidates: the product is formed in float,
// as upstream's ColumnSampler multiplies its float fraction by the set size
// (so 0.7 of 10 keeps 7: 0.7f * 10 rounds to 7.0f), then truncated.
__host__ __device__ inline int32_t stage_keep(float fraction, int32_t m) {
  if (!(fraction < 1.0f)) return m;
  const float x = fraction * float(m);
  const int32_t n = int32_t(x);  // truncation: x >= 0
  return n < 1 ? 1 : n;
}

// Row sampling of one round: kept iff draw < threshold; threshold 2^32 keeps
// every row (no draw is made).
struct RowSample {
  uint64_t seed = 0;
  uint64_t threshold = uint64_t(1) << 32;
  const int32_t* round = nullptr;  // device: the round's index
  __host__ __device__ bool active() const { return threshold < (uint64_t(1) << 32); }
};

// Column sampling of one tree (all fractions 1: inactive).
struct ColSample {
  uint64_t seed = 0;
  const int32_t* round = nullptr;  // device: the round's index
  int32_t output = 0;              // the tree's output (class) index
  float bytree = 1.0f, bylevel = 1.0f, bynode = 1.0f;
  __host__ __device__ bool active() const {
    return bytree < 1.0f || bylevel < 1.0f || bynode < 1.0f;
  }
};

}  // namespace dp
