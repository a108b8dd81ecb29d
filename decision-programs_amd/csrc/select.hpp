// Candidate records and the per-node argmax over feature candidates, shared by
// the split-selection kernel (split.hip) and the partition count kernel
// (partition.hip), which selects a node's split itself when the evaluation
// left per-feature candidates (one launch fewer per level).
//
// Order (upstream's tie rule, reached through XGBoosterUpdateOneIter,
// class_native_training.cuh:67): the larger loss wins; equal losses go to the
// lower feature, then the lower bin.
#pragma once

#include <cmath>

#include "dp_internal.hpp"

namespace dp {

struct Cand {
  double loss;
  long long gl, hl;
  int feature, bin, dl;
};

// a strictly better than b.
__device__ __forceinline__ bool better(const Cand& a, const Cand& b) {
  if (a.loss > b.loss) return true;
  if (a.loss < b.loss) return false;
  if (a.feature != b.feature) return unsigned(a.feature) < unsigned(b.feature);
  return unsigned(a.bin) < unsigned(b.bin);
}

__device__ __forceinline__ Cand shfl_xor_cand(const Cand& c, int mask) {
  Cand o;
  o.loss = __shfl_xor(c.loss, mask, 64);
  o.gl = __shfl_xor(c.gl, mask, 64);
  o.hl = __shfl_xor(c.hl, mask, 64);
  o.feature = __shfl_xor(c.feature, mask, 64);
  o.bin = __shfl_xor(c.bin, mask, 64);
  o.dl = __shfl_xor(c.dl, mask, 64);
  return o;
}

// The split record of a node's best candidate.
__device__ __forceinline__ dp_split_record make_record(const Cand& r, double gamma) {
  dp_split_record rec;
  rec.loss_chg = r.loss;
  rec.gl = r.gl;
  rec.hl = r.hl;
  rec.feature = r.feature;
  rec.bin = r.bin;
  rec.default_left = r.dl;
  rec.valid = r.loss > -INFINITY ? 1 : 0;
  rec.expand = rec.valid && r.loss > kRtEps && r.loss >= gamma;
  rec.pad = 0;
  return rec;
}

// Cross-lane moves on the DPP path (VALU lane swizzles, no LDS round trip):
// row_shr 1, 2, 4, 8 within each 16-lane row, then row_bcast15 (lane 15 of
// rows 0 and 2 into rows 1 and 3) and row_bcast31 (lane 31 into rows 2 and 3).
// Lanes whose source is out of range or whose row is masked off keep `old`.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ long long dpp64(long long v, long long old) {
  const int lo = __builtin_amdgcn_update_dpp(int(old), int(v), CTRL, ROW_MASK, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(int(old >> 32), int(v >> 32), CTRL, ROW_MASK, 0xf,
                                             false);
  return (long long)((uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
}

__device__ __forceinline__ long long readlane64(long long v, int lane) {
  const int lo = __builtin_amdgcn_readlane(int(v), lane);
  const int hi = __builtin_amdgcn_readlane(int(v >> 32), lane);
  return (long long)((uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
}

// Inclusive wavefront scan: row_shr 1, 2, 4, 8 within each 16-lane row, then
// row_bcast15 (lane 15 of rows 0 and 2 into rows 1 and 3) and row_bcast31
// (lane 31 into rows 2 and 3).
__device__ __forceinline__ long long wave_inclusive_sum(long long x) {
  x += dpp64<0x111>(x, 0);
  x += dpp64<0x112>(x, 0);
  x += dpp64<0x114>(x, 0);
  x += dpp64<0x118>(x, 0);
  x += dpp64<0x142, 0xa>(x, 0);
  x += dpp64<0x143, 0xc>(x, 0);
  return x;
}

// The same scan of 32-bit values (half the lane moves of the 64-bit one).
__device__ __forceinline__ int wave_inclusive_sum32(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);
  return x;
}

// The largest double of the wavefront, returned to every lane.
__device__ __forceinline__ double wave_max_f64(double v) {
  long long b = __double_as_longlong(v);
  auto step = [&](long long o) {
    if (__longlong_as_double(o) > __longlong_as_double(b)) b = o;
  };
  step(dpp64<0x111>(b, b));
  step(dpp64<0x112>(b, b));
  step(dpp64<0x114>(b, b));
  step(dpp64<0x118>(b, b));
  step(dpp64<0x142, 0xa>(b, b));
  step(dpp64<0x143, 0xc>(b, b));
  return __longlong_as_double(readlane64(b, 63));
}

// The smallest unsigned value of the wavefront, returned to every lane.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  int b = int(v);
  auto step = [&](int o) {
    if (uint32_t(o) < uint32_t(b)) b = o;
  };
  step(__builtin_amdgcn_update_dpp(b, b, 0x111, 0xf, 0xf, false));
  step(__builtin_amdgcn_update_dpp(b, b, 0x112, 0xf, 0xf, false));
  step(__builtin_amdgcn_update_dpp(b, b, 0x114, 0xf, 0xf, false));
  step(__builtin_amdgcn_update_dpp(b, b, 0x118, 0xf, 0xf, false));
  step(__builtin_amdgcn_update_dpp(b, b, 0x142, 0xa, 0xf, false));
  step(__builtin_amdgcn_update_dpp(b, b, 0x143, 0xc, 0xf, false));
  return uint32_t(__builtin_amdgcn_readlane(b, 63));
}

// The wavefront's best candidate in better()'s order, returned to every lane,
// when no two lanes hold the same feature: the largest loss, then among the
// lanes holding it the smallest feature (as unsigned, so -1 is last); that
// lane's fields are read back.
__device__ __forceinline__ Cand wave_best_by_feature(const Cand& c) {
  const double loss = wave_max_f64(c.loss);
  const bool top = c.loss == loss;
  const uint32_t feat = wave_min_u32(top ? uint32_t(c.feature) : 0xffffffffu);
  const unsigned long long hit = __ballot(top && uint32_t(c.feature) == feat);
  const int w = __builtin_ctzll(hit);
  Cand r;
  r.loss = __longlong_as_double(readlane64(__double_as_longlong(c.loss), w));
  r.gl = readlane64(c.gl, w);
  r.hl = readlane64(c.hl, w);
  r.feature = __builtin_amdgcn_readlane(c.feature, w);
  r.bin = __builtin_amdgcn_readlane(c.bin, w);
  r.dl = __builtin_amdgcn_readlane(c.dl, w);
  return r;
}

// The split record of `node` from its n_features candidates, computed by a
// whole workgroup of THREADS threads (every thread must call it; it holds two
// barriers).  wave_best: THREADS / 64 entries of LDS.  Returned to every thread.
template <int THREADS>
__device__ __forceinline__ dp_split_record select_node(const FeatCand* __restrict__ cand,
                                                       int32_t node, int32_t n_features,
                                                       double gamma, Cand* wave_best,
                                                       dp_split_record* shared_rec) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  Cand best;
  best.loss = -INFINITY;
  best.gl = best.hl = 0;
  best.feature = -1;
  best.bin = -1;
  best.dl = 0;
  for (int32_t f = threadIdx.x; f < n_features; f += THREADS) {
    const FeatCand fc = cand[int64_t(node) * n_features + f];
    Cand c;
    c.loss = fc.loss;
    c.gl = fc.gl;
    c.hl = fc.hl;
    c.feature = f;
    c.bin = fc.bin;
    c.dl = fc.dl;
    if (fc.loss > -INFINITY && better(c, best)) best = c;
  }
  // Threads hold disjoint feature sets (f = thread + k * THREADS).
  best = wave_best_by_feature(best);
  if (lane == 0) wave_best[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    Cand r = wave_best[0];
    for (int k = 1; k < THREADS / 64; ++k)
      if (better(wave_best[k], r)) r = wave_best[k];
    *shared_rec = make_record(r, gamma);
  }
  __syncthreads();
  return *shared_rec;
}

}  // namespace dp
