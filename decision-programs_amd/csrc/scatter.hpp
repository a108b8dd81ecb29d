// The partition's stable scatter (the second of its two passes; the count pass
// and the row rule are in partition.hip), shared by the scatter launch of
// partition.hip and by the launch of grow.hip that runs a level's scatter beside
// its planner (the planner needs only the count pass's results).
//
// Each item sums the counts of its node's items (the node's left total, and
// the lefts in the node's items before it), ranks its rows in position order
// and writes lefts to [begin + left rank) and rights to
// [begin + n_left + right rank) of ridx_out.  Lane l of every wavefront holds
// ballot l of the item (step l / 4, wavefront l % 4), which is also position
// order; an exclusive scan of their counts gives each (step, wavefront) its
// lefts before it in the item, so the steps need no barrier.  The item's two
// barriers share the node-level sums.  No atomics: a node can have thousands
// of items.
//
// A workgroup of Q * 256 threads takes Q items at a time, one per 256-thread
// quarter; every quarter passes the same barriers, also when it has no item.
#pragma once

#include "dp_internal.hpp"
#include "select.hpp"

namespace dp {

constexpr int kPartThreads = 256;
constexpr int kPartSteps = int(kPartChunk / kPartThreads);  // 16 rows per lane
static_assert(kPartSteps * (kPartThreads / 64) == kPartMasks, "one mask per wave and step");

__device__ __forceinline__ int popc64(unsigned long long m) { return __popcll(m); }

// A leaf's weight as the planner records it (upstream's CalcWeight with
// max_delta_step 0): -T(g) / (h + lambda), T the L1 soft threshold alpha; 0
// when h < min_child_weight or h <= 0.  Double, compiled without contraction.
__device__ inline double leaf_weight(double g, double h, double lambda, double alpha,
                                     double mcw) {
  if (h < mcw || h <= 0.0) return 0.0;
  const double t = g > alpha ? g - alpha : (g < -alpha ? g + alpha : 0.0);
  return -t / (h + lambda);
}

// Items block * Q + quarter + k * n_blocks * Q.  Rows of a group of G steps:
// the first group's ids are loaded with the item's other inputs; with G > 1
// (large matrices) each later group's while the group before it is written.
template <int G, int Q>
__device__ void scatter_items(const ScatterArgs& a, int32_t block, int32_t n_blocks) {
  __shared__ int64_t wave_sum[Q][2][kPartThreads / 64];
  const int q = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kPartThreads);
  const int t = int(threadIdx.x) - q * kPartThreads;  // thread within the quarter
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int32_t item0 = block * Q + q;
  const PartWork w_first = item0 < a.n_work_host ? a.work[item0] : PartWork{0, 0, 0, 0};
  const int32_t n_work = a.n_work_dev ? *a.n_work_dev : a.n_work_host;
  for (int32_t base = block * Q; base < n_work; base += n_blocks * Q) {
    const int32_t item = base + q;
    const bool have = item < n_work;  // uniform per quarter (always true for Q = 1)
    const PartWork w = !have ? PartWork{0, 0, 0, 0} : (item == item0 ? w_first : a.work[item]);
    uint32_t row[G], nxt[G];
    auto load_rows = [&](uint32_t (&r)[G], int g0) {
#pragma unroll
      for (int k = 0; k < G; ++k) {
        const int64_t i = w.begin + int64_t(g0 + k) * kPartThreads + t;
        r[k] = i < w.end ? a.ridx_in[i] : 0u;
      }
    };
    bool act = false;
    if (have) {
      load_rows(row, 0);
      act = a.splits[w.node].expand != 0;
    }
    if (Q == 1 && !act) continue;  // uniform per workgroup
    unsigned long long my_mask = 0;
    int64_t begin = 0;
    int32_t first = 0;
    long long before = 0, total = 0;  // lefts in the node's items before this one; node total
    if (act) {
      my_mask = a.masks[int64_t(item) * kPartMasks + lane];
      begin = a.seg_begin[w.node];
      first = a.node_first_work[w.node];
      const int32_t last = a.node_first_work[w.node + 1];
      for (int32_t k0 = first + t; k0 < last; k0 += 4 * kPartThreads) {
        int64_t v[4];  // four counts in flight, at indexes clamped below last
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int32_t k = k0 + u * kPartThreads;
          v[u] = a.work_left[k < last ? k : last - 1] & 0xffffffffll;  // the left rows
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int32_t k = k0 + u * kPartThreads;
          if (k < last) {
            total += v[u];
            if (k < item) before += v[u];
          }
        }
      }
    }
    before = wave_inclusive_sum(before);
    total = wave_inclusive_sum(total);
    if (lane == 63) {
      wave_sum[q][0][wave] = before;
      wave_sum[q][1][wave] = total;
    }
    // lefts before each ballot of the item, in position order
    const long long c = popc64(my_mask);
    const int excl = int(wave_inclusive_sum(c) - c);
    __syncthreads();
    int64_t lefts_before = 0, n_left = 0;
    for (int k = 0; k < kPartThreads / 64; ++k) {
      lefts_before += wave_sum[q][0][k];
      n_left += wave_sum[q][1][k];
    }
    __syncthreads();  // wave_sum is rewritten by the next items
    if (!act) continue;  // after the barriers every quarter passes
    if (a.node_left && item == first && t == 0) a.node_left[w.node] = n_left;
#pragma unroll 1
    for (int g0 = 0; g0 < kPartSteps; g0 += G) {
      if (w.begin + int64_t(g0) * kPartThreads >= w.end) break;  // uniform per quarter
      if (g0 > 0 && G == 1) load_rows(row, g0);
      if (G > 1 && g0 + G < kPartSteps) load_rows(nxt, g0 + G);
#pragma unroll
      for (int k = 0; k < G; ++k) {
        const int64_t i = w.begin + int64_t(g0 + k) * kPartThreads + t;
        const int idx = (g0 + k) * (kPartThreads / 64) + wave;
        const unsigned long long mask = (unsigned long long)readlane64((long long)my_mask, idx);
        const int64_t prefix =
            lefts_before + __builtin_amdgcn_readlane(excl, idx) + popc64(mask & below);
        const int64_t dst = ((mask >> lane) & 1ull) ? begin + prefix
                                                    : begin + n_left + ((i - begin) - prefix);
        if (i < w.end) a.ridx_out[dst] = row[k];
      }
      if (G > 1)
#pragma unroll
        for (int k = 0; k < G; ++k) row[k] = nxt[k];
    }
  }
}

}  // namespace dp
