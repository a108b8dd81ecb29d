// Stable row partition of split nodes and the leaf margin update.
//
// Upstream applies a level's splits by moving each node's row ids so the left
// child's rows precede the right child's (inside XGBoosterUpdateOneIter,
// class_native_training.cuh:67).  Here every expanding node's segment of
// ridx_in is split in two launches:
//   1. count: one workgroup per chunk of <= kPartChunk rows counts its left
//      rows with wavefront ballots and keeps the ballots (one 64-bit mask per
//      wavefront and 256-row step, 64 per chunk), so the split feature's bins
//      are gathered once per level;
//   2. scatter (scatter.hpp): each chunk sums the counts of its node's chunks
//      (the node's left total, and its own exclusive offset from the earlier
//      ones; the node's first chunk publishes the total in node_left), ranks
//      its rows in position order (an exclusive scan of the chunk's 64 ballot
//      counts, one per lane, plus the lane's prefix in its ballot) and writes
//      lefts to [begin + left rank) and rights to [begin + n_left + right rank)
//      of ridx_out.  No atomics: a node can have thousands of chunks.  A caller
//      may take the scatter's arguments instead and launch it beside the level
//      planner (grow.hip).
// The row goes left iff its bin of the split feature is <= the split bin, or it
// is missing and the split's default is left.
#include "dp_internal.hpp"
#include "scatter.hpp"
#include "select.hpp"

namespace dp {
namespace {

// The split feature's bin of `row`: from the column-major copy when there is
// one (one symbol per row, contiguous within a feature; uint16 symbols for
// matrices whose missing marker is kWideMissing), else from the tiles.
template <bool COLS, typename SYM>
__device__ __forceinline__ int split_bin_of(const SYM* __restrict__ bins, int64_t n_rows,
                                            int tile_width, uint32_t row, int feature) {
  if (COLS) return bins[int64_t(feature) * n_rows + row];
  const int64_t tile = feature / tile_width;
  const int within = feature - int(tile) * tile_width;
  return bins[tile * n_rows * tile_width + int64_t(row) * tile_width + within];
}

// The margin (and leaf id) update of one leaf chunk (taken by value: the
// margin stores cannot alias it).  Row ids are loaded a batch ahead of their
// margins, at indexes clamped into the chunk (i0 < end), so the loads need no
// branch and overlap; a chunk's rows are distinct, so all margins of a batch
// are read before any is written.  With lp.store (uniform) the value is
// stored into the leaf-value plane and nothing is read: a row's scattered
// access is then one write instead of a read and a write of its sector.
__device__ __forceinline__ void apply_leaf(const LeafPass& lp, const LeafWork w) {
  constexpr int kBatch = 8;
  for (int64_t i0 = w.begin + threadIdx.x; i0 < w.end; i0 += int64_t(kBatch) * blockDim.x) {
    uint32_t row[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int64_t i = i0 + int64_t(k) * blockDim.x;
      row[k] = lp.ridx[i < w.end ? i : w.end - 1];
    }
    float m[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
      m[k] = lp.store ? 0.0f : lp.margin[int64_t(row[k]) * lp.stride];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (i0 + int64_t(k) * blockDim.x >= w.end) break;
      lp.margin[int64_t(row[k]) * lp.stride] = lp.store ? w.value : m[k] + w.value;
      if (lp.positions) lp.positions[row[k]] = w.pad;
    }
  }
}

// The partition kernels loop over their items (item = blockIdx.x + k * gridDim.x).
// The count kernel also takes the previous level's leaf chunks as items
// [n_work, n_work + n_leaves): their margin update rides in the same launch.
// With sel.cand set, the split records are not written yet: each item selects
// its node's split from the per-feature candidates (every chunk of a node gets
// the same record) and the node's first item writes it to splits.
// A lane handles rows begin + step * 256 + threadIdx.x, step = 0..15, in
// groups of G steps whose row ids, then bins, are loaded together
// (part_group: G = 4 keeps more loads in flight and pays on large levels;
// smaller matrices take the steps of one item).
// MARGIN (the last split level, LastLevel): each row's child leaf value is
// stored into the leaf-value plane once the side is known; the rows of a node
// that does not expand get the node's own leaf value.
template <bool COLS, int G, bool MARGIN, typename SYM = uint8_t>
__global__ __launch_bounds__(kPartThreads) void part_count_kernel(
    const SYM* __restrict__ bins, int64_t n_rows, int tile_width, int missing_bin,
    const uint32_t* __restrict__ ridx, const PartWork* __restrict__ work, int32_t n_work_host,
    const int32_t* __restrict__ n_work_dev, dp_split_record* __restrict__ splits,
    SplitSelect sel, const int32_t* __restrict__ node_first_work,
    int64_t* __restrict__ work_left, unsigned long long* __restrict__ masks, LeafPass lp,
    LastLevel ll) {
  __shared__ int wave_count[kPartThreads / 64];
  __shared__ Cand wave_best[kPartThreads / 64];
  __shared__ dp_split_record sel_rec;
  // The first item is loaded alongside the device counts (the host bound keeps
  // it in range), so the loads overlap instead of chaining.
  const PartWork w_first =
      int32_t(blockIdx.x) < n_work_host ? work[blockIdx.x] : PartWork{0, 0, 0, 0};
  const int32_t n_work = n_work_dev ? *n_work_dev : n_work_host;
  const int32_t n_leaves = lp.work ? (lp.n_dev ? *lp.n_dev : lp.n_host) : 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int32_t item = blockIdx.x; item < n_work + n_leaves; item += gridDim.x) {
  if (item >= n_work) {  // uniform per workgroup; no barriers on this path
    apply_leaf(lp, lp.work[item - n_work]);
    continue;
  }
  const PartWork w = item == int32_t(blockIdx.x) ? w_first : work[item];
  // Row ids of a group; the first group's are loaded before the split is
  // known, each later group's while the group before it is gathered.
  uint32_t row[G];
  auto load_rows = [&](int g0) {
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int64_t i = w.begin + int64_t(g0 + k) * kPartThreads + threadIdx.x;
      row[k] = i < w.end ? ridx[i] : 0u;
    }
  };
  load_rows(0);
  dp_split_record s;
  if (sel.cand) {  // uniform per launch
    s = select_node<kPartThreads>(sel.cand, w.node, sel.n_features, sel.gamma, wave_best,
                                  &sel_rec);
    if (threadIdx.x == 0 && item == node_first_work[w.node]) splits[w.node] = s;
  } else {
    s = splits[w.node];
  }
  // MARGIN: the leaf values of this item's rows (uniform per workgroup), in
  // the level planner's arithmetic (double, rounded to float once).
  float v_left = 0.0f, v_right = 0.0f;
  if constexpr (MARGIN) {
    const LevelNode nd = ll.nodes[w.node];
    const double ug = ldexp(1.0, -ll.exps[0]), uh = ldexp(1.0, -ll.exps[1]);
    if (s.expand) {
      v_left = float(leaf_weight(double(s.gl) * ug, double(s.hl) * uh, ll.lambda, ll.alpha,
                                 ll.mcw) * ll.eta);
      v_right = float(leaf_weight(double(nd.g - s.gl) * ug, double(nd.h - s.hl) * uh, ll.lambda,
                                  ll.alpha, ll.mcw) * ll.eta);
    } else {
      v_left = float(leaf_weight(double(nd.g) * ug, double(nd.h) * uh, ll.lambda, ll.alpha,
                                 ll.mcw) * ll.eta);
    }
  }
  if (!s.expand) {
    if (threadIdx.x == 0) work_left[item] = int64_t(w.node) << 32;
    if constexpr (MARGIN)  // the node is a leaf: its rows get its own value
      apply_leaf(LeafPass{ridx, nullptr, nullptr, 0, ll.values, 1, nullptr, true},
                 LeafWork{v_left, 0, w.begin, w.end});
    continue;
  }
  int count = 0;
  unsigned long long* item_masks = masks + int64_t(item) * kPartMasks + wave;
#pragma unroll 1
  for (int g0 = 0; g0 < kPartSteps; g0 += G) {
    if (w.begin + int64_t(g0) * kPartThreads >= w.end) break;  // uniform per workgroup
    int bin[G];
    uint32_t mrow[G];  // MARGIN: this group's rows (row[] is refilled below)
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int64_t i = w.begin + int64_t(g0 + k) * kPartThreads + threadIdx.x;
      bin[k] = i < w.end ? split_bin_of<COLS, SYM>(bins, n_rows, tile_width, row[k], s.feature)
                         : -1;
      if constexpr (MARGIN) mrow[k] = row[k];
    }
    if (g0 + G < kPartSteps) load_rows(g0 + G);
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int b = bin[k];
      const bool left = b >= 0 && (b == missing_bin ? s.default_left != 0 : b <= s.bin);
      const unsigned long long m = __ballot(left);
      if (lane == 0) item_masks[(g0 + k) * (kPartThreads / 64)] = m;
      count += popc64(m);
      if constexpr (MARGIN) {
        if (b >= 0) ll.values[mrow[k]] = left ? v_left : v_right;
      }
    }
  }
  if (lane == 0) wave_count[wave] = count;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t t = 0;
    for (int k = 0; k < kPartThreads / 64; ++k) t += wave_count[k];
    work_left[item] = (int64_t(w.node) << 32) | t;  // the node, then its left rows
  }
  __syncthreads();
  }
}

template <int G>
__global__ __launch_bounds__(kPartThreads) void part_scatter_kernel(ScatterArgs a) {
  scatter_items<G, 1>(a, int32_t(blockIdx.x), int32_t(gridDim.x));
}

// Two leaf lists (the second may be empty): items [0, n0) are list 0's,
// [n0, n0 + n1) list 1's, each list with its own row-id buffer.  store: the
// values are stored (a leaf-value plane) rather than added.
__global__ void update_margin_kernel(LeafList l0, LeafList l1, float* __restrict__ margin,
                                     int64_t stride, int32_t store) {
  const int32_t n0 = l0.n_dev ? *l0.n_dev : l0.n_host;
  const int32_t n1 = l1.work ? (l1.n_dev ? *l1.n_dev : l1.n_host) : 0;
  constexpr int kBatch = 8;  // as apply_leaf: row ids, then margins, then stores
  for (int32_t item = blockIdx.x; item < n0 + n1; item += gridDim.x) {
    const bool first = item < n0;  // uniform per workgroup
    const uint32_t* __restrict__ ridx = first ? l0.ridx : l1.ridx;
    const LeafWork w = first ? l0.work[item] : l1.work[item - n0];
    for (int64_t i0 = w.begin + threadIdx.x; i0 < w.end; i0 += int64_t(kBatch) * blockDim.x) {
      uint32_t row[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {  // clamped into the chunk: no branch
        const int64_t i = i0 + int64_t(k) * blockDim.x;
        row[k] = ridx[i < w.end ? i : w.end - 1];
      }
      // A leaf's rows are distinct: all margins are read before any is written.
      float m[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) m[k] = store ? 0.0f : margin[int64_t(row[k]) * stride];
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (i0 + int64_t(k) * blockDim.x < w.end)
          margin[int64_t(row[k]) * stride] = store ? w.value : m[k] + w.value;
    }
  }
}

// margin[row * K + k] += values[k * n + row]: one thread per row (grid-stride),
// the K planes read in row order, so every access is coalesced (K = 1: a
// float4 of rows per thread).
__global__ void add_leaf_values_kernel(float* __restrict__ margin, int32_t n_groups,
                                       const float* __restrict__ values, int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  const int64_t t0 = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (n_groups == 1) {
    const int64_t n4 = n / 4;
    auto* m4 = reinterpret_cast<float4*>(margin);
    const auto* v4 = reinterpret_cast<const float4*>(values);
    for (int64_t i = t0; i < n4; i += stride) {
      float4 m = m4[i];
      const float4 v = v4[i];
      m.x = m.x + v.x;
      m.y = m.y + v.y;
      m.z = m.z + v.z;
      m.w = m.w + v.w;
      m4[i] = m;
    }
    for (int64_t r = n4 * 4 + t0; r < n; r += stride) margin[r] = margin[r] + values[r];
    return;
  }
  for (int64_t r = t0; r < n; r += stride)
    for (int32_t k = 0; k < n_groups; ++k)
      margin[r * n_groups + k] = margin[r * n_groups + k] + values[int64_t(k) * n + r];
}

__global__ void leaf_positions_kernel(const uint32_t* __restrict__ ridx,
                                      const LeafWork* __restrict__ work, int32_t n_work_host,
                                      const int32_t* __restrict__ n_work_dev,
                                      int32_t* __restrict__ positions) {
  const int32_t n_work = n_work_dev ? *n_work_dev : n_work_host;
  for (int32_t item = blockIdx.x; item < n_work; item += gridDim.x) {
    const LeafWork w = work[item];
    for (int64_t i = w.begin + threadIdx.x; i < w.end; i += blockDim.x)
      positions[ridx[i]] = w.pad;
  }
}

}  // namespace

void launch_leaf_positions(const uint32_t* ridx, const LeafWork* work, int32_t n_work,
                           const int32_t* n_work_dev, int32_t* positions, hipStream_t s) {
  if (n_work <= 0) return;
  hipLaunchKernelGGL(leaf_positions_kernel, dim3(n_work < 2048 ? n_work : 2048), dim3(256), 0, s,
                     ridx, work, n_work, n_work_dev, positions);
  DP_HIP(hipGetLastError());
}

void launch_partition(const uint8_t* bins, const void* cols, const dp_bin_layout& layout,
                      const uint32_t* ridx_in, uint32_t* ridx_out, const PartWork* work,
                      int32_t n_work, const int32_t* n_work_dev, const int64_t* seg_begin,
                      dp_split_record* splits, const int32_t* node_first_work,
                      int32_t n_nodes, const int32_t* n_nodes_dev, int64_t* work_left,
                      unsigned long long* masks, int64_t* node_left, bool node_left_zeroed,
                      hipStream_t s, const LeafPass* leaves, const SplitSelect* select,
                      ScatterArgs* deferred, const LastLevel* last) {
  if (deferred) *deferred = ScatterArgs{};  // nothing to scatter unless filled below
  if (n_nodes <= 0) return;
  (void)n_nodes_dev;
  const int missing = layout.missing_bin;
  const LeafPass lp = leaves ? *leaves : LeafPass{};
  const int64_t items = int64_t(n_work) + (lp.work ? lp.n_host : 0);
  const int gc = int(items < 2048 ? items : 2048);
  const int gw = n_work < 2048 ? n_work : 2048;
  const bool wide = missing == kWideMissing;
  need(!wide || cols, "16-bit symbols are read from the column copy");
  if (!node_left_zeroed) launch_fill_i64(node_left, n_nodes, 0, s);
  if (items <= 0) return;
  const SplitSelect sel = select ? *select : SplitSelect{};
  const int group = part_group(layout.n_rows);
  const LastLevel ll = last ? *last : LastLevel{};
  need(!last || (ll.values && ll.nodes && ll.exps), "last-level leaf value arguments");
  auto pick = [&](auto k1, auto k2, auto k4) { return group == 4 ? k4 : (group == 2 ? k2 : k1); };
  if (wide) {
    auto count = last ? pick(part_count_kernel<true, 1, true, uint16_t>,
                             part_count_kernel<true, 2, true, uint16_t>,
                             part_count_kernel<true, 4, true, uint16_t>)
                      : pick(part_count_kernel<true, 1, false, uint16_t>,
                             part_count_kernel<true, 2, false, uint16_t>,
                             part_count_kernel<true, 4, false, uint16_t>);
    hipLaunchKernelGGL(count, dim3(gc), dim3(kPartThreads), 0, s,
                       static_cast<const uint16_t*>(cols), layout.n_rows, layout.tile_width,
                       missing, ridx_in, work, n_work, n_work_dev, splits, sel, node_first_work,
                       work_left, masks, lp, ll);
  } else {
    const uint8_t* src = cols ? static_cast<const uint8_t*>(cols) : bins;
    auto count =
        cols ? (last ? pick(part_count_kernel<true, 1, true>, part_count_kernel<true, 2, true>,
                            part_count_kernel<true, 4, true>)
                     : pick(part_count_kernel<true, 1, false>, part_count_kernel<true, 2, false>,
                            part_count_kernel<true, 4, false>))
             : (last ? pick(part_count_kernel<false, 1, true>, part_count_kernel<false, 2, true>,
                            part_count_kernel<false, 4, true>)
                     : pick(part_count_kernel<false, 1, false>, part_count_kernel<false, 2, false>,
                            part_count_kernel<false, 4, false>));
    hipLaunchKernelGGL(count, dim3(gc), dim3(kPartThreads), 0, s, src, layout.n_rows,
                       layout.tile_width, missing, ridx_in, work, n_work, n_work_dev, splits,
                       sel, node_first_work, work_left, masks, lp, ll);
  }
  DP_HIP(hipGetLastError());
  if (last) return;  // every child is a leaf: no new row order
  const ScatterArgs sa{ridx_in, ridx_out,   work,      n_work, n_work_dev, splits,
                       seg_begin, node_first_work, work_left, masks, node_left};
  if (deferred) {
    *deferred = sa;
    return;
  }
  if (n_work <= 0) return;
  hipLaunchKernelGGL(pick(part_scatter_kernel<1>, part_scatter_kernel<2>, part_scatter_kernel<4>),
                     dim3(gw), dim3(kPartThreads), 0, s, sa);
  DP_HIP(hipGetLastError());
}

void launch_update_margin(const uint32_t* ridx, const LeafWork* work, int32_t n_work,
                          const int32_t* n_work_dev, float* margin, int64_t stride,
                          hipStream_t s, const LeafList* second, bool store) {
  const LeafList l1 = second ? *second : LeafList{};
  const int64_t items = int64_t(n_work) + (l1.work ? l1.n_host : 0);
  if (items <= 0) return;
  const LeafList l0{ridx, work, n_work, n_work_dev};
  hipLaunchKernelGGL(update_margin_kernel, dim3(items < 2048 ? items : 2048), dim3(256), 0, s, l0,
                     l1, margin, stride, store ? 1 : 0);
  DP_HIP(hipGetLastError());
}

void launch_add_leaf_values(float* margin, int32_t n_groups, const float* values, int64_t n_rows,
                            hipStream_t s) {
  if (n_rows <= 0 || n_groups <= 0) return;
  need(margin && values, "leaf-value addition needs the margins and the planes");
  need(n_groups > 1 || (reinterpret_cast<uintptr_t>(margin) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(values) % 16 == 0),
       "single-output margins and leaf values must be 16-byte aligned");
  const int64_t per = n_groups == 1 ? (n_rows + 3) / 4 : n_rows;
  const int64_t blocks = (per + 255) / 256;
  hipLaunchKernelGGL(add_leaf_values_kernel, dim3(unsigned(blocks < 2048 ? blocks : 2048)),
                     dim3(256), 0, s, margin, n_groups, values, n_rows);
  DP_HIP(hipGetLastError());
}

}  // namespace dp
