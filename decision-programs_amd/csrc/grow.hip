// Device-side level planning for depth-wise tree growth.
//
// After a level has been evaluated and partitioned, one workgroup turns the
// split records and left counts into
//   * the tree's node records (split or leaf value), numbered as upstream's
//     depth-wise driver numbers them: children of the k-th expanded node of a
//     level get the next two ids (left > parent, right = left + 1,
//     native/class_native_source_contract.hpp:24-31);
//   * the next level's nodes, their quantised sums and segment starts;
//   * the next level's histogram work (the smaller child of every pair, rows
//     chunked and ordered for the XCD-aware dispatch), the subtraction jobs
//     deriving each sibling, and the partition work;
//   * the margin-update work of this level's leaves.
// Nothing goes back to the host until the tree is complete, so a whole tree
// is enqueued without a host round trip per level.
//
// Leaf weights use the same double arithmetic as the CPU restatement
// (-T(G)/(H + lambda), times eta, rounded to float), compiled with
// -ffp-contract=off.
#include "dp_internal.hpp"

#include <cmath>

namespace dp {
namespace {

constexpr int kPlanThreads = 1024;
constexpr int64_t kHistMinChunk = 4096;

__device__ double plan_threshold_l1(double g, double alpha) {
  if (g > alpha) return g - alpha;
  if (g < -alpha) return g + alpha;
  return 0.0;
}

__device__ double plan_weight(const PlanArgs& a, double g, double h) {
  if (h < a.mcw || h <= 0.0) return 0.0;
  return -plan_threshold_l1(g, a.alpha) / (h + a.lambda);
}

// Exclusive scan of one int64 per thread over the workgroup; returns this
// thread's prefix and writes the total to *total.
__device__ int64_t block_scan(int64_t v, int64_t* lds, int64_t* total) {
  const int t = threadIdx.x;
  lds[t] = v;
  __syncthreads();
  for (int d = 1; d < kPlanThreads; d <<= 1) {
    const int64_t add = t >= d ? lds[t - d] : 0;
    __syncthreads();
    lds[t] += add;
    __syncthreads();
  }
  const int64_t incl = lds[t];
  *total = lds[kPlanThreads - 1];
  __syncthreads();
  return incl - v;
}

__device__ bool node_expands(const PlanArgs& a, int32_t i, int64_t rows) {
  if (!a.splits || !a.splits[i].expand) return false;
  const int64_t nl = a.node_left[i];
  return nl > 0 && nl < rows;
}

__global__ __launch_bounds__(kPlanThreads) void plan_level_kernel(PlanArgs a) {
  __shared__ int64_t scan[kPlanThreads];
  __shared__ int32_t s_error;
  const int tid = threadIdx.x;
  const int32_t n = a.counts->n_level;
  const int32_t n_nodes0 = a.counts->n_nodes;
  const double ug = ldexp(1.0, -a.exps[0]), uh = ldexp(1.0, -a.exps[1]);
  if (tid == 0) s_error = 0;
  __syncthreads();

  // ---- A: numbering, node records, next-level nodes ----------------------
  int64_t carry = 0;
  for (int32_t base = 0; base < n; base += kPlanThreads) {
    const int32_t i = base + tid;
    bool e = false;
    LevelNode nd{};
    if (i < n) {
      nd = a.cur[i];
      e = node_expands(a, i, nd.end - nd.begin);
      if (a.splits && a.splits[i].expand && !e) s_error = 1;
    }
    int64_t total;
    const int64_t rank = carry + block_scan(e ? 1 : 0, scan, &total);
    carry += total;
    if (i < n) {
      NodeInfo info{};
      info.g = nd.g;
      info.h = nd.h;
      info.begin = nd.begin;
      info.end = nd.end;
      info.parity = a.depth & 1;
      const double G = double(nd.g) * ug, H = double(nd.h) * uh;
      const double w = plan_weight(a, G, H);
      info.base_weight = float(w);
      info.sum_hess = float(H);
      info.bin = -1;
      if (e) {
        const dp_split_record s = a.splits[i];
        const int32_t left = n_nodes0 + int32_t(2 * rank);
        const int64_t nl = a.node_left[i];
        info.left = left;
        info.feature = s.feature;
        info.bin = s.bin;
        info.default_left = s.default_left;
        info.loss_chg = s.loss_chg;
        const int64_t slot = 2 * rank;
        if (left + 1 < a.info_capacity && slot + 1 < a.level_capacity) {
          a.next[slot] = LevelNode{nd.begin, nd.begin + nl, s.gl, s.hl, left, i};
          a.next[slot + 1] = LevelNode{nd.begin + nl, nd.end, nd.g - s.gl, nd.h - s.hl, left + 1, i};
          a.next_sums[2 * slot] = s.gl;
          a.next_sums[2 * slot + 1] = s.hl;
          a.next_sums[2 * slot + 2] = nd.g - s.gl;
          a.next_sums[2 * slot + 3] = nd.h - s.hl;
          a.next_seg_begin[slot] = nd.begin;
          a.next_seg_begin[slot + 1] = nd.begin + nl;
        } else {
          s_error = 2;
        }
      } else {
        info.left = -1;
        info.leaf_value = float(w * a.eta);
      }
      if (nd.nid >= 0 && nd.nid < a.info_capacity) a.info[nd.nid] = info;
      else s_error = 2;
    }
  }
  const int32_t n_expand = int32_t(carry);
  const int32_t n_next = 2 * n_expand;
  __syncthreads();
  if (s_error) {  // inconsistent level or capacity exceeded: stop this tree
    if (tid == 0) {
      PlanCounts* c = a.counts;
      c->n_level = c->n_hist = c->n_sub = c->n_part = c->n_leaf = 0;
      if (!c->error) c->error = s_error;
    }
    return;
  }

  // ---- B: leaf work of this level -----------------------------------------
  carry = 0;
  for (int32_t base = 0; base < n; base += kPlanThreads) {
    const int32_t i = base + tid;
    int64_t chunks = 0;
    LevelNode nd{};
    if (i < n) {
      nd = a.cur[i];
      if (!node_expands(a, i, nd.end - nd.begin))
        chunks = (nd.end - nd.begin + kLeafChunk - 1) / kLeafChunk;
    }
    int64_t total;
    const int64_t off = carry + block_scan(chunks, scan, &total);
    carry += total;
    if (chunks > 0) {
      const float value = a.info[nd.nid].leaf_value;
      for (int64_t j = 0; j < chunks; ++j) {
        const int64_t at = off + j;
        if (at >= a.leaf_capacity) { s_error = 3; break; }
        const int64_t b = nd.begin + j * kLeafChunk;
        a.leaf_work[at] = LeafWork{value, nd.nid, b, b + kLeafChunk < nd.end ? b + kLeafChunk : nd.end};
      }
    }
  }
  const int64_t n_leaf = carry;

  // ---- C: histogram work and subtraction jobs of the next level ----------
  const bool next_hist = n_next > 0 && a.depth + 1 < a.max_depth;
  int64_t n_hist = 0;
  int32_t n_sub = 0;
  if (next_hist) {
    // total rows of the smaller children
    int64_t mine = 0;
    for (int32_t j = tid; j < n_expand; j += kPlanThreads) {
      const LevelNode l = a.next[2 * j], r = a.next[2 * j + 1];
      const int64_t rl = l.end - l.begin, rr = r.end - r.begin;
      mine += rr < rl ? rr : rl;
    }
    int64_t small_total;
    (void)block_scan(mine, scan, &small_total);
    int64_t chunk = (small_total * a.n_tiles + 1023) / 1024;
    if (chunk < kHistMinChunk) chunk = kHistMinChunk;
    int64_t* cstart = a.pair_chunk;
    carry = 0;
    for (int32_t base = 0; base < n_expand; base += kPlanThreads) {
      const int32_t j = base + tid;
      int64_t nc = 0;
      if (j < n_expand) {
        const LevelNode l = a.next[2 * j], r = a.next[2 * j + 1];
        const int64_t rl = l.end - l.begin, rr = r.end - r.begin;
        const int64_t rows = rr < rl ? rr : rl;
        nc = (rows + chunk - 1) / chunk;
      }
      int64_t total;
      const int64_t off = carry + block_scan(nc, scan, &total);
      carry += total;
      if (j < n_expand) cstart[j] = off;
    }
    const int64_t C = carry;
    if (tid == 0) cstart[n_expand] = C;
    __syncthreads();
    const int64_t padded = (C + 7) / 8 * 8;
    n_hist = padded * a.n_tiles;
    if (n_hist > a.hist_capacity) {
      if (tid == 0) s_error = 4;
      n_hist = 0;
    } else {
      for (int64_t c = tid; c < padded; c += kPlanThreads) {
        HistWork item{0, 0, 0, 0};
        if (c < C) {
          int32_t lo = 0, hi = n_expand;  // last pair with cstart <= c
          while (hi - lo > 1) {
            const int32_t mid = (lo + hi) >> 1;
            if (cstart[mid] <= c) lo = mid; else hi = mid;
          }
          const int32_t j = lo;
          const LevelNode l = a.next[2 * j], r = a.next[2 * j + 1];
          const bool right_small = (r.end - r.begin) < (l.end - l.begin);
          const LevelNode sm = right_small ? r : l;
          const int64_t b = sm.begin + (c - cstart[j]) * chunk;
          item = HistWork{2 * j + (right_small ? 1 : 0), 0, b, b + chunk < sm.end ? b + chunk : sm.end};
        }
        for (int32_t t = 0; t < a.n_tiles; ++t) {
          item.tile = t;
          a.hist_work[((c / 8) * a.n_tiles + t) * 8 + (c % 8)] = item;
        }
      }
    }
    for (int32_t j = tid; j < n_expand; j += kPlanThreads) {
      const LevelNode l = a.next[2 * j], r = a.next[2 * j + 1];
      const bool right_small = (r.end - r.begin) < (l.end - l.begin);
      const int32_t small = 2 * j + (right_small ? 1 : 0), large = 2 * j + (right_small ? 0 : 1);
      a.sub_jobs[j] = SubtractJob{int64_t(l.parent_slot) * a.hist_elems,
                                  int64_t(small) * a.hist_elems, int64_t(large) * a.hist_elems};
    }
    n_sub = n_expand;
  }

  // ---- D: partition work of the next level ----------------------------------
  int64_t n_part = 0;
  if (next_hist) {
    carry = 0;
    for (int32_t base = 0; base < n_next; base += kPlanThreads) {
      const int32_t i = base + tid;
      int64_t chunks = 0;
      LevelNode nd{};
      if (i < n_next) {
        nd = a.next[i];
        chunks = (nd.end - nd.begin + kPartChunk - 1) / kPartChunk;
      }
      int64_t total;
      const int64_t off = carry + block_scan(chunks, scan, &total);
      carry += total;
      if (i < n_next) {
        a.part_first[i] = int32_t(off);
        for (int64_t j = 0; j < chunks; ++j) {
          if (off + j >= a.part_capacity) { s_error = 5; break; }
          const int64_t b = nd.begin + j * kPartChunk;
          a.part_work[off + j] = PartWork{i, 0, b, b + kPartChunk < nd.end ? b + kPartChunk : nd.end};
        }
      }
    }
    n_part = carry;
    if (tid == 0) a.part_first[n_next] = int32_t(n_part);
  }

  __syncthreads();
  if (tid == 0) {
    PlanCounts* c = a.counts;
    c->n_level = n_next;
    c->n_nodes = n_nodes0 + n_next;
    c->n_hist = int32_t(n_hist);
    c->n_sub = n_sub;
    c->n_part = int32_t(n_part > a.part_capacity ? 0 : n_part);
    c->n_leaf = int32_t(n_leaf > a.leaf_capacity ? 0 : n_leaf);
    if (s_error && !c->error) c->error = s_error;
  }
}

__global__ void plan_root_kernel(LevelNode* cur, int64_t* sums, int64_t* seg_begin,
                                 PartWork* part_work, int32_t* part_first, PlanCounts* counts,
                                 int64_t n_rows, const int64_t* root_sums) {
  const int64_t chunks = (n_rows + kPartChunk - 1) / kPartChunk;
  for (int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; j < chunks;
       j += int64_t(blockDim.x) * gridDim.x) {
    const int64_t b = j * kPartChunk;
    part_work[j] = PartWork{0, 0, b, b + kPartChunk < n_rows ? b + kPartChunk : n_rows};
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const int64_t g = root_sums[0], h = root_sums[1];
    cur[0] = LevelNode{0, n_rows, g, h, 0, -1};
    sums[0] = g;
    sums[1] = h;
    seg_begin[0] = 0;
    part_first[0] = 0;
    part_first[1] = int32_t(chunks);
    PlanCounts c{};
    c.n_level = 1;
    c.n_nodes = 1;
    c.n_part = int32_t(chunks);
    *counts = c;
  }
}

}  // namespace

void launch_plan_level(const PlanArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(plan_level_kernel, dim3(1), dim3(kPlanThreads), 0, s, a);
  DP_HIP(hipGetLastError());
}

void launch_plan_root(LevelNode* cur, int64_t* sums, int64_t* seg_begin, PartWork* part_work,
                      int32_t* part_first, PlanCounts* counts, int64_t n_rows,
                      const int64_t* root_sums, hipStream_t s) {
  const int64_t chunks = (n_rows + kPartChunk - 1) / kPartChunk;
  hipLaunchKernelGGL(plan_root_kernel, dim3(grid_for(chunks, 256, 1024)), dim3(256), 0, s, cur,
                     sums, seg_begin, part_work, part_first, counts, n_rows, root_sums);
  DP_HIP(hipGetLastError());
}

}  // namespace dp
