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
//     chunked and ordered for the XCD-aware dispatch; a pair with one chunk
//     per tile writes its histogram directly, larger ones use partial slots),
//     the reduce jobs that finish the built histograms and derive each
//     sibling, and the partition work;
//   * the leaf-value work of this level's leaves.
// Counts are scanned over the workgroup and every work item is then written
// by its own thread, which finds its node by binary search over the offsets.
// Nothing goes back to the host until the tree is complete, so a whole tree
// is enqueued without a host round trip per level.
//
// Leaf weights use the same double arithmetic as the CPU restatement
// (-T(G)/(H + lambda), times eta, rounded to float), compiled with
// -ffp-contract=off.
#include "dp_internal.hpp"
#include "scatter.hpp"
#include "select.hpp"

#include <cmath>

namespace dp {
namespace {

constexpr int kPlanThreads = 1024;
// Offsets of levels up to this many segments are also kept in LDS, so the
// per-item binary searches do not chase dependent global loads.
constexpr int kLdsOffsets = 4096;

__device__ double plan_weight(const PlanArgs& a, double g, double h) {
  return leaf_weight(g, h, a.lambda, a.alpha, a.mcw);
}

// ceil(rows / chunk) for 0 <= rows < 2^32 (row ids are 32-bit) and chunk >= 1:
// a 32-bit division, far shorter than the 64-bit one.
__device__ __forceinline__ int64_t ceil_rows(int64_t rows, int64_t chunk) {
  if (chunk >> 32) return rows > 0 ? 1 : 0;
  const uint32_t r = uint32_t(rows), c = uint32_t(chunk);
  const uint32_t q = r / c;
  return int64_t(q) + (r - q * c != 0u ? 1 : 0);
}

// Exclusive scans of V int64 values per thread over the workgroup (out) and
// their totals.  Each wavefront scans with DPP lane moves; lane 63 leaves the
// wavefront's totals in lds; after a barrier every wavefront scans the
// (kPlanThreads / 64) totals the same way and reads its own prefix and the
// grand total by readlane.  lds holds at least 16 * V values; two barriers.
template <int V>
__device__ void block_scan_n(const int64_t (&v)[V], int64_t (&out)[V], int64_t (&total)[V],
                             int64_t* lds) {
  constexpr int W = kPlanThreads / 64;
  static_assert(W <= 64, "one wavefront scans the wavefront totals");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  int64_t x[V];
#pragma unroll
  for (int k = 0; k < V; ++k) x[k] = wave_inclusive_sum(v[k]);
  if (lane == 63)
#pragma unroll
    for (int k = 0; k < V; ++k) lds[k * W + wave] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int64_t w = wave_inclusive_sum(lane < W ? lds[k * W + lane] : 0);
    out[k] = (wave ? readlane64(w, wave - 1) : 0) + x[k] - v[k];
    total[k] = readlane64(w, W - 1);
  }
  __syncthreads();  // lds is reused by the next scan
}

// block_scan_n over the first nw wavefronts only (nw uniform, 1 <= nw <= 16):
// the others hold no values, skip the scans (a wavefront's VALU work costs the
// same whether its lanes are live or not) and pass the same two barriers;
// their out is 0, and every thread gets the totals, through tot_lds.
template <int V>
__device__ void block_scan_live(const int64_t (&v)[V], int64_t (&out)[V], int64_t (&total)[V],
                                int64_t* lds, int64_t* tot_lds, int nw) {
  constexpr int W = kPlanThreads / 64;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const bool live = wave < nw;  // uniform per wavefront
  int64_t x[V];
  if (live) {
#pragma unroll
    for (int k = 0; k < V; ++k) x[k] = wave_inclusive_sum(v[k]);
    if (lane == 63)
#pragma unroll
      for (int k = 0; k < V; ++k) lds[k * W + wave] = x[k];
  }
  __syncthreads();
  if (live) {
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int64_t w = wave_inclusive_sum(lane < nw ? lds[k * W + lane] : 0);
      out[k] = (wave ? readlane64(w, wave - 1) : 0) + x[k] - v[k];
      total[k] = readlane64(w, nw - 1);
    }
    if (wave == 0 && lane == 0)
#pragma unroll
      for (int k = 0; k < V; ++k) tot_lds[k] = total[k];
  }
  __syncthreads();  // lds is reused by the next scan; tot_lds is read below
  if (!live)
#pragma unroll
    for (int k = 0; k < V; ++k) {
      out[k] = 0;
      total[k] = tot_lds[k];
    }
}

// Exclusive scan of one int64 per thread over the workgroup; returns this
// thread's prefix and writes the total to *total (two barriers).
__device__ int64_t block_scan(int64_t v, int64_t* lds, int64_t* total) {
  int64_t out[1], tot[1];
  const int64_t in[1] = {v};
  block_scan_n<1>(in, out, tot, lds);
  *total = tot[0];
  return out[0];
}

// Index of the segment holding item k: the last i in [0, n) with off[i] <= k
// (off nondecreasing, off[0] <= k).
template <class T>
__device__ int32_t owner(const T* off, int32_t n, int64_t k) {
  int32_t lo = 0, hi = n;
  while (hi - lo > 1) {
    const int32_t mid = (lo + hi) >> 1;
    if (int64_t(off[mid]) <= k) lo = mid; else hi = mid;
  }
  return lo;
}

__device__ bool node_expands(const PlanArgs& a, int32_t i, int64_t rows) {
  if (!a.splits || !a.splits[i].expand) return false;
  const int64_t nl = a.node_left[i];
  return nl > 0 && nl < rows;
}

__global__ __launch_bounds__(kPlanThreads) void plan_level_kernel(PlanArgs a) {
  __shared__ int64_t scan[kPlanThreads];
  __shared__ int64_t s_off[kLdsOffsets + 1];
  __shared__ int32_t s_error;
  const int tid = threadIdx.x;
  const int32_t n = a.counts->n_level;
  const int32_t n_leaf_old = a.counts->n_leaf;
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
          a.next_node_left[slot] = 0;
          a.next_node_left[slot + 1] = 0;
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
      c->n_level = c->n_hist = c->n_reduce = c->n_leaf = c->n_leaf_prev = 0;
      c->n_part[(a.depth + 1) & 1] = 0;
      if (!c->error) c->error = s_error;
    }
    return;
  }

  // ---- B: leaf work of this level -----------------------------------------
  int64_t* off = a.pair_chunk;  // [n + 1]: first leaf chunk of each node
  carry = 0;
  for (int32_t base = 0; base < n; base += kPlanThreads) {
    const int32_t i = base + tid;
    int64_t chunks = 0;
    if (i < n) {
      const LevelNode nd = a.cur[i];
      if (!node_expands(a, i, nd.end - nd.begin))
        chunks = ceil_rows(nd.end - nd.begin, a.leaf_chunk);
    }
    int64_t total;
    const int64_t o = carry + block_scan(chunks, scan, &total);
    carry += total;
    if (i < n) {
      off[i] = o;
      if (n <= kLdsOffsets) s_off[i] = o;
    }
  }
  int64_t n_leaf = carry;
  if (tid == 0) {
    off[n] = n_leaf;
    if (n <= kLdsOffsets) s_off[n] = n_leaf;
  }
  __syncthreads();
  const int64_t* leaf_off = n <= kLdsOffsets ? s_off : off;
  if (n_leaf > a.leaf_capacity) {
    if (tid == 0) s_error = 3;
    n_leaf = 0;
  }
  for (int64_t k = tid; k < n_leaf; k += kPlanThreads) {
    const int32_t i = owner(leaf_off, n, k);
    const LevelNode nd = a.cur[i];
    const int64_t b = nd.begin + (k - leaf_off[i]) * a.leaf_chunk;
    a.leaf_work[k] = LeafWork{a.info[nd.nid].leaf_value, nd.nid, b,
                              b + a.leaf_chunk < nd.end ? b + a.leaf_chunk : nd.end};
  }
  __syncthreads();  // off is reused below

  // ---- C: histogram work and reduce jobs of the next level ----------------
  const bool next_hist = n_next > 0 && a.depth + 1 < a.max_depth;
  int64_t n_hist = 0;
  int32_t n_reduce = 0;
  if (next_hist) {
    const int32_t T = a.n_tiles;
    int64_t mine = 0;  // rows of the smaller children
    for (int32_t j = tid; j < n_expand; j += kPlanThreads) {
      const LevelNode l = a.next[2 * j], r = a.next[2 * j + 1];
      const int64_t rl = l.end - l.begin, rr = r.end - r.begin;
      mine += rr < rl ? rr : rl;
    }
    int64_t small_total;
    (void)block_scan(mine, scan, &small_total);
    const int32_t TPW = a.hist_tiles;
    const int32_t G = hist_groups(T, TPW, a.hist_pairs);  // items per row chunk
    const int64_t chunk = hist_chunk_fit(small_total, n_expand, G, a.hist_items, a.hist_slots);
    int64_t* cstart = a.pair_chunk;                 // [n_expand + 1]
    int64_t* pstart = a.pair_chunk + n_expand + 1;  // [n_expand + 1]
    int64_t pcarry = 0;
    carry = 0;
    for (int32_t base = 0; base < n_expand; base += kPlanThreads) {
      const int32_t j = base + tid;
      int64_t nc = 0;
      if (j < n_expand) {
        const LevelNode l = a.next[2 * j], r = a.next[2 * j + 1];
        const int64_t rl = l.end - l.begin, rr = r.end - r.begin;
        nc = ceil_rows(rr < rl ? rr : rl, chunk);
      }
      int64_t total, ptotal;
      const int64_t o = carry + block_scan(nc, scan, &total);
      const int64_t po = pcarry + block_scan(nc >= 2 ? nc : 0, scan, &ptotal);
      carry += total;
      pcarry += ptotal;
      if (j < n_expand) {
        cstart[j] = o;
        pstart[j] = po;
        if (n_expand <= kLdsOffsets) s_off[j] = o;
      }
    }
    const int64_t C = carry;
    if (tid == 0) {
      cstart[n_expand] = C;
      if (n_expand <= kLdsOffsets) s_off[n_expand] = C;
    }
    __syncthreads();
    const int64_t* pair_off = n_expand <= kLdsOffsets ? s_off : cstart;
    const int64_t padded = (C + 7) / 8 * 8;
    n_hist = padded * G;
    if (n_hist > a.hist_capacity || pcarry * T > a.partial_capacity) {
      if (tid == 0) s_error = 4;
      n_hist = 0;
    } else {
      for (int64_t c = tid; c < padded; c += kPlanThreads) {
        HistWork item{0, 0, 0, 0, -1, 0};
        int64_t p = -1;
        if (c < C) {
          const int32_t j = owner(pair_off, n_expand, c);
          const LevelNode l = a.next[2 * j], r = a.next[2 * j + 1];
          const bool right_small = (r.end - r.begin) < (l.end - l.begin);
          const LevelNode sm = right_small ? r : l;
          const int64_t k = c - pair_off[j];
          const int64_t b = sm.begin + k * chunk;
          item = HistWork{2 * j + (right_small ? 1 : 0), 0, b,
                          b + chunk < sm.end ? b + chunk : sm.end, -1, l.parent_slot};
          if (pair_off[j + 1] - pair_off[j] >= 2) p = (pstart[j] + k) * T;
        }
        int32_t g = 0;  // tile group g: its first tile t
        for (int32_t t = 0; t < T; t += TPW) {
          if (pair_second(a.hist_pairs, t)) continue;
          item.tile = t;
          item.partial = p < 0 ? -1 : int32_t(p + t);
          a.hist_work[((c / 8) * G + g) * 8 + (c % 8)] = item;
          ++g;
        }
      }
      for (int32_t j = tid; j < n_expand; j += kPlanThreads) {
        const LevelNode l = a.next[2 * j], r = a.next[2 * j + 1];
        const bool right_small = (r.end - r.begin) < (l.end - l.begin);
        const int32_t nc = int32_t(pair_off[j + 1] - pair_off[j]);
        a.reduce_jobs[j] = HistReduce{2 * j + (right_small ? 1 : 0), 2 * j + (right_small ? 0 : 1),
                                      int64_t(l.parent_slot) * a.hist_elems,
                                      nc >= 2 ? int32_t(pstart[j]) : -1, nc};
      }
      n_reduce = n_expand;
    }
  }

  // ---- D: partition work of the next level ----------------------------------
  int64_t n_part = 0;
  if (next_hist) {
    carry = 0;
    for (int32_t base = 0; base < n_next; base += kPlanThreads) {
      const int32_t i = base + tid;
      int64_t chunks = 0;
      if (i < n_next) {
        const LevelNode nd = a.next[i];
        chunks = ceil_rows(nd.end - nd.begin, a.part_chunk);
      }
      int64_t total;
      const int64_t o = carry + block_scan(chunks, scan, &total);
      carry += total;
      if (i < n_next) {
        a.part_first[i] = int32_t(o);
        if (n_next <= kLdsOffsets) s_off[i] = o;
      }
    }
    n_part = carry;
    if (tid == 0) {
      a.part_first[n_next] = int32_t(n_part);
      if (n_next <= kLdsOffsets) s_off[n_next] = n_part;
    }
    __syncthreads();
    if (n_part > a.part_capacity) {
      if (tid == 0) s_error = 5;
      n_part = 0;
    }
    for (int64_t k = tid; k < n_part; k += kPlanThreads) {
      const int32_t i = n_next <= kLdsOffsets ? owner(s_off, n_next, k) : owner(a.part_first, n_next, k);
      const LevelNode nd = a.next[i];
      const int64_t first = n_next <= kLdsOffsets ? s_off[i] : int64_t(a.part_first[i]);
      const int64_t b = nd.begin + (k - first) * a.part_chunk;
      a.part_work[k] = PartWork{i, 0, b, b + a.part_chunk < nd.end ? b + a.part_chunk : nd.end};
    }
  }

  __syncthreads();
  if (tid == 0) {
    PlanCounts* c = a.counts;
    c->n_level = n_next;
    c->n_nodes = n_nodes0 + n_next;
    c->n_hist = int32_t(n_hist);
    c->n_reduce = n_reduce;
    c->n_part[(a.depth + 1) & 1] = int32_t(n_part);
    c->n_leaf_prev = n_leaf_old;  // the previous planner's leaves
    c->n_leaf = int32_t(n_leaf);
    if (s_error && !c->error) c->error = s_error;
  }
}

// The planner for levels of at most kPlanThreads nodes: thread i owns node i
// for the whole level and keeps the node and its split in registers.  Every
// per-node count the level's work lists need is known once the split is
// read, so two multi-value scans give all offsets (the second depends on the
// histogram chunk, which depends on the first's totals); the offsets and
// segments then sit in LDS, read-only, for the item loops.  Its work lists
// are identical to plan_level_kernel's.  With a.work_left set it sums each
// node's left rows from the partition count's per-item words (node << 32 |
// left rows) itself, so it can run beside the level's scatter (which
// publishes the totals in node_left).
__device__ void plan_small_level(const PlanArgs& a) {
  __shared__ int64_t scan[2 * (kPlanThreads / 64) * 4];
  __shared__ int64_t s_left[kPlanThreads];      // left rows per node (a.work_left set)
  __shared__ int64_t s_tot[4];                  // scan totals for wavefronts without nodes
  __shared__ int64_t s_leaf[kPlanThreads + 1];  // first leaf chunk per node
  __shared__ int64_t s_cs[kPlanThreads + 1];    // first histogram chunk per node
  __shared__ int64_t s_ps[kPlanThreads];        // first partial chunk per node
  __shared__ int64_t s_po[kPlanThreads + 1];    // first partition item per node
  __shared__ int64_t s_begin[kPlanThreads], s_mid[kPlanThreads], s_end[kPlanThreads];
  __shared__ int32_t s_nid[kPlanThreads];
  __shared__ int32_t s_slot[kPlanThreads];  // 2 * rank + (right child is the smaller)
  __shared__ float s_val[kPlanThreads];
  __shared__ int32_t s_error;
  const int tid = threadIdx.x;
  // This thread's node is loaded alongside the counts (the host bound keeps the
  // index inside the level's buffers; the count decides whether it is used).
  LevelNode nd_s{};
  dp_split_record sp_s{};
  int64_t nl_s = 0;
  const bool sum_left = a.splits && a.work_left;
  // This level's partition item words (node << 32 | left rows), kSumBatch per
  // thread at a time; the first batch is loaded with the counts (the host
  // bound keeps the indexes in the buffer, the device count decides which are
  // used).
  constexpr int kSumBatch = 4;
  int64_t item_word[kSumBatch];
  auto load_items = [&](int32_t k0) {
#pragma unroll
    for (int u = 0; u < kSumBatch; ++u) {
      const int32_t k = k0 + u * kPlanThreads < a.part_bound ? k0 + u * kPlanThreads
                                                               : a.part_bound - 1;
      item_word[u] = a.work_left[k];
    }
  };
  if (sum_left && a.part_bound > 0) load_items(tid);
  if (tid < a.cur_bound) {
    nd_s = a.cur[tid];
    if (a.splits) {
      sp_s = a.splits[tid];
      if (!sum_left) nl_s = a.node_left[tid];
    }
  }
  const int32_t n = a.counts->n_level;  // <= kPlanThreads (the host bound)
  const int32_t n_leaf_old = a.counts->n_leaf;
  const int32_t n_nodes0 = a.counts->n_nodes;
  const int32_t n_items = sum_left ? a.counts->n_part[a.depth & 1] : 0;
  const double ug = ldexp(1.0, -a.exps[0]), uh = ldexp(1.0, -a.exps[1]);
  if (sum_left) s_left[tid] = 0;
  __syncthreads();  // every thread has read the counts before any is rewritten
  if (sum_left) {  // item k's count goes to its node
    // Lanes of a wavefront hold consecutive items, which the partition work
    // lists by node: each run of one node is summed in the wavefront (its
    // inclusive prefix minus the prefix before the run's head) and only the
    // run's last lane adds it to the node, instead of one LDS atomic per item
    // on a few addresses.
    const int lane = tid & 63;
    for (int32_t base = 0; base < a.part_bound; base += kSumBatch * kPlanThreads) {
      if (base) load_items(base + tid);
#pragma unroll
      for (int u = 0; u < kSumBatch; ++u) {
        if (base + u * kPlanThreads >= n_items) break;  // uniform (the device count)
        const int32_t k = base + tid + u * kPlanThreads;
        const uint32_t node = uint32_t(uint64_t(item_word[u]) >> 32);
        const bool valid = k < n_items && node < uint32_t(kPlanThreads);
        const int key = valid ? int(node) : -1;
        const int v = valid ? int(item_word[u] & 0xffffffffll) : 0;  // <= kPartChunk
        const int prefix = wave_inclusive_sum32(v);                    // <= 64 * kPartChunk
        const int prev = __shfl_up(key, 1), next = __shfl_down(key, 1);
        const bool head = lane == 0 || prev != key, tail = lane == 63 || next != key;
        const unsigned long long heads = __ballot(head);
        const unsigned long long upto = lane == 63 ? ~0ull : ((2ull << lane) - 1ull);
        const int h = 63 - __clzll(heads & upto);  // the run's head lane
        const int before = __shfl(prefix - v, h);  // the prefix before the run
        if (tail && key >= 0)
          atomicAdd(reinterpret_cast<unsigned long long*>(&s_left[key]),
                    static_cast<unsigned long long>(prefix - before));
      }
    }
    __syncthreads();
    nl_s = s_left[tid];
  }
  if (n > kPlanThreads) {  // the host chose this kernel on a wrong bound
    if (tid == 0) {
      PlanCounts* c = a.counts;
      c->n_level = c->n_hist = c->n_reduce = c->n_leaf = c->n_leaf_prev = 0;
      c->n_part[(a.depth + 1) & 1] = 0;
      if (!c->error) c->error = 6;
    }
    return;
  }
  if (tid == 0) s_error = 0;

  // ---- per-node state and counts ----------------------------------------------
  // Only the wavefronts that hold nodes run the per-node phases (the item
  // loops below use every thread).
  const int n_waves = n > 0 ? (n + 63) >> 6 : 1;
  const bool wave_live = (tid >> 6) < n_waves;  // uniform per wavefront
  const bool live = tid < n;
  LevelNode nd{};
  dp_split_record sp{};
  int64_t nl = 0;
  bool e = false;
  if (live) {
    nd = nd_s;
    if (a.splits) {
      sp = sp_s;
      if (sp.expand) {
        nl = nl_s;
        e = nl > 0 && nl < nd.end - nd.begin;
      }
    }
  }
  const bool next_hist = a.depth + 1 < a.max_depth;  // children get histograms
  const int64_t rows = nd.end - nd.begin, lrows = nl, rrows = rows - nl;
  const bool right_small = rrows < lrows;
  int64_t cnt[4] = {0, 0, 0, 0};
  if (wave_live) {
    cnt[0] = e ? 1 : 0;                                                               // expanded
    cnt[1] = (live && !e) ? ceil_rows(rows, a.leaf_chunk) : 0;                        // leaf chunks
    cnt[2] = (e && next_hist) ? (right_small ? rrows : lrows) : 0;                    // smaller child
    cnt[3] = (e && next_hist)                                                         // partition
                 ? ceil_rows(lrows, a.part_chunk) + ceil_rows(rrows, a.part_chunk)
                 : 0;
  }
  int64_t off[4], tot[4];
  block_scan_live<4>(cnt, off, tot, scan, s_tot, n_waves);  // its barriers also publish s_error = 0
  if (live && a.splits && sp.expand && !e) s_error = 1;
  if (tid == 0 && n_items > a.part_bound) s_error = 7;  // items beyond the host bound
  const int64_t rank = off[0];
  const int32_t n_expand = int32_t(tot[0]);
  const int32_t n_next = 2 * n_expand;

  // ---- A: node records and next-level nodes ----------------------------------
  float leaf_value = 0.0f;
  if (live) {
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
      const int32_t left = n_nodes0 + int32_t(2 * rank);
      info.left = left;
      info.feature = sp.feature;
      info.bin = sp.bin;
      info.default_left = sp.default_left;
      info.loss_chg = sp.loss_chg;
      const int64_t slot = 2 * rank;
      if (left + 1 < a.info_capacity && slot + 1 < a.level_capacity) {
        a.next[slot] = LevelNode{nd.begin, nd.begin + nl, sp.gl, sp.hl, left, tid};
        a.next[slot + 1] = LevelNode{nd.begin + nl, nd.end, nd.g - sp.gl, nd.h - sp.hl, left + 1, tid};
        a.next_sums[2 * slot] = sp.gl;
        a.next_sums[2 * slot + 1] = sp.hl;
        a.next_sums[2 * slot + 2] = nd.g - sp.gl;
        a.next_sums[2 * slot + 3] = nd.h - sp.hl;
        a.next_seg_begin[slot] = nd.begin;
        a.next_seg_begin[slot + 1] = nd.begin + nl;
        a.next_node_left[slot] = 0;
        a.next_node_left[slot + 1] = 0;
        if (a.leaf_children) {  // the children's records, as the next level's planner writes leaves
          for (int c = 0; c < 2; ++c) {
            const LevelNode ch = a.next[slot + c];
            NodeInfo li{};
            li.g = ch.g;
            li.h = ch.h;
            li.begin = ch.begin;
            li.end = ch.end;
            li.parity = (a.depth + 1) & 1;
            const double cg = double(ch.g) * ug, chh = double(ch.h) * uh;
            const double cw = plan_weight(a, cg, chh);
            li.base_weight = float(cw);
            li.sum_hess = float(chh);
            li.bin = -1;
            li.left = -1;
            li.leaf_value = float(cw * a.eta);
            a.info[left + c] = li;
          }
        }
      } else {
        s_error = 2;
      }
    } else {
      info.left = -1;
      leaf_value = float(w * a.eta);
      info.leaf_value = leaf_value;
    }
    if (nd.nid >= 0 && nd.nid < a.info_capacity) a.info[nd.nid] = info;
    else s_error = 2;
  }

  // ---- second scan: histogram chunks of the smaller children -----------------
  const int32_t T = a.n_tiles;
  const int32_t TPW = a.hist_tiles;
  const int32_t G = hist_groups(T, TPW, a.hist_pairs);  // items per row chunk
  const int64_t chunk = hist_chunk_fit(tot[2], tot[0], G, a.hist_items, a.hist_slots);
  const int64_t nc = wave_live ? ceil_rows(cnt[2], chunk) : 0;
  int64_t cnt2[2] = {nc, nc >= 2 ? nc : 0}, off2[2], tot2[2];
  if (live) {
    s_leaf[tid] = off[1];
    s_po[tid] = off[3];
    s_begin[tid] = nd.begin;
    s_mid[tid] = nd.begin + nl;
    s_end[tid] = nd.end;
    s_nid[tid] = nd.nid;
    s_slot[tid] = int32_t(2 * rank) + (right_small ? 1 : 0);
    s_val[tid] = leaf_value;
  }
  if (tid == 0) {
    s_leaf[n] = tot[1];
    s_po[n] = tot[3];
  }
  block_scan_live<2>(cnt2, off2, tot2, scan, s_tot, n_waves);  // its barriers also publish the arrays above
  if (live) {
    s_cs[tid] = off2[0];
    s_ps[tid] = off2[1];
  }
  if (tid == 0) s_cs[n] = tot2[0];
  __syncthreads();
  if (s_error) {  // inconsistent level or capacity exceeded: stop this tree
    if (tid == 0) {
      PlanCounts* c = a.counts;
      c->n_level = c->n_hist = c->n_reduce = c->n_leaf = c->n_leaf_prev = 0;
      c->n_part[(a.depth + 1) & 1] = 0;
      if (!c->error) c->error = s_error;
    }
    return;
  }
  int32_t error = 0;

  // ---- B: leaf work of this level -----------------------------------------
  int64_t n_leaf = tot[1];
  if (n_leaf > a.leaf_capacity) {
    error = 3;
    n_leaf = 0;
  }
  for (int64_t k = tid; k < n_leaf; k += kPlanThreads) {
    const int32_t j = owner(s_leaf, n, k);
    const int64_t b = s_begin[j] + (k - s_leaf[j]) * a.leaf_chunk;
    a.leaf_work[k] = LeafWork{s_val[j], s_nid[j], b,
                              b + a.leaf_chunk < s_end[j] ? b + a.leaf_chunk : s_end[j]};
  }

  // ---- C: histogram work and reduce jobs of the next level ----------------
  int64_t n_hist = 0;
  int32_t n_reduce = 0;
  if (next_hist && n_next > 0) {
    const int64_t C = tot2[0];
    const int64_t padded = (C + 7) / 8 * 8;
    n_hist = padded * G;
    if (n_hist > a.hist_capacity || tot2[1] * T > a.partial_capacity) {
      error = 4;
      n_hist = 0;
    } else {
      for (int64_t c = tid; c < padded; c += kPlanThreads) {
        HistWork item{0, 0, 0, 0, -1, 0};
        int64_t p = -1;
        if (c < C) {
          const int32_t j = owner(s_cs, n, c);
          const int64_t k = c - s_cs[j];
          const bool rs = s_slot[j] & 1;
          const int64_t sb = rs ? s_mid[j] : s_begin[j], se = rs ? s_end[j] : s_mid[j];
          const int64_t b = sb + k * chunk;
          item = HistWork{s_slot[j], 0, b, b + chunk < se ? b + chunk : se, -1, j};
          if (s_cs[j + 1] - s_cs[j] >= 2) p = (s_ps[j] + k) * T;
        }
        int32_t g = 0;  // tile group g: its first tile t
        for (int32_t t = 0; t < T; t += TPW) {
          if (pair_second(a.hist_pairs, t)) continue;
          item.tile = t;
          item.partial = p < 0 ? -1 : int32_t(p + t);
          a.hist_work[((c / 8) * G + g) * 8 + (c % 8)] = item;
          ++g;
        }
      }
      if (e)
        a.reduce_jobs[rank] = HistReduce{int32_t(2 * rank) + (right_small ? 1 : 0),
                                         int32_t(2 * rank) + (right_small ? 0 : 1),
                                         int64_t(tid) * a.hist_elems,
                                         nc >= 2 ? int32_t(off2[1]) : -1, int32_t(nc)};
      n_reduce = n_expand;
    }
  }

  // ---- D: partition work of the next level ----------------------------------
  int64_t n_part = 0;
  if (next_hist && n_next > 0) {
    n_part = tot[3];
    if (e) {
      const int64_t cl = ceil_rows(lrows, a.part_chunk);
      a.part_first[2 * rank] = int32_t(off[3]);
      a.part_first[2 * rank + 1] = int32_t(off[3] + cl);
    }
    if (tid == 0) a.part_first[n_next] = int32_t(n_part);
    if (n_part > a.part_capacity) {
      error = 5;
      n_part = 0;
    }
    for (int64_t k = tid; k < n_part; k += kPlanThreads) {
      const int32_t j = owner(s_po, n, k);
      const int64_t cl = ceil_rows(s_mid[j] - s_begin[j], a.part_chunk);
      int64_t kk = k - s_po[j];
      int32_t node = s_slot[j] & ~1;
      int64_t b, end;
      if (kk < cl) {
        b = s_begin[j] + kk * a.part_chunk;
        end = s_mid[j];
      } else {
        kk -= cl;
        node += 1;
        b = s_mid[j] + kk * a.part_chunk;
        end = s_end[j];
      }
      a.part_work[k] = PartWork{node, 0, b, b + a.part_chunk < end ? b + a.part_chunk : end};
    }
  }

  if (tid == 0) {
    PlanCounts* c = a.counts;
    c->n_level = n_next;
    c->n_nodes = n_nodes0 + n_next;
    c->n_hist = int32_t(n_hist);
    c->n_reduce = n_reduce;
    c->n_part[(a.depth + 1) & 1] = int32_t(n_part);
    c->n_leaf_prev = n_leaf_old;  // the previous planner's leaves
    c->n_leaf = int32_t(n_leaf);
    if (error && !c->error) c->error = error;
  }
}

__global__ __launch_bounds__(kPlanThreads) void plan_small_kernel(PlanArgs a) {
  plan_small_level(a);
}

// A level's planner (workgroup 0) and its scatter (the other workgroups, four
// items at a time) in one launch: both read only what the partition count
// left, and write disjoint buffers (the planner writes the next level's, and
// the next level's partition count in counts->n_part).
template <int G>
__global__ __launch_bounds__(kPlanThreads) void plan_scatter_kernel(PlanArgs a, ScatterArgs sa) {
  if (blockIdx.x == 0) {
    plan_small_level(a);
    return;
  }
  scatter_items<G, kPlanThreads / kPartThreads>(sa, int32_t(blockIdx.x) - 1,
                                                int32_t(gridDim.x) - 1);
}

__global__ __launch_bounds__(256) void plan_root_kernel(
    LevelNode* cur, int64_t* sums, int64_t* seg_begin, PartWork* part_work, int32_t* part_first,
    int64_t* node_left, PlanCounts* counts, int64_t n_rows, const int64_t* __restrict__ root_slots,
    int32_t root_blocks, int64_t part_chunk, uint32_t* __restrict__ ridx,
    const int32_t* __restrict__ exps) {
  __shared__ int64_t part[2][4];
  const int64_t chunks = (n_rows + part_chunk - 1) / part_chunk;
  const int64_t stride = int64_t(blockDim.x) * gridDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n_rows; i += stride)
    ridx[i] = uint32_t(i);
  for (int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; j < chunks; j += stride) {
    const int64_t b = j * part_chunk;
    part_work[j] = PartWork{0, 0, b, b + part_chunk < n_rows ? b + part_chunk : n_rows};
  }
  if (blockIdx.x != 0) return;  // uniform per workgroup: the barrier below is block 0's alone
  int64_t g = 0, h = 0;
  for (int32_t k = threadIdx.x; k < root_blocks; k += blockDim.x) {
    g += root_slots[2 * k];
    h += root_slots[2 * k + 1];
  }
  g = wave_inclusive_sum(g);
  h = wave_inclusive_sum(h);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 63) {
    part[0][wave] = g;
    part[1][wave] = h;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    g = (part[0][0] + part[0][1]) + (part[0][2] + part[0][3]);
    h = (part[1][0] + part[1][1]) + (part[1][2] + part[1][3]);
    cur[0] = LevelNode{0, n_rows, g, h, 0, -1};
    sums[0] = g;
    sums[1] = h;
    seg_begin[0] = 0;
    node_left[0] = 0;
    part_first[0] = 0;
    part_first[1] = int32_t(chunks);
    PlanCounts c{};
    c.n_level = 1;
    c.n_nodes = 1;
    c.n_part[0] = int32_t(chunks);
    if (exps) {  // the tree's records then carry its exponents to the host
      c.exps[0] = exps[0];
      c.exps[1] = exps[1];
    }
    *counts = c;
  }
}

}  // namespace

void launch_plan_level(const PlanArgs& a, int64_t level_bound, hipStream_t s) {
  need(!a.leaf_children || level_bound <= kPlanThreads,
       "the children's leaf records are written by the small planner only");
  if (level_bound <= kPlanThreads)
    hipLaunchKernelGGL(plan_small_kernel, dim3(1), dim3(kPlanThreads), 0, s, a);
  else
    hipLaunchKernelGGL(plan_level_kernel, dim3(1), dim3(kPlanThreads), 0, s, a);
  DP_HIP(hipGetLastError());
}

void launch_plan_scatter(const PlanArgs& a, const ScatterArgs& sa, int64_t n_rows,
                         hipStream_t s) {
  need(a.work_left && a.splits, "the merged planner sums the left counts");
  need(a.cur_bound <= kPlanThreads, "the merged planner takes levels of at most 1024 nodes");
  const int32_t items = sa.n_work_host < 2048 ? sa.n_work_host : 2048;
  constexpr int Q = kPlanThreads / kPartThreads;
  const int blocks = 1 + (items + Q - 1) / Q;
  const int group = part_group(n_rows);  // load groups as the partition's
  auto k = group == 4 ? plan_scatter_kernel<4>
                      : (group == 2 ? plan_scatter_kernel<2> : plan_scatter_kernel<1>);
  hipLaunchKernelGGL(k, dim3(blocks), dim3(kPlanThreads), 0, s, a, sa);
  DP_HIP(hipGetLastError());
}

void launch_plan_root(LevelNode* cur, int64_t* sums, int64_t* seg_begin, PartWork* part_work,
                      int32_t* part_first, int64_t* node_left, PlanCounts* counts,
                      int64_t n_rows, const int64_t* root_slots, int32_t root_blocks,
                      int64_t part_chunk, uint32_t* ridx, hipStream_t s,
                      const int32_t* exps) {
  need(part_chunk >= 1 && part_chunk <= kPartChunk, "partition chunk out of range");
  need(root_blocks >= 1, "root sums need at least one slot");
  hipLaunchKernelGGL(plan_root_kernel, dim3(grid_for(n_rows, 256, 1024)), dim3(256), 0, s, cur,
                     sums, seg_begin, part_work, part_first, node_left, counts, n_rows, root_slots,
                     root_blocks, part_chunk, ridx, exps);
  DP_HIP(hipGetLastError());
}

}  // namespace dp
