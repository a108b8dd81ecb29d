// Internal declarations shared by the HIP kernel files and the host library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/dpgbdt.h"
#include "sample.hpp"

namespace dp {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

[[noreturn]] inline void fail(const std::string& message) { throw Error(message); }
inline void need(bool ok, const std::string& message) {
  if (!ok) fail(message);
}
inline void hip_check(hipError_t status, const char* what) {
  if (status != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(status));
}
#define DP_HIP(call) ::dp::hip_check((call), #call)

// Cached allocations for the booster's training buffers (pool.cpp).  A block
// handed back is kept, by device and exact size, for the next allocation of
// that size (a new booster on the same configuration, a study's next trial)
// instead of going through hipMalloc / hipHostMalloc again.  Only buffers
// whose last use has completed may be handed back: their owners synchronise
// their streams first.  A miss that the device cannot serve empties the cache
// and retries.
// device_pool_get reports the device the block belongs to (the current one);
// device_pool_put files the block under that device, whichever is current.
void* device_pool_get(size_t bytes, int* device);
void device_pool_put(void* p, size_t bytes, int device);
void* pinned_pool_get(size_t bytes);
void pinned_pool_put(void* p, size_t bytes);

// Owning device allocation (POOLED: through the cache above).
template <class T, bool POOLED = false>
struct DeviceBuffer {
  T* p = nullptr;
  size_t n = 0;
  int dev = 0;  // POOLED: the device the block belongs to
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t count) { resize(count); }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& o) noexcept : p(o.p), n(o.n), dev(o.dev) { o.p = nullptr; o.n = 0; }
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
      release();
      p = o.p;
      n = o.n;
      dev = o.dev;
      o.p = nullptr;
      o.n = 0;
    }
    return *this;
  }
  ~DeviceBuffer() { release(); }
  void release() {
    if (p) {
      if (POOLED) device_pool_put(p, n * sizeof(T), dev);
      else (void)hipFree(p);
    }
    p = nullptr;
    n = 0;
  }
  void resize(size_t count) {
    release();
    if (count) {
      if (POOLED) p = static_cast<T*>(device_pool_get(count * sizeof(T), &dev));
      else DP_HIP(hipMalloc(reinterpret_cast<void**>(&p), count * sizeof(T)));
    }
    n = count;
  }
  // Grows (discarding contents) when smaller than `count`.
  void reserve(size_t count) {
    if (count > n) resize(count);
  }
  size_t bytes() const { return n * sizeof(T); }
};
template <class T>
using PooledBuffer = DeviceBuffer<T, true>;

// Pinned host allocation (hipHostMalloc; never hipHostRegister).
template <bool POOLED = false>
struct PinnedBufferT {
  uint8_t* p = nullptr;
  size_t n = 0;
  PinnedBufferT() = default;
  PinnedBufferT(const PinnedBufferT&) = delete;
  PinnedBufferT& operator=(const PinnedBufferT&) = delete;
  ~PinnedBufferT() { release(); }
  void release() {
    if (p) {
      if (POOLED) pinned_pool_put(p, n);
      else (void)hipHostFree(p);
    }
    p = nullptr;
    n = 0;
  }
  void reserve(size_t count) {
    if (count <= n) return;
    release();
    if (POOLED) p = static_cast<uint8_t*>(pinned_pool_get(count));
    else DP_HIP(hipHostMalloc(reinterpret_cast<void**>(&p), count, hipHostMallocDefault));
    n = count;
  }
};
using PinnedBuffer = PinnedBufferT<false>;
using PooledPinnedBuffer = PinnedBufferT<true>;

// Fixed-point quantiser precision: |q| <= 2^kQuantBits.
constexpr int kQuantBits = 30;
constexpr double kRtEps = 1e-6;

// Best candidate of one (node, feature) from the split evaluation, or loss
// -inf when the feature has none.
struct FeatCand {
  double loss;
  long long gl, hl;
  int32_t bin, dl;
};
constexpr int kMaxBins = 256;
// Missing symbol of 16-bit bins: a matrix with missing values some of whose
// features use all 256 bins keeps 16-bit columns (the layout's missing_bin is
// then kWideMissing) and histograms from the present-value layout, which
// stores no missing values.
constexpr int32_t kWideMissing = 256;

// One histogram work item: rows [begin, end) of node `slot` for one tile.
// partial >= 0: the workgroup stores its tile histogram in partial slot
// `partial` (summed later by the reduce pass); partial < 0: the item is the
// node's only chunk and writes the node histogram's tile directly.  parent:
// the parent's histogram slot in the previous level (the node's sibling is
// slot ^ 1), or -1 when the node has no sibling (the root).
struct HistWork {
  int32_t slot;
  int32_t tile;
  int64_t begin;
  int64_t end;
  int32_t partial;
  int32_t parent;
};

// One reduce job (all tiles of one built node): node histogram `slot` = sum
// of the partial tiles (p0 + k) * n_tiles + tile, k < nc (or, for nc == 1 with
// a direct item, what that item wrote); then, when sibling >= 0, node
// `sibling` = parent histogram at element offset `parent` - node `slot`.
struct HistReduce {
  int32_t slot;
  int32_t sibling;
  int64_t parent;
  int32_t p0;
  int32_t nc;
};

// One partition work item: rows [begin, end) of ridx, belonging to `node`.
struct PartWork {
  int32_t node;
  int32_t pad;
  int64_t begin;
  int64_t end;
};

// One margin-update work item.
struct LeafWork {
  float value;
  int32_t pad;
  int64_t begin;
  int64_t end;
};

// A node of the level being grown (device-side planning).
struct LevelNode {
  int64_t begin, end;  // segment of ridx (buffer = depth & 1)
  int64_t g, h;        // quantised sums
  int32_t nid;         // tree node id
  int32_t parent_slot; // index of the parent in the previous level
};

// Everything the host needs about one tree node, written by the planner.
struct NodeInfo {
  int64_t g, h;        // quantised sums
  int64_t begin, end;  // final segment (leaves) / segment when split
  double loss_chg;
  int32_t left;        // left child id, -1 for a leaf
  int32_t feature, bin, default_left;
  float leaf_value, base_weight, sum_hess;
  int32_t parity;      // ridx buffer holding the segment
};

// Device counters of the planner (one struct per tree).
struct PlanCounts {
  int32_t n_level;     // nodes of the current level
  int32_t n_nodes;     // nodes allocated in the tree so far
  int32_t n_hist;      // histogram work items for the current level
  int32_t n_reduce;    // histogram reduce jobs for the current level
  int32_t n_leaf;      // leaf work items produced by the last planner run
  int32_t error;       // nonzero: inconsistent partition counts
  int32_t n_leaf_prev; // leaf work items of the planner run before the last
  int32_t pad;
  int32_t exps[2];     // the tree's quantiser exponents (g, h), stored by its root planner
  // Partition work items of the level of depth d in n_part[d & 1]: the planner
  // of level d writes level d + 1's while that level's scatter, in the same
  // launch, still reads level d's.
  int32_t n_part[2];
};

}  // namespace dp

// Device scratch shared by the operator entry points.  Host-side data for a
// call is staged into pinned memory and copied with one async copy; the
// staging buffer is reused only after the previous copy has completed.
struct dp_workspace_s {
  int device = 0;
  dp::DeviceBuffer<uint8_t> staged_dev;
  dp::PinnedBuffer staged_host;
  dp::DeviceBuffer<uint8_t> scratch;
  hipEvent_t staged_done = nullptr;
  size_t staged_used = 0;
  size_t scratch_used = 0;

  dp_workspace_s();
  ~dp_workspace_s();
  // Starts a call: waits for the previous staging copy, resets bump offsets
  // and makes room for `staging_bytes` of staged data (each stage() call adds
  // up to 255 bytes of alignment).
  void begin(size_t staging_bytes = 0);
  // Reserves room for `count` T in the staging area; returns the host pointer.
  template <class T>
  T* stage(size_t count, T** device_ptr) {
    size_t offset = (staged_used + 255) & ~size_t(255);
    size_t bytes = count * sizeof(T);
    grow_staging(offset + bytes);
    staged_used = offset + bytes;
    *device_ptr = reinterpret_cast<T*>(staged_dev.p + offset);
    return reinterpret_cast<T*>(staged_host.p + offset);
  }
  // Copies everything staged since begin() to the device on `stream`, unless
  // the device area already holds exactly these bytes from the previous
  // commit (a repeated call with the same work lists issues no copy).
  void commit(hipStream_t stream);
  // Device-only scratch, valid until the next begin().
  template <class T>
  T* take(size_t count) {
    size_t offset = (scratch_used + 255) & ~size_t(255);
    size_t bytes = count * sizeof(T);
    if (offset + bytes > scratch.n) {
      need_scratch(offset + bytes);
    }
    scratch_used = offset + bytes;
    return reinterpret_cast<T*>(scratch.p + offset);
  }
  void reserve_scratch(size_t bytes);

 private:
  std::vector<uint8_t> committed_;  // the bytes the device staging area holds
  void grow_staging(size_t bytes);
  [[noreturn]] void need_scratch(size_t bytes);
};

namespace dp {

// ---- kernel launchers (implemented in the .hip files) -------------------
// Kernels that take (n_host, n_dev) process n_dev ? *n_dev : n_host items; the
// host value is then an upper bound used to size a persistent grid.
void launch_fill_i64(int64_t* p, int64_t n, int64_t value, hipStream_t s);
// p[0 .. (*n_dev) * per) = 0, at most bound * per elements.
void launch_zero_i64_dev(int64_t* p, const int32_t* n_dev, int64_t per, int64_t bound,
                         hipStream_t s);
void launch_fill_u8(uint8_t* p, int64_t n, uint8_t value, hipStream_t s);
void launch_iota_u32(uint32_t* p, int64_t n, hipStream_t s);

// Launch shape of the dense histogram kernel, chosen per matrix shape by the
// autotuner (tune.cpp) or forced by booster parameters: 16-feature tiles per
// work item (1 or 2), rows per lane per pipeline step (1 or 2), the work
// items a pass aims at (which sets the rows per item), and with two tiles the
// lane bit (4 or 5; 0 = none) that swaps a lane's tile order.
struct HistConfig {
  int32_t tiles = 1;
  int32_t unroll = 2;
  int32_t items = 1024;
  int32_t split = 0;
  int32_t deep = 0;  // 1: three blocks of rows in flight per workgroup (split 0 only)
};

// Paired tiles (dp_bin_layout::paired_tiles): bit t joins tiles t and t + 1
// into one work item whose rows add one joint byte per feature pair.
// hist_pairs gives the pairs a configuration uses: with one tile per item
// every pair (the pair's item replaces two), with two every pair that is an
// item's two tiles (t even).
__host__ __device__ inline uint64_t hist_pairs(uint64_t paired_tiles, int32_t tiles) {
  return tiles == 1 ? paired_tiles : paired_tiles & 0x5555555555555555ull;
}
// Work items per row chunk: tile groups of `tiles` tiles (one tile: less one
// per pair).
__host__ __device__ inline int32_t hist_groups(int32_t n_tiles, int32_t tiles, uint64_t pairs) {
  return tiles == 1 ? n_tiles - __builtin_popcountll(pairs) : (n_tiles + tiles - 1) / tiles;
}
// Tile t is the second of a pair (its rows go with tile t - 1's item).
__host__ __device__ inline bool pair_second(uint64_t pairs, int32_t t) {
  return t >= 1 && t <= 64 && ((pairs >> (t - 1)) & 1ull);
}
// The pairs of a matrix: tiles t, t + 1 (left to right, t < 63) whose
// features all have at most 16 bins (n_bins[f], f < n_features; pad features
// count as such); none when the matrix has missing values.
uint64_t pair_tiles(const int32_t* n_bins, int32_t n_features, int32_t n_tiles, bool missing);
// Rejects a layout whose paired_tiles the histogram kernel cannot take.
void check_pairs(const dp_bin_layout& layout);

// Histograms: every work item accumulates into hist[slot]; hist must be zero.
// Direct items write hist; the others write partial (int64 [slot][bin_stride * 32]).
// row_major: optional row-major copy of the bins (launch_tiles_to_rows), read
// for gathered rows; when the configuration uses the layout's pairs (one tile
// per item), it must be the copy that holds each pair's joint tile in place of
// its first tile (launch_tiles_to_rows with that layout), else the plain copy.
// The work items must come from the same cfg.tiles and layout (its
// paired_tiles: launch_hist pairs what make_hist_work paired).
// skip (matrices without missing values): per tile, the 16 features' skip
// bins ([n_tiles][16] bytes); rows in a feature's skip bin add nothing, so that
// bin's sums stay zero (the split evaluation restores them from the node's
// totals: launch_evaluate's skip argument).  fmaj: partial slots are stored
// feature-major, [16 features][bin_stride][g, h] (the node histogram's layout
// restricted to the tile), for launch_reduce_evaluate_dense; otherwise as the
// LDS image [bin][g of 16 features, h of 16 features] (launch_hist_reduce).
// Histogram workgroups the device holds at once for launch_hist's kernel of
// this configuration (gathered or contiguous rows; missing values; skip bins;
// paired tiles in use).
int hist_resident(bool gather, bool missing, bool skip, const HistConfig& cfg,
                  bool paired = false);
void launch_hist(const uint8_t* bins, const dp_bin_layout& layout, const int32_t* gpair,
                 const uint32_t* ridx, const HistWork* work, int32_t n_work,
                 const int32_t* n_work_dev, int32_t bin_stride, int64_t* hist,
                 int64_t* partial, hipStream_t s, const uint8_t* row_major = nullptr,
                 const HistConfig& cfg = HistConfig{}, const uint8_t* skip = nullptr,
                 bool fmaj = false);
// counts[f][b] = rows whose bin of feature f is b ([n_features][256] uint32),
// from the column copy cols[f][row].
void launch_bin_counts(const uint8_t* cols, int64_t n_rows, int32_t n_features,
                       unsigned int* counts, hipStream_t s);
// Completes the histograms of launch_hist: sums partial tiles, writes built
// and sibling node histograms.  accumulate: add the sums to hist instead of
// storing them (then no job may rely on a direct item).
void launch_hist_reduce(const int64_t* partial, const HistReduce* jobs, int32_t n_jobs,
                        const int32_t* n_jobs_dev, int32_t n_tiles, int32_t n_features,
                        int32_t bin_stride, const int64_t* parent_base, int64_t* hist,
                        bool accumulate, hipStream_t s);
// Minimum rows per histogram chunk and the chunk size for `rows` rows when
// each row chunk makes `groups` work items: at most `items` work items in all
// on large levels (items / groups row chunks, rounded down to a multiple of 8,
// the XCD interleave's unit, so that a group count that does not divide
// `items` -- seven with one pair of eight tiles -- leaves no real item behind
// the padding of a last partial block of 8 chunks, past the workgroups the
// chip holds at once).  On smaller levels of matrices
// with at most four groups, about k * 256 items (k whole items per CU, k =
// 1..3), so that no CU is left with one more item after the others finish
// (with more groups the item count moves in steps of the group count, and the
// rule measured no better).
constexpr int64_t kHistMinChunk = 4096;
__host__ __device__ inline int64_t hist_chunk(int64_t rows, int32_t groups, int32_t items) {
  const int64_t units = rows * groups;
  int64_t c;
  if (groups <= 4 && units < int64_t(items) * kHistMinChunk &&
      units < (int64_t(1) << 31)) {  // 32-bit division
    const uint32_t u = uint32_t(units);
    const uint32_t k = u < 256u * kHistMinChunk ? 1u : u / uint32_t(256 * kHistMinChunk);
    c = int64_t((u + 256u * k - 1u) / (256u * k));
  } else {
    int64_t per = items >= groups ? items / groups : 1;  // row chunks
    if (per >= 8) per = per / 8 * 8;
    c = (rows + per - 1) / per;
  }
  return c < kHistMinChunk ? kHistMinChunk : c;
}
// A level's chunk: hist_chunk's, enlarged when that moves the level's items
// into one round fewer of the `slots` workgroups the chip holds at once (the
// last round of items, if only partly filled, takes as long as a full one:
// measured on C3's gathered passes, 264-276 items on 256 slots took two rounds
// for one round's work).  The items are at most (ceil(rows / chunk) + nodes) *
// groups (rows: the built nodes' rows, nodes: their count); the larger chunk
// keeps that bound within (rounds - 1) * slots, and only replaces hist_chunk's
// when (rounds - 1) * chunk is the shorter time.  It is never smaller, so the
// level's items and partial slots stay within hist_chunk's capacity bounds.
// slots <= 0: hist_chunk's chunk.
__host__ __device__ inline int64_t hist_chunk_fit(int64_t rows, int64_t nodes, int32_t groups,
                                                  int32_t items, int32_t slots) {
  const int64_t c = hist_chunk(rows, groups, items);
  if (slots <= 0 || rows <= 0 || groups <= 0) return c;
  const int64_t per_round = slots / groups;  // chunks that fit one round
  const int64_t bound = (rows + c - 1) / c + nodes;
  const int64_t rounds = (bound * groups + slots - 1) / slots;
  if (rounds < 2) return c;
  const int64_t avail = (rounds - 1) * per_round - nodes;
  if (avail <= 0) return c;
  const int64_t c2 = (rows + avail - 1) / avail;
  return c2 > c && (rounds - 1) * c2 < rounds * c ? c2 : c;
}
// Partial slots needed by one level: the chunks of nodes with two or more
// chunks number at most 2 * items / groups, each with n_tiles slots (groups:
// hist_groups, at least n_tiles / 2 with pairs).
inline int64_t hist_partial_capacity(int32_t n_tiles, const HistConfig& cfg, uint64_t pairs) {
  const int64_t g = hist_groups(n_tiles, cfg.tiles, hist_pairs(pairs, cfg.tiles));
  return (2 * int64_t(cfg.items) * n_tiles + g - 1) / g + int64_t(n_tiles);
}
// Work items and reduce jobs for the histograms of n_nodes row sets (node i:
// [begin[i], end[i]) of ridx, written to hist slot slots[i], or i when slots
// is null), chunked and ordered for the XCD-aware dispatch; the work may hold
// empty padding items.  allow_direct: single-chunk nodes write directly.
// n_tiles > 0 overrides the layout's tile count (present-value tiles).
// Returns the number of partial slots used.
// n_tiles > 0: present-value tiles, one per item; otherwise cfg.tiles of the
// layout's 16-feature tiles per item, and with one tile per item one item for
// each pair of paired_tiles (its partial slots stay one per tile).
int32_t make_hist_work(const dp_bin_layout& layout, const int64_t* begin, const int64_t* end,
                       const int32_t* slots, int32_t n_nodes, bool allow_direct,
                       std::vector<HistWork>& work, std::vector<HistReduce>& jobs,
                       int32_t n_tiles = 0, const HistConfig& cfg = HistConfig{});
void launch_subtract(const int64_t* parent, const int64_t* built, int64_t* sibling, int64_t n,
                     hipStream_t s);


// Split evaluation; scratch holds evaluate_scratch_bytes(n_nodes, n_features)
// (the per-feature candidates, as FeatCand [node][feature]).  Returns whether
// the split records were written: always with select; without it, only for
// matrices few enough features for one workgroup per node -- otherwise the
// caller selects from the candidates (SplitSelect in launch_partition).
// With at most kEvalNodeFeatures features the evaluation writes the split
// records itself (one workgroup per node) and uses no scratch.
constexpr int kEvalNodeFeatures = 16;
size_t evaluate_scratch_bytes(int32_t n_nodes, int32_t n_features);
bool launch_evaluate(const int64_t* hist, int32_t n_nodes, const int32_t* n_nodes_dev,
                     int32_t n_features, int32_t bin_stride, const int32_t* n_bins,
                     const int64_t* node_sums, const int32_t* exps, int32_t exp_g, int32_t exp_h,
                     const dp_train_param& param, void* scratch, dp_split_record* out,
                     hipStream_t s, bool select = true, const uint32_t* fmask = nullptr,
                     const uint8_t* skip_bins = nullptr);
// skip_bins ([n_features] bytes, matrices without missing values): the
// histograms leave each feature's skip bin at zero (launch_hist's skip); the
// node's remaining sums (totals minus the bins) are that bin's.
// Present-value layout (at most 64 bins, tiles of a multiple of 16 features):
// launch_hist_reduce_flat and launch_evaluate(..., select = false) in one
// launch -- the same node histograms (built and sibling) and the same
// per-feature candidates in scratch.  exps: the quantiser exponents in device
// memory.  skip_direct: jobs whose node was built by one direct item are left
// alone (launch_hist_sparse's evaluation did them).
void launch_reduce_evaluate_flat(const int64_t* partial, const HistReduce* jobs, int32_t n_jobs,
                                 const int32_t* n_jobs_dev, int32_t n_tiles, int32_t tile_features,
                                 int32_t n_features, int32_t bin_stride,
                                 const int64_t* parent_base, int64_t* hist, const int32_t* n_bins,
                                 const int64_t* node_sums, const int32_t* exps,
                                 const dp_train_param& param, const uint32_t* fmask,
                                 const uint8_t* skip_bins, void* scratch, bool store,
                                 hipStream_t s, bool skip_direct = false);
// Feature counts from which the booster's dense levels below the root use
// feature-major partial slots and launch_reduce_evaluate_dense, and from which
// that launch takes four features per workgroup instead of one.
constexpr int32_t kDenseFuseFeatures = 17;
constexpr int32_t kDenseWideFeatures = 256;
// Dense levels whose partial slots are feature-major (launch_hist's fmaj):
// launch_hist_reduce and launch_evaluate(..., select = false) in one launch --
// the same node histograms (built and sibling; none stored when !store) and the
// same per-feature candidates in scratch.  At most 256 bins.
void launch_reduce_evaluate_dense(const int64_t* partial, const HistReduce* jobs, int32_t n_jobs,
                                  const int32_t* n_jobs_dev, int32_t n_tiles, int32_t n_features,
                                  int32_t bin_stride, const int64_t* parent_base, int64_t* hist,
                                  const int32_t* n_bins, const int64_t* node_sums,
                                  const int32_t* exps, const dp_train_param& param,
                                  const uint32_t* fmask, const uint8_t* skip_bins, void* scratch,
                                  bool store, hipStream_t s);
// Column sampling of one level (ColSample active): masks[node][ceil(F / 32)]
// gets each node's feature sample (bit f set: feature f is a candidate), for
// the node count *n_dev (n_host when null; n_host bounds the grid).  depth is
// the level's depth; nodes supply the node ids.
void launch_colsample(const LevelNode* nodes, int32_t n_host, const int32_t* n_dev,
                      int32_t n_features, const ColSample& cs, int32_t depth, uint32_t* masks,
                      hipStream_t s);

// Margin (and optional leaf id) update of leaf chunks: margin[ridx[i] *
// stride] += value, positions[ridx[i]] = leaf id; work count from n_dev when
// set, else n_host (an upper bound for grid sizing either way).  With store
// set, margin[ridx[i] * stride] = value instead: `margin` is then the tree's
// leaf-value plane, which launch_add_leaf_values adds to the margins.
struct LeafPass {
  const uint32_t* ridx = nullptr;
  const LeafWork* work = nullptr;
  const int32_t* n_dev = nullptr;
  int32_t n_host = 0;
  float* margin = nullptr;
  int64_t stride = 1;
  int32_t* positions = nullptr;
  bool store = false;
};

// The partition scatter's arguments (scatter.hpp).
struct ScatterArgs {
  const uint32_t* ridx_in;
  uint32_t* ridx_out;
  const PartWork* work;
  int32_t n_work_host;       // bound of the item count (grid sizing, first-item prefetch)
  const int32_t* n_work_dev; // the item count; n_work_host when null
  const dp_split_record* splits;
  const int64_t* seg_begin;
  const int32_t* node_first_work;
  const int64_t* work_left;
  const unsigned long long* masks;
  int64_t* node_left;        // the node's first item writes the node's left total; may be null
};

// The last split level's leaf values, stored by its count launch (every child
// is a leaf, so the rows need no new order): a row of an expanding node gets
// values[row] = its child's leaf value, eta times the leaf weight of the
// child's quantised sums (split record and nodes[node]); a row of a node that
// does not expand gets the node's own leaf value.
struct LastLevel {
  float* values;  // the tree's leaf-value plane, one float per row
  const LevelNode* nodes;
  const int32_t* exps;  // quantiser exponents (gradient, hessian)
  double eta, lambda, alpha, mcw;
};

// Partition: counts, then scatter (which writes the left totals of the
// expanding nodes into node_left).  cols: column-major copy of the bins
// (launch_tiles_to_columns) or null to read the tiles.  work_left: one word
// per work item, the item's node in the upper 32 bits and its left rows in the
// lower 32 (zero for a node that does not expand); masks: kPartMasks words per
// work item (the count kernel's ballots, read back by the scatter).  node_left_zeroed: the caller has zeroed
// node_left[0, nodes) (non-expanding nodes keep 0); else it is cleared here
// for n_nodes nodes.  deferred: when given, the scatter is not launched; its
// arguments are written there (n_work_host = 0: nothing to scatter) for
// launch_plan_scatter.  last: the last split level's margin update is done by
// the count launch, and no scatter is launched or deferred (ridx_out is not
// written; the count still writes work_left for the level's planner).
// Per-feature candidates left by launch_evaluate(..., select = false): the
// partition count selects each node's split from them and writes the records.
struct SplitSelect {
  const FeatCand* cand = nullptr;
  int32_t n_features = 0;
  double gamma = 0.0;
};
// cols: the column copy, uint8 symbols, or uint16 when layout.missing_bin is
// kWideMissing (such a layout has no tile-major bins: cols is required).
void launch_partition(const uint8_t* bins, const void* cols, const dp_bin_layout& layout,
                      const uint32_t* ridx_in, uint32_t* ridx_out, const PartWork* work,
                      int32_t n_work, const int32_t* n_work_dev, const int64_t* seg_begin,
                      dp_split_record* splits, const int32_t* node_first_work,
                      int32_t n_nodes, const int32_t* n_nodes_dev, int64_t* work_left,
                      unsigned long long* masks, int64_t* node_left, bool node_left_zeroed,
                      hipStream_t s, const LeafPass* leaves = nullptr,
                      const SplitSelect* select = nullptr, ScatterArgs* deferred = nullptr,
                      const LastLevel* last = nullptr);
constexpr int64_t kPartChunk = 4096;
constexpr int kPartMasks = 64;  // ballot words per partition work item (kPartChunk / 64)

// A list of leaf chunks over the rows of one row-id buffer; count from n_dev
// when set, else n_host (an upper bound for grid sizing either way).
struct LeafList {
  const uint32_t* ridx = nullptr;
  const LeafWork* work = nullptr;
  int32_t n_host = 0;
  const int32_t* n_dev = nullptr;
};
// margin[ridx[i] * stride] += value for the chunks of the list (ridx, work,
// n_work, n_work_dev) and, in the same launch, of `second` when given; with
// store, margin[ridx[i] * stride] = value (a leaf-value plane).
void launch_update_margin(const uint32_t* ridx, const LeafWork* work, int32_t n_work,
                          const int32_t* n_work_dev, float* margin, int64_t stride, hipStream_t s,
                          const LeafList* second = nullptr, bool store = false);
// margin[row * n_groups + k] += values[k * n_rows + row] for every row and
// output group k: a round's trees' leaf-value planes (each row of each plane
// stored once by its tree's leaf passes) added to the margins in row order.
void launch_add_leaf_values(float* margin, int32_t n_groups, const float* values, int64_t n_rows,
                            hipStream_t s);
void launch_leaf_positions(const uint32_t* ridx, const LeafWork* work, int32_t n_work,
                           const int32_t* n_work_dev, int32_t* positions, hipStream_t s);

// Device-side level planner (grow.hip): one workgroup turns the evaluated
// level (split records, left counts) into the tree's node records, the next
// level's nodes, and the next level's histogram / subtraction / partition work
// plus this level's leaf work.  Counts live in `counts`.
struct PlanArgs {
  const LevelNode* cur;
  const dp_split_record* splits;  // null: every node of this level is a leaf
  const int64_t* node_left;
  int64_t* next_node_left;  // zeroed for the next level's nodes
  LevelNode* next;
  int64_t* next_sums;      // [slot][2]
  int64_t* next_seg_begin; // [slot]
  NodeInfo* info;          // indexed by node id
  HistWork* hist_work;
  HistReduce* reduce_jobs;
  PartWork* part_work;
  int32_t* part_first;     // [n_next + 1]
  int64_t* pair_chunk;     // scratch: 2 x [n_pairs + 1] first chunk / first partial chunk
  LeafWork* leaf_work;
  PlanCounts* counts;
  const int32_t* exps;     // quantiser exponents (gradient, hessian)
  int32_t depth, max_depth;
  int32_t n_tiles;
  int32_t hist_tiles;      // tiles per histogram work item (HistConfig::tiles; 1 for present-value)
  uint64_t hist_pairs;     // paired tiles of the level's items (hist_pairs; 0 for present-value)
  int32_t hist_items;      // work items a histogram pass aims at (HistConfig::items)
  int32_t hist_slots;      // histogram workgroups the chip holds at once (hist_chunk_fit; 0: off)
  int64_t hist_elems;      // int64 values per node histogram
  int64_t part_chunk, leaf_chunk;  // rows per partition / margin-update item
  double eta, lambda, alpha, mcw;
  int32_t info_capacity, level_capacity;
  int32_t hist_capacity, partial_capacity, part_capacity, leaf_capacity;
  // Entries of cur, splits and node_left that may be read before the level's
  // node count is known (the host's bound of this level's size).
  int32_t cur_bound;
  // Set: left rows are summed from the partition count's per-item words (node
  // << 32 | left rows) instead of read from node_left.
  const int64_t* work_left;
  int32_t part_bound;  // host bound of this level's partition items (sizes work_left)
  // Set on the last split level when no planner runs for the next level: the
  // children's node records are written here, as leaves (the small planner).
  int32_t leaf_children;
};
// level_bound: an upper bound of the level's node count (selects the planner).
void launch_plan_level(const PlanArgs& a, int64_t level_bound, hipStream_t s);
// The planner of a level of at most 1024 nodes (a.work_left set) and the
// level's partition scatter (the arguments launch_partition deferred) in one
// launch.
void launch_plan_scatter(const PlanArgs& a, const ScatterArgs& sa, int64_t n_rows,
                         hipStream_t s);
// ridx[i] = i for i < n_rows; counts->n_level = 1, n_nodes = 1, ...; cur[0] =
// root {0, n_rows, g, h, 0, -1} with (g, h) the sum of the root_blocks (g, h)
// pairs of root_slots (the quantiser's per-workgroup sums of this output);
// sums[0..1] = (g, h), seg_begin[0] = 0, node_left[0] = 0; root partition work
// over [0, n_rows).
void launch_plan_root(LevelNode* cur, int64_t* sums, int64_t* seg_begin, PartWork* part_work,
                      int32_t* part_first, int64_t* node_left, PlanCounts* counts,
                      int64_t n_rows, const int64_t* root_slots, int32_t root_blocks,
                      int64_t part_chunk, uint32_t* ridx, hipStream_t s,
                      const int32_t* exps = nullptr);
// Upper bounds of the planner's outputs for a level of at most `nodes` nodes.
inline int64_t plan_hist_capacity(int64_t nodes, int32_t groups, int32_t items) {
  return items + int64_t(groups) + (nodes / 2 + 8) * int64_t(groups);
}
// Rows per partition / leaf-value work item of the planner: about 1024 items
// over the matrix, a multiple of 256 in [256, kPartChunk] (measured against
// about 2048, 1536 and 768 items: C2 at 1M rows 2,290 / 2,414 / 2,449 against
// 2,460 trees/s here, C5 at 2M rows 615 / 630 / 627 against 634).
inline int64_t row_chunk(int64_t n_rows) {
  const int64_t c = (n_rows / 1024 + 255) / 256 * 256;
  return c < 256 ? 256 : (c > kPartChunk ? kPartChunk : c);
}
// 256-row steps whose row ids, then bins, a partition lane loads together
// (count and scatter): four once items have 1024 rows or more (more loads in
// flight; C2 2,460 -> 2,483 trees/s against two), else the steps of one
// row_chunk item, at most two.
inline int part_group(int64_t n_rows) {
  const int64_t c = row_chunk(n_rows);
  return c >= 1024 ? 4 : (c >= 512 ? 2 : 1);
}
inline int64_t plan_part_capacity(int64_t nodes, int64_t n_rows, int64_t chunk) {
  return n_rows / chunk + 1 + nodes;
}
inline int64_t plan_leaf_capacity(int64_t nodes, int64_t n_rows, int64_t chunk) {
  return n_rows / chunk + 1 + nodes;
}
// Histogram work items of a level of at most `nodes` nodes with `groups`
// items per row chunk: C <= min(items / groups + 1, n_rows / (2 kHistMinChunk))
// + nodes / 2 row chunks, padded to 8.
inline int64_t plan_hist_items(int64_t nodes, int64_t n_rows, int32_t groups, int32_t items) {
  const int64_t a = items / groups + 1, b = n_rows / (2 * kHistMinChunk);
  return ((a < b ? a : b) + nodes / 2 + 8) * int64_t(groups);
}
constexpr int64_t kLeafChunk = 16384;  // margin-update items of the operator API

// margin[r * n_outputs + k] = base[k] (base: n_outputs device floats).
void launch_init_margin(float* margin, int64_t n_rows, int32_t n_outputs, const float* base,
                        hipStream_t s);

// Objective gradients.  With quant_scratch (quantise_scratch_bytes) and one
// output, the per-workgroup maxima the quantiser needs are written too and
// true is returned (pass maxima_ready to launch_quantise).
// values (optional, planes [n_classes][n_rows]): leaf values added to the
// margins first (margin[r * n_classes + k] += values[k * n_rows + r], stored),
// as launch_add_leaf_values would, so a round's add rides in the next round's
// gradients.
bool launch_gradients(int32_t objective, float* margin, const float* label,
                      int64_t n_rows, int32_t n_classes, float* grad, float* hess,
                      void* quant_scratch, hipStream_t s, const float* values = nullptr);
// Quantiser: exps int32 [n_classes][2]; gpair int32 [n_classes][n_rows][2];
// sums int64 [n_classes][2]; scratch holds quantise_scratch_bytes.
// Most workgroups (and reduction slots) per class: eight 256-thread workgroups
// per CU keep enough loads in flight for the streaming passes over 10M rows.
constexpr int kQuantBlocks = 2048;
int quantise_blocks(int64_t n_rows);
// The quantiser's int64 sum slots in its scratch: class k's quantise_blocks
// (g, h) pairs start at pair k * quantise_blocks(n_rows).
const int64_t* quantise_sum_slots(const void* scratch, int64_t n_rows, int32_t n_classes);
size_t quantise_scratch_bytes(int64_t n_rows, int32_t n_classes);
// rows: row sampling of the round (inactive by default): a dropped row's
// (g, h) count as zero in the maxima, the pairs and the sums of its class.
void launch_quantise(const float* grad, const float* hess, int64_t n_rows, int32_t n_classes,
                     void* scratch, bool maxima_ready, int32_t* exps, int32_t* gpair,
                     int64_t* sums, hipStream_t s, const RowSample& rows = RowSample{});
// *p = value (one thread), e.g. the round index the sampling kernels read.
void launch_store_i32(int32_t* p, int32_t value, hipStream_t s);

void launch_bin_values(const float* values, const dp_bin_layout& layout, const int32_t* cut_ptr,
                       const float* cut_values, uint8_t* bins, hipStream_t s);
// cols[f * n_rows + r] = bin of (r, f), from the tile-major bins.
// Present-value layout of a mostly-missing matrix.  Features are grouped in
// tiles of tile_features (a multiple of 16, at most 256, sized so that one
// tile's histogram fills kSparseLdsBytes of LDS).  For tile t and row r the
// row's present values in the tile are
//   entries[ptr[t * n_rows + r] .. ptr[t * n_rows + r + 1])
// in feature order, each the word index of its (feature, bin) in one LDS plane
// of the tile's histogram: (feature - t * tile_features) * (bin_stride + 1) +
// bin (one word of pad per feature; see hist_sparse_kernel).
struct SparseBins {
  int32_t tile_features = 0, n_tiles = 0;  // n_tiles 0: not built
  int32_t bin_stride = 0;                  // the stride the entries' indexes use
  int64_t nnz = 0;
  DeviceBuffer<uint32_t> ptr;      // [n_tiles * n_rows + 1]: (tile t, row r) at t * n_rows + r
  DeviceBuffer<uint16_t> entries;  // [nnz], tile-major (the root pass's contiguous runs)
  // The same entries row-major, for gathered rows: (row r, tile t) at
  // rptr[r * n_tiles + t], so the tile items of one row chunk, which run on one
  // XCD, read each row's offsets and entries from the same L2 lines.
  DeviceBuffer<uint32_t> rptr;      // [n_rows * n_tiles + 1]
  DeviceBuffer<uint16_t> rentries;  // [nnz]
};
constexpr int64_t kSparseLdsBytes = 64 * 1024;
// LDS of one present-value tile in the histogram kernel: g and h in planes of
// their own, each feature's bins padded by one word.  A plane holds
// tile_features * (bin_stride + 1) words, at most kSparsePlaneWords for every
// tile sparse_tile_features makes (tile_features * bin_stride <= 4096 and
// tile_features <= 256), followed by kSparseTrashWords words that the
// histogram kernel adds its masked lanes' values to (never read); the h plane
// starts at word kSparsePlaneStride, so an entry's h address is its g address
// plus an instruction offset.
constexpr int64_t kSparsePlaneWords = 4352;
constexpr int64_t kSparseTrashWords = 64;
constexpr int64_t kSparsePlaneStride = kSparsePlaneWords + kSparseTrashWords;
constexpr int64_t kSparseLdsAlloc = 2 * kSparsePlaneStride * 8;
// Entries past the last one that the histogram kernel's aligned 8-byte loads
// may read (their values are not used).
constexpr int64_t kSparseEntryPad = 4;
constexpr double kSparseDensity = 0.25;  // automatic use: at most this share present
int32_t sparse_tile_features(int32_t bin_stride);
// Counts the present values of `bins` (16-feature tiles, missing byte 255) and
// builds `out` when their share is at most max_density (and the count fits
// 32-bit offsets); returns the share.  Synchronises the stream.
double build_sparse_bins(const uint8_t* bins, const dp_bin_layout& layout, int32_t bin_stride,
                         double max_density, SparseBins& out, hipStream_t s);
// The same layout from 16-bit columns (cols[f * n_rows + r], kWideMissing for
// missing values), whatever the density; fails when the present values do not
// fit 32-bit offsets.  Synchronises the stream.
void build_sparse_bins_wide(const uint16_t* cols, int64_t n_rows, int32_t n_features,
                            int32_t bin_stride, SparseBins& out, hipStream_t s);
// cols[f * n_rows + r] = bin of values[r * n_features + f] (first cut > x,
// clamped), kWideMissing for NaN: the 16-bit columns of such a matrix.
void launch_bin_columns16(const float* values, int64_t n_rows, int32_t n_features,
                          const int32_t* cut_ptr, const float* cut_values, uint16_t* cols,
                          hipStream_t s);
// Histograms from the present-value layout: work items as for launch_hist,
// with `tile` a sparse tile; partial slots of tile_features * bin_stride * 2
// words in the node histogram's layout.  Finished by launch_hist_reduce_flat.
// The evaluation a present-value pass does for the nodes it builds in one
// chunk (HistWork::partial < 0; HistWork::parent names the sibling): the
// node's and its sibling's words and per-feature candidates of
// launch_reduce_evaluate_flat, computed from the LDS tile; that launch then
// skips these jobs (skip_direct).
// store false: nothing is written but the candidates (no later level reads
// the histograms).  At most 64 bins.
struct SparseEval {
  const int64_t* parent_base = nullptr;  // previous level's node histograms
  const int32_t* n_bins = nullptr;
  const int64_t* node_sums = nullptr;
  const int32_t* exps = nullptr;  // quantiser exponents, device memory
  dp_train_param param{};
  const uint32_t* fmask = nullptr;
  const uint8_t* skip_bins = nullptr;
  void* cand = nullptr;  // evaluate_scratch_bytes of per-feature candidates
  bool store = true;
};
void launch_hist_sparse(const SparseBins& sp, int64_t n_rows, int32_t n_features,
                        const int32_t* gpair, const uint32_t* ridx, const HistWork* work,
                        int32_t n_work, const int32_t* n_work_dev, int32_t bin_stride,
                        int64_t* hist, int64_t* partial, hipStream_t s,
                        const SparseEval* eval = nullptr);
void launch_hist_reduce_flat(const int64_t* partial, const HistReduce* jobs, int32_t n_jobs,
                             const int32_t* n_jobs_dev, int32_t n_tiles, int32_t tile_features,
                             int32_t n_features, int32_t bin_stride, const int64_t* parent_base,
                             int64_t* hist, hipStream_t s);

void launch_tiles_to_columns(const uint8_t* bins, const dp_bin_layout& layout, uint8_t* cols,
                             hipStream_t s);
// rows[r * n_tiles * 16 + t * 16 + j] = tile t's byte j of row r; for the
// first tile t of each of the layout's pairs, the pair's joint tile instead
// (from the tile-major bins, which hold it): the copy the gathered passes of
// one-tile items read with the pairs in use (launch_hist).
void launch_tiles_to_rows(const uint8_t* bins, const dp_bin_layout& layout, uint8_t* rows,
                          hipStream_t s);
// Writes the joint tiles of the layout's pairs (after its n_tiles tiles) from
// the tiles they pair: per row and feature slot i, the byte (tile t's bin <<
// 4) | (tile t + 1's bin & 15).
void launch_join_tiles(uint8_t* bins, const dp_bin_layout& layout, hipStream_t s);

// Quantile cuts on the device; host outputs as in dp_sketch_cuts.
void sketch_cuts(dp_workspace_s& ws, const float* values, int64_t n_rows, int32_t n_features,
                 int32_t max_bin, int32_t* cut_ptr, float* cut_values, float* min_values,
                 int32_t* has_missing, hipStream_t s);

void launch_synth(int32_t config, uint64_t seed, int64_t n_rows, int32_t n_features,
                  float* values, float* labels, float* grad, float* hess, hipStream_t s);

// Device memory of the entry points that allocate nothing (noalloc.hip): a
// file-scope array of this many bytes per GPU.  Returns its device address on
// the current device (looked up once per device); fails when `bytes` exceeds
// the array.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
void* noalloc_scratch(size_t bytes);

inline int grid_for(int64_t n, int threads, int64_t cap = 65536) {
  int64_t g = (n + threads - 1) / threads;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return int(g);
}

}  // namespace dp
