// Training objects: quantised matrix cache, depth-wise tree grower, booster.
//
// The booster reproduces what the reference obtains from XGBoost 3.4.1 through
// XGBoosterUpdateOneIter with tree_method=hist on the GPU
// (native/class_native_training.cuh:54-67): one depth-wise tree per output per
// round, grown level by level.  Per level the device runs
//   histogram build of the smaller child of every pair (gather by row ids)
//   -> sibling = parent - built -> split evaluation -> stable partition
//   -> planner (node records, child numbering, next level's work, leaf work)
//   -> the leaf values of the level's leaves, stored per row
// with every count read from device memory, so a round's trees are enqueued
// back to back and the host reads the node records once per round.  The round
// ends by adding its trees' per-row leaf values to the margins in row order.
#include "booster.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <charconv>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>

#include "json.hpp"
#include "predict.hpp"
#include "tune.hpp"

namespace dp {

void launch_any_nan(const float* values, int64_t n, int32_t* flag, hipStream_t s);
void launch_check_labels(const float* label, int64_t n, int32_t objective, int32_t n_classes,
                         int32_t* bad, hipStream_t s);

namespace {

float parse_float(const std::string& key, const std::string& v) {
  char* end = nullptr;
  const double x = std::strtod(v.c_str(), &end);
  need(end && *end == '\0' && !v.empty(), "invalid numeric value for " + key + ": " + v);
  need(std::isfinite(x), "non-finite value for " + key);
  return float(x);
}

int32_t parse_int(const std::string& key, const std::string& v) {
  char* end = nullptr;
  const long long x = std::strtoll(v.c_str(), &end, 10);
  need(end && *end == '\0' && !v.empty(), "invalid integer value for " + key + ": " + v);
  need(x >= INT_MIN && x <= INT_MAX, "integer out of range for " + key);
  return int32_t(x);
}

}  // namespace

// ---------------------------------------------------------------------------
// Hyperparameter validation (the reference's rules, class_native_training.cuh:16-33)
// ---------------------------------------------------------------------------
std::string validate_hyperparameters(const std::string& text, uint32_t classes) {
  const json::Value in = json::parse(text);
  need(in.kind == json::Value::Object, "hyperparameters must be an object");
  static const char* allowed[] = {"rounds", "max_depth", "eta", "lambda", "alpha", "gamma",
                                  "min_child_weight", "max_bin", "seed", "subsample",
                                  "colsample_bytree", "colsample_bylevel", "colsample_bynode"};
  for (const auto& m : in.members) {
    bool ok = false;
    for (const char* a : allowed) ok = ok || m.first == a;
    need(ok, "unsupported training hyperparameter: " + m.first);
  }
  auto integer = [&](const json::Value& v, const std::string& name, uint64_t maximum) {
    need(v.kind == json::Value::Number && v.text.find_first_of(".eEn") == std::string::npos &&
             v.text != "Infinity" && v.text != "+Infinity",
         name + " must be an integer");
    need(v.text[0] != '-', name + " must be nonnegative");
    uint64_t x = 0;
    auto r = std::from_chars(v.text.data() + (v.text[0] == '+'), v.text.data() + v.text.size(), x);
    need(r.ec == std::errc() && r.ptr == v.text.data() + v.text.size() && x <= maximum,
         name + " exceeds native metadata capacity");
    return x;
  };
  auto numeric = [&](const json::Value& v, const std::string& name, double low, double high,
                     bool strict_low) {
    need(v.kind == json::Value::Number, name + " must be numeric");
    const double x = v.number();
    need(std::isfinite(x) && (strict_low ? x > low : x >= low) && x <= high,
         name + " is outside the supported native parameter range");
    return x;
  };
  auto get = [&](const char* k) { return in.find(k); };
  need(get("rounds") != nullptr, "missing JSON key: rounds");
  need(get("max_depth") != nullptr, "missing JSON key: max_depth");
  const uint64_t rounds = integer(*get("rounds"), "rounds", uint64_t(INT_MAX) / classes);
  const uint64_t depth = integer(*get("max_depth"), "max_depth", INT_MAX);
  need(rounds > 0 && depth > 0, "positive rounds and max_depth required");
  json::Value dflt;
  dflt.kind = json::Value::Number;
  auto or_default = [&](const char* k, const char* d) -> json::Value {
    if (const auto* v = get(k)) return *v;
    json::Value x = dflt;
    x.text = d;
    return x;
  };
  const uint64_t max_bin = integer(or_default("max_bin", "256"), "max_bin", INT_MAX);
  need(max_bin >= 2, "max_bin must be at least 2");
  need(max_bin <= uint64_t(kMaxBins),
       "max_bin above 256 is not supported by this library: bins are stored as uint8");
  const uint64_t seed = integer(or_default("seed", "0"), "seed", INT_MAX);
  const double eta = numeric(or_default("eta", "0.3"), "eta", 0, 1, true);
  std::string o = "{\"rounds\":" + std::to_string(rounds) + ",\"max_depth\":" +
                  std::to_string(depth) + ",\"max_bin\":" + std::to_string(max_bin) +
                  ",\"seed\":" + std::to_string(seed) + ",\"eta\":";
  json::put_double(o, eta);
  for (const char* k : {"lambda", "alpha", "gamma", "min_child_weight"}) {
    const bool one = std::string(k) == "lambda" || std::string(k) == "min_child_weight";
    const double x = numeric(or_default(k, one ? "1" : "0"), k, 0,
                             std::numeric_limits<double>::max(), false);
    o += ",\"" + std::string(k) + "\":";
    json::put_double(o, x);
  }
  for (const char* k : {"subsample", "colsample_bytree", "colsample_bylevel", "colsample_bynode"}) {
    if (const auto* v = get(k)) {
      const double x = numeric(*v, k, 0, 1, true);
      o += ",\"" + std::string(k) + "\":";
      json::put_double(o, x);
    }
  }
  return o + "}";
}

// ---------------------------------------------------------------------------
// DMatrix quantisation
// ---------------------------------------------------------------------------
Quantized& DMatrix::quantize(int32_t max_bin, dp_workspace_s& ws, hipStream_t s) {
  auto it = quantized.find(max_bin);
  if (it != quantized.end()) return *it->second;
  need(max_bin >= 2, "max_bin must be at least 2");
  auto q = std::make_unique<Quantized>();
  DeviceBuffer<int32_t> flag(1);
  launch_any_nan(values.p, n_rows * n_features, flag.p, s);
  int32_t has_nan = 0;
  DP_HIP(hipMemcpyAsync(&has_nan, flag.p, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  DP_HIP(hipStreamSynchronize(s));
  // Cuts for up to 256 bins, with or without missing values.  uint8 bins keep
  // byte 255 for missing values, so a matrix with NaN whose features use all
  // 256 bins keeps 16-bit columns instead (below).
  const int32_t eff = std::min(max_bin, kMaxBins);
  q->max_bin = eff;
  q->cut_ptr.assign(size_t(n_features) + 1, 0);
  q->cut_values.assign(size_t(n_features) * eff, 0.0f);
  q->min_values.assign(size_t(n_features), 0.0f);
  int32_t sketch_missing = 0;
  sketch_cuts(ws, values.p, n_rows, n_features, eff, q->cut_ptr.data(), q->cut_values.data(),
              q->min_values.data(), &sketch_missing, s);
  q->cut_values.resize(size_t(q->cut_ptr[size_t(n_features)]));
  std::vector<int32_t> nbins(static_cast<size_t>(n_features));
  int32_t widest = 1;
  for (int32_t f = 0; f < n_features; ++f) {
    nbins[size_t(f)] = q->cut_ptr[size_t(f) + 1] - q->cut_ptr[size_t(f)];
    widest = std::max(widest, nbins[size_t(f)]);
  }
  q->bin_stride = widest;
  const bool wide = has_nan && widest > 255;
  need(dp_layout_init(n_rows, n_features, 0, has_nan ? 255 : -1, &q->layout) == 0,
       "bin layout");
  if (wide) q->layout.missing_bin = kWideMissing;
  q->d_cut_ptr.resize(q->cut_ptr.size());
  q->d_cut_values.resize(std::max<size_t>(q->cut_values.size(), 1));
  q->d_nbins.resize(nbins.size());
  DP_HIP(hipMemcpyAsync(q->d_cut_ptr.p, q->cut_ptr.data(), q->d_cut_ptr.bytes(),
                        hipMemcpyHostToDevice, s));
  DP_HIP(hipMemcpyAsync(q->d_cut_values.p, q->cut_values.data(),
                        sizeof(float) * q->cut_values.size(), hipMemcpyHostToDevice, s));
  DP_HIP(hipMemcpyAsync(q->d_nbins.p, nbins.data(), q->d_nbins.bytes(), hipMemcpyHostToDevice, s));
  if (wide) {
    q->cols16.resize(size_t(n_rows) * size_t(n_features));
    launch_bin_columns16(values.p, n_rows, n_features, q->d_cut_ptr.p, q->d_cut_values.p,
                         q->cols16.p, s);
  } else {
    // The tiles whose features all have at most 16 bins are paired: their
    // joint tiles follow the matrix's tiles in q->bins (the histograms use
    // them unless the round's histograms skip bins or pairing is off).
    dp_bin_layout paired = q->layout;
    paired.paired_tiles = pair_tiles(nbins.data(), n_features, q->layout.n_tiles, has_nan);
    q->pairs = paired.paired_tiles;
    q->bins.resize(dp_layout_bytes(&paired));
    launch_bin_values(values.p, q->layout, q->d_cut_ptr.p, q->d_cut_values.p, q->bins.p, s);
    launch_join_tiles(q->bins.p, paired, s);
    q->cols.resize(size_t(n_rows) * size_t(n_features));
    launch_tiles_to_columns(q->bins.p, q->layout, q->cols.p, s);
  }
  DP_HIP(hipStreamSynchronize(s));
  auto& ref = *q;
  quantized.emplace(max_bin, std::move(q));
  return ref;
}

// Each feature's most frequent bin (ties: the lowest) over all rows, as skip
// bins per feature and per 16-feature tile (pad features: bin 0, the byte the
// tiles hold for them, so their atomics are skipped too), and the share of
// the element atomics skipped: the rows in those bins plus the pad features.
void build_skip_bins(Quantized& q, hipStream_t s) {
  const int64_t N = q.layout.n_rows;
  const int32_t F = q.layout.n_features, T = q.layout.n_tiles;
  DeviceBuffer<unsigned int> counts(size_t(F) * 256);
  launch_bin_counts(q.cols.p, N, F, counts.p, s);
  std::vector<unsigned int> host(counts.n);
  DP_HIP(hipMemcpyAsync(host.data(), counts.p, counts.bytes(), hipMemcpyDeviceToHost, s));
  DP_HIP(hipStreamSynchronize(s));
  std::vector<uint8_t> per_feature(static_cast<size_t>(F), 0);
  std::vector<uint8_t> per_tile(static_cast<size_t>(T) * 16, 0);
  double share = 0.0;
  for (int32_t f = 0; f < F; ++f) {
    const unsigned int* c = host.data() + size_t(f) * 256;
    int32_t best = 0;
    for (int32_t b = 1; b < 256; ++b)
      if (c[b] > c[best]) best = b;
    per_feature[size_t(f)] = uint8_t(best);
    per_tile[size_t(f)] = uint8_t(best);  // tile-major: feature f at byte f
    share += double(c[best]) / double(N);
  }
  q.skip_features.resize(per_feature.size());
  q.skip_tiles.resize(per_tile.size());
  DP_HIP(hipMemcpy(q.skip_features.p, per_feature.data(), per_feature.size(),
                   hipMemcpyHostToDevice));
  DP_HIP(hipMemcpy(q.skip_tiles.p, per_tile.data(), per_tile.size(), hipMemcpyHostToDevice));
  const double slots = double(T) * 16.0;
  q.skip_share = T > 0 ? (share + (slots - double(F))) / slots : 0.0;
}

int32_t Tree::alloc(int32_t parent_id) {
  const int32_t id = size();
  left.push_back(-1);
  right.push_back(-1);
  parent.push_back(parent_id);
  feature.push_back(0);
  split_bin.push_back(-1);
  cond.push_back(0.0f);
  base_weight.push_back(0.0f);
  loss_chg.push_back(0.0f);
  sum_hess.push_back(0.0f);
  default_left.push_back(0);
  sum_qg.push_back(0);
  sum_qh.push_back(0);
  rows.push_back(-1);
  return id;
}

// ---------------------------------------------------------------------------
// Grower
// ---------------------------------------------------------------------------
namespace {

// Trees whose widest level can hold more nodes than this, or whose two
// histogram levels would take more bytes, are grown level-synced.
constexpr int64_t kEagerNodes = int64_t(1) << 16;
constexpr int64_t kEagerHistBytes = int64_t(8) << 30;

// Present-value levels of at least this many nodes evaluate their single-chunk
// nodes in the histogram pass (Grower::grow).
constexpr int64_t kInPassNodes = 128;

int64_t level_bound(int32_t depth, int64_t n_rows) {
  return depth >= 62 ? n_rows : std::min<int64_t>(int64_t(1) << depth, n_rows);
}

int32_t* field(PlanCounts* c, int32_t PlanCounts::*m) { return &(c->*m); }

}  // namespace

Grower::Grower() = default;
Grower::~Grower() = default;

void Grower::ensure_level(const Quantized& q, int64_t nb, int32_t d, int32_t D) {
  const int64_t N = q.layout.n_rows;
  const int32_t T = tiles_;
  const int64_t S = int64_t(q.layout.n_features) * q.bin_stride * 2;
  const int cur = d & 1, nxt = cur ^ 1;
  const int64_t nn = d < D ? std::min(2 * nb, N) : 0;  // next level's bound
  // items per row chunk
  const int32_t G = hist_groups(T, level_cfg_.tiles, hist_pairs(lay_.paired_tiles, level_cfg_.tiles));
  need(plan_hist_capacity(nn, G, level_cfg_.items) < INT32_MAX &&
           plan_part_capacity(nb, N, chunk_) < INT32_MAX &&
           plan_part_capacity(nn, N, chunk_) < INT32_MAX && plan_leaf_capacity(nb, N, chunk_) < INT32_MAX,
       "tree level too wide for the planner's 32-bit work counts");
  if (d < D) {
    hist_[cur].reserve(size_t(nb * S));
    splits_.reserve(size_t(nb));
    eval_scratch_.reserve(evaluate_scratch_bytes(int32_t(nb), q.layout.n_features));
    if (colsample_) fmask_.reserve(size_t(nb) * size_t((q.layout.n_features + 31) / 32));
    work_left_.reserve(size_t(plan_part_capacity(nb, N, chunk_)));
    part_masks_.reserve(size_t(plan_part_capacity(nb, N, chunk_)) * kPartMasks);
  }
  node_left_[nxt].reserve(size_t(std::max<int64_t>(nn, 1)));
  level_[nxt].reserve(size_t(std::max<int64_t>(nn, 1)));
  sums_[nxt].reserve(size_t(2 * std::max<int64_t>(nn, 1)));
  seg_begin_[nxt].reserve(size_t(std::max<int64_t>(nn, 1)));
  hist_work_[nxt].reserve(size_t(plan_hist_capacity(nn, G, level_cfg_.items)));
  reduce_jobs_[nxt].reserve(size_t(nn / 2 + 1));
  pair_chunk_.reserve(size_t(2 * (std::max(nb, nn) + 1)));
  part_work_[nxt].reserve(size_t(plan_part_capacity(nn, N, chunk_)));
  part_first_[nxt].reserve(size_t(nn + 1));
  leaf_work_[cur].reserve(size_t(plan_leaf_capacity(nb, N, chunk_)));
}

void Grower::prepare(const Quantized& q, const TrainParam& p, int32_t n_slots, bool sparse,
                     const HistConfig& root_cfg, const HistConfig& level_cfg, bool skip,
                     uint64_t pairs, hipStream_t s) {
  const dp_bin_layout& L = q.layout;
  rows_major_ = sparse ? nullptr : q.row_major(hist_pairs(pairs, level_cfg.tiles));
  need(sparse ? q.sparse.n_tiles > 0 : rows_major_ != nullptr, "histogram layout not built");
  need(!skip || (!sparse && q.skip_tiles.n > 0 && q.skip_features.n > 0),
       "skip bins not built");
  need(!pairs || (!sparse && !skip && (pairs & ~q.pairs) == 0), "tile pairs out of place");
  lay_ = L;
  lay_.paired_tiles = pairs;
  check_pairs(lay_);
  sparse_ = sparse;
  skip_tiles_ = skip ? q.skip_tiles.p : nullptr;
  skip_features_ = skip ? q.skip_features.p : nullptr;
  root_cfg_ = root_cfg;
  level_cfg_ = level_cfg;
  if (sparse) root_cfg_.tiles = level_cfg_.tiles = 1;  // one present-value tile per item
  colsample_ = p.colsample();
  tiles_ = sparse ? q.sparse.n_tiles : L.n_tiles;
  const int64_t N = L.n_rows;
  const int32_t D = p.max_depth;
  const int64_t S = int64_t(L.n_features) * q.bin_stride * 2;
  need(N >= 1, "training matrix has no rows");
  need(N <= int64_t(UINT32_MAX), "row ids are 32-bit");
  need(D >= 1 && D <= 30, "max_depth out of supported range");
  chunk_ = row_chunk(N);
  if (cus_ == 0) {
    int dev = 0;
    DP_HIP(hipGetDevice(&dev));
    DP_HIP(hipDeviceGetAttribute(&cus_, hipDeviceAttributeMultiprocessorCount, dev));
  }
  ridx_[0].reserve(size_t(N));
  ridx_[1].reserve(size_t(N));
  counts_.reserve(1);
  level_count_.reserve(sizeof(PlanCounts));
  // level 0: the root
  level_[0].reserve(1);
  sums_[0].reserve(2);
  seg_begin_[0].reserve(1);
  part_work_[0].reserve(size_t(plan_part_capacity(1, N, chunk_)));
  part_first_[0].reserve(2);
  node_left_[0].reserve(1);
  const int64_t slot_words = sparse ? int64_t(q.sparse.tile_features) * q.bin_stride * 2
                                    : int64_t(q.bin_stride) * 32;
  partial_.reserve(size_t(std::max(hist_partial_capacity(tiles_, root_cfg_, pairs),
                                    hist_partial_capacity(tiles_, level_cfg_, pairs)) *
                           slot_words));
  if (root_rows_ != N || root_tiles_ != tiles_ || root_sparse_ != sparse ||
      root_made_.tiles != root_cfg_.tiles || root_made_.items != root_cfg_.items ||
      root_pairs_ != pairs) {
    const int64_t b = 0, e = N;
    const int32_t slot = 0;
    std::vector<HistWork> w;
    std::vector<HistReduce> j;
    make_hist_work(lay_, &b, &e, &slot, 1, true, w, j, sparse ? tiles_ : 0, root_cfg_);
    root_work_.resize(w.size());
    root_job_.resize(j.size());
    DP_HIP(hipMemcpy(root_work_.p, w.data(), sizeof(HistWork) * w.size(), hipMemcpyHostToDevice));
    DP_HIP(hipMemcpy(root_job_.p, j.data(), sizeof(HistReduce) * j.size(), hipMemcpyHostToDevice));
    root_items_ = int32_t(w.size());
    root_rows_ = N;
    root_tiles_ = tiles_;
    root_sparse_ = sparse;
    root_made_ = root_cfg_;
    root_pairs_ = pairs;
  }
  const int64_t widest = level_bound(D, N), widest_hist = level_bound(D - 1, N);
  eager_ = widest <= kEagerNodes && 2 * widest_hist * S * int64_t(sizeof(int64_t)) <= kEagerHistBytes;
  if (eager_) {
    int64_t cap = 0;
    for (int32_t d = 0; d <= D; ++d) {
      ensure_level(q, level_bound(d, N), d, D);
      cap += level_bound(d, N);
    }
    node_cap_ = std::min(cap, 2 * N - 1);
    slot_bytes_ = (sizeof(PlanCounts) + sizeof(NodeInfo) * size_t(node_cap_) + 255) & ~size_t(255);
    slots_.reserve(slot_bytes_ * size_t(n_slots));
    readback_.reserve(2 * slot_bytes_ * size_t(n_slots));
    readback_slots_ = n_slots;
  } else {
    ensure_level(q, 1, 0, D);
    info_.reserve(3);
    spill_.resize(size_t(n_slots));
    spill_counts_.resize(size_t(n_slots));
  }
  (void)s;
}

void Grower::grow(const Quantized& q, const int32_t* gpair, const int32_t* exps,
                  const int64_t* root_slots, int32_t root_blocks, const TrainParam& p,
                  float* values, int32_t* positions, int32_t slot, hipStream_t s) {
  const dp_bin_layout& L = q.layout;
  const int64_t N = L.n_rows;
  const int32_t F = L.n_features, B = q.bin_stride, T = tiles_, D = p.max_depth;
  const int64_t S = int64_t(F) * B * 2;  // int64 values per node histogram
  const dp_train_param dtp{p.eta, p.lambda, p.alpha, p.gamma, p.min_child_weight, p.max_depth};
  // Eager trees keep their counters and node records in their own slot, so
  // the slots of a round come back to the host in one copy.
  uint8_t* slot_dev = eager_ ? slots_.p + slot_bytes_ * size_t(slot) : nullptr;
  PlanCounts* c = eager_ ? reinterpret_cast<PlanCounts*>(slot_dev) : counts_.p;
  NodeInfo* info = eager_ ? reinterpret_cast<NodeInfo*>(slot_dev + sizeof(PlanCounts)) : info_.p;
  auto* host_counts = reinterpret_cast<PlanCounts*>(level_count_.p);

  launch_plan_root(level_[0].p, sums_[0].p, seg_begin_[0].p, part_work_[0].p, part_first_[0].p,
                   node_left_[0].p, c, N, root_slots, root_blocks, chunk_, ridx_[0].p, s, exps);
  int64_t nb = 1;  // bound of the current level's node count
  int64_t nb_prev = 0;
  // The last split level's count launch stores every leaf value of levels
  // D - 1 and D (rows of expanding nodes and of D - 1's leaves).  Every leaf
  // pass stores into the leaf-value plane: no margin is read here.
  bool last_level_applied = false;
  for (int32_t d = 0; d <= D; ++d) {
    const int cur = d & 1, nxt = cur ^ 1;
    if (!eager_ && d > 0) {
      DP_HIP(hipMemcpyAsync(host_counts, c, sizeof(PlanCounts), hipMemcpyDeviceToHost, s));
      DP_HIP(hipStreamSynchronize(s));
      nb = host_counts->n_level;
      if (nb == 0) {  // the tree ended: apply the previous level's deferred leaves
        const int32_t bound = int32_t(plan_leaf_capacity(nb_prev, N, chunk_));
        if (!last_level_applied)  // else the last split level's count launch did
          launch_update_margin(ridx_[nxt].p, leaf_work_[nxt].p, bound,
                               field(c, &PlanCounts::n_leaf), values, 1, s, nullptr, true);
        if (positions)
          launch_leaf_positions(ridx_[nxt].p, leaf_work_[nxt].p, bound,
                                field(c, &PlanCounts::n_leaf), positions, s);
        break;
      }
      ensure_level(q, nb, d, D);
      const int64_t need_nodes = int64_t(host_counts->n_nodes) + 2 * nb;
      if (int64_t(info_.n) < need_nodes) {
        PooledBuffer<NodeInfo> grown(size_t(std::max<int64_t>(need_nodes, 2 * int64_t(info_.n))));
        DP_HIP(hipMemcpyAsync(grown.p, info_.p, info_.bytes(), hipMemcpyDeviceToDevice, s));
        DP_HIP(hipStreamSynchronize(s));
        info_ = std::move(grown);
      }
    }
    const bool split = d < D;
    // A split level of at most 1024 nodes runs its planner and its partition
    // scatter in one launch.
    const bool merged = split && nb <= 1024;
    // On the last split level of such a tree the rows need no new order: the
    // count launch stores the leaf values and the planner runs alone (unless leaf
    // ids are wanted, which the scatter's segments give).
    const bool fuse_last = merged && d + 1 == D && values && !positions;
    ScatterArgs scatter{};
    int64_t* h = hist_[cur].p;
    if (split) {
      const int32_t tf = q.sparse.tile_features;
      // Column sampling: each node's feature sample, read by the evaluation.
      const uint32_t* fmask = nullptr;
      if (colsample.active()) {
        need(colsample_, "column sampling buffers were not prepared");
        launch_colsample(level_[cur].p, int32_t(nb), field(c, &PlanCounts::n_level), F,
                         colsample, d, fmask_.p, s);
        fmask = fmask_.p;
      }
      // The present-value layout's partial slots hold node-histogram words: its
      // levels reduce and evaluate in one launch (up to 64 bins).
      const bool fused = sparse_ && B <= 64 && tf % 16 == 0 && exps;
      // The last split level's histograms have no readers: a fused launch
      // evaluates them without storing them.
      const bool keep = d + 1 < D;
      bool dense_fused = false;  // set below for dense passes with at least kDenseFuseFeatures features
      if (d == 0 && sparse_) {
        launch_hist_sparse(q.sparse, N, F, gpair, nullptr, root_work_.p, root_items_, nullptr, B,
                           h, partial_.p, s);
        if (fused)
          launch_reduce_evaluate_flat(partial_.p, root_job_.p, 1, nullptr, T, tf, F, B, nullptr, h,
                                      q.d_nbins.p, sums_[cur].p, exps, dtp, fmask,
                                      skip_features_, eval_scratch_.p, keep, s);
        else
          launch_hist_reduce_flat(partial_.p, root_job_.p, 1, nullptr, T, tf, F, B, nullptr, h, s);
      } else if (d == 0) {
        // The root, as the levels below it: feature-major partial slots, and
        // the reduce and the evaluation in one launch (one job, no sibling).
        dense_fused = F >= kDenseFuseFeatures && B <= 256 && exps;
        launch_hist(q.bins.p, lay_, gpair, nullptr, root_work_.p, root_items_, nullptr, B, h,
                    partial_.p, s, nullptr, root_cfg_, skip_tiles_, dense_fused);
        if (dense_fused)
          launch_reduce_evaluate_dense(partial_.p, root_job_.p, 1, nullptr, T, F, B, nullptr, h,
                                       q.d_nbins.p, sums_[cur].p, exps, dtp, fmask,
                                       skip_features_, eval_scratch_.p, keep, s);
        else
          launch_hist_reduce(partial_.p, root_job_.p, 1, nullptr, T, F, B, nullptr, h, false, s);
      } else if (sparse_) {
        // On the last split level of a fused tree, and on levels of at least
        // kInPassNodes nodes (mostly small ones), the nodes built in one chunk
        // are evaluated by the histogram pass itself, from LDS (on the last
        // level never stored); the reduce-evaluate takes the rest.  (On
        // levels of fewer, larger nodes the pass's 512-thread workgroups
        // accumulate the multi-chunk items more slowly than the evaluation
        // saves: measured on C5.)
        const bool in_pass = fused && (!keep || nb >= kInPassNodes);
        SparseEval ev;
        ev.parent_base = hist_[nxt].p;
        ev.n_bins = q.d_nbins.p;
        ev.node_sums = sums_[cur].p;
        ev.exps = exps;
        ev.param = dtp;
        ev.fmask = fmask;
        ev.skip_bins = skip_features_;
        ev.cand = eval_scratch_.p;
        ev.store = keep;
        launch_hist_sparse(q.sparse, N, F, gpair, ridx_[cur].p, hist_work_[cur].p,
                           int32_t(plan_hist_items(nb, N, T, level_cfg_.items)),
                           field(c, &PlanCounts::n_hist), B, h, partial_.p, s,
                           in_pass ? &ev : nullptr);
        if (fused)
          launch_reduce_evaluate_flat(partial_.p, reduce_jobs_[cur].p, int32_t(nb / 2 + 1),
                                      field(c, &PlanCounts::n_reduce), T, tf, F, B, hist_[nxt].p,
                                      h, q.d_nbins.p, sums_[cur].p, exps, dtp, fmask,
                                      skip_features_, eval_scratch_.p, keep, s, in_pass);
        else
          launch_hist_reduce_flat(partial_.p, reduce_jobs_[cur].p, int32_t(nb / 2 + 1),
                                  field(c, &PlanCounts::n_reduce), T, tf, F, B, hist_[nxt].p, h,
                                  s);
      } else {
        const int32_t G =
            hist_groups(T, level_cfg_.tiles, hist_pairs(lay_.paired_tiles, level_cfg_.tiles));
        // Levels below the root with more features than one evaluation
        // workgroup takes: feature-major partial slots, and the reduce and the
        // evaluation in one launch (measured: C2 2,474 -> 2,560, C3 455 ->
        // 463, C4 3,321 -> 3,886 trees/s).
        dense_fused = F >= kDenseFuseFeatures && B <= 256 && exps;
        launch_hist(q.bins.p, lay_, gpair, ridx_[cur].p, hist_work_[cur].p,
                    int32_t(plan_hist_items(nb, N, G, level_cfg_.items)),
                    field(c, &PlanCounts::n_hist), B, h, partial_.p, s, rows_major_, level_cfg_,
                    skip_tiles_, dense_fused);
        if (dense_fused)
          launch_reduce_evaluate_dense(partial_.p, reduce_jobs_[cur].p, int32_t(nb / 2 + 1),
                                       field(c, &PlanCounts::n_reduce), T, F, B, hist_[nxt].p, h,
                                       q.d_nbins.p, sums_[cur].p, exps, dtp, fmask,
                                       skip_features_, eval_scratch_.p, keep, s);
        else
          launch_hist_reduce(partial_.p, reduce_jobs_[cur].p, int32_t(nb / 2 + 1),
                             field(c, &PlanCounts::n_reduce), T, F, B, hist_[nxt].p, h, false, s);
      }
      // Without records from the evaluation, the count launch selects them.
      const bool records =
          fused || dense_fused
              ? false
              : launch_evaluate(h, int32_t(nb), field(c, &PlanCounts::n_level), F, B,
                                q.d_nbins.p, sums_[cur].p, exps, 0, 0, dtp, eval_scratch_.p,
                                splits_.p, s, false, fmask, skip_features_);
      SplitSelect sel;
      sel.cand = reinterpret_cast<const FeatCand*>(eval_scratch_.p);
      sel.n_features = F;
      sel.gamma = double(p.gamma);
      // The previous level's leaves (its planner wrote their chunks; their rows
      // sit in that level's ridx buffer, untouched by this level's scatter)
      // are applied by this level's count launch.
      LeafPass prev;
      if (d > 0) {
        prev.ridx = ridx_[nxt].p;
        prev.work = leaf_work_[nxt].p;
        prev.n_dev = field(c, &PlanCounts::n_leaf);
        prev.n_host = int32_t(plan_leaf_capacity(nb_prev, N, chunk_));
        prev.margin = values;
        prev.stride = 1;
        prev.store = true;
        prev.positions = positions;
      }
      LastLevel ll{};
      if (fuse_last) {
        ll.values = values;
        ll.nodes = level_[cur].p;
        ll.exps = exps;
        ll.eta = double(p.eta);
        ll.lambda = double(p.lambda);
        ll.alpha = double(p.alpha);
        ll.mcw = double(p.min_child_weight);
        last_level_applied = true;
      }
      launch_partition(q.bins.p,
                       L.missing_bin == kWideMissing ? static_cast<const void*>(q.cols16.p)
                                                     : static_cast<const void*>(q.cols.p),
                       L, ridx_[cur].p, ridx_[nxt].p, part_work_[cur].p,
                       int32_t(plan_part_capacity(nb, N, chunk_)), &c->n_part[d & 1],
                       seg_begin_[cur].p, splits_.p, part_first_[cur].p, int32_t(nb),
                       field(c, &PlanCounts::n_level), work_left_.p, part_masks_.p,
                       node_left_[cur].p, true, s, d > 0 ? &prev : nullptr,
                       records ? nullptr : &sel, merged && !fuse_last ? &scatter : nullptr,
                       fuse_last ? &ll : nullptr);
    }
    PlanArgs a{};
    a.cur = level_[cur].p;
    a.splits = split ? splits_.p : nullptr;
    a.node_left = node_left_[cur].p;
    a.next_node_left = node_left_[nxt].p;
    a.next = level_[nxt].p;
    a.next_sums = sums_[nxt].p;
    a.next_seg_begin = seg_begin_[nxt].p;
    a.info = eager_ ? info : info_.p;
    a.hist_work = hist_work_[nxt].p;
    a.reduce_jobs = reduce_jobs_[nxt].p;
    a.part_work = part_work_[nxt].p;
    a.part_first = part_first_[nxt].p;
    a.pair_chunk = pair_chunk_.p;
    a.leaf_work = leaf_work_[cur].p;
    a.counts = c;
    a.exps = exps;
    a.depth = d;
    a.max_depth = D;
    a.n_tiles = T;
    a.hist_tiles = level_cfg_.tiles;
    a.hist_pairs = hist_pairs(lay_.paired_tiles, level_cfg_.tiles);
    a.hist_items = level_cfg_.items;
    // Histogram workgroups resident at once: two per CU for present-value
    // tiles; for dense tiles, what the level kernel's LDS and registers allow.
    a.hist_slots = sparse_ ? cus_ * 2
                           : hist_resident(true, L.missing_bin >= 0, skip_tiles_ != nullptr,
                                           level_cfg_, a.hist_pairs != 0);
    a.hist_elems = S;
    a.part_chunk = chunk_;
    a.leaf_chunk = chunk_;
    a.eta = double(p.eta);
    a.lambda = double(p.lambda);
    a.alpha = double(p.alpha);
    a.mcw = double(p.min_child_weight);
    a.info_capacity = int32_t(eager_ ? node_cap_ : int64_t(info_.n));
    a.level_capacity = int32_t(level_[nxt].n);
    a.hist_capacity = int32_t(hist_work_[nxt].n);
    a.partial_capacity = int32_t(hist_partial_capacity(T, level_cfg_, lay_.paired_tiles));
    a.part_capacity = int32_t(part_work_[nxt].n);
    a.leaf_capacity = int32_t(leaf_work_[cur].n);
    a.cur_bound = int32_t(std::min<int64_t>(nb, INT32_MAX));
    if (merged) {  // the planner sums the count launch's left counts itself
      a.work_left = work_left_.p;
      a.part_bound = int32_t(plan_part_capacity(nb, N, chunk_));
    }
    // The last split level's planner also writes its children's records (all
    // leaves, their values already stored): no planner for level D.
    a.leaf_children = fuse_last ? 1 : 0;
    if (merged && !fuse_last) launch_plan_scatter(a, scatter, N, s);
    else if (!(d == D && last_level_applied)) launch_plan_level(a, nb, s);
    // No later count launch carries the leaves of the last two levels: level
    // D - 1's are applied with level D's, in one launch after the last planner
    // (which keeps their count in n_leaf_prev).  A level-synced tree that ends
    // before level D applies them when it stops, above.
    if (d == D) {
      const int32_t leaf_bound = int32_t(plan_leaf_capacity(nb, N, chunk_));
      LeafList prev_leaves;
      if (D >= 1) {
        prev_leaves.ridx = ridx_[nxt].p;
        prev_leaves.work = leaf_work_[nxt].p;
        prev_leaves.n_host = int32_t(plan_leaf_capacity(nb_prev, N, chunk_));
        prev_leaves.n_dev = field(c, &PlanCounts::n_leaf_prev);
      }
      if (!last_level_applied)
        launch_update_margin(ridx_[cur].p, leaf_work_[cur].p, leaf_bound,
                             field(c, &PlanCounts::n_leaf), values, 1, s,
                             D >= 1 ? &prev_leaves : nullptr, true);
      if (positions) {
        if (D >= 1)
          launch_leaf_positions(prev_leaves.ridx, prev_leaves.work, prev_leaves.n_host,
                                prev_leaves.n_dev, positions, s);
        launch_leaf_positions(ridx_[cur].p, leaf_work_[cur].p, leaf_bound,
                              field(c, &PlanCounts::n_leaf), positions, s);
      }
    }
    nb_prev = nb;
    nb = split ? std::min(2 * nb, N) : 0;
  }

  if (!eager_) {
    DP_HIP(hipMemcpyAsync(host_counts, c, sizeof(PlanCounts), hipMemcpyDeviceToHost, s));
    DP_HIP(hipStreamSynchronize(s));
    spill_counts_[size_t(slot)] = *host_counts;
    auto& v = spill_[size_t(slot)];
    v.resize(size_t(std::max(host_counts->n_nodes, 0)));
    if (!v.empty())
      DP_HIP(hipMemcpy(v.data(), info_.p, sizeof(NodeInfo) * v.size(), hipMemcpyDeviceToHost));
  }
}

void Grower::readback(int32_t n_slots, int32_t buffer, hipStream_t s) {
  if (!eager_ || n_slots <= 0) return;
  need(n_slots <= readback_slots_ && (buffer == 0 || buffer == 1),
       "readback beyond the prepared slots");
  DP_HIP(hipMemcpyAsync(readback_.p + size_t(buffer) * slot_bytes_ * size_t(readback_slots_),
                        slots_.p, slot_bytes_ * size_t(n_slots), hipMemcpyDeviceToHost, s));
}

uint64_t Grower::signature() const {
  uint64_t h = 1469598103934665603ull;  // FNV-1a over the buffers' addresses and sizes
  auto mix = [&h](uint64_t v) {
    for (int i = 0; i < 8; ++i) {
      h ^= (v >> (8 * i)) & 0xffu;
      h *= 1099511628211ull;
    }
  };
  auto buf = [&mix](const auto& b) {
    mix(reinterpret_cast<uint64_t>(b.p));
    mix(uint64_t(b.n));
  };
  for (int i = 0; i < 2; ++i) {
    buf(ridx_[i]); buf(hist_[i]); buf(level_[i]); buf(sums_[i]); buf(seg_begin_[i]);
    buf(hist_work_[i]); buf(reduce_jobs_[i]); buf(part_work_[i]); buf(part_first_[i]);
    buf(node_left_[i]); buf(leaf_work_[i]);
  }
  buf(root_work_); buf(root_job_); buf(partial_); buf(pair_chunk_); buf(work_left_);
  buf(part_masks_);
  buf(splits_); buf(eval_scratch_); buf(fmask_); buf(info_); buf(counts_); buf(slots_);
  mix(uint64_t(eager_)); mix(uint64_t(sparse_)); mix(uint64_t(colsample_)); mix(uint64_t(tiles_));
  mix(reinterpret_cast<uint64_t>(skip_tiles_)); mix(reinterpret_cast<uint64_t>(skip_features_));
  mix(reinterpret_cast<uint64_t>(rows_major_));
  mix(uint64_t(node_cap_)); mix(uint64_t(chunk_));
  mix(uint64_t(slot_bytes_)); mix(uint64_t(root_rows_)); mix(uint64_t(root_tiles_));
  mix(uint64_t(root_items_));
  for (const HistConfig* c : {&root_cfg_, &level_cfg_}) {
    mix(uint64_t(c->tiles));
    mix(uint64_t(c->unroll));
    mix(uint64_t(c->items));
    mix(uint64_t(c->split));
    mix(uint64_t(c->deep));
  }
  mix(lay_.paired_tiles);
  return h;
}

void Grower::exponents(int32_t slot, int32_t buffer, int32_t* out) const {
  const PlanCounts* c =
      eager_ ? reinterpret_cast<const PlanCounts*>(
                   readback_.p +
                   slot_bytes_ * (size_t(buffer) * size_t(readback_slots_) + size_t(slot)))
             : &spill_counts_[size_t(slot)];
  out[0] = c->exps[0];
  out[1] = c->exps[1];
}

void Grower::collect(const Quantized& q, int32_t slot, int32_t buffer, Tree& tree) const {
  const PlanCounts* c;
  const NodeInfo* info;
  if (eager_) {
    const uint8_t* src =
        readback_.p + slot_bytes_ * (size_t(buffer) * size_t(readback_slots_) + size_t(slot));
    c = reinterpret_cast<const PlanCounts*>(src);
    info = reinterpret_cast<const NodeInfo*>(src + sizeof(PlanCounts));
  } else {
    c = &spill_counts_[size_t(slot)];
    info = spill_[size_t(slot)].data();
  }
  need(c->error != 1, "partition produced an empty child");
  need(c->error == 0, "tree planner capacity exceeded (code " + std::to_string(c->error) + ")");
  const int32_t n = c->n_nodes;
  need(n >= 1 && (!eager_ || n <= node_cap_), "tree planner reported an invalid node count");
  tree = Tree{};
  for (int32_t i = 0; i < n; ++i) tree.alloc(-1);
  for (int32_t i = 0; i < n; ++i) {
    const NodeInfo& r = info[i];
    const size_t id = size_t(i);
    tree.base_weight[id] = r.base_weight;
    tree.sum_hess[id] = r.sum_hess;
    tree.sum_qg[id] = r.g;
    tree.sum_qh[id] = r.h;
    tree.rows[id] = r.end - r.begin;
    if (r.left >= 0) {
      need(r.left > i && r.left + 1 < n, "tree planner produced an invalid child id");
      need(r.feature >= 0 && r.feature < q.layout.n_features && r.bin >= 0 &&
               q.cut_ptr[size_t(r.feature)] + r.bin < q.cut_ptr[size_t(r.feature) + 1],
           "tree planner produced an invalid split");
      tree.left[id] = r.left;
      tree.right[id] = r.left + 1;
      tree.parent[size_t(r.left)] = tree.parent[size_t(r.left) + 1] = i;
      tree.feature[id] = r.feature;
      tree.split_bin[id] = r.bin;
      tree.default_left[id] = uint8_t(r.default_left);
      tree.cond[id] = q.cut_values[size_t(q.cut_ptr[size_t(r.feature)] + r.bin)];
      tree.loss_chg[id] = float(r.loss_chg);
    } else {
      tree.cond[id] = r.leaf_value;
    }
  }
}

// ---------------------------------------------------------------------------
// Booster
// ---------------------------------------------------------------------------
Booster::Booster(std::vector<DMatrix*> cache) : cache_(std::move(cache)) {}

void DMatrix::release_pending() {
  const std::vector<const Booster*> users = pending;
  for (const Booster* b : users) {
    try {
      b->flush();
    } catch (...) {
      // the booster keeps its last good rounds; the matrix is freed regardless
    }
  }
  pending.clear();
  (void)hipDeviceSynchronize();
}

Booster::~Booster() {
  if (pending_ && pending_d_) {  // the round in flight is dropped, not collected
    auto& v = pending_d_->pending;
    v.erase(std::remove(v.begin(), v.end(), this), v.end());
  }
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (hipEvent_t& e : round_done_)
    if (e) (void)hipEventDestroy(e);
  clear_graphs();
  growers_.clear();
  for (hipStream_t t : tree_streams_) (void)hipStreamDestroy(t);
  for (hipEvent_t e : tree_done_) (void)hipEventDestroy(e);
  if (fork_) (void)hipEventDestroy(fork_);
  if (caller_read_) (void)hipEventDestroy(caller_read_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

void Booster::clear_graphs() {
  for (auto& g : graphs_) (void)hipGraphExecDestroy(g.second);
  graphs_.clear();
}

void Booster::set_param(const std::string& key, const std::string& value) {
  static const char* known[] = {
      "objective", "num_class", "tree_method", "device", "booster", "max_bin", "max_depth",
      "eta", "learning_rate", "lambda", "reg_lambda", "alpha", "reg_alpha", "gamma",
      "min_split_loss", "min_child_weight", "subsample", "colsample_bytree", "colsample_bylevel",
      "colsample_bynode", "base_score", "boost_from_average", "seed", "seed_per_iteration",
      "nthread", "verbosity", "validate_parameters", "grow_policy", "dp_record_positions",
      "dp_graphs", "dp_sparse_hist", "dp_concurrent_trees", "dp_autotune", "dp_hist_tiles",
      "dp_hist_unroll", "dp_hist_items", "dp_hist_split", "dp_hist_deep", "dp_hist_pair",
      "dp_skip_bin"};
  bool ok = false;
  for (const char* k : known) ok = ok || key == k;
  need(ok, "unsupported parameter: " + key);
  if (model_only_ && key == "objective") {
    const std::string cur = effective_objective();
    const bool multi = [](const std::string& o) {
      return o == "multi:softmax" || o == "multi:softprob";
    }(cur);
    need(value == cur || (multi && (value == "multi:softmax" || value == "multi:softprob")),
         "a loaded model can only switch between multi:softmax and multi:softprob");
  } else if (configured_ && (key == "objective" || key == "num_class" || key == "max_bin")) {
    auto it = params_.find(key);
    need(it != params_.end() && it->second == value,
         "parameter " + key + " cannot change after training started");
  }
  params_[key] = value;
  if (key == "dp_record_positions") record_positions_ = parse_int(key, value) != 0;
  if (key == "dp_graphs") use_graphs_ = parse_int(key, value) != 0;
  if (key == "dp_concurrent_trees") {
    const int32_t m = parse_int(key, value);
    need(m >= 1 && m <= 8, "dp_concurrent_trees must be in [1, 8]");
    concurrent_trees_ = m;
  }
  if (key == "dp_autotune") autotune_ = parse_int(key, value) != 0;
  if (key == "dp_skip_bin") {
    const int32_t m = parse_int(key, value);
    need(m >= 0 && m <= 2, "dp_skip_bin must be 0, 1 or 2");
    skip_mode_ = m;
  }
  if (key == "dp_hist_tiles") {
    const int32_t m = parse_int(key, value);
    need(m == 0 || m == 1 || m == 2, "dp_hist_tiles must be 0 (tuned), 1 or 2");
    forced_hist_.tiles = m;
  }
  if (key == "dp_hist_unroll") {
    const int32_t m = parse_int(key, value);
    need(m == 0 || m == 1 || m == 2, "dp_hist_unroll must be 0 (tuned), 1 or 2");
    forced_hist_.unroll = m;
  }
  if (key == "dp_hist_items") {
    const int32_t m = parse_int(key, value);
    need(m == 0 || (m >= 256 && m <= 4096), "dp_hist_items must be 0 (tuned) or in [256, 4096]");
    forced_hist_.items = m;
  }
  if (key == "dp_hist_split") {
    const int32_t m = parse_int(key, value);
    need(m == 0 || m == 4 || m == 5, "dp_hist_split must be 0, 4 or 5");
    forced_hist_.split = m;
  }
  if (key == "dp_hist_deep") {
    const int32_t m = parse_int(key, value);
    need(m == 0 || m == 1, "dp_hist_deep must be 0 or 1");
    forced_hist_.deep = m;
  }
  if (key == "dp_hist_pair") {
    const int32_t m = parse_int(key, value);
    need(m == 0 || m == 1, "dp_hist_pair must be 0 or 1");
    pair_tiles_ = m != 0;
  }
  if (key == "dp_sparse_hist") {
    const int32_t m = parse_int(key, value);
    need(m >= 0 && m <= 2, "dp_sparse_hist must be 0, 1 or 2");
    sparse_mode_ = m;
  }
}

void Booster::configure(DMatrix* d) {
  auto get = [&](const char* k, const char* dflt) {
    auto it = params_.find(k);
    return it == params_.end() ? std::string(dflt) : it->second;
  };
  auto first_of = [&](std::initializer_list<const char*> keys, const char* dflt) {
    for (const char* k : keys) {
      auto it = params_.find(k);
      if (it != params_.end()) return it->second;
    }
    return std::string(dflt);
  };
  TrainParam tp;
  tp.eta = parse_float("eta", first_of({"eta", "learning_rate"}, "0.3"));
  tp.lambda = parse_float("lambda", first_of({"lambda", "reg_lambda"}, "1"));
  tp.alpha = parse_float("alpha", first_of({"alpha", "reg_alpha"}, "0"));
  tp.gamma = parse_float("gamma", first_of({"gamma", "min_split_loss"}, "0"));
  tp.min_child_weight = parse_float("min_child_weight", get("min_child_weight", "1"));
  tp.max_depth = parse_int("max_depth", get("max_depth", "6"));
  tp.max_bin = parse_int("max_bin", get("max_bin", "256"));
  need(tp.eta > 0.0f, "eta must be positive");
  need(tp.lambda >= 0 && tp.alpha >= 0 && tp.gamma >= 0 && tp.min_child_weight >= 0,
       "regularisation parameters must be non-negative");
  need(tp.max_depth >= 1 && tp.max_depth <= 30, "max_depth must be in [1, 30]");
  need(tp.max_bin >= 2, "max_bin must be at least 2");
  need(tp.max_bin <= kMaxBins, "max_bin above 256 is not supported: bins are stored as uint8");
  // Row and column sampling (draws defined in sample.hpp).
  float* fractions[] = {&tp.subsample, &tp.colsample_bytree, &tp.colsample_bylevel,
                        &tp.colsample_bynode};
  const char* fraction_keys[] = {"subsample", "colsample_bytree", "colsample_bylevel",
                                 "colsample_bynode"};
  for (int i = 0; i < 4; ++i) {
    *fractions[i] = parse_float(fraction_keys[i], get(fraction_keys[i], "1"));
    need(*fractions[i] > 0.0f && *fractions[i] <= 1.0f,
         std::string(fraction_keys[i]) + " must be in (0, 1]");
  }
  {
    const std::string v = get("seed", "0");
    char* end = nullptr;
    const long long x = std::strtoll(v.c_str(), &end, 10);
    need(end && *end == '\0' && !v.empty(), "invalid integer value for seed: " + v);
    tp.seed = uint64_t(x);
  }
  const std::string method = get("tree_method", "hist");
  need(method == "hist" || method == "gpu_hist" || method == "auto",
       "tree_method must be hist");
  const std::string booster = get("booster", "gbtree");
  need(booster == "gbtree", "booster must be gbtree");
  const std::string policy = get("grow_policy", "depthwise");
  need(policy == "depthwise", "grow_policy must be depthwise");
  tp_ = tp;
  if (configured_) {
    need(train_ == d, "training on a second DMatrix is not supported");
    return;
  }
  objective_ = get("objective", "reg:squarederror");
  if (objective_ == "binary:logistic") {
    objective_id_ = DP_OBJ_LOGISTIC;
    n_groups_ = 1;
  } else if (objective_ == "multi:softmax" || objective_ == "multi:softprob") {
    objective_id_ = DP_OBJ_SOFTPROB;
    num_class_ = parse_int("num_class", get("num_class", "0"));
    need(num_class_ >= 2, "multi-class objectives need num_class >= 2");
    n_groups_ = num_class_;
  } else if (objective_ == "reg:squarederror") {
    objective_id_ = DP_OBJ_SQUARED;
    n_groups_ = 1;
  } else {
    fail("unsupported objective: " + objective_);
  }
  // base_score: scalar or JSON array; defaults 0.5 (logistic) / 0.
  base_score_.assign(size_t(n_groups_), objective_id_ == DP_OBJ_LOGISTIC ? 0.5f : 0.0f);
  auto bs = params_.find("base_score");
  if (bs != params_.end()) {
    json::Value v = json::parse(bs->second);
    if (v.kind == json::Value::Array) {
      need(v.items.size() == 1 || v.items.size() == size_t(n_groups_), "base_score size");
      for (int32_t k = 0; k < n_groups_; ++k)
        base_score_[size_t(k)] = float(v.items[v.items.size() == 1 ? 0 : size_t(k)].number());
    } else {
      for (auto& x : base_score_) x = float(v.number());
    }
  }
  for (float x : base_score_) need(std::isfinite(x), "base_score must be finite");
  if (objective_id_ == DP_OBJ_LOGISTIC)
    for (float x : base_score_) need(x > 0.0f && x < 1.0f, "logistic base_score must be in (0,1)");

  train_ = d;
  n_features_ = d->n_features;
  const int64_t N = d->n_rows;
  DP_HIP(hipStreamCreateWithFlags(&stream_, hipStreamDefault));  // orders with the null stream
  margin_.resize(size_t(N) * n_groups_);
  leaf_values_.resize(size_t(N) * n_groups_);
  grad_.resize(size_t(N) * n_groups_);
  hess_.resize(size_t(N) * n_groups_);
  gpair_.resize(size_t(N) * n_groups_ * 2);
  // The autotuner times the first round's histogram passes on gpair_ before
  // that round's quantiser writes it: zero it once so the timing passes read
  // defined values (their sums are discarded either way).
  launch_fill_u8(reinterpret_cast<uint8_t*>(gpair_.p), int64_t(gpair_.bytes()), 0, stream_);
  exps_.resize(size_t(2 * n_groups_));
  quant_scratch_.resize(quantise_scratch_bytes(N, n_groups_));
  std::vector<float> init(static_cast<size_t>(n_groups_));
  for (int32_t k = 0; k < n_groups_; ++k) {
    const float b = base_score_[size_t(k)];
    init[size_t(k)] =
        objective_id_ == DP_OBJ_LOGISTIC ? float(std::log(double(b) / (1.0 - double(b)))) : b;
  }
  DeviceBuffer<float> base(init.size());
  DP_HIP(hipMemcpy(base.p, init.data(), base.bytes(), hipMemcpyHostToDevice));
  launch_init_margin(margin_.p, N, n_groups_, base.p, stream_);
  DP_HIP(hipStreamSynchronize(stream_));  // before `base` is freed
  configured_ = true;
}

void Booster::update_one_iter(int iter, DMatrix* d) {
  need(d != nullptr, "null DMatrix");
  need(!model_only_, "continuing training of a loaded or sliced model is not supported");
  need(iter == rounds_, "iteration index must equal the number of boosted rounds");
  configure(d);
  need(d->has_labels, "training DMatrix has no labels");
  if (!labels_checked_) {
    DeviceBuffer<int32_t> bad(1);
    launch_check_labels(d->labels.p, d->n_rows, objective_id_, n_groups_, bad.p, stream_);
    int32_t flag = 0;
    DP_HIP(hipMemcpyAsync(&flag, bad.p, sizeof flag, hipMemcpyDeviceToHost, stream_));
    DP_HIP(hipStreamSynchronize(stream_));
    need(flag == 0, objective_id_ == DP_OBJ_SOFTPROB
                        ? "labels must be exact class ids in [0, num_class)"
                        : objective_id_ == DP_OBJ_LOGISTIC ? "logistic labels must be in [0, 1]"
                                                           : "labels must be finite");
    labels_checked_ = true;
  }
  caller_gradients_ = false;
  run_round(d, true);
}

void Booster::train_one_iter(DMatrix* d, int iter, const float* grad, const float* hess,
                             int64_t n, int32_t k) {
  need(d != nullptr, "null DMatrix");
  need(!model_only_, "continuing training of a loaded or sliced model is not supported");
  need(iter == rounds_, "iteration index must equal the number of boosted rounds");
  configure(d);
  need(n == d->n_rows && k == n_groups_, "gradient shape differs from [rows, outputs]");
  need(grad && hess, "null gradient buffer");
  // The round's quantiser reads the caller's buffers in place, in stream
  // order after the previous round, and the call returns once it has run: the
  // caller may then overwrite them from any stream, as upstream's call, which
  // consumes the gradients before it returns, allows.
  caller_grad_ = grad;
  caller_hess_ = hess;
  caller_gradients_ = true;
  if (!caller_read_) DP_HIP(hipEventCreateWithFlags(&caller_read_, hipEventDisableTiming));
  run_round(d, false);
  DP_HIP(hipEventSynchronize(caller_read_));
}

void Booster::enqueue(const std::vector<uint64_t>& key, bool capturable,
                      const std::function<void()>& body) {
  if (!use_graphs_ || !capturable) {
    body();
    return;
  }
  for (auto& g : graphs_)
    if (g.first == key) {
      DP_HIP(hipGraphLaunch(g.second, stream_));
      return;
    }
  // Capture: nothing in body() allocates, synchronises or reads device
  // memory on the host, so the captured launches are exactly the direct ones.
  // A capture does not run its launches, so when the runtime refuses any step
  // of it the body is simply launched directly (and graphs stay off).
  auto direct = [&] {
    (void)hipGetLastError();
    use_graphs_ = false;
    body();
  };
  hipGraph_t graph = nullptr;
  if (hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal) != hipSuccess)
    return direct();
  try {
    body();
  } catch (...) {
    if (hipStreamEndCapture(stream_, &graph) == hipSuccess && graph) (void)hipGraphDestroy(graph);
    throw;
  }
  if (hipStreamEndCapture(stream_, &graph) != hipSuccess || !graph) {
    if (graph) (void)hipGraphDestroy(graph);
    return direct();
  }
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) return direct();
  constexpr size_t kMaxGraphs = 4;
  if (graphs_.size() >= kMaxGraphs) {
    DP_HIP(hipStreamSynchronize(stream_));  // the oldest may still be running
    (void)hipGraphExecDestroy(graphs_.front().second);
    graphs_.erase(graphs_.begin());
  }
  graphs_.emplace_back(key, exec);
  DP_HIP(hipGraphLaunch(exec, stream_));
}

void Booster::run_round(DMatrix* d, bool with_gradients) {
  const int64_t N = d->n_rows;
  // Host inputs that size buffers: when they change, the round in flight is
  // collected first, so no buffer it uses moves under it.
  std::vector<uint64_t> inputs = {reinterpret_cast<uint64_t>(d), uint64_t(record_positions_),
                                  uint64_t(n_groups_), uint64_t(sparse_mode_),
                                  uint64_t(concurrent_trees_), uint64_t(autotune_),
                                  uint64_t(forced_hist_.tiles), uint64_t(forced_hist_.unroll),
                                  uint64_t(forced_hist_.items), uint64_t(forced_hist_.split),
                                  uint64_t(forced_hist_.deep), uint64_t(skip_mode_)};
  auto words = [](std::vector<uint64_t>& v, const void* p, size_t n) {
    for (size_t i = 0; i < n; i += 8) {
      uint64_t w = 0;
      std::memcpy(&w, static_cast<const uint8_t*>(p) + i, std::min<size_t>(8, n - i));
      v.push_back(w);
    }
  };
  words(inputs, &tp_, sizeof tp_);
  if (inputs != last_round_inputs_) flush();
  Quantized* qp;
  {
    dp_workspace_s scratch;
    qp = &d->quantize(tp_.max_bin, scratch, stream_);
  }
  Quantized& q = *qp;
  effective_max_bin_ = q.max_bin;
  // Histogram layout: the present-value layout for mostly-missing matrices,
  // else the row-major copy of the tiles for gathered rows.
  bool sparse = false;
  if (q.layout.missing_bin == kWideMissing) {
    // 16-bit symbols: the present-value layout is the only histogram layout
    // (whatever dp_sparse_hist says), built from the columns.
    if (q.sparse.n_tiles == 0) {
      build_sparse_bins_wide(q.cols16.p, N, q.layout.n_features, q.bin_stride, q.sparse, stream_);
      q.sparse_limit = 1.0;
    }
    sparse = true;
  } else if (sparse_mode_ != 0 && q.layout.missing_bin >= 0) {
    const double limit = sparse_mode_ == 2 ? 1.0 : kSparseDensity;
    if (q.sparse.n_tiles == 0 && q.sparse_limit < limit) {
      q.density = build_sparse_bins(q.bins.p, q.layout, q.bin_stride, limit, q.sparse, stream_);
      q.sparse_limit = limit;
    }
    sparse = q.sparse.n_tiles > 0;
  }
  // Skip bins (matrices without missing values): counted once per matrix.
  bool skip = false;
  if (!sparse && q.layout.missing_bin < 0 && skip_mode_ != 0) {
    if (q.skip_share < 0.0) build_skip_bins(q, stream_);
    skip = skip_mode_ == 2 || q.skip_share >= kSkipShare;
  }
  // Paired tiles (dense histograms without skip bins): the tuner times and the
  // growers launch with this layout.
  dp_bin_layout hl = q.layout;
  hl.paired_tiles = !sparse && !skip && pair_tiles_ ? q.pairs : 0;
  if (record_positions_) positions_.reserve(size_t(N));
  // Histogram launch shapes: forced by dp_hist_* (0 = default for the rest),
  // else tuned on this matrix shape (once per process), else the defaults.
  HistConfig root_cfg, level_cfg;
  if (forced_hist_.tiles || forced_hist_.unroll || forced_hist_.items || forced_hist_.split ||
      forced_hist_.deep) {
    need(!(forced_hist_.deep && forced_hist_.split), "dp_hist_deep 1 needs dp_hist_split 0");
    if (forced_hist_.tiles) root_cfg.tiles = forced_hist_.tiles;
    if (forced_hist_.unroll) root_cfg.unroll = forced_hist_.unroll;
    if (forced_hist_.items) root_cfg.items = forced_hist_.items;
    root_cfg.split = forced_hist_.split;
    root_cfg.deep = forced_hist_.deep;
    level_cfg = root_cfg;
    tuning_report_ = "{\"forced\":true}";
  } else if (autotune_) {
    const HistTuning& t =
        sparse ? tune_sparse_hist(q.sparse, N, q.layout.n_features, q.bin_stride, gpair_.p,
                                  stream_)
               : tune_dense_hist(hl, q.bins.p, true, q.bin_stride, gpair_.p, stream_,
                                 skip ? q.skip_tiles.p : nullptr);
    root_cfg = t.root;
    level_cfg = t.level;
    tuning_report_ = t.report;
  } else {
    tuning_report_ = "{\"defaults\":true}";
  }
  // The gathered passes' row-major copy: with the pairs' joint tiles in place
  // of their first tiles when the level shape uses the pairs, else plain.
  const uint64_t rows_pairs = sparse ? 0 : hist_pairs(hl.paired_tiles, level_cfg.tiles);
  if (!sparse && !q.row_major(rows_pairs)) {
    dp_bin_layout rl = q.layout;
    rl.paired_tiles = rows_pairs;
    auto& copy = q.rows.emplace(rows_pairs, DeviceBuffer<uint8_t>(dp_layout_bytes(&q.layout)))
                     .first->second;
    launch_tiles_to_rows(q.bins.p, rl, copy.p, stream_);
  }
  {  // the histogram mode beside the launch shapes
    std::string mode = "{\"layout\":\"";
    mode += sparse ? "present-value" : "dense";
    mode += "\",\"skip_bins\":";
    mode += skip ? "true" : "false";
    char pairs[40];
    std::snprintf(pairs, sizeof pairs, ",\"paired_tiles\":%llu",
                  static_cast<unsigned long long>(hl.paired_tiles));
    mode += pairs;
    if (q.skip_share >= 0.0) {
      mode += ",\"skip_share\":";
      json::put_double(mode, q.skip_share);
    }
    tuning_report_ = mode + "," + tuning_report_.substr(1);
  }
  const int32_t K = n_groups_;
  int32_t S = std::min(K, concurrent_trees_);
  while (int32_t(growers_.size()) < S) growers_.push_back(std::make_unique<Grower>());
  if (growers_.empty()) growers_.push_back(std::make_unique<Grower>());
  growers_[0]->prepare(q, tp_, (K + S - 1) / S, sparse, root_cfg, level_cfg, skip,
                       hl.paired_tiles, stream_);
  const bool eager = growers_[0]->eager();
  if (!eager && S > 1) {  // level-synced trees synchronise per level: one at a time
    S = 1;
    growers_[0]->prepare(q, tp_, K, sparse, root_cfg, level_cfg, skip, hl.paired_tiles,
                         stream_);
  }
  for (int32_t l = 1; l < S; ++l)
    growers_[size_t(l)]->prepare(q, tp_, (K - l + S - 1) / S, sparse, root_cfg, level_cfg,
                                 skip, hl.paired_tiles, stream_);
  while (S > 1 && int32_t(tree_streams_.size()) < S) {
    hipStream_t t;
    DP_HIP(hipStreamCreateWithFlags(&t, hipStreamNonBlocking));
    tree_streams_.push_back(t);
    hipEvent_t e;
    DP_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    tree_done_.push_back(e);
  }
  if (S > 1 && !fork_) DP_HIP(hipEventCreateWithFlags(&fork_, hipEventDisableTiming));
  // Level-synced trees copy their records during grow(): collect the round in
  // flight before they are overwritten.
  if (!eager) flush();
  last_round_inputs_ = inputs;
  int32_t* positions = record_positions_ ? positions_.p : nullptr;
  // Everything the enqueued launches depend on: a change of any of it gives
  // a new graph.
  std::vector<uint64_t> key = {
      uint64_t(with_gradients), reinterpret_cast<uint64_t>(d), reinterpret_cast<uint64_t>(&q),
      reinterpret_cast<uint64_t>(q.bins.p), reinterpret_cast<uint64_t>(q.cols.p),
      reinterpret_cast<uint64_t>(q.cols16.p),
      reinterpret_cast<uint64_t>(q.row_major(rows_pairs)), reinterpret_cast<uint64_t>(q.d_nbins.p),
      uint64_t(q.bin_stride), uint64_t(N), reinterpret_cast<uint64_t>(d->labels.p),
      uint64_t(objective_id_), uint64_t(n_groups_), reinterpret_cast<uint64_t>(margin_.p),
      reinterpret_cast<uint64_t>(leaf_values_.p), reinterpret_cast<uint64_t>(grad_.p), reinterpret_cast<uint64_t>(hess_.p),
      reinterpret_cast<uint64_t>(gpair_.p), reinterpret_cast<uint64_t>(exps_.p),
      reinterpret_cast<uint64_t>(quant_scratch_.p),
      reinterpret_cast<uint64_t>(positions), reinterpret_cast<uint64_t>(q.sparse.ptr.p),
      reinterpret_cast<uint64_t>(q.sparse.entries.p), uint64_t(sparse), uint64_t(S)};
  // Sampling kernels read the round's index from device memory, stored ahead
  // of the (possibly replayed) round.
  RowSample rows;
  if (tp_.subsample < 1.0f || tp_.colsample()) {
    round_dev_.reserve(1);
    launch_store_i32(round_dev_.p, rounds_, stream_);
    if (tp_.subsample < 1.0f) {
      rows.seed = tp_.seed;
      rows.threshold = uint64_t(std::ldexp(double(tp_.subsample), 32));
      rows.round = round_dev_.p;
    }
  }
  key.push_back(reinterpret_cast<uint64_t>(round_dev_.p));
  for (int32_t l = 0; l < S; ++l) key.push_back(growers_[size_t(l)]->signature());
  words(key, &q.layout, sizeof q.layout);
  words(key, &tp_, sizeof tp_);
  // A round that computes gradients leaves its leaf values for the next round's
  // gradient kernel to add to the margins (one launch fewer per round);
  // values_pending_ says so, and margins() adds them when asked first.
  const bool add_first = values_pending_ && !with_gradients;  // caller gradients follow
  key.push_back(uint64_t(values_pending_) | uint64_t(with_gradients) << 1);
  // The per-workgroup sums stay in the quantiser's slots: each tree's first
  // launch adds up its output's.  Caller gradients are quantised by direct
  // launches ahead of the round's graph, so that the call can wait for their
  // last read (caller_read_) without waiting for the trees.
  if (!with_gradients) {
    launch_quantise(caller_grad_, caller_hess_, N, K, quant_scratch_.p, false, exps_.p,
                    gpair_.p, nullptr, stream_, rows);
    DP_HIP(hipEventRecord(caller_read_, stream_));
  }
  enqueue(key, eager, [&] {
    if (add_first) launch_add_leaf_values(margin_.p, K, leaf_values_.p, N, stream_);
    if (with_gradients) {
      // With row sampling the quantiser takes the maxima over the kept rows.
      const bool maxima =
          launch_gradients(objective_id_, margin_.p, d->labels.p, N, K, grad_.p, hess_.p,
                           rows.active() ? nullptr : quant_scratch_.p, stream_,
                           values_pending_ ? leaf_values_.p : nullptr);
      launch_quantise(grad_.p, hess_.p, N, K, quant_scratch_.p, maxima, exps_.p, gpair_.p,
                      nullptr, stream_, rows);
    }
    const int32_t blocks = quantise_blocks(N);
    const int64_t* slots = quantise_sum_slots(quant_scratch_.p, N, K);
    auto sample_columns = [&](Grower& g, int32_t k) {
      g.colsample = ColSample{};
      if (tp_.colsample()) {
        g.colsample.seed = tp_.seed;
        g.colsample.round = round_dev_.p;
        g.colsample.output = k;
        g.colsample.bytree = tp_.colsample_bytree;
        g.colsample.bylevel = tp_.colsample_bylevel;
        g.colsample.bynode = tp_.colsample_bynode;
      }
    };
    if (S == 1) {
      for (int32_t k = 0; k < K; ++k) {
        sample_columns(*growers_[0], k);
        growers_[0]->grow(q, gpair_.p + int64_t(k) * N * 2, exps_.p + 2 * k,
                          slots + int64_t(k) * blocks * 2, blocks, tp_,
                          leaf_values_.p + int64_t(k) * N, positions, k, stream_);
      }
      if (!with_gradients) launch_add_leaf_values(margin_.p, K, leaf_values_.p, N, stream_);
      return;
    }
    // Each tree stores its own leaf-value plane; only the last writes the row
    // positions (the round's positions are its last tree's).
    DP_HIP(hipEventRecord(fork_, stream_));
    for (int32_t l = 0; l < S; ++l) DP_HIP(hipStreamWaitEvent(tree_streams_[size_t(l)], fork_, 0));
    for (int32_t k = 0; k < K; ++k) {
      sample_columns(*growers_[size_t(k % S)], k);
      growers_[size_t(k % S)]->grow(q, gpair_.p + int64_t(k) * N * 2, exps_.p + 2 * k,
                                    slots + int64_t(k) * blocks * 2, blocks, tp_,
                                    leaf_values_.p + int64_t(k) * N,
                                    k == K - 1 ? positions : nullptr, k / S,
                                    tree_streams_[size_t(k % S)]);
    }
    for (int32_t l = 0; l < S; ++l) {
      DP_HIP(hipEventRecord(tree_done_[size_t(l)], tree_streams_[size_t(l)]));
      DP_HIP(hipStreamWaitEvent(stream_, tree_done_[size_t(l)], 0));
    }
    if (!with_gradients) launch_add_leaf_values(margin_.p, K, leaf_values_.p, N, stream_);
  });
  values_pending_ = with_gradients;
  // This round's records go to the buffer the round in flight does not use.
  const int32_t buffer = pending_ ? 1 - pending_buffer_ : 0;
  for (int32_t l = 0; l < S; ++l)
    growers_[size_t(l)]->readback(S == 1 ? K : (K - l + S - 1) / S, buffer, stream_);
  if (!round_done_[buffer])
    DP_HIP(hipEventCreateWithFlags(&round_done_[buffer], hipEventDisableTiming));
  DP_HIP(hipEventRecord(round_done_[buffer], stream_));
  flush();  // the previous round, which completed before this one started
  pending_ = true;
  pending_buffer_ = buffer;
  pending_q_ = &q;
  pending_d_ = d;
  pending_lanes_ = S;
  d->pending.push_back(this);
  ++rounds_;
  if (!eager) flush();
}

void Booster::flush() const {
  if (!pending_) return;
  pending_ = false;
  if (pending_d_) {
    auto& v = pending_d_->pending;
    v.erase(std::remove(v.begin(), v.end(), this), v.end());
  }
  const int32_t b = pending_buffer_;
  DP_HIP(hipEventSynchronize(round_done_[b]));
  // Each tree's records carry its output's quantiser exponents.
  last_exps_.assign(size_t(2 * n_groups_), 0);
  for (int32_t k = 0; k < n_groups_; ++k)
    growers_[size_t(k % pending_lanes_)]->exponents(k / pending_lanes_, b,
                                                   &last_exps_[2 * size_t(k)]);
  std::vector<Tree> round(static_cast<size_t>(n_groups_));
  try {
    const int32_t S = pending_lanes_;
    for (int32_t k = 0; k < n_groups_; ++k)
      growers_[size_t(k % S)]->collect(*pending_q_, k / S, b, round[size_t(k)]);
  } catch (...) {
    rounds_ = int(iteration_indptr_.size()) - 1;  // the failed round is not part of the model
    throw;
  }
  for (int32_t k = 0; k < n_groups_; ++k) {
    trees_.push_back(std::move(round[size_t(k)]));
    tree_info_.push_back(k);
  }
  iteration_indptr_.push_back(int32_t(trees_.size()));
}

void Booster::margins(float* out, size_t n) const {
  flush();
  need(configured_, "booster has not been trained");
  need(n == margin_.n, "margin buffer size differs");
  if (values_pending_) {  // the last round's leaf values, left for the next gradients
    launch_add_leaf_values(margin_.p, n_groups_, leaf_values_.p, train_->n_rows, stream_);
    values_pending_ = false;
  }
  DP_HIP(hipStreamSynchronize(stream_));
  DP_HIP(hipMemcpy(out, margin_.p, margin_.bytes(), hipMemcpyDeviceToHost));
}

void Booster::last_gradients(float* grad, float* hess, size_t n, int32_t* exps) const {
  flush();
  need(configured_, "booster has not been trained");
  need(!caller_gradients_,
       "the last round's gradients were supplied by the caller (XGBoosterTrainOneIter)");
  need(n == grad_.n, "gradient buffer size differs");
  if (grad) DP_HIP(hipMemcpy(grad, grad_.p, grad_.bytes(), hipMemcpyDeviceToHost));
  if (hess) DP_HIP(hipMemcpy(hess, hess_.p, hess_.bytes(), hipMemcpyDeviceToHost));
  if (exps) std::copy(last_exps_.begin(), last_exps_.end(), exps);
}

void Booster::last_positions(int32_t* out, size_t n) const {
  flush();
  need(record_positions_ && positions_.p, "set dp_record_positions=1 before training");
  need(n == size_t(train_->n_rows), "positions buffer size differs");
  DP_HIP(hipMemcpy(out, positions_.p, sizeof(int32_t) * n, hipMemcpyDeviceToHost));
}

// ---------------------------------------------------------------------------
// Model and configuration JSON (XGBoost 3.4.1 schema; the fields the
// reference's readers consume are listed at native/class_io.hpp:99-240).
// ---------------------------------------------------------------------------
namespace {

std::string objective_json(const std::string& name, int32_t num_class) {
  std::string o = "{\"name\":";
  json::put_string(o, name);
  if (name == "multi:softmax" || name == "multi:softprob")
    o += ",\"softmax_multiclass_param\":{\"num_class\":\"" + std::to_string(num_class) + "\"}";
  else
    o += ",\"reg_loss_param\":{\"scale_pos_weight\":\"1\"}";
  o += '}';
  return o;
}

std::string base_score_text(const std::vector<float>& b) {
  std::string s = "[";
  for (size_t i = 0; i < b.size(); ++i) {
    if (i) s += ',';
    json::put_float(s, b[i]);
  }
  return s + "]";
}

}  // namespace

std::string Booster::save_model() const {
  flush();
  std::string o;
  o.reserve(1 << 16);
  o += "{\"learner\":{\"attributes\":{},\"feature_names\":[],\"feature_types\":[],";
  o += "\"gradient_booster\":{\"model\":{\"gbtree_model_param\":{\"num_parallel_tree\":\"1\","
       "\"num_trees\":\"";
  o += std::to_string(trees_.size()) + "\"},\"iteration_indptr\":";
  json::put_int_array(o, iteration_indptr_);
  o += ",\"tree_info\":";
  json::put_int_array(o, tree_info_);
  o += ",\"trees\":[";
  for (size_t t = 0; t < trees_.size(); ++t) {
    const Tree& tr = trees_[t];
    const size_t n = size_t(tr.size());
    if (t) o += ',';
    std::vector<int32_t> parents(n), split_idx(n), dl(n), split_type(n, 0);
    std::vector<float> loss(n);
    for (size_t i = 0; i < n; ++i) {
      parents[i] = tr.parent[i] < 0 ? INT_MAX : tr.parent[i];
      const bool leaf = tr.left[i] == -1;
      split_idx[i] = leaf ? 0 : tr.feature[i];
      dl[i] = leaf ? 0 : tr.default_left[i];
      loss[i] = leaf ? 0.0f : tr.loss_chg[i];
    }
    o += "{\"base_weights\":";
    json::put_float_array(o, tr.base_weight);
    o += ",\"categories\":[],\"categories_nodes\":[],\"categories_segments\":[],"
         "\"categories_sizes\":[],\"default_left\":";
    json::put_int_array(o, dl);
    o += ",\"id\":" + std::to_string(t) + ",\"left_children\":";
    json::put_int_array(o, tr.left);
    o += ",\"loss_changes\":";
    json::put_float_array(o, loss);
    o += ",\"parents\":";
    json::put_int_array(o, parents);
    o += ",\"right_children\":";
    json::put_int_array(o, tr.right);
    o += ",\"split_conditions\":";
    json::put_float_array(o, tr.cond);
    o += ",\"split_indices\":";
    json::put_int_array(o, split_idx);
    o += ",\"split_type\":";
    json::put_int_array(o, split_type);
    o += ",\"sum_hessian\":";
    json::put_float_array(o, tr.sum_hess);
    o += ",\"tree_param\":{\"num_deleted\":\"0\",\"num_feature\":\"" + std::to_string(n_features_) +
         "\",\"num_nodes\":\"" + std::to_string(n) + "\",\"size_leaf_vector\":\"1\"}}";
  }
  o += "]},\"name\":\"gbtree\"},\"learner_model_param\":{\"base_score\":";
  json::put_string(o, base_score_text(base_score_));
  o += ",\"boost_from_average\":\"0\",\"num_class\":\"" + std::to_string(num_class_) +
       "\",\"num_feature\":\"" + std::to_string(n_features_) +
       "\",\"num_target\":\"1\"},\"objective\":" +
       objective_json(effective_objective(), num_class_) + "},\"version\":[3,4,1]}";
  return o;
}

std::string Booster::save_config() const {
  flush();
  auto get = [&](const char* k, const char* dflt) {
    auto it = params_.find(k);
    return it == params_.end() ? std::string(dflt) : it->second;
  };
  std::string device = get("device", "cuda:0");
  if (device == "cuda" || device == "gpu") device = "cuda:0";
  std::string o = "{\"learner\":{\"generic_param\":{\"device\":";
  json::put_string(o, device);
  o += ",\"nthread\":";
  json::put_string(o, get("nthread", "0"));
  o += ",\"seed\":";
  json::put_string(o, get("seed", "0"));
  o += ",\"seed_per_iteration\":";
  json::put_string(o, get("seed_per_iteration", "0"));
  o += ",\"validate_parameters\":";
  json::put_string(o, get("validate_parameters", "0"));
  o += "},\"gradient_booster\":{\"gbtree_model_param\":{\"num_parallel_tree\":\"1\",\"num_trees\":\"" +
       std::to_string(trees_.size()) +
       "\"},\"gbtree_train_param\":{\"process_type\":\"default\",\"tree_method\":\"hist\","
       "\"updater\":\"grow_gpu_hist\",\"updater_seq\":\"grow_gpu_hist\"},\"name\":\"gbtree\","
       "\"updater\":[{\"hist_train_param\":{\"max_bin\":\"";
  // The bins the cuts were computed with (max_bin, at most 256, also with
  // missing values).
  o += std::to_string(effective_max_bin_ > 0 ? effective_max_bin_ : tp_.max_bin) +
       "\"},\"name\":\"grow_gpu_hist\",\"train_param\":{";
  auto kv = [&](const char* k, const std::string& v, bool comma = true) {
    if (comma) o += ',';
    json::put_string(o, k);
    o += ':';
    json::put_string(o, v);
  };
  kv("alpha", get("alpha", "0"), false);
  kv("eta", get("eta", "0.3"));
  kv("gamma", get("gamma", "0"));
  kv("lambda", get("lambda", "1"));
  kv("max_depth", get("max_depth", "6"));
  kv("min_child_weight", get("min_child_weight", "1"));
  kv("subsample", get("subsample", "1"));
  kv("colsample_bytree", get("colsample_bytree", "1"));
  kv("colsample_bylevel", get("colsample_bylevel", "1"));
  kv("colsample_bynode", get("colsample_bynode", "1"));
  o += "}}]},\"learner_model_param\":{\"base_score\":";
  json::put_string(o, base_score_text(base_score_));
  o += ",\"boost_from_average\":\"0\",\"num_class\":\"" + std::to_string(num_class_) +
       "\",\"num_feature\":\"" + std::to_string(n_features_) +
       "\",\"num_target\":\"1\"},\"learner_train_param\":{\"booster\":\"gbtree\",\"objective\":";
  json::put_string(o, effective_objective());
  o += "},\"objective\":" + objective_json(effective_objective(), num_class_) +
       "},\"version\":[3,4,1]}";
  return o;
}


// ---------------------------------------------------------------------------
// Prediction, loading and slicing
// ---------------------------------------------------------------------------
std::string Booster::effective_objective() const {
  auto it = params_.find("objective");
  if (model_only_ && it != params_.end()) return it->second;
  return objective_;
}

void Booster::upload_forest(int32_t tree_begin, int32_t tree_end) {
  flush();
  if (forest_begin_ == tree_begin && forest_end_ == tree_end && forest_trees_ == trees_.size())
    return;
  std::vector<PredNode> nodes;
  std::vector<int32_t> roots;
  std::vector<std::vector<int32_t>> per_group(size_t(std::max(n_groups_, 1)));
  for (int32_t t = tree_begin; t < tree_end; ++t) {
    const Tree& tr = trees_[size_t(t)];
    const int32_t base = int32_t(nodes.size());
    for (int32_t i = 0; i < tr.size(); ++i) {
      const bool leaf = tr.left[size_t(i)] == -1;
      nodes.push_back({leaf ? -1 : base + tr.left[size_t(i)], leaf ? 0 : tr.feature[size_t(i)],
                       tr.cond[size_t(i)], leaf ? 0 : int32_t(tr.default_left[size_t(i)])});
    }
    per_group[size_t(tree_info_[size_t(t)])].push_back(base);
  }
  std::vector<int32_t> group_ptr{0};
  for (const auto& g : per_group) {
    roots.insert(roots.end(), g.begin(), g.end());
    group_ptr.push_back(int32_t(roots.size()));
  }
  std::vector<float> base(size_t(std::max(n_groups_, 1)));
  for (size_t k = 0; k < base.size(); ++k) {
    const float b = base_score_.empty() ? 0.0f : base_score_[k < base_score_.size() ? k : 0];
    base[k] = objective_id_ == DP_OBJ_LOGISTIC ? float(std::log(double(b) / (1.0 - double(b)))) : b;
  }
  forest_nodes_.resize(std::max<size_t>(nodes.size(), 1) * sizeof(PredNode));
  forest_roots_.resize(std::max<size_t>(roots.size(), 1));
  forest_group_ptr_.resize(group_ptr.size());
  forest_base_.resize(base.size());
  if (!nodes.empty())
    DP_HIP(hipMemcpy(forest_nodes_.p, nodes.data(), nodes.size() * sizeof(PredNode),
                     hipMemcpyHostToDevice));
  if (!roots.empty())
    DP_HIP(hipMemcpy(forest_roots_.p, roots.data(), roots.size() * sizeof(int32_t),
                     hipMemcpyHostToDevice));
  DP_HIP(hipMemcpy(forest_group_ptr_.p, group_ptr.data(), group_ptr.size() * sizeof(int32_t),
                   hipMemcpyHostToDevice));
  DP_HIP(hipMemcpy(forest_base_.p, base.data(), base.size() * sizeof(float),
                   hipMemcpyHostToDevice));
  forest_begin_ = tree_begin;
  forest_end_ = tree_end;
  forest_trees_ = trees_.size();
}

const float* Booster::predict(const PredictRequest& req, std::vector<uint64_t>& shape) {
  flush();
  need(configured_ || model_only_, "booster holds no model");
  need(req.features == n_features_, "prediction input has " + std::to_string(req.features) +
                                        " features, the model " + std::to_string(n_features_));
  need(req.rows >= 0 && req.row_stride >= req.features, "prediction input shape");
  const int32_t begin = req.iteration_begin;
  const int32_t end = req.iteration_end == 0 ? rounds_ : req.iteration_end;
  need(begin >= 0 && begin <= end && end <= rounds_, "iteration range outside the model");
  const std::string obj = effective_objective();
  int32_t transform = kPredIdentity, outputs = n_groups_;
  if (req.type == 0) {
    if (obj == "binary:logistic") transform = kPredSigmoid;
    else if (obj == "multi:softprob") transform = kPredSoftmax;
    else if (obj == "multi:softmax") { transform = kPredArgmax; outputs = 1; }
  } else {
    need(req.type == 1, "prediction type must be 0 (value) or 1 (margin)");
  }
  upload_forest(iteration_indptr_[size_t(begin)], iteration_indptr_[size_t(end)]);
  pred_out_.reserve(size_t(std::max<int64_t>(req.rows, 1)) * size_t(n_groups_));
  hipStream_t s = stream_;
  launch_predict(req.values, req.rows, req.features, req.row_stride, req.missing,
                 reinterpret_cast<const PredNode*>(forest_nodes_.p), forest_roots_.p,
                 forest_group_ptr_.p, n_groups_, forest_base_.p, transform, pred_out_.p, s);
  DP_HIP(hipStreamSynchronize(s));
  shape.clear();
  shape.push_back(uint64_t(req.rows));
  if (req.strict_shape || outputs > 1) shape.push_back(uint64_t(outputs));
  return pred_out_.p;
}

void Booster::load_model(const std::string& text) {
  flush();
  need(!configured_, "cannot load into a booster that is training");
  const json::Value doc = json::parse(text);
  const auto& learner = doc.at("learner");
  const auto& mp = learner.at("learner_model_param");
  auto decimal = [](const json::Value& v, const char* what) {
    need(v.kind == json::Value::String, std::string(what) + " must be a decimal string");
    char* e = nullptr;
    const long long x = std::strtoll(v.text.c_str(), &e, 10);
    need(e && *e == '\0' && !v.text.empty() && x >= 0, std::string("invalid ") + what);
    return int64_t(x);
  };
  n_features_ = int32_t(decimal(mp.at("num_feature"), "num_feature"));
  num_class_ = int32_t(decimal(mp.at("num_class"), "num_class"));
  objective_ = learner.at("objective").at("name").text;
  if (objective_ == "binary:logistic") objective_id_ = DP_OBJ_LOGISTIC;
  else if (objective_ == "multi:softmax" || objective_ == "multi:softprob") objective_id_ = DP_OBJ_SOFTPROB;
  else if (objective_ == "reg:squarederror") objective_id_ = DP_OBJ_SQUARED;
  else fail("unsupported objective in model: " + objective_);
  n_groups_ = objective_id_ == DP_OBJ_SOFTPROB ? num_class_ : 1;
  need(n_groups_ >= 1, "model output count");
  json::Value bs = mp.at("base_score");
  if (bs.kind == json::Value::String) bs = json::parse(bs.text);
  base_score_.clear();
  if (bs.kind == json::Value::Array)
    for (const auto& x : bs.items) base_score_.push_back(float(x.number()));
  else
    base_score_.push_back(float(bs.number()));
  need(base_score_.size() == 1 || base_score_.size() == size_t(n_groups_), "base_score size");
  if (base_score_.size() == 1) base_score_.resize(size_t(n_groups_), base_score_[0]);
  const auto& model = learner.at("gradient_booster").at("model");
  const auto& trees = model.at("trees").items;
  const auto& info = model.at("tree_info").items;
  need(trees.size() == info.size(), "tree_info size differs from the tree count");
  trees_.clear();
  tree_info_.clear();
  for (size_t t = 0; t < trees.size(); ++t) {
    const json::Value& jt = trees[t];
    auto ints = [&](const char* k) {
      std::vector<int32_t> v;
      for (const auto& x : jt.at(k).items) v.push_back(int32_t(x.i64()));
      return v;
    };
    auto floats = [&](const char* k) {
      std::vector<float> v;
      if (const auto* a = jt.find(k))
        for (const auto& x : a->items) v.push_back(float(x.number()));
      return v;
    };
    Tree tr;
    tr.left = ints("left_children");
    tr.right = ints("right_children");
    tr.feature = ints("split_indices");
    tr.cond = floats("split_conditions");
    const size_t n = tr.left.size();
    need(n > 0 && tr.right.size() == n && tr.feature.size() == n && tr.cond.size() == n,
         "tree node arrays differ in size");
    for (const auto& x : jt.at("default_left").items)
      tr.default_left.push_back(uint8_t(x.kind == json::Value::Bool ? x.boolean : x.i64() != 0));
    need(tr.default_left.size() == n, "default_left size");
    tr.base_weight = floats("base_weights");
    tr.loss_chg = floats("loss_changes");
    tr.sum_hess = floats("sum_hessian");
    tr.base_weight.resize(n, 0.0f);
    tr.loss_chg.resize(n, 0.0f);
    tr.sum_hess.resize(n, 0.0f);
    tr.parent.assign(n, -1);
    tr.split_bin.assign(n, -1);
    tr.sum_qg.assign(n, 0);
    tr.sum_qh.assign(n, 0);
    for (size_t i = 0; i < n; ++i) {
      if (tr.left[i] == -1) continue;
      need(tr.left[i] > int32_t(i) && tr.right[i] == tr.left[i] + 1 && tr.right[i] < int32_t(n),
           "split successors must advance and be consecutive");
      need(tr.feature[i] >= 0 && tr.feature[i] < n_features_, "split feature out of range");
      tr.parent[size_t(tr.left[i])] = tr.parent[size_t(tr.right[i])] = int32_t(i);
    }
    const int32_t group = int32_t(info[t].i64());
    need(group >= 0 && group < n_groups_, "tree_info class out of range");
    trees_.push_back(std::move(tr));
    tree_info_.push_back(group);
  }
  iteration_indptr_.clear();
  if (const auto* ip = model.find("iteration_indptr")) {
    for (const auto& x : ip->items) iteration_indptr_.push_back(int32_t(x.i64()));
  } else {
    for (size_t t = 0; t <= trees_.size(); t += size_t(n_groups_))
      iteration_indptr_.push_back(int32_t(t));
  }
  need(iteration_indptr_.size() >= 1 && iteration_indptr_.front() == 0 &&
           iteration_indptr_.back() == int32_t(trees_.size()),
       "iteration_indptr does not cover the trees");
  rounds_ = int(iteration_indptr_.size()) - 1;
  model_only_ = true;
  forest_begin_ = forest_end_ = -1;
  if (!stream_) DP_HIP(hipStreamCreateWithFlags(&stream_, hipStreamDefault));
}

std::unique_ptr<Booster> Booster::slice(int begin, int end, int step) const {
  flush();
  need(configured_ || model_only_, "booster holds no model");
  if (end == 0) end = rounds_;
  need(step >= 1 && begin >= 0 && begin <= end && end <= rounds_, "slice range outside the model");
  auto out = std::make_unique<Booster>(std::vector<DMatrix*>{});
  out->params_ = params_;
  out->params_.erase("dp_record_positions");
  out->params_.erase("dp_graphs");
  out->params_.erase("dp_sparse_hist");
  out->params_.erase("dp_concurrent_trees");
  out->objective_ = effective_objective();
  out->objective_id_ = objective_id_;
  out->n_groups_ = n_groups_;
  out->num_class_ = num_class_;
  out->n_features_ = n_features_;
  out->base_score_ = base_score_;
  out->tp_ = tp_;
  out->effective_max_bin_ = effective_max_bin_;
  out->iteration_indptr_ = {0};
  for (int r = begin; r < end; r += step) {
    for (int32_t t = iteration_indptr_[size_t(r)]; t < iteration_indptr_[size_t(r) + 1]; ++t) {
      out->trees_.push_back(trees_[size_t(t)]);
      out->tree_info_.push_back(tree_info_[size_t(t)]);
    }
    out->iteration_indptr_.push_back(int32_t(out->trees_.size()));
  }
  out->rounds_ = int(out->iteration_indptr_.size()) - 1;
  out->model_only_ = true;
  DP_HIP(hipStreamCreateWithFlags(&out->stream_, hipStreamDefault));
  return out;
}

}  // namespace dp
