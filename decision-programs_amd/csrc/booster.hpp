// Host-side training objects behind the XGBoost-compatible C API.
#pragma once

#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "dp_internal.hpp"

namespace dp {

// Quantised view of a matrix for one max_bin: cuts plus tile-major bins.
struct Quantized {
  dp_bin_layout layout{};
  int32_t max_bin = 0;     // effective max_bin used for the cuts
  int32_t bin_stride = 0;  // largest per-feature bin count
  std::vector<int32_t> cut_ptr;
  std::vector<float> cut_values, min_values;
  DeviceBuffer<int32_t> d_cut_ptr, d_nbins;
  DeviceBuffer<float> d_cut_values;
  DeviceBuffer<uint8_t> bins;
  DeviceBuffer<uint8_t> cols;  // column-major copy: cols[f * n_rows + r]
  // A matrix with missing values some of whose features use all 256 bins
  // (layout.missing_bin == kWideMissing): no uint8 bins; 16-bit columns
  // (missing: kWideMissing) for the partition, and every histogram from the
  // present-value layout built from them.
  DeviceBuffer<uint16_t> cols16;
  // Row-major copies, rows[(r * n_tiles + t) * 16 + j], by the pairs whose
  // joint tiles replace their first tiles (0: the plain copy); each made on
  // first use and kept, so boosters sharing the matrix never rewrite one.
  std::map<uint64_t, DeviceBuffer<uint8_t>> rows;
  const uint8_t* row_major(uint64_t pairs) const {
    const auto it = rows.find(pairs);
    return it == rows.end() ? nullptr : it->second.p;
  }
  SparseBins sparse;           // present-value layout (on demand, mostly-missing matrices)
  // Skip bins (matrices without missing values, on demand): each feature's most
  // frequent bin, per feature and per 16-feature tile, and the share of the
  // histogram's element atomics they remove: the rows in those bins plus the
  // last tile's padding features, over n_tiles * 16 (-1: not counted yet).
  DeviceBuffer<uint8_t> skip_features, skip_tiles;
  double skip_share = -1.0;
  double sparse_limit = -1.0;  // largest density limit the layout was tried with
  double density = -1.0;       // share of present values, once counted
  // Tiles the dense histograms may pair (dp_bin_layout::paired_tiles, from
  // pair_tiles: none with missing values); their joint tiles follow the
  // n_tiles tiles in `bins`.
  uint64_t pairs = 0;
};

// Counts each feature's bins (column copy) and fills q.skip_features,
// q.skip_tiles and q.skip_share; synchronises the stream.
void build_skip_bins(Quantized& q, hipStream_t s);
// dp_skip_bin 1 uses skip bins when they remove at least this share of the
// element atomics (C4's zero pixels: about 0.8; C1's 8 features in a 16-wide
// tile: 0.5; quantile-binned features filling their tiles: about 1 / bins).
constexpr double kSkipShare = 0.2;

class Booster;

struct DMatrix {
  int64_t n_rows = 0;
  int32_t n_features = 0;
  DeviceBuffer<float> values;  // row-major copy
  DeviceBuffer<float> labels;
  bool has_labels = false;
  std::map<int32_t, std::unique_ptr<Quantized>> quantized;  // by requested max_bin
  Quantized& quantize(int32_t max_bin, dp_workspace_s& ws, hipStream_t s);
  // Boosters with a round in flight on this matrix.  Freeing the matrix
  // collects those rounds first (release_pending) and waits for the device.
  std::vector<const Booster*> pending;
  void release_pending();
};

// One regression tree in XGBoost's RegTree JSON field order plus parity data.
struct Tree {
  std::vector<int32_t> left, right, parent, feature, split_bin;
  std::vector<float> cond, base_weight, loss_chg, sum_hess;
  std::vector<uint8_t> default_left;
  std::vector<int64_t> sum_qg, sum_qh;
  std::vector<int64_t> rows;  // training rows reaching the node; -1 when unknown (loaded)
  int32_t size() const { return int32_t(left.size()); }
  int32_t alloc(int32_t parent_id);
};

struct TrainParam {
  float eta = 0.3f, lambda = 1.0f, alpha = 0.0f, gamma = 0.0f, min_child_weight = 1.0f;
  int32_t max_depth = 6, max_bin = 256;
  // Sampling (sample.hpp): fractions in (0, 1], 1 = off; seed of the draws.
  float subsample = 1.0f, colsample_bytree = 1.0f, colsample_bylevel = 1.0f,
        colsample_bynode = 1.0f;
  int32_t pad = 0;  // no padding bytes: the struct's words key the cached round graphs
  uint64_t seed = 0;
  bool colsample() const {
    return colsample_bytree < 1.0f || colsample_bylevel < 1.0f || colsample_bynode < 1.0f;
  }
};

// Depth-wise tree growth on one quantised matrix (reusable device buffers).
//
// A tree is grown without a host round trip per level: every level's launches
// take their item counts from device counters that a one-workgroup planner
// kernel writes after the level's partition.  The host enqueues all levels,
// then the tree's node records (and counters) are copied into a pinned slot;
// collect() turns them into a Tree once the caller has synchronised the
// stream.  Trees wider than the eager bound fall back to reading the level
// size back before each level to size the buffers.
class Grower {
 public:
  Grower();
  ~Grower();
  // Sizes the buffers for trees over `q` with parameters `p`, with `n_slots`
  // trees in flight before the caller synchronises.
  // sparse: build histograms from q.sparse (which must be built) instead of
  // the 16-feature tiles and the row-major copy (which must then be built).
  // root_cfg / level_cfg: launch shapes of the root (contiguous) and gathered
  // histogram passes (present-value histograms use their items only).
  // skip: histograms leave each feature's skip bin out (q.skip_tiles and
  // q.skip_features, which must be built) and the evaluation restores it.
  // pairs: the paired tiles of the dense histograms (a subset of q.pairs; 0
  // with sparse or skip).
  void prepare(const Quantized& q, const TrainParam& p, int32_t n_slots, bool sparse,
               const HistConfig& root_cfg, const HistConfig& level_cfg, bool skip,
               uint64_t pairs, hipStream_t s);
  // Column sampling of the trees grow() enqueues next (inactive: every
  // feature is a candidate at every node); cs.output is set per tree.
  ColSample colsample;
  // Enqueues one tree.  gpair: [n_rows][2] fixed-point gradients of one output;
  // exps (device): its two quantiser exponents; root_slots (device): the
  // quantiser's root_blocks per-workgroup (g, h) sums of gpair, added up by the
  // tree's first launch.  Stores each row's leaf value into values[row] (every
  // row once; the caller adds the plane to the margins) and, when `positions`
  // is set, writes each row's leaf id.
  void grow(const Quantized& q, const int32_t* gpair, const int32_t* exps,
            const int64_t* root_slots, int32_t root_blocks, const TrainParam& p, float* values,
            int32_t* positions, int32_t slot, hipStream_t s);
  // Copies the node records of slots [0, n_slots) to host buffer `buffer`
  // (0 or 1; one copy; eager trees only, level-synced trees were copied by
  // grow).
  void readback(int32_t n_slots, int32_t buffer, hipStream_t s);
  // The tree grown into `slot`; readback() into `buffer` has completed.
  void collect(const Quantized& q, int32_t slot, int32_t buffer, Tree& tree) const;
  // The quantiser exponents (g, h) of the tree in `slot`, as collect() finds it.
  void exponents(int32_t slot, int32_t buffer, int32_t* out) const;
  // False when trees are grown level-synced (grow() then synchronises).
  bool eager() const { return eager_; }
  // Changes whenever a buffer that grow() passes to a kernel moves or resizes.
  uint64_t signature() const;

 private:
  void ensure_level(const Quantized& q, int64_t nodes, int32_t depth, int32_t max_depth);
  PooledBuffer<uint32_t> ridx_[2];
  PooledBuffer<int64_t> hist_[2];
  PooledBuffer<LevelNode> level_[2];
  PooledBuffer<int64_t> sums_[2], seg_begin_[2];
  PooledBuffer<HistWork> hist_work_[2], root_work_;
  PooledBuffer<HistReduce> reduce_jobs_[2], root_job_;
  PooledBuffer<int64_t> partial_;
  PooledBuffer<PartWork> part_work_[2];
  PooledBuffer<int32_t> part_first_[2];
  PooledBuffer<int64_t> pair_chunk_, work_left_, node_left_[2];
  PooledBuffer<unsigned long long> part_masks_;  // count ballots, kPartMasks per item
  PooledBuffer<dp_split_record> splits_;
  PooledBuffer<uint8_t> eval_scratch_;
  PooledBuffer<uint32_t> fmask_;  // column sampling: [level node][ceil(F / 32)] bits
  PooledBuffer<LeafWork> leaf_work_[2];  // by level parity: applied one level later
  PooledBuffer<NodeInfo> info_;
  PooledBuffer<PlanCounts> counts_;
  PooledBuffer<uint8_t> slots_;  // eager: per slot, PlanCounts then NodeInfo[node_cap_]
  PooledPinnedBuffer readback_;        // host copies of slots_: two buffers of readback_slots_ slots
  int32_t readback_slots_ = 0;
  PooledPinnedBuffer level_count_;
  std::vector<std::vector<NodeInfo>> spill_;  // slots of trees grown level-synced
  std::vector<PlanCounts> spill_counts_;
  bool eager_ = true;
  bool sparse_ = false;  // histograms from the present-value layout
  bool colsample_ = false;  // column sampling buffers sized (prepare)
  int32_t tiles_ = 0;    // histogram tiles per row chunk (16-feature or sparse tiles)
  int64_t node_cap_ = 0;
  int64_t chunk_ = kPartChunk;  // rows per partition / margin-update item
  int32_t cus_ = 0;             // compute units of the device (histogram slots per round)
  size_t slot_bytes_ = 0;
  int64_t root_rows_ = -1;
  int32_t root_tiles_ = 0, root_items_ = 0;
  bool root_sparse_ = false;
  HistConfig root_cfg_, level_cfg_, root_made_;
  uint64_t root_pairs_ = 0;                 // the paired tiles root_work_ was made for
  dp_bin_layout lay_{};                     // the matrix's layout with the pairs in use
  const uint8_t* rows_major_ = nullptr;     // the row-major copy the gathered passes read
  const uint8_t* skip_tiles_ = nullptr;     // the matrix's skip bins when in use
  const uint8_t* skip_features_ = nullptr;
};

// Normalised hyperparameter JSON (see DPValidateHyperparameters).
std::string validate_hyperparameters(const std::string& text, uint32_t classes);

struct PredictRequest {
  const float* values = nullptr;  // device, row-major
  int64_t rows = 0, row_stride = 0;
  int32_t features = 0;
  float missing = 0.0f;  // NaN: only NaN is missing
  int32_t type = 0;      // 0 = transformed value, 1 = margin
  int32_t iteration_begin = 0, iteration_end = 0;  // rounds; end 0 = all
  bool strict_shape = true;
};

class Booster {
 public:
  explicit Booster(std::vector<DMatrix*> cache);
  ~Booster();
  Booster(const Booster&) = delete;
  Booster& operator=(const Booster&) = delete;
  void set_param(const std::string& key, const std::string& value);
  void update_one_iter(int iter, DMatrix* d);
  void train_one_iter(DMatrix* d, int iter, const float* grad, const float* hess, int64_t n,
                      int32_t k);
  int boosted_rounds() const {
    flush();
    return rounds_;
  }
  // num_feature of the trained or loaded model, else of the first training
  // matrix (XGBoosterGetNumFeature); 0 with neither.
  int64_t num_features() const {
    if (configured_ || model_only_) return n_features_;
    return cache_.empty() || !cache_[0] ? 0 : cache_[0]->n_features;
  }
  std::string save_config() const;
  std::string save_model() const;
  const std::vector<Tree>& trees() const {
    flush();
    return trees_;
  }
  // Collects the trees of a round still in flight (rounds are pipelined: a
  // round's trees come back while the next round runs on the GPU).
  void flush() const;
  void margins(float* out, size_t n) const;
  void last_gradients(float* grad, float* hess, size_t n, int32_t* exps) const;
  void last_positions(int32_t* out, size_t n) const;
  // JSON of the histogram launch shapes of the last round (the autotuner's
  // timings and choice, or the forced / default shapes).
  const std::string& tuning() const { return tuning_report_; }
  // Model from an XGBoost-schema JSON document (prediction / export only).
  void load_model(const std::string& text);
  // Rounds [begin, end) with the given step, as a new prediction-only booster.
  std::unique_ptr<Booster> slice(int begin, int end, int step) const;
  // Device output (library-owned, valid until the next predict) and its shape.
  const float* predict(const PredictRequest& req, std::vector<uint64_t>& shape);

 private:
  std::string effective_objective() const;
  void upload_forest(int32_t tree_begin, int32_t tree_end);
  void configure(DMatrix* d);
  // One boosting round: quantise + sizes the buffers (host), then enqueues
  // the round's device work (gradients when `with_gradients`, the quantiser
  // and the K trees) through a cached HIP graph, then collects the trees.
  void run_round(DMatrix* d, bool with_gradients);
  // Enqueues body() on stream_: replays the graph cached for `key`, or
  // captures body() into a new graph and launches it (direct launches when
  // graphs are off or the trees are grown level-synced).
  void enqueue(const std::vector<uint64_t>& key, bool capturable, const std::function<void()>& body);
  void clear_graphs();
  std::map<std::string, std::string> params_;
  std::vector<DMatrix*> cache_;
  // configured state
  bool configured_ = false;
  std::string objective_ = "reg:squarederror";
  int32_t objective_id_ = DP_OBJ_SQUARED;
  int32_t n_groups_ = 1;  // outputs (trees per round)
  int32_t num_class_ = 0;
  int32_t n_features_ = 0;
  std::vector<float> base_score_;  // as stored in the model (probability for logistic)
  TrainParam tp_;
  int32_t effective_max_bin_ = 0;  // the quantiser's max_bin of the last round (0: none yet)
  DMatrix* train_ = nullptr;
  // training state
  PooledBuffer<float> margin_, grad_, hess_;
  // The last round's leaf values are not in margin_ yet: the next round's
  // gradient kernel (or margins()) adds them.
  mutable bool values_pending_ = false;
  // The round's leaf-value planes, [n_groups][n_rows]: tree k stores each
  // row's leaf value in plane k; they are added to margin_ by the next round's
  // gradient kernel, or at the end of a round of caller-supplied gradients.
  PooledBuffer<float> leaf_values_;
  PooledBuffer<int32_t> gpair_, exps_;
  PooledBuffer<uint8_t> quant_scratch_;  // quantiser reduction slots
  PooledBuffer<int32_t> positions_;
  PooledBuffer<int32_t> round_dev_;  // the round's index, read by the sampling kernels
  // The caller's (grad, hess) buffers of an XGBoosterTrainOneIter round: its
  // quantiser reads them in place, launched outside the round's graph, and
  // caller_read_ (recorded after it) is waited on before the call returns.
  const float* caller_grad_ = nullptr;
  const float* caller_hess_ = nullptr;
  hipEvent_t caller_read_ = nullptr;
  bool caller_gradients_ = false;  // the last round's gradients came from the caller
  mutable std::vector<int32_t> last_exps_;
  bool record_positions_ = false;
  bool use_graphs_ = true;
  bool autotune_ = true;        // dp_autotune: time the histogram launch shapes (tune.cpp)
  HistConfig forced_hist_{0, 0, 0, 0, 0};  // dp_hist_tiles / _unroll / _items / _split / _deep; 0 = not forced
  bool pair_tiles_ = true;      // dp_hist_pair: pair the tiles whose features have <= 16 bins
  std::string tuning_report_ = "{}";
  int32_t sparse_mode_ = 1;  // dp_sparse_hist: 0 never, 1 when <= 1/4 present, 2 with any NaN
  // dp_skip_bin (matrices without missing values): 0 never, 1 when the skip
  // bins remove at least kSkipShare of the element atomics, 2 always.
  int32_t skip_mode_ = 1;
  bool labels_checked_ = false;
  std::vector<std::pair<std::vector<uint64_t>, hipGraphExec_t>> graphs_;  // newest last
  hipStream_t stream_ = nullptr;
  // Trees of a round run concurrently: tree k on growers_[k % S] and, when S
  // > 1, on tree_streams_[k % S] (forked from and joined back to stream_ by
  // events).  S = min(outputs, dp_concurrent_trees).
  std::vector<std::unique_ptr<Grower>> growers_;
  std::vector<hipStream_t> tree_streams_;
  std::vector<hipEvent_t> tree_done_;
  hipEvent_t fork_ = nullptr;
  int32_t concurrent_trees_ = 4;
  int32_t pending_lanes_ = 1;  // S of the round in flight
  mutable std::vector<Tree> trees_;
  mutable std::vector<int32_t> tree_info_;
  mutable std::vector<int32_t> iteration_indptr_{0};
  // The round in flight: its readback buffer, matrix and completion event.
  mutable bool pending_ = false;
  int32_t pending_buffer_ = 0;
  const Quantized* pending_q_ = nullptr;
  DMatrix* pending_d_ = nullptr;
  hipEvent_t round_done_[2] = {nullptr, nullptr};
  std::vector<uint64_t> last_round_inputs_;  // host inputs of the last round enqueued
  mutable int rounds_ = 0;
  bool model_only_ = false;  // loaded or sliced: predicts, cannot train
  // device forest for prediction
  DeviceBuffer<uint8_t> forest_nodes_;
  DeviceBuffer<int32_t> forest_roots_, forest_group_ptr_;
  DeviceBuffer<float> forest_base_, pred_out_;
  int32_t forest_begin_ = -1, forest_end_ = -1;
  size_t forest_trees_ = 0;
};

}  // namespace dp
