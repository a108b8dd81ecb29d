// Training objects: quantised matrix cache, level-wise tree grower, booster.
//
// The booster reproduces what the reference obtains from XGBoost 3.4.1 through
// XGBoosterUpdateOneIter with tree_method=hist on the GPU
// (native/class_native_training.cuh:54-67): one depth-wise tree per output per
// round, grown level by level.  Per level the device runs
//   histogram build of the smaller child of every pair (gather by row ids)
//   -> sibling = parent - built -> split evaluation -> stable partition
// and the host reads back one small record per node (split and left count)
// to number the children and compute leaf weights.
#include "booster.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>

#include "json.hpp"

namespace dp {

void launch_any_nan(const float* values, int64_t n, int32_t* flag, hipStream_t s);
void launch_leaf_positions(const uint32_t* ridx, const LeafWork* work, int32_t n_work,
                           int32_t* positions, hipStream_t s);

namespace {

double threshold_l1(double g, double alpha) {
  if (g > alpha) return g - alpha;
  if (g < -alpha) return g + alpha;
  return 0.0;
}

// Leaf weight -T(G)/(H + lambda); 0 when H < min_child_weight or H <= 0.
double calc_weight(const TrainParam& p, double g, double h) {
  if (h < double(p.min_child_weight) || h <= 0.0) return 0.0;
  return -threshold_l1(g, double(p.alpha)) / (h + double(p.lambda));
}

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
  // uint8 storage: with NaN present byte 255 marks missing, leaving 255 bins.
  const int32_t eff = std::min(max_bin, has_nan ? 255 : 256);
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
  need(dp_layout_init(n_rows, n_features, 0, has_nan ? 255 : -1, &q->layout) == 0,
       "bin layout");
  q->d_cut_ptr.resize(q->cut_ptr.size());
  q->d_cut_values.resize(std::max<size_t>(q->cut_values.size(), 1));
  q->d_nbins.resize(nbins.size());
  DP_HIP(hipMemcpyAsync(q->d_cut_ptr.p, q->cut_ptr.data(), q->d_cut_ptr.bytes(),
                        hipMemcpyHostToDevice, s));
  DP_HIP(hipMemcpyAsync(q->d_cut_values.p, q->cut_values.data(),
                        sizeof(float) * q->cut_values.size(), hipMemcpyHostToDevice, s));
  DP_HIP(hipMemcpyAsync(q->d_nbins.p, nbins.data(), q->d_nbins.bytes(), hipMemcpyHostToDevice, s));
  q->bins.resize(dp_layout_bytes(&q->layout));
  launch_bin_values(values.p, q->layout, q->d_cut_ptr.p, q->d_cut_values.p, q->bins.p, s);
  DP_HIP(hipStreamSynchronize(s));
  auto& ref = *q;
  quantized.emplace(max_bin, std::move(q));
  return ref;
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
  return id;
}

// ---------------------------------------------------------------------------
// Grower
// ---------------------------------------------------------------------------
Grower::Grower() = default;
Grower::~Grower() = default;

void Grower::grow(const Quantized& q, const int32_t* gpair, int32_t exp_g, int32_t exp_h,
                  int64_t root_g, int64_t root_h, const TrainParam& p, float* margin,
                  int64_t stride, Tree& tree, int32_t* positions, hipStream_t s) {
  const dp_bin_layout& L = q.layout;
  const int64_t N = L.n_rows;
  const int32_t F = L.n_features, B = q.bin_stride;
  const int64_t S = int64_t(F) * B * 2;  // int64 values per node histogram
  const double ug = std::ldexp(1.0, -exp_g), uh = std::ldexp(1.0, -exp_h);
  need(p.max_depth >= 0 && p.max_depth <= 30, "max_depth out of supported range");
  dp_train_param dtp{p.eta, p.lambda, p.alpha, p.gamma, p.min_child_weight, p.max_depth};

  ridx_[0].reserve(size_t(N));
  ridx_[1].reserve(size_t(N));
  launch_iota_u32(ridx_[0].p, N, s);
  tree = Tree{};
  tree.alloc(-1);

  struct LNode {
    int32_t nid;
    int32_t parent_slot;
    int64_t begin, end, g, h;
  };
  struct Leaf {
    float value;
    int32_t parity;
    int64_t begin, end;
    int32_t nid;
  };
  std::vector<LNode> level{{0, -1, 0, N, root_g, root_h}};
  std::vector<Leaf> leaves;

  for (int32_t depth = 0; !level.empty(); ++depth) {
    const int32_t n = int32_t(level.size());
    const bool can_split = depth < p.max_depth;
    const dp_split_record* rec = nullptr;
    const int64_t* lefts = nullptr;
    if (can_split) {
      const int cur = depth & 1;
      hist_[cur].reserve(size_t(n) * size_t(S));
      sums_.reserve(size_t(2 * n));
      splits_.reserve(size_t(n));
      node_left_.reserve(size_t(n));

      // Nodes whose histogram is built: the root, else the smaller child of
      // every pair (ties: the left child).
      std::vector<int32_t> build;
      std::vector<SubtractJob> jobs;
      if (depth == 0) {
        build.push_back(0);
      } else {
        for (int32_t j = 0; j + 1 < n; j += 2) {
          const LNode& a = level[size_t(j)];
          const LNode& b = level[size_t(j) + 1];
          const bool right_small = (b.end - b.begin) < (a.end - a.begin);
          const int32_t small = right_small ? j + 1 : j, large = right_small ? j : j + 1;
          build.push_back(small);
          jobs.push_back({int64_t(a.parent_slot) * S, int64_t(small) * S, int64_t(large) * S});
        }
      }
      std::vector<int64_t> bb, be;
      for (int32_t k : build) {
        bb.push_back(level[size_t(k)].begin);
        be.push_back(level[size_t(k)].end);
      }
      const std::vector<HistWork> hw =
          make_hist_work(L, bb.data(), be.data(), build.data(), int32_t(build.size()));

      std::vector<PartWork> pw;
      std::vector<int32_t> first(static_cast<size_t>(n) + 1);
      for (int32_t i = 0; i < n; ++i) {
        first[size_t(i)] = int32_t(pw.size());
        for (int64_t b = level[size_t(i)].begin; b < level[size_t(i)].end; b += kPartChunk)
          pw.push_back({i, 0, b, std::min(b + kPartChunk, level[size_t(i)].end)});
      }
      first[size_t(n)] = int32_t(pw.size());

      ws_.begin(sizeof(HistWork) * hw.size() + sizeof(SubtractJob) * jobs.size() +
                sizeof(int64_t) * size_t(3 * n) + sizeof(PartWork) * pw.size() +
                sizeof(int32_t) * first.size() + 6 * 256);
      ws_.reserve_scratch(2 * sizeof(int64_t) * pw.size() + 1024);
      HistWork* d_hw;
      SubtractJob* d_jobs;
      int64_t* d_sums;
      PartWork* d_pw;
      int64_t* d_segb;
      int32_t* d_first;
      std::copy(hw.begin(), hw.end(), ws_.stage(hw.size(), &d_hw));
      std::copy(jobs.begin(), jobs.end(), ws_.stage(jobs.size(), &d_jobs));
      int64_t* h_sums = ws_.stage(size_t(2 * n), &d_sums);
      int64_t* h_segb = ws_.stage(size_t(n), &d_segb);
      for (int32_t i = 0; i < n; ++i) {
        h_sums[2 * i] = level[size_t(i)].g;
        h_sums[2 * i + 1] = level[size_t(i)].h;
        h_segb[i] = level[size_t(i)].begin;
      }
      std::copy(pw.begin(), pw.end(), ws_.stage(pw.size(), &d_pw));
      std::copy(first.begin(), first.end(), ws_.stage(first.size(), &d_first));
      ws_.commit(s);
      int64_t* work_left = ws_.take<int64_t>(pw.size());
      int64_t* work_offset = ws_.take<int64_t>(pw.size());

      launch_fill_i64(hist_[cur].p, int64_t(n) * S, 0, s);
      launch_hist(q.bins.p, L, gpair, depth == 0 ? nullptr : ridx_[cur].p, d_hw,
                  int32_t(hw.size()), B, hist_[cur].p, s);
      if (!jobs.empty())
        launch_subtract_many(hist_[cur ^ 1].p, hist_[cur].p, hist_[cur].p, d_jobs,
                             int32_t(jobs.size()), S, s);
      launch_evaluate(hist_[cur].p, n, F, B, q.d_nbins.p, d_sums, nullptr, exp_g, exp_h, dtp,
                      splits_.p, s);
      launch_partition(q.bins.p, L, ridx_[cur].p, ridx_[cur ^ 1].p, d_pw, int32_t(pw.size()),
                       d_segb, splits_.p, d_first, n, work_left, work_offset, node_left_.p, s);
      readback_.reserve(size_t(n) * (sizeof(dp_split_record) + sizeof(int64_t)));
      auto* h_rec = reinterpret_cast<dp_split_record*>(readback_.p);
      auto* h_left = reinterpret_cast<int64_t*>(readback_.p + size_t(n) * sizeof(dp_split_record));
      DP_HIP(hipMemcpyAsync(h_rec, splits_.p, sizeof(dp_split_record) * size_t(n),
                            hipMemcpyDeviceToHost, s));
      DP_HIP(hipMemcpyAsync(h_left, node_left_.p, sizeof(int64_t) * size_t(n),
                            hipMemcpyDeviceToHost, s));
      DP_HIP(hipStreamSynchronize(s));
      rec = h_rec;
      lefts = h_left;
    }

    std::vector<LNode> next;
    for (int32_t i = 0; i < n; ++i) {
      const LNode nd = level[size_t(i)];
      const double G = double(nd.g) * ug, H = double(nd.h) * uh;
      const double w = calc_weight(p, G, H);
      tree.base_weight[size_t(nd.nid)] = float(w);
      tree.sum_hess[size_t(nd.nid)] = float(H);
      tree.sum_qg[size_t(nd.nid)] = nd.g;
      tree.sum_qh[size_t(nd.nid)] = nd.h;
      if (can_split && rec[i].expand) {
        const dp_split_record& r = rec[i];
        const int64_t nl = lefts[i];
        need(nl > 0 && nl < nd.end - nd.begin, "partition produced an empty child");
        const int32_t l = tree.alloc(nd.nid), rr = tree.alloc(nd.nid);
        const size_t id = size_t(nd.nid);
        tree.left[id] = l;
        tree.right[id] = rr;
        tree.feature[id] = r.feature;
        tree.split_bin[id] = r.bin;
        tree.default_left[id] = uint8_t(r.default_left);
        tree.cond[id] = q.cut_values[size_t(q.cut_ptr[size_t(r.feature)] + r.bin)];
        tree.loss_chg[id] = float(r.loss_chg);
        next.push_back({l, i, nd.begin, nd.begin + nl, r.gl, r.hl});
        next.push_back({rr, i, nd.begin + nl, nd.end, nd.g - r.gl, nd.h - r.hl});
      } else {
        const float v = float(w * double(p.eta));
        tree.cond[size_t(nd.nid)] = v;
        leaves.push_back({v, depth & 1, nd.begin, nd.end, nd.nid});
      }
    }
    level.swap(next);
  }

  // Leaf values into the margins (and leaf ids into positions).
  constexpr int64_t kLeafChunk = 16384;
  std::vector<LeafWork> lw[2];
  for (const Leaf& lf : leaves)
    for (int64_t b = lf.begin; b < lf.end; b += kLeafChunk)
      lw[lf.parity].push_back({lf.value, lf.nid, b, std::min(b + kLeafChunk, lf.end)});
  ws_.begin(sizeof(LeafWork) * (lw[0].size() + lw[1].size()) + 2 * 256);
  LeafWork* d_lw[2];
  for (int par = 0; par < 2; ++par)
    std::copy(lw[par].begin(), lw[par].end(), ws_.stage(lw[par].size(), &d_lw[par]));
  ws_.commit(s);
  for (int par = 0; par < 2; ++par) {
    launch_update_margin(ridx_[par].p, d_lw[par], int32_t(lw[par].size()), margin, stride, s);
    if (positions)
      launch_leaf_positions(ridx_[par].p, d_lw[par], int32_t(lw[par].size()), positions, s);
  }
}

// ---------------------------------------------------------------------------
// Booster
// ---------------------------------------------------------------------------
Booster::Booster(std::vector<DMatrix*> cache) : cache_(std::move(cache)) {}

Booster::~Booster() {
  grower_.reset();
  if (stream_) {
    (void)hipStreamSynchronize(stream_);
    (void)hipStreamDestroy(stream_);
  }
}

void Booster::set_param(const std::string& key, const std::string& value) {
  static const char* known[] = {
      "objective", "num_class", "tree_method", "device", "booster", "max_bin", "max_depth",
      "eta", "learning_rate", "lambda", "reg_lambda", "alpha", "reg_alpha", "gamma",
      "min_split_loss", "min_child_weight", "subsample", "colsample_bytree", "colsample_bylevel",
      "colsample_bynode", "base_score", "boost_from_average", "seed", "seed_per_iteration",
      "nthread", "verbosity", "validate_parameters", "grow_policy", "dp_record_positions"};
  bool ok = false;
  for (const char* k : known) ok = ok || key == k;
  need(ok, "unsupported parameter: " + key);
  if (rounds_ > 0 && (key == "objective" || key == "num_class" || key == "max_bin"))
    need(params_[key] == value, "parameter " + key + " cannot change after training started");
  params_[key] = value;
  if (key == "dp_record_positions") record_positions_ = parse_int(key, value) != 0;
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
  for (const char* k : {"subsample", "colsample_bytree", "colsample_bylevel", "colsample_bynode"})
    need(parse_float(k, get(k, "1")) == 1.0f, std::string(k) + " other than 1 is not supported");
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
  grad_.resize(size_t(N) * n_groups_);
  hess_.resize(size_t(N) * n_groups_);
  gpair_.resize(size_t(N) * n_groups_ * 2);
  exps_.resize(size_t(2 * n_groups_));
  sums_.resize(size_t(2 * n_groups_));
  maxima_.resize(size_t(2 * n_groups_));
  std::vector<float> init(static_cast<size_t>(N) * n_groups_);
  for (int64_t r = 0; r < N; ++r)
    for (int32_t k = 0; k < n_groups_; ++k) {
      const float b = base_score_[size_t(k)];
      init[size_t(r * n_groups_ + k)] =
          objective_id_ == DP_OBJ_LOGISTIC ? float(std::log(double(b) / (1.0 - double(b)))) : b;
    }
  DP_HIP(hipMemcpy(margin_.p, init.data(), margin_.bytes(), hipMemcpyHostToDevice));
  grower_ = std::make_unique<Grower>();
  configured_ = true;
}

void Booster::update_one_iter(int iter, DMatrix* d) {
  need(d != nullptr, "null DMatrix");
  need(iter == rounds_, "iteration index must equal the number of boosted rounds");
  configure(d);
  need(d->has_labels, "training DMatrix has no labels");
  launch_gradients(objective_id_, margin_.p, d->labels.p, d->n_rows, n_groups_, grad_.p, hess_.p,
                   stream_);
  boost_from_gradients(d, grad_.p, hess_.p);
}

void Booster::train_one_iter(DMatrix* d, int iter, const float* grad, const float* hess,
                             int64_t n, int32_t k) {
  need(d != nullptr, "null DMatrix");
  need(iter == rounds_, "iteration index must equal the number of boosted rounds");
  configure(d);
  need(n == d->n_rows && k == n_groups_, "gradient shape differs from [rows, outputs]");
  // Keep a copy so the parity hook can report the gradients of this round.
  DP_HIP(hipMemcpyAsync(grad_.p, grad, grad_.bytes(), hipMemcpyDeviceToDevice, stream_));
  DP_HIP(hipMemcpyAsync(hess_.p, hess, hess_.bytes(), hipMemcpyDeviceToDevice, stream_));
  boost_from_gradients(d, grad_.p, hess_.p);
}

void Booster::boost_from_gradients(DMatrix* d, const float* grad, const float* hess) {
  dp_workspace_s scratch;
  Quantized& q = d->quantize(tp_.max_bin, scratch, stream_);
  const int64_t N = d->n_rows;
  launch_quantise(grad, hess, N, n_groups_, maxima_.p, exps_.p, gpair_.p, sums_.p, stream_);
  std::vector<int32_t> exps(static_cast<size_t>(2 * n_groups_));
  std::vector<int64_t> sums(static_cast<size_t>(2 * n_groups_));
  DP_HIP(hipMemcpyAsync(exps.data(), exps_.p, exps_.bytes(), hipMemcpyDeviceToHost, stream_));
  DP_HIP(hipMemcpyAsync(sums.data(), sums_.p, sums_.bytes(), hipMemcpyDeviceToHost, stream_));
  DP_HIP(hipStreamSynchronize(stream_));
  last_exps_ = exps;
  if (record_positions_) positions_.reserve(size_t(N));
  for (int32_t k = 0; k < n_groups_; ++k) {
    Tree tree;
    grower_->grow(q, gpair_.p + int64_t(k) * N * 2, exps[size_t(2 * k)], exps[size_t(2 * k + 1)],
                  sums[size_t(2 * k)], sums[size_t(2 * k + 1)], tp_, margin_.p + k, n_groups_,
                  tree, record_positions_ ? positions_.p : nullptr, stream_);
    trees_.push_back(std::move(tree));
    tree_info_.push_back(k);
  }
  iteration_indptr_.push_back(int32_t(trees_.size()));
  ++rounds_;
  DP_HIP(hipStreamSynchronize(stream_));
}

void Booster::margins(float* out, size_t n) const {
  need(configured_, "booster has not been trained");
  need(n == margin_.n, "margin buffer size differs");
  DP_HIP(hipMemcpy(out, margin_.p, margin_.bytes(), hipMemcpyDeviceToHost));
}

void Booster::last_gradients(float* grad, float* hess, size_t n, int32_t* exps) const {
  need(configured_, "booster has not been trained");
  need(n == grad_.n, "gradient buffer size differs");
  if (grad) DP_HIP(hipMemcpy(grad, grad_.p, grad_.bytes(), hipMemcpyDeviceToHost));
  if (hess) DP_HIP(hipMemcpy(hess, hess_.p, hess_.bytes(), hipMemcpyDeviceToHost));
  if (exps) std::copy(last_exps_.begin(), last_exps_.end(), exps);
}

void Booster::last_positions(int32_t* out, size_t n) const {
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
       "\",\"num_target\":\"1\"},\"objective\":" + objective_json(objective_, num_class_) +
       "},\"version\":[3,4,1]}";
  return o;
}

std::string Booster::save_config() const {
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
  o += std::to_string(tp_.max_bin) + "\"},\"name\":\"grow_gpu_hist\",\"train_param\":{";
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
  json::put_string(o, objective_);
  o += "},\"objective\":" + objective_json(objective_, num_class_) + "},\"version\":[3,4,1]}";
  return o;
}

}  // namespace dp
