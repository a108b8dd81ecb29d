// Host-side training objects behind the XGBoost-compatible C API.
#pragma once

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
};

struct DMatrix {
  int64_t n_rows = 0;
  int32_t n_features = 0;
  DeviceBuffer<float> values;  // row-major copy
  DeviceBuffer<float> labels;
  bool has_labels = false;
  std::map<int32_t, std::unique_ptr<Quantized>> quantized;  // by requested max_bin
  Quantized& quantize(int32_t max_bin, dp_workspace_s& ws, hipStream_t s);
};

// One regression tree in XGBoost's RegTree JSON field order plus parity data.
struct Tree {
  std::vector<int32_t> left, right, parent, feature, split_bin;
  std::vector<float> cond, base_weight, loss_chg, sum_hess;
  std::vector<uint8_t> default_left;
  std::vector<int64_t> sum_qg, sum_qh;
  int32_t size() const { return int32_t(left.size()); }
  int32_t alloc(int32_t parent_id);
};

struct TrainParam {
  float eta = 0.3f, lambda = 1.0f, alpha = 0.0f, gamma = 0.0f, min_child_weight = 1.0f;
  int32_t max_depth = 6, max_bin = 256;
};

// Level-wise tree growth on one quantised matrix (reusable device buffers).
class Grower {
 public:
  Grower();
  ~Grower();
  // gpair: [n_rows][2] fixed-point gradients of one output; (root_g, root_h)
  // their int64 sums; exps the quantiser exponents.  Adds the leaf values to
  // margin[r * stride] and, when `positions` is set, writes each row's leaf id.
  void grow(const Quantized& q, const int32_t* gpair, int32_t exp_g, int32_t exp_h,
            int64_t root_g, int64_t root_h, const TrainParam& p, float* margin, int64_t stride,
            Tree& tree, int32_t* positions, hipStream_t s);

 private:
  dp_workspace_s ws_;
  DeviceBuffer<uint32_t> ridx_[2];
  DeviceBuffer<int64_t> hist_[2];
  DeviceBuffer<int64_t> sums_;
  DeviceBuffer<dp_split_record> splits_;
  DeviceBuffer<int64_t> node_left_;
  PinnedBuffer readback_;
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
  int boosted_rounds() const { return rounds_; }
  std::string save_config() const;
  std::string save_model() const;
  const std::vector<Tree>& trees() const { return trees_; }
  void margins(float* out, size_t n) const;
  void last_gradients(float* grad, float* hess, size_t n, int32_t* exps) const;
  void last_positions(int32_t* out, size_t n) const;

 private:
  void configure(DMatrix* d);
  void boost_from_gradients(DMatrix* d, const float* grad, const float* hess);
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
  DMatrix* train_ = nullptr;
  // training state
  DeviceBuffer<float> margin_, grad_, hess_;
  DeviceBuffer<int32_t> gpair_, exps_;
  DeviceBuffer<int64_t> sums_;
  DeviceBuffer<uint32_t> maxima_;
  DeviceBuffer<int32_t> positions_;
  std::vector<int32_t> last_exps_;
  bool record_positions_ = false;
  hipStream_t stream_ = nullptr;
  std::unique_ptr<Grower> grower_;
  std::vector<Tree> trees_;
  std::vector<int32_t> tree_info_;
  std::vector<int32_t> iteration_indptr_{0};
  int rounds_ = 0;
};

}  // namespace dp
