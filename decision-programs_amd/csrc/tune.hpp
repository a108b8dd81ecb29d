// Histogram autotuner (tune.cpp): launch shapes of the histogram passes of one
// matrix shape, chosen by timing candidates on the matrix itself.
#pragma once

#include <string>

#include "dp_internal.hpp"

namespace dp {

struct HistTuning {
  HistConfig root;    // the contiguous root pass
  HistConfig level;   // the gathered passes of the levels below the root
  bool tuned = false;
  std::string report;  // JSON: every candidate's time and the choice
};

// Dense 16-feature tiles (bins: tile-major, with the joint tiles of the
// layout's pairs).  gathered: also tune the gathered passes, which read a
// row-major copy (made here for the timing: the plain copy, and the one with
// the pairs' joint tiles for one-tile candidates); otherwise level = root.
// gpair: any [n_rows][2] pairs (the timing does not depend on their values).
// Cached per process by (rows, features, bins, missing, gathered, skip,
// pairs); synchronises `s`.  skip: the matrix's skip bins per tile when the
// histograms leave them out.
const HistTuning& tune_dense_hist(const dp_bin_layout& layout, const uint8_t* bins,
                                  bool gathered, int32_t bin_stride, const int32_t* gpair,
                                  hipStream_t s, const uint8_t* skip = nullptr);
// The cached dense tuning of a shape, or null when it has not been tuned.
const HistTuning* find_dense_tuning(const dp_bin_layout& layout, int32_t bin_stride,
                                    bool gathered);
// Present-value layout: the work-item count of its passes.
const HistTuning& tune_sparse_hist(const SparseBins& sp, int64_t n_rows, int32_t n_features,
                                   int32_t bin_stride, const int32_t* gpair, hipStream_t s);

}  // namespace dp
