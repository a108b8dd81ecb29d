// Flattened forest for device prediction.
#pragma once

#include <cstdint>

#include <hip/hip_runtime.h>

namespace dp {

struct PredNode {
  int32_t left;     // absolute index of the left child, -1 for a leaf
  int32_t feature;  // split feature
  float cond;       // threshold (x < cond goes left), or the leaf value
  int32_t flags;    // bit 0: missing goes left
};

enum PredTransform : int32_t {
  kPredIdentity = 0,  // margins (type 1) or regression values
  kPredSigmoid = 1,   // binary:logistic probabilities
  kPredSoftmax = 2,   // multi:softprob probabilities
  kPredArgmax = 3,    // multi:softmax class ids
};

void launch_predict(const float* values, int64_t n_rows, int32_t n_features, int64_t row_stride,
                    float missing, const PredNode* nodes, const int32_t* group_roots,
                    const int32_t* group_ptr, int32_t n_groups, const float* base,
                    int32_t transform, float* out, hipStream_t s);

}  // namespace dp
