// Forest prediction on the device (the XGBoosterPredictFromCudaArray path the
// reference's study code uses for VALID scoring and probability views,
// native/class_study_train.cu:151-163, native/class_model_native_adapter.cuh:30).
//
// Trees are flattened into one node array; a node holds its left child's
// absolute index (right = left + 1, the order XGBoost's readers require,
// native/class_native_source_contract.hpp:24-31), the split feature, the
// threshold (or the leaf value) and the default direction.  One thread per row
// walks, for each output group, that group's trees in boosting order and sums
// the leaves in float, so on the training rows the margins equal the ones the
// trainer accumulated, bit for bit.
#include "dp_internal.hpp"
#include "predict.hpp"

#include <cmath>

namespace dp {
namespace {

__device__ __forceinline__ float pred_expf(float x) {
  // Same exp as the gradient kernels (Cody & Waite reduction, degree-7 Taylor).
  if (x != x) return x;
  if (x > 88.72283f) return INFINITY;
  if (x < -87.0f) return 0.0f;
  const float k = rintf(x * 1.44269504088896341f);
  float r = fmaf(-k, 0.693145751953125f, x);
  r = fmaf(-k, 1.42860682030941723212e-6f, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, int(k));
}

__global__ void predict_kernel(const float* __restrict__ values, int64_t n_rows,
                               int32_t n_features, int64_t row_stride, float missing,
                               const PredNode* __restrict__ nodes,
                               const int32_t* __restrict__ group_roots,
                               const int32_t* __restrict__ group_ptr, int32_t n_groups,
                               const float* __restrict__ base, int32_t transform,
                               float* __restrict__ out) {
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n_rows;
       r += int64_t(blockDim.x) * gridDim.x) {
    const float* x = values + r * row_stride;
    float best = -INFINITY;
    int best_k = 0;
    float mx = -INFINITY;
    for (int g = 0; g < n_groups; ++g) {
      float m = base[g];
      for (int t = group_ptr[g]; t < group_ptr[g + 1]; ++t) {
        int node = group_roots[t];
        PredNode nd = nodes[node];
        while (nd.left >= 0) {
          float v = x[nd.feature];
          if (v == missing) v = __builtin_nanf("");
          const bool left = (v != v) ? (nd.flags & 1) : (v < nd.cond);
          node = left ? nd.left : nd.left + 1;
          nd = nodes[node];
        }
        m += nd.cond;
      }
      if (transform == kPredArgmax) {
        if (m > best) { best = m; best_k = g; }
      } else if (transform == kPredSigmoid) {
        out[r * n_groups + g] = 1.0f / (1.0f + pred_expf(-m));
      } else {
        out[r * n_groups + g] = m;
      }
      mx = fmaxf(mx, m);
    }
    if (transform == kPredArgmax) {
      out[r] = float(best_k);
    } else if (transform == kPredSoftmax) {
      float s = 0.0f;
      for (int g = 0; g < n_groups; ++g) s += pred_expf(out[r * n_groups + g] - mx);
      for (int g = 0; g < n_groups; ++g)
        out[r * n_groups + g] = pred_expf(out[r * n_groups + g] - mx) / s;
    }
  }
}

}  // namespace

void launch_predict(const float* values, int64_t n_rows, int32_t n_features, int64_t row_stride,
                    float missing, const PredNode* nodes, const int32_t* group_roots,
                    const int32_t* group_ptr, int32_t n_groups, const float* base,
                    int32_t transform, float* out, hipStream_t s) {
  if (n_rows <= 0) return;
  hipLaunchKernelGGL(predict_kernel, dim3(grid_for(n_rows, 256, 16384)), dim3(256), 0, s, values,
                     n_rows, n_features, row_stride, missing, nodes, group_roots, group_ptr,
                     n_groups, base, transform, out);
  DP_HIP(hipGetLastError());
}

}  // namespace dp
