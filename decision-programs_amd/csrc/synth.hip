// Synthetic inputs for the five benchmark configurations.  Not part of the
// training path: these kernels only create benchmark and test data on the
// device, deterministically from (config, seed), so any run can rebuild the
// exact same matrix.
//
// Random numbers are counter based: u = mix(mix(seed ^ stream*phi) + i*c) with
// SplitMix64's finaliser `mix`; uniforms use the top 24 bits, normals use the
// Box-Muller transform.
//   C1  10k x 8: x ~ U(0,1); y ~ Bernoulli(sigmoid(w.x + 0.5 x0 x1)), w ~ N(0,1)
//   C2  1M x 28: f0-20 ~ N(0,1); f21-27 alternate x_a*x_b and |x_a - x_b| over
//       seeded pairs of f0-20; y ~ Bernoulli(sigmoid(8 seeded N(0,1)-weighted
//       features + 3 seeded pairwise products with N(0,1) weights))
//   C3  10M x 128: f0-63 N(0,1), f64-95 lognormal(0,1), f96-127 U{0..15};
//       grad ~ N(0,1), hess ~ U(0.01, 0.25)
//   C4  60k x 784 (28x28): label r mod 10; pixel nonzero with probability
//       0.05 + 0.6*exp(-d^2/50), d the distance to a seeded class centre;
//       nonzero values U{1..255}
//   C5  2M x 1000: NaN with probability 0.95 else N(0,1);
//       y = sum of 20 seeded features (NaN -> 0) + N(0, 0.1)
#include "dp_internal.hpp"

#include <cmath>

namespace dp {
namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t rnd(uint64_t seed, uint64_t stream, uint64_t i) {
  return mix64(mix64(seed ^ (stream * 0x9e3779b97f4a7c15ull)) + i * 0xd1b54a32d192ed03ull);
}

__device__ __forceinline__ float uniform(uint64_t seed, uint64_t stream, uint64_t i) {
  return float(rnd(seed, stream, i) >> 40) * 5.9604644775390625e-8f;  // [0, 1)
}

__device__ __forceinline__ float normal(uint64_t seed, uint64_t stream, uint64_t i) {
  const float u1 = 1.0f - uniform(seed, stream, 2 * i);  // (0, 1]
  const float u2 = uniform(seed, stream, 2 * i + 1);
  return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// Seeded pair (a, b), a != b, both in [0, 21).
__device__ __forceinline__ void c2_pair(uint64_t seed, uint64_t stream, int* a, int* b) {
  *a = int(rnd(seed, stream, 0) % 21);
  *b = int((uint64_t(*a) + 1 + rnd(seed, stream, 1) % 20) % 21);
}

__device__ float c2_base(uint64_t seed, int64_t r, int j) { return normal(seed, uint64_t(j), uint64_t(r)); }

__device__ float c2_value(uint64_t seed, int64_t r, int j) {
  if (j < 21) return c2_base(seed, r, j);
  int a, b;
  c2_pair(seed, 3000 + uint64_t(j), &a, &b);
  const float xa = c2_base(seed, r, a), xb = c2_base(seed, r, b);
  return (j & 1) ? fabsf(xa - xb) : xa * xb;
}

__device__ float value_of(int config, uint64_t seed, int64_t r, int j) {
  switch (config) {
    case 1:
      return uniform(seed, uint64_t(j), uint64_t(r));
    case 2:
      return c2_value(seed, r, j);
    case 3:
      if (j < 64) return normal(seed, uint64_t(j), uint64_t(r));
      if (j < 96) return expf(normal(seed, uint64_t(j), uint64_t(r)));
      return floorf(uniform(seed, uint64_t(j), uint64_t(r)) * 16.0f);
    case 4: {
      const int c = int(r % 10);
      const int py = j / 28, px = j % 28;
      const float cy = float(6 + rnd(seed, 7000 + uint64_t(c), 0) % 16);
      const float cx = float(6 + rnd(seed, 7000 + uint64_t(c), 1) % 16);
      const float d2 = (float(py) - cy) * (float(py) - cy) + (float(px) - cx) * (float(px) - cx);
      const float q = fminf(1.0f, 0.05f + 0.6f * expf(-d2 / 50.0f));
      if (uniform(seed, uint64_t(j), uint64_t(r)) >= q) return 0.0f;
      return float(1 + rnd(seed, 10000 + uint64_t(j), uint64_t(r)) % 255);
    }
    case 5:
      if (uniform(seed, 20000 + uint64_t(j), uint64_t(r)) < 0.95f) return NAN;
      return normal(seed, uint64_t(j), uint64_t(r));
    default:
      return 0.0f;
  }
}

__global__ void synth_values_kernel(int config, uint64_t seed, int64_t n_rows, int n_features,
                                    float* __restrict__ values) {
  const int64_t total = n_rows * n_features;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(blockDim.x) * gridDim.x) {
    const int64_t r = i / n_features;
    const int j = int(i - r * n_features);
    values[i] = value_of(config, seed, r, j);
  }
}

__global__ void synth_rows_kernel(int config, uint64_t seed, int64_t n_rows, int n_features,
                                  float* __restrict__ labels, float* __restrict__ grad,
                                  float* __restrict__ hess) {
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n_rows;
       r += int64_t(blockDim.x) * gridDim.x) {
    float y = 0.0f;
    if (config == 1) {
      float logit = 0.5f * value_of(1, seed, r, 0) * value_of(1, seed, r, 1);
      for (int j = 0; j < n_features && j < 8; ++j)
        logit += normal(seed, 1000 + uint64_t(j), 0) * value_of(1, seed, r, j);
      y = uniform(seed, 2000, uint64_t(r)) < sigmoid(logit) ? 1.0f : 0.0f;
    } else if (config == 2) {
      float logit = 0.0f;
      for (int i = 0; i < 8; ++i) {
        const int j = int(rnd(seed, 4000 + uint64_t(i), 0) % uint64_t(n_features));
        logit += normal(seed, 4000 + uint64_t(i), 1) * value_of(2, seed, r, j);
      }
      for (int p = 0; p < 3; ++p) {
        int a, b;
        c2_pair(seed, 5000 + uint64_t(p), &a, &b);
        logit += normal(seed, 5000 + uint64_t(p), 2) * c2_base(seed, r, a) * c2_base(seed, r, b);
      }
      y = uniform(seed, 2000, uint64_t(r)) < sigmoid(logit) ? 1.0f : 0.0f;
    } else if (config == 4) {
      y = float(r % 10);
    } else if (config == 5) {
      for (int i = 0; i < 20; ++i) {
        const int j = int(rnd(seed, 8000 + uint64_t(i), 0) % uint64_t(n_features));
        const float x = value_of(5, seed, r, j);
        if (x == x) y += x;
      }
      y += 0.1f * normal(seed, 9000, uint64_t(r));
    }
    if (labels) labels[r] = y;
    if (grad) grad[r] = normal(seed, 6000, uint64_t(r));
    if (hess) hess[r] = 0.01f + 0.24f * uniform(seed, 6001, uint64_t(r));
  }
}

}  // namespace

void launch_synth(int32_t config, uint64_t seed, int64_t n_rows, int32_t n_features,
                  float* values, float* labels, float* grad, float* hess, hipStream_t s) {
  need(config >= 1 && config <= 5, "synthetic config must be 1..5");
  need(n_rows > 0 && n_features > 0, "synthetic shape must be positive");
  if (config == 2) need(n_features == 28, "config 2 has 28 features");
  if (config == 3) need(n_features == 128, "config 3 has 128 features");
  if (config == 4) need(n_features == 784, "config 4 has 784 features");
  if (values)
    hipLaunchKernelGGL(synth_values_kernel, dim3(grid_for(n_rows * n_features, 256, 65536)),
                       dim3(256), 0, s, config, seed, n_rows, n_features, values);
  DP_HIP(hipGetLastError());
  if (labels || grad || hess)
    hipLaunchKernelGGL(synth_rows_kernel, dim3(grid_for(n_rows, 256, 16384)), dim3(256), 0, s,
                       config, seed, n_rows, n_features, labels, grad, hess);
  DP_HIP(hipGetLastError());
}

}  // namespace dp
