// Objective gradients and the fixed-point gradient quantiser.
//
// Objectives (upstream's; the reference trainer pins multi:softmax with a zero
// base margin, class_native_training.cuh:60-64):
//   binary:logistic  p = 1/(1+e^-m), g = p - y, h = max(p(1-p), 1e-16)
//   multi:softprob   p = softmax(m), g = p_k - [y==k], h = max(2p(1-p), 1e-16)
//   reg:squarederror g = m - y, h = 1
// exp is computed by dp_expf below: Cody & Waite range reduction with a float
// head/tail split of ln 2 and the degree-7 Taylor polynomial of e^r in Horner
// form with fused multiply-adds, scaled by 2^k.  It uses only IEEE-exact
// operations, so GPU and CPU produce the same bits.
//
// Quantiser: per class, e = frexp exponent of max|x| (max|x| < 2^e), exp =
// 30 - e, q = rint(x * 2^exp), so |q| <= 2^30 and the sum of any row set is an
// exact int64.  The maxima are reduced with integer atomicMax on the bit
// patterns of |x| (order-independent, hence deterministic).
#include "dp_internal.hpp"

#include <cmath>

namespace dp {
namespace {

__device__ __forceinline__ float dp_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283f) return INFINITY;
  if (x < -87.0f) return 0.0f;
  const float log2e = 1.44269504088896341f;
  const float ln2_hi = 0.693145751953125f;
  const float ln2_lo = 1.42860682030941723212e-6f;
  const float k = rintf(x * log2e);
  float r = fmaf(-k, ln2_hi, x);
  r = fmaf(-k, ln2_lo, r);
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

__global__ void gradients_kernel(int objective, const float* __restrict__ margin,
                                 const float* __restrict__ label, int64_t n_rows, int n_classes,
                                 float* __restrict__ grad, float* __restrict__ hess) {
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n_rows;
       r += int64_t(blockDim.x) * gridDim.x) {
    if (objective == DP_OBJ_LOGISTIC) {
      const float p = 1.0f / (1.0f + dp_expf(-margin[r]));
      grad[r] = p - label[r];
      hess[r] = fmaxf(p * (1.0f - p), 1e-16f);
    } else if (objective == DP_OBJ_SQUARED) {
      grad[r] = margin[r] - label[r];
      hess[r] = 1.0f;
    } else {
      const float* m = margin + r * n_classes;
      float mx = m[0];
      for (int k = 1; k < n_classes; ++k) mx = fmaxf(mx, m[k]);
      float s = 0.0f;
      for (int k = 0; k < n_classes; ++k) s += dp_expf(m[k] - mx);
      const int y = int(label[r]);
      for (int k = 0; k < n_classes; ++k) {
        const float p = dp_expf(m[k] - mx) / s;
        grad[r * n_classes + k] = p - (k == y ? 1.0f : 0.0f);
        hess[r * n_classes + k] = fmaxf(2.0f * p * (1.0f - p), 1e-16f);
      }
    }
  }
}

__global__ void absmax_kernel(const float* __restrict__ grad, const float* __restrict__ hess,
                              int64_t n_rows, int n_classes, unsigned* __restrict__ maxima) {
  // blockIdx.y = class
  const int k = blockIdx.y;
  unsigned mg = 0, mh = 0;
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n_rows;
       r += int64_t(blockDim.x) * gridDim.x) {
    mg = max(mg, __float_as_uint(fabsf(grad[r * n_classes + k])));
    mh = max(mh, __float_as_uint(fabsf(hess[r * n_classes + k])));
  }
  for (int d = 32; d >= 1; d >>= 1) {
    mg = max(mg, __shfl_xor(mg, d, 64));
    mh = max(mh, __shfl_xor(mh, d, 64));
  }
  // one atomic per workgroup: per-wave atomics on two addresses serialise
  __shared__ unsigned wave_max[2][4];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    wave_max[0][wave] = mg;
    wave_max[1][wave] = mh;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < int(blockDim.x >> 6); ++w) {
      mg = max(mg, wave_max[0][w]);
      mh = max(mh, wave_max[1][w]);
    }
    atomicMax(&maxima[2 * k], mg);
    atomicMax(&maxima[2 * k + 1], mh);
  }
}

__device__ __forceinline__ int quant_exp(unsigned bits) {
  const float m = __uint_as_float(bits);
  if (!(m > 0.0f)) return kQuantBits;
  int e;
  frexpf(m, &e);
  return kQuantBits - e;
}

__global__ void quantise_kernel(const float* __restrict__ grad, const float* __restrict__ hess,
                                int64_t n_rows, int n_classes, const unsigned* __restrict__ maxima,
                                int32_t* __restrict__ exps, int2* __restrict__ gpair,
                                long long* __restrict__ sums) {
  __shared__ long long wave_sum[2][4];
  const int k = blockIdx.y;
  const int eg = quant_exp(maxima[2 * k]), eh = quant_exp(maxima[2 * k + 1]);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    exps[2 * k] = eg;
    exps[2 * k + 1] = eh;
  }
  long long sg = 0, sh = 0;
  int2* out = gpair + int64_t(k) * n_rows;
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n_rows;
       r += int64_t(blockDim.x) * gridDim.x) {
    const int qg = int(rintf(ldexpf(grad[r * n_classes + k], eg)));
    const int qh = int(rintf(ldexpf(hess[r * n_classes + k], eh)));
    out[r] = make_int2(qg, qh);
    sg += qg;
    sh += qh;
  }
  for (int d = 32; d >= 1; d >>= 1) {
    sg += __shfl_xor(sg, d, 64);
    sh += __shfl_xor(sh, d, 64);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    wave_sum[0][wave] = sg;
    wave_sum[1][wave] = sh;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    long long tg = 0, th = 0;
    for (int w = 0; w < int(blockDim.x >> 6); ++w) {
      tg += wave_sum[0][w];
      th += wave_sum[1][w];
    }
    atomicAdd(reinterpret_cast<unsigned long long*>(&sums[2 * k]), (unsigned long long)tg);
    atomicAdd(reinterpret_cast<unsigned long long*>(&sums[2 * k + 1]), (unsigned long long)th);
  }
}

// Label checks in the spirit of the reference's prepare_labels
// (class_native_training.cuh:36-41): class ids must be exact integers in [0, K),
// logistic labels in [0, 1], regression labels finite.
__global__ void check_labels_kernel(const float* __restrict__ label, int64_t n, int objective,
                                    int n_classes, int32_t* __restrict__ bad) {
  bool wrong = false;
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n;
       r += int64_t(blockDim.x) * gridDim.x) {
    const float y = label[r];
    if (objective == DP_OBJ_SOFTPROB)
      wrong = wrong || !(y >= 0.0f) || !(y < float(n_classes)) || y != floorf(y);
    else if (objective == DP_OBJ_LOGISTIC)
      wrong = wrong || !(y >= 0.0f && y <= 1.0f);
    else
      wrong = wrong || !isfinite(y);
  }
  if (__ballot(wrong) && (threadIdx.x & 63) == 0) atomicOr(bad, 1);
}

}  // namespace

void launch_check_labels(const float* label, int64_t n, int32_t objective, int32_t n_classes,
                         int32_t* bad, hipStream_t s) {
  launch_fill_u8(reinterpret_cast<uint8_t*>(bad), 4, 0, s);
  if (n <= 0) return;
  hipLaunchKernelGGL(check_labels_kernel, dim3(grid_for(n, 256, 4096)), dim3(256), 0, s, label, n,
                     objective, n_classes, bad);
  DP_HIP(hipGetLastError());
}

void launch_gradients(int32_t objective, const float* margin, const float* label,
                      int64_t n_rows, int32_t n_classes, float* grad, float* hess,
                      hipStream_t s) {
  if (n_rows <= 0) return;
  need(objective == DP_OBJ_LOGISTIC || objective == DP_OBJ_SOFTPROB ||
           objective == DP_OBJ_SQUARED,
       "unknown objective id");
  hipLaunchKernelGGL(gradients_kernel, dim3(grid_for(n_rows, 256, 8192)), dim3(256), 0, s,
                     objective, margin, label, n_rows, n_classes, grad, hess);
  DP_HIP(hipGetLastError());
}

void launch_quantise(const float* grad, const float* hess, int64_t n_rows, int32_t n_classes,
                     uint32_t* maxima, int32_t* exps, int32_t* gpair, int64_t* sums,
                     hipStream_t s) {
  need(n_classes >= 1 && n_classes <= 65535, "class count out of range");
  launch_fill_u8(reinterpret_cast<uint8_t*>(maxima), int64_t(sizeof(uint32_t)) * 2 * n_classes, 0, s);
  launch_fill_i64(sums, 2 * int64_t(n_classes), 0, s);
  // A few hundred workgroups cover HBM; more only adds atomics on the totals.
  const int blocks = grid_for(n_rows, 256, 512);
  hipLaunchKernelGGL(absmax_kernel, dim3(blocks, n_classes), dim3(256), 0, s, grad, hess, n_rows,
                     n_classes, reinterpret_cast<unsigned*>(maxima));
  DP_HIP(hipGetLastError());
  hipLaunchKernelGGL(quantise_kernel, dim3(blocks, n_classes), dim3(256), 0, s, grad, hess,
                     n_rows, n_classes, reinterpret_cast<const unsigned*>(maxima), exps,
                     reinterpret_cast<int2*>(gpair), reinterpret_cast<long long*>(sums));
  DP_HIP(hipGetLastError());
}

}  // namespace dp
