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
// exact int64.  Maxima (integer max of the bit patterns of |x|) and sums are
// reduced through per-workgroup slots, never by same-address atomics (512
// workgroups on one word serialise): each quantiser workgroup reduces the
// maxima slots itself, and a finishing kernel reduces the sum slots.  Single-
// output objectives produce the maxima slots in the gradient kernel.
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

constexpr int kQuantThreads = 256;

// Max of two values over a 256-thread workgroup; thread 0 gets the result.
__device__ __forceinline__ void block_max2(unsigned& a, unsigned& b) {
  __shared__ unsigned part[2][kQuantThreads / 64];
  for (int d = 32; d >= 1; d >>= 1) {
    a = max(a, __shfl_xor(a, d, 64));
    b = max(b, __shfl_xor(b, d, 64));
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    part[0][wave] = a;
    part[1][wave] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < kQuantThreads / 64; ++w) {
      a = max(a, part[0][w]);
      b = max(b, part[1][w]);
    }
  __syncthreads();
}

// MAXIMA: single-output objectives also write this workgroup's max|g|, max|h|
// bit patterns to max_slots[2 * blockIdx.x ..].
template <bool MAXIMA>
__global__ __launch_bounds__(kQuantThreads) void gradients_kernel(
    int objective, float* __restrict__ margin, const float* __restrict__ label,
    int64_t n_rows, int n_classes, float* __restrict__ grad, float* __restrict__ hess,
    unsigned* __restrict__ max_slots, const float* __restrict__ values) {
  unsigned mg = 0, mh = 0;
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n_rows;
       r += int64_t(blockDim.x) * gridDim.x) {
    // The previous round's leaf values first (values: planes [n_classes][n_rows]):
    // margin + value, the add add_leaf_values_kernel would have made.
    if (values)
      for (int k = 0; k < n_classes; ++k)
        margin[r * n_classes + k] = margin[r * n_classes + k] + values[int64_t(k) * n_rows + r];
    if (objective == DP_OBJ_LOGISTIC) {
      const float p = 1.0f / (1.0f + dp_expf(-margin[r]));
      const float g = p - label[r], h = fmaxf(p * (1.0f - p), 1e-16f);
      grad[r] = g;
      hess[r] = h;
      mg = max(mg, __float_as_uint(fabsf(g)));
      mh = max(mh, __float_as_uint(fabsf(h)));
    } else if (objective == DP_OBJ_SQUARED) {
      const float g = margin[r] - label[r];
      grad[r] = g;
      hess[r] = 1.0f;
      mg = max(mg, __float_as_uint(fabsf(g)));
      mh = max(mh, __float_as_uint(1.0f));
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
  if constexpr (MAXIMA) {
    block_max2(mg, mh);
    if (threadIdx.x == 0) {
      max_slots[2 * blockIdx.x] = mg;
      max_slots[2 * blockIdx.x + 1] = mh;
    }
  }
}

// Per-workgroup max|g|, max|h| of class blockIdx.y into its slots.
// With row sampling, a dropped row's values count as zero.
__device__ __forceinline__ uint64_t row_prefix(const RowSample& rs, int k) {
  return rs.active() ? sample_prefix(rs.seed, kRowStream, uint64_t(uint32_t(*rs.round)),
                                     uint64_t(uint32_t(k)) << 32)
                     : 0;
}

__device__ __forceinline__ bool row_kept(const RowSample& rs, uint64_t prefix, int64_t r) {
  return !rs.active() || uint64_t(sample_draw(prefix, uint64_t(r))) < rs.threshold;
}

__global__ __launch_bounds__(kQuantThreads) void absmax_kernel(
    const float* __restrict__ grad, const float* __restrict__ hess, int64_t n_rows,
    int n_classes, unsigned* __restrict__ max_slots, RowSample rs) {
  const int k = blockIdx.y;
  const uint64_t prefix = row_prefix(rs, k);
  unsigned mg = 0, mh = 0;
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n_rows;
       r += int64_t(blockDim.x) * gridDim.x) {
    if (!row_kept(rs, prefix, r)) continue;
    mg = max(mg, __float_as_uint(fabsf(grad[r * n_classes + k])));
    mh = max(mh, __float_as_uint(fabsf(hess[r * n_classes + k])));
  }
  block_max2(mg, mh);
  if (threadIdx.x == 0) {
    unsigned* slot = max_slots + (int64_t(k) * gridDim.x + blockIdx.x) * 2;
    slot[0] = mg;
    slot[1] = mh;
  }
}

__device__ __forceinline__ int quant_exp(unsigned bits) {
  const float m = __uint_as_float(bits);
  if (!(m > 0.0f)) return kQuantBits;
  int e;
  frexpf(m, &e);
  return kQuantBits - e;
}

// Reduces class blockIdx.y's maxima slots, quantises its rows and writes this
// workgroup's sums to the sum slots.
__global__ __launch_bounds__(kQuantThreads) void quantise_kernel(
    const float* __restrict__ grad, const float* __restrict__ hess, int64_t n_rows,
    int n_classes, const unsigned* __restrict__ max_slots, int32_t* __restrict__ exps,
    int2* __restrict__ gpair, long long* __restrict__ sum_slots, RowSample rs) {
  __shared__ long long wave_sum[2][kQuantThreads / 64];
  __shared__ int s_exp[2];
  const int k = blockIdx.y;
  unsigned mg = 0, mh = 0;
  const unsigned* slots = max_slots + int64_t(k) * gridDim.x * 2;
  for (int b = threadIdx.x; b < int(gridDim.x); b += kQuantThreads) {
    mg = max(mg, slots[2 * b]);
    mh = max(mh, slots[2 * b + 1]);
  }
  block_max2(mg, mh);
  if (threadIdx.x == 0) {
    s_exp[0] = quant_exp(mg);
    s_exp[1] = quant_exp(mh);
    if (blockIdx.x == 0) {
      exps[2 * k] = s_exp[0];
      exps[2 * k + 1] = s_exp[1];
    }
  }
  __syncthreads();
  const int eg = s_exp[0], eh = s_exp[1];
  long long sg = 0, sh = 0;
  int2* out = gpair + int64_t(k) * n_rows;
  const uint64_t prefix = row_prefix(rs, k);
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n_rows;
       r += int64_t(blockDim.x) * gridDim.x) {
    const bool kept = row_kept(rs, prefix, r);
    const int qg = kept ? int(rintf(ldexpf(grad[r * n_classes + k], eg))) : 0;
    const int qh = kept ? int(rintf(ldexpf(hess[r * n_classes + k], eh))) : 0;
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
    for (int w = 0; w < kQuantThreads / 64; ++w) {
      tg += wave_sum[0][w];
      th += wave_sum[1][w];
    }
    long long* slot = sum_slots + (int64_t(k) * gridDim.x + blockIdx.x) * 2;
    slot[0] = tg;
    slot[1] = th;
  }
}

// One workgroup per class: sums[k] = the class's sum slots added up.
__global__ __launch_bounds__(kQuantThreads) void finish_sums_kernel(
    const long long* __restrict__ sum_slots, int blocks, long long* __restrict__ sums) {
  __shared__ long long part[2][kQuantThreads / 64];
  const int k = blockIdx.x;
  long long sg = 0, sh = 0;
  for (int b = threadIdx.x; b < blocks; b += kQuantThreads) {
    sg += sum_slots[(int64_t(k) * blocks + b) * 2];
    sh += sum_slots[(int64_t(k) * blocks + b) * 2 + 1];
  }
  for (int d = 32; d >= 1; d >>= 1) {
    sg += __shfl_xor(sg, d, 64);
    sh += __shfl_xor(sh, d, 64);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    part[0][wave] = sg;
    part[1][wave] = sh;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    long long tg = 0, th = 0;
    for (int w = 0; w < kQuantThreads / 64; ++w) {
      tg += part[0][w];
      th += part[1][w];
    }
    sums[2 * k] = tg;
    sums[2 * k + 1] = th;
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

// margin[r * K + k] = base[k]: the starting margins of every row.
__global__ void init_margin_kernel(float* __restrict__ margin, int64_t n, int32_t k,
                                   const float* __restrict__ base) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    margin[i] = base[i % k];
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

// At least four rows per thread: every quantise workgroup re-reads all the
// maxima slots, so a 1M-row pass keeps about 1,000 of them (four per CU; eight
// rows per thread measured 0.8 % slower on C2's trees), a 10M-row one 2048.
int quantise_blocks(int64_t n_rows) {
  return grid_for(n_rows, kQuantThreads * 4, kQuantBlocks);
}

size_t quantise_scratch_bytes(int64_t n_rows, int32_t n_classes) {
  const size_t slots = size_t(n_classes) * size_t(quantise_blocks(n_rows));
  return slots * 2 * sizeof(uint32_t) + 256 + slots * 2 * sizeof(int64_t);
}

void launch_init_margin(float* margin, int64_t n_rows, int32_t n_outputs, const float* base,
                        hipStream_t s) {
  if (n_rows <= 0 || n_outputs <= 0) return;
  hipLaunchKernelGGL(init_margin_kernel, dim3(grid_for(n_rows * n_outputs, 256, 8192)), dim3(256),
                     0, s, margin, n_rows * n_outputs, n_outputs, base);
  DP_HIP(hipGetLastError());
}

bool launch_gradients(int32_t objective, float* margin, const float* label,
                      int64_t n_rows, int32_t n_classes, float* grad, float* hess,
                      void* quant_scratch, hipStream_t s, const float* values) {
  if (n_rows <= 0) return false;
  need(objective == DP_OBJ_LOGISTIC || objective == DP_OBJ_SOFTPROB ||
           objective == DP_OBJ_SQUARED,
       "unknown objective id");
  if (quant_scratch && n_classes == 1) {
    hipLaunchKernelGGL(gradients_kernel<true>, dim3(quantise_blocks(n_rows)), dim3(kQuantThreads),
                       0, s, objective, margin, label, n_rows, n_classes, grad, hess,
                       static_cast<unsigned*>(quant_scratch), values);
    DP_HIP(hipGetLastError());
    return true;
  }
  hipLaunchKernelGGL(gradients_kernel<false>, dim3(grid_for(n_rows, kQuantThreads, 8192)),
                     dim3(kQuantThreads), 0, s, objective, margin, label, n_rows, n_classes, grad,
                     hess, nullptr, values);
  DP_HIP(hipGetLastError());
  return false;
}

__global__ void store_i32_kernel(int32_t* p, int32_t value) { *p = value; }

void launch_store_i32(int32_t* p, int32_t value, hipStream_t s) {
  hipLaunchKernelGGL(store_i32_kernel, dim3(1), dim3(1), 0, s, p, value);
  DP_HIP(hipGetLastError());
}

void launch_quantise(const float* grad, const float* hess, int64_t n_rows, int32_t n_classes,
                     void* scratch, bool maxima_ready, int32_t* exps, int32_t* gpair,
                     int64_t* sums, hipStream_t s, const RowSample& rows) {
  need(!rows.active() || rows.round != nullptr, "row sampling needs the device round index");
  need(!(rows.active() && maxima_ready), "row sampling needs the sampled maxima");
  need(n_classes >= 1 && n_classes <= 65535, "class count out of range");
  need(n_rows >= 1, "quantiser needs at least one row");
  const int blocks = quantise_blocks(n_rows);
  const size_t slots = size_t(n_classes) * size_t(blocks);
  auto* max_slots = static_cast<unsigned*>(scratch);
  auto* sum_slots = reinterpret_cast<long long*>(static_cast<uint8_t*>(scratch) +
                                                 ((slots * 2 * sizeof(uint32_t) + 255) & ~size_t(255)));
  if (!maxima_ready) {
    hipLaunchKernelGGL(absmax_kernel, dim3(blocks, n_classes), dim3(kQuantThreads), 0, s, grad,
                       hess, n_rows, n_classes, max_slots, rows);
    DP_HIP(hipGetLastError());
  }
  hipLaunchKernelGGL(quantise_kernel, dim3(blocks, n_classes), dim3(kQuantThreads), 0, s, grad,
                     hess, n_rows, n_classes, max_slots, exps, reinterpret_cast<int2*>(gpair),
                     sum_slots, rows);
  DP_HIP(hipGetLastError());
  if (!sums) return;  // the caller reduces the sum slots itself
  hipLaunchKernelGGL(finish_sums_kernel, dim3(n_classes), dim3(kQuantThreads), 0, s, sum_slots,
                     blocks, reinterpret_cast<long long*>(sums));
  DP_HIP(hipGetLastError());
}

const int64_t* quantise_sum_slots(const void* scratch, int64_t n_rows, int32_t n_classes) {
  const size_t slots = size_t(n_classes) * size_t(quantise_blocks(n_rows));
  return reinterpret_cast<const int64_t*>(static_cast<const uint8_t*>(scratch) +
                                          ((slots * 2 * sizeof(uint32_t) + 255) & ~size_t(255)));
}

}  // namespace dp
