// Node histogram construction and sibling subtraction for gfx950.
//
// The reference reaches this step only inside XGBoost's grow_gpu_hist updater
// (native/class_native_training.cuh:67).  Design for CDNA4:
//  * bins are uint8 in feature tiles of FT bytes per row (tile-major), so one
//    lane reads 16 features of a row with one 128-bit load and a wavefront
//    covers 64*16 contiguous bytes for contiguous rows;
//  * each workgroup privatises the histogram of one tile in LDS as two int64
//    planes (sum qg, sum qh) laid out [bin][feature], so the LDS word of
//    (bin, f) sits in bank pair f mod 16 whatever the bin;
//  * every lane walks its 16 features starting at a lane-dependent rotation,
//    so at each step the 16 lanes of a group touch 16 different features and
//    therefore 16 different bank pairs: the layout plus the rotation make the
//    64-bit LDS atomics bank-conflict free for any bin values;
//  * sums are exact integers (fixed-point gradients), so the result does not
//    depend on atomic order and equals the CPU restatement bit for bit;
//  * the workgroup merges its LDS histogram into the node histogram with
//    64-bit global atomics, skipping empty bins.
#include "dp_internal.hpp"

namespace dp {
namespace {

__global__ void fill_i64_kernel(int64_t* p, int64_t n, int64_t value) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    p[i] = value;
}

__global__ void fill_u8_kernel(uint8_t* p, int64_t n, uint8_t value) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    p[i] = value;
}

__global__ void iota_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    p[i] = uint32_t(i);
}

// Rotates a 16-byte vector so that output byte k is input byte (k + rot) & 15.
__device__ __forceinline__ void rotate16(uint32_t w[4], uint32_t rot) {
  const uint32_t d = rot >> 2, s = rot & 3u;
  const uint32_t a0 = (d & 1u) ? w[1] : w[0];
  const uint32_t a1 = (d & 1u) ? w[2] : w[1];
  const uint32_t a2 = (d & 1u) ? w[3] : w[2];
  const uint32_t a3 = (d & 1u) ? w[0] : w[3];
  const uint32_t b0 = (d & 2u) ? a2 : a0;
  const uint32_t b1 = (d & 2u) ? a3 : a1;
  const uint32_t b2 = (d & 2u) ? a0 : a2;
  const uint32_t b3 = (d & 2u) ? a1 : a3;
  w[0] = __builtin_amdgcn_alignbyte(b1, b0, s);
  w[1] = __builtin_amdgcn_alignbyte(b2, b1, s);
  w[2] = __builtin_amdgcn_alignbyte(b3, b2, s);
  w[3] = __builtin_amdgcn_alignbyte(b0, b3, s);
}

__device__ __forceinline__ void lds_add(unsigned long long* p, unsigned long long v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void global_add(unsigned long long* p, unsigned long long v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// FT: features per tile (16 or 32).  THREADS: workgroup size.  MISSING: the
// matrix holds NaN, whose bin byte is skipped.
template <int FT, int THREADS, bool MISSING>
__global__ __launch_bounds__(THREADS) void hist_kernel(
    const uint8_t* __restrict__ bins, int64_t n_rows, int32_t n_features,
    const int2* __restrict__ gpair, const uint32_t* __restrict__ ridx,
    const HistWork* __restrict__ work, int32_t bin_stride, int32_t missing_bin,
    unsigned long long* __restrict__ hist) {
  extern __shared__ unsigned long long lds[];
  constexpr int TPR = FT / 16;          // lanes per row
  constexpr int ROWS = THREADS / TPR;   // rows per sweep of the workgroup
  const HistWork w = work[blockIdx.x];
  const int plane = bin_stride * FT;
  unsigned long long* gpl = lds;
  unsigned long long* hpl = lds + plane;
  for (int e = threadIdx.x; e < 2 * plane; e += THREADS) lds[e] = 0ull;
  __syncthreads();

  const int sub = threadIdx.x % TPR;
  const uint32_t rot = threadIdx.x & 15u;
  const uint8_t* tile = bins + int64_t(w.tile) * n_rows * FT + sub * 16;
  // byte offset of feature slot (sub*16 + ((k + rot) & 15)) in a plane row
  uint32_t slot[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) slot[k] = uint32_t(sub * 16) + ((uint32_t(k) + rot) & 15u);

  int64_t i = w.begin + threadIdx.x / TPR;
  // Two rows in flight per lane.
  for (; i + ROWS < w.end; i += 2 * ROWS) {
    const uint32_t r0 = ridx ? ridx[i] : uint32_t(i);
    const uint32_t r1 = ridx ? ridx[i + ROWS] : uint32_t(i + ROWS);
    const uint4 v0 = *reinterpret_cast<const uint4*>(tile + int64_t(r0) * FT);
    const uint4 v1 = *reinterpret_cast<const uint4*>(tile + int64_t(r1) * FT);
    const int2 q0 = gpair[r0];
    const int2 q1 = gpair[r1];
    uint32_t a[4] = {v0.x, v0.y, v0.z, v0.w};
    uint32_t b[4] = {v1.x, v1.y, v1.z, v1.w};
    rotate16(a, rot);
    rotate16(b, rot);
    const unsigned long long g0 = (unsigned long long)(long long)q0.x;
    const unsigned long long h0 = (unsigned long long)(long long)q0.y;
    const unsigned long long g1 = (unsigned long long)(long long)q1.x;
    const unsigned long long h1 = (unsigned long long)(long long)q1.y;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const uint32_t bin = (a[k >> 2] >> ((k & 3) * 8)) & 0xffu;
      if (!MISSING || int(bin) != missing_bin) {
        const uint32_t idx = bin * FT + slot[k];
        lds_add(&gpl[idx], g0);
        lds_add(&hpl[idx], h0);
      }
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const uint32_t bin = (b[k >> 2] >> ((k & 3) * 8)) & 0xffu;
      if (!MISSING || int(bin) != missing_bin) {
        const uint32_t idx = bin * FT + slot[k];
        lds_add(&gpl[idx], g1);
        lds_add(&hpl[idx], h1);
      }
    }
  }
  if (i < w.end) {
    const uint32_t r0 = ridx ? ridx[i] : uint32_t(i);
    const uint4 v0 = *reinterpret_cast<const uint4*>(tile + int64_t(r0) * FT);
    const int2 q0 = gpair[r0];
    uint32_t a[4] = {v0.x, v0.y, v0.z, v0.w};
    rotate16(a, rot);
    const unsigned long long g0 = (unsigned long long)(long long)q0.x;
    const unsigned long long h0 = (unsigned long long)(long long)q0.y;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const uint32_t bin = (a[k >> 2] >> ((k & 3) * 8)) & 0xffu;
      if (!MISSING || int(bin) != missing_bin) {
        const uint32_t idx = bin * FT + slot[k];
        lds_add(&gpl[idx], g0);
        lds_add(&hpl[idx], h0);
      }
    }
  }
  __syncthreads();

  const int f0 = w.tile * FT;
  unsigned long long* out = hist + int64_t(w.slot) * n_features * bin_stride * 2;
  for (int e = threadIdx.x; e < plane; e += THREADS) {
    const int bin = e / FT, f = f0 + e % FT;
    if (f >= n_features) continue;
    const unsigned long long g = gpl[e], h = hpl[e];
    if ((g | h) == 0ull) continue;
    unsigned long long* cell = out + (int64_t(f) * bin_stride + bin) * 2;
    global_add(cell, g);
    global_add(cell + 1, h);
  }
}

__global__ void subtract_kernel(const int64_t* __restrict__ parent,
                                const int64_t* __restrict__ built, int64_t* __restrict__ sibling,
                                int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    sibling[i] = parent[i] - built[i];
}

// blockIdx.y selects the job; the x dimension strides over its n elements.
__global__ void subtract_many_kernel(const int64_t* __restrict__ base_parent,
                                     const int64_t* __restrict__ base_child,
                                     int64_t* __restrict__ base_out,
                                     const SubtractJob* __restrict__ jobs, int64_t n) {
  const SubtractJob j = jobs[blockIdx.y];
  const int64_t* p = base_parent + j.parent;
  const int64_t* c = base_child + j.built;
  int64_t* s = base_out + j.sibling;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    s[i] = p[i] - c[i];
}

template <int FT, int THREADS, bool MISSING>
void launch_hist_t(const uint8_t* bins, const dp_bin_layout& layout, const int32_t* gpair,
                   const uint32_t* ridx, const HistWork* work, int32_t n_work, int32_t bin_stride,
                   int64_t* hist, hipStream_t s) {
  const size_t lds = size_t(2) * bin_stride * FT * sizeof(unsigned long long);
  auto kernel = hist_kernel<FT, THREADS, MISSING>;
  static bool configured = false;
  if (!configured) {
    DP_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    configured = true;
  }
  hipLaunchKernelGGL(kernel, dim3(n_work), dim3(THREADS), lds, s, bins, layout.n_rows,
                     layout.n_features, reinterpret_cast<const int2*>(gpair), ridx, work,
                     bin_stride, layout.missing_bin,
                     reinterpret_cast<unsigned long long*>(hist));
  DP_HIP(hipGetLastError());
}

}  // namespace

void launch_fill_i64(int64_t* p, int64_t n, int64_t value, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_i64_kernel, dim3(grid_for(n, 256, 4096)), dim3(256), 0, s, p, n, value);
  DP_HIP(hipGetLastError());
}

void launch_fill_u8(uint8_t* p, int64_t n, uint8_t value, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_u8_kernel, dim3(grid_for(n, 256, 4096)), dim3(256), 0, s, p, n, value);
  DP_HIP(hipGetLastError());
}

void launch_iota_u32(uint32_t* p, int64_t n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(iota_kernel, dim3(grid_for(n, 256, 4096)), dim3(256), 0, s, p, n);
  DP_HIP(hipGetLastError());
}

int64_t hist_chunk_rows(const dp_bin_layout& layout, int64_t total_rows, int32_t n_nodes) {
  // Aim for about 1024 work items over the whole launch, with at least 2048
  // rows per item so the LDS merge stays small next to the row work.
  const int64_t items = 1024;
  int64_t per = (total_rows * layout.n_tiles + items - 1) / items;
  (void)n_nodes;
  if (per < 2048) per = 2048;
  return per;
}

void launch_hist(const uint8_t* bins, const dp_bin_layout& layout, const int32_t* gpair,
                 const uint32_t* ridx, const HistWork* work, int32_t n_work, int32_t bin_stride,
                 int64_t* hist, hipStream_t s) {
  if (n_work <= 0) return;
  need(bin_stride >= 1 && bin_stride <= kMaxBins, "histogram bin stride out of range");
  const bool missing = layout.missing_bin >= 0;
  switch (layout.tile_width) {
    case 16:
      if (missing) launch_hist_t<16, 512, true>(bins, layout, gpair, ridx, work, n_work, bin_stride, hist, s);
      else launch_hist_t<16, 512, false>(bins, layout, gpair, ridx, work, n_work, bin_stride, hist, s);
      break;
    case 32:
      if (missing) launch_hist_t<32, 1024, true>(bins, layout, gpair, ridx, work, n_work, bin_stride, hist, s);
      else launch_hist_t<32, 1024, false>(bins, layout, gpair, ridx, work, n_work, bin_stride, hist, s);
      break;
    default:
      fail("unsupported tile width " + std::to_string(layout.tile_width));
  }
}

void launch_subtract(const int64_t* parent, const int64_t* built, int64_t* sibling, int64_t n,
                     hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(subtract_kernel, dim3(grid_for(n, 256, 8192)), dim3(256), 0, s, parent,
                     built, sibling, n);
  DP_HIP(hipGetLastError());
}

void launch_subtract_many(const int64_t* base_parent, const int64_t* base_child,
                          int64_t* base_out, const SubtractJob* jobs, int32_t n_jobs, int64_t n,
                          hipStream_t s) {
  if (n_jobs <= 0 || n <= 0) return;
  hipLaunchKernelGGL(subtract_many_kernel, dim3(grid_for(n, 256, 64), n_jobs), dim3(256), 0, s,
                     base_parent, base_child, base_out, jobs, n);
  DP_HIP(hipGetLastError());
}

}  // namespace dp
