// Quantile cuts and uint8 binning on the device.
//
// The reference obtains both inside XGDMatrixCreateFromCudaArrayInterface and
// the first update (class_native_training.cuh:51).  This build fixes an exact
// definition (upstream's sketch is approximate and cannot be run here):
//   v = sorted non-missing values of a feature (-0.0 folded into +0.0),
//   u = its distinct values, m = |u|;
//   m <= max_bin: cuts = u[1..m-1] then `last`;
//   m >  max_bin: cuts = the strictly increasing subsequence (above u[0]) of
//                 v[floor(i*n/max_bin)], i = 1..max_bin-1, then `last`;
//   last = max + (|max| + 1e-5f); an all-missing feature gets the one cut 1e-5f.
//   bin(x) = index of the first cut > x, clamped to the last bin.
// Sorting uses rocPRIM's radix sort on order-preserving 32-bit keys (NaN maps
// to 0xffffffff and sorts last); one workgroup per feature then extracts cuts.
#include "dp_internal.hpp"

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>
#include <rocprim/device/device_reduce.hpp>

#include <cmath>

namespace dp {
namespace {

__device__ __forceinline__ uint32_t order_key(float x) {
  if (x != x) return 0xffffffffu;
  if (x == 0.0f) return 0x80000000u;
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ float end_cut(float v) { return v + (fabsf(v) + 1e-5f); }

__global__ void keys_kernel(const float* __restrict__ values, int64_t n_rows, int32_t n_features,
                            int32_t f_begin, int32_t f_count, uint32_t* __restrict__ keys) {
  const int64_t total = n_rows * f_count;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(blockDim.x) * gridDim.x) {
    const int64_t r = i / f_count;
    const int32_t j = int32_t(i - r * f_count);
    keys[int64_t(j) * n_rows + r] = order_key(values[r * n_features + f_begin + j]);
  }
}

constexpr int kCutThreads = 256;

// One workgroup per feature of the sorted key block.
__global__ __launch_bounds__(kCutThreads) void cuts_kernel(const uint32_t* __restrict__ sorted,
                                                           int64_t n_rows, int32_t f_begin,
                                                           int32_t max_bin,
                                                           int32_t* __restrict__ counts,
                                                           float* __restrict__ cuts,
                                                           float* __restrict__ mins,
                                                           int32_t* __restrict__ any_missing) {
  __shared__ int64_t s_valid;
  __shared__ int64_t s_distinct;
  __shared__ int s_wave[kCutThreads / 64];
  __shared__ float s_cand[kMaxBins];
  const int j = blockIdx.x;
  const int f = f_begin + j;
  const uint32_t* v = sorted + int64_t(j) * n_rows;
  float* out = cuts + int64_t(f) * max_bin;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) {
    int64_t lo = 0, hi = n_rows;  // first NaN key
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (v[mid] == 0xffffffffu) hi = mid; else lo = mid + 1;
    }
    s_valid = lo;
    if (lo < n_rows) atomicOr(any_missing, 1);
    s_distinct = 0;
  }
  __syncthreads();
  const int64_t n = s_valid;
  if (n == 0) {
    if (threadIdx.x == 0) {
      out[0] = end_cut(0.0f);
      counts[f] = 1;
      mins[f] = 0.0f;
    }
    return;
  }
  // Distinct count, stopping once it exceeds max_bin.
  for (int64_t base = 0; base < n; base += kCutThreads) {
    const int64_t i = base + threadIdx.x;
    const bool first = i < n && (i == 0 || v[i] != v[i - 1]);
    const unsigned long long m = __ballot(first);
    if (lane == 0) s_wave[wave] = __popcll(m);
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 0; w < kCutThreads / 64; ++w) s_distinct += s_wave[w];
    }
    __syncthreads();
    if (s_distinct > max_bin) break;
  }
  const int64_t distinct = s_distinct;
  if (distinct <= max_bin) {
    // Every distinct value after the first is a cut, in order.
    int64_t written = 0;  // distinct values seen before this sweep
    for (int64_t base = 0; base < n; base += kCutThreads) {
      const int64_t i = base + threadIdx.x;
      const bool first = i < n && (i == 0 || v[i] != v[i - 1]);
      const unsigned long long m = __ballot(first);
      if (lane == 0) s_wave[wave] = __popcll(m);
      __syncthreads();
      int64_t rank = written;
      int64_t sweep = 0;
      for (int w = 0; w < kCutThreads / 64; ++w) {
        if (w < wave) rank += s_wave[w];
        sweep += s_wave[w];
      }
      const unsigned long long below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
      rank += __popcll(m & below);
      if (first && rank >= 1) out[rank - 1] = key_value(v[i]);
      written += sweep;
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      out[distinct - 1] = end_cut(key_value(v[n - 1]));
      counts[f] = int32_t(distinct);
      mins[f] = key_value(v[0]);
    }
    return;
  }
  for (int i = 1 + threadIdx.x; i < max_bin; i += kCutThreads)
    s_cand[i] = key_value(v[(int64_t(i) * n) / max_bin]);
  __syncthreads();
  if (threadIdx.x == 0) {
    float prev = key_value(v[0]);
    int32_t c = 0;
    for (int i = 1; i < max_bin; ++i) {
      const float x = s_cand[i];
      if (x > prev) {
        out[c++] = x;
        prev = x;
      }
    }
    out[c++] = end_cut(key_value(v[n - 1]));
    counts[f] = c;
    mins[f] = key_value(v[0]);
  }
}

// Bins for one tile of FT features; cuts of the tile staged in LDS.
template <int FT>
__global__ __launch_bounds__(256) void bin_kernel(const float* __restrict__ values,
                                                  int64_t n_rows, int32_t n_features,
                                                  const int32_t* __restrict__ cut_ptr,
                                                  const float* __restrict__ cut_values,
                                                  int32_t stride, int32_t missing_bin,
                                                  uint8_t* __restrict__ bins) {
  extern __shared__ float s_cuts[];  // [FT][stride]
  __shared__ int s_count[FT];
  const int tile = blockIdx.y;
  const int f0 = tile * FT;
  for (int e = threadIdx.x; e < FT; e += blockDim.x) {
    const int f = f0 + e;
    s_count[e] = f < n_features ? cut_ptr[f + 1] - cut_ptr[f] : 0;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < FT * stride; e += blockDim.x) {
    const int jf = e / stride, b = e % stride;
    const int f = f0 + jf;
    s_cuts[e] = (f < n_features && b < s_count[jf]) ? cut_values[cut_ptr[f] + b] : 0.0f;
  }
  __syncthreads();
  constexpr int TPR = FT / 16;
  const int sub = threadIdx.x % TPR;
  const int64_t rows_per_block = blockDim.x / TPR;
  uint8_t* tile_base = bins + int64_t(tile) * n_rows * FT;
  for (int64_t r = int64_t(blockIdx.x) * rows_per_block + threadIdx.x / TPR; r < n_rows;
       r += int64_t(gridDim.x) * rows_per_block) {
    uint32_t word[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int jf = sub * 16 + k;
      const int f = f0 + jf;
      uint32_t b = 0;
      if (f < n_features) {
        const float x = values[r * n_features + f];
        if (x != x) {
          b = uint32_t(missing_bin);
        } else {
          const float* c = s_cuts + jf * stride;
          int lo = 0, hi = s_count[jf];
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (c[mid] > x) hi = mid; else lo = mid + 1;
          }
          b = uint32_t(lo < s_count[jf] ? lo : s_count[jf] - 1);
        }
      }
      word[k >> 2] |= (b & 0xffu) << ((k & 3) * 8);
    }
    *reinterpret_cast<uint4*>(tile_base + r * FT + sub * 16) =
        make_uint4(word[0], word[1], word[2], word[3]);
  }
}

__global__ void any_nan_kernel(const float* __restrict__ values, int64_t n,
                               int32_t* __restrict__ flag) {
  bool found = false;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    found = found || (values[i] != values[i]);
  if (__ballot(found) && (threadIdx.x & 63) == 0) atomicOr(flag, 1);
}

// Dense row-major copy; values equal to `missing` become NaN, +-inf is flagged
// (the reference's prepare_values kernel rejects inf the same way,
// class_native_training.cuh:42-46).
__global__ void copy_matrix_kernel(const float* __restrict__ src, int64_t row_stride,
                                   int64_t n_rows, int32_t n_features, float missing,
                                   float* __restrict__ dst, int32_t* __restrict__ bad) {
  const int64_t total = n_rows * n_features;
  bool inf = false;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(blockDim.x) * gridDim.x) {
    const int64_t r = i / n_features;
    const int64_t f = i - r * n_features;
    float x = src[r * row_stride + f];
    if (x == missing) x = __builtin_nanf("");
    inf = inf || isinf(x);
    dst[i] = x;
  }
  if (__ballot(inf) && (threadIdx.x & 63) == 0) atomicOr(bad, 1);
}

// Column-major copy of tile-major bins: cols[f * n_rows + r].  A workgroup
// stages 256 rows x 16 features in LDS and writes 16 runs of 256 bytes.
__global__ __launch_bounds__(256) void tiles_to_columns_kernel(const uint8_t* __restrict__ bins,
                                                               int64_t n_rows, int32_t n_features,
                                                               uint8_t* __restrict__ cols) {
  __shared__ uint8_t s[16][256 + 4];
  const int tile = blockIdx.y;
  const int f0 = tile * 16;
  const uint8_t* tb = bins + int64_t(tile) * n_rows * 16;
  for (int64_t r0 = int64_t(blockIdx.x) * 256; r0 < n_rows; r0 += int64_t(gridDim.x) * 256) {
    const int64_t r = r0 + threadIdx.x;
    if (r < n_rows) {
      const uint4 v = *reinterpret_cast<const uint4*>(tb + r * 16);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 16; ++k) s[k][threadIdx.x] = uint8_t(w[k >> 2] >> (8 * (k & 3)));
    }
    __syncthreads();
    if (r < n_rows)
      for (int k = 0; k < 16 && f0 + k < n_features; ++k)
        cols[int64_t(f0 + k) * n_rows + r] = s[k][threadIdx.x];
    __syncthreads();
  }
}

// Joint tiles of the paired tiles (dp_bin_layout::paired_tiles): joint tile
// n_tiles + k, for the k-th pair (tiles t, t + 1; blockIdx.y = k), holds per
// row and feature slot i the byte (tile t's bin << 4) | (tile t + 1's bin &
// 15).  One row per thread: two 16-byte loads, one store.
__global__ void join_tiles_kernel(uint8_t* __restrict__ bins, int64_t n_rows, int32_t n_tiles,
                                  uint64_t pairs) {
  const int32_t k = int32_t(blockIdx.y);
  uint64_t m = pairs;
  for (int32_t j = 0; j < k; ++j) m &= m - 1ull;  // drop the first k pairs
  const int64_t t = __builtin_ctzll(m);
  const uint8_t* hi = bins + t * n_rows * 16;
  const uint8_t* lo = hi + n_rows * 16;
  uint8_t* out = bins + int64_t(n_tiles + k) * n_rows * 16;
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n_rows;
       r += int64_t(blockDim.x) * gridDim.x) {
    const uint4 x = *reinterpret_cast<const uint4*>(hi + r * 16);
    const uint4 y = *reinterpret_cast<const uint4*>(lo + r * 16);
    uint4 z;
    z.x = ((x.x << 4) & 0xf0f0f0f0u) | (y.x & 0x0f0f0f0fu);
    z.y = ((x.y << 4) & 0xf0f0f0f0u) | (y.y & 0x0f0f0f0fu);
    z.z = ((x.z << 4) & 0xf0f0f0f0u) | (y.z & 0x0f0f0f0fu);
    z.w = ((x.w << 4) & 0xf0f0f0f0u) | (y.w & 0x0f0f0f0fu);
    *reinterpret_cast<uint4*>(out + r * 16) = z;
  }
}

// Row-major copy of tile-major bins: one 16-byte piece per thread.  The first
// tile of each pair takes the pair's joint tile (tile n_tiles + k of the
// tile-major bins for the k-th pair).
__global__ void tiles_to_rows_kernel(const uint8_t* __restrict__ bins, int64_t n_rows,
                                     int32_t n_tiles, uint64_t pairs, uint8_t* __restrict__ rows) {
  const int64_t n = n_rows * n_tiles;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x) {
    const int64_t t = i / n_rows, r = i - t * n_rows;
    const int64_t src = t < 63 && ((pairs >> t) & 1ull)
                            ? n_tiles + __builtin_popcountll(pairs & ((1ull << t) - 1ull))
                            : t;
    *reinterpret_cast<uint4*>(rows + (r * n_tiles + t) * 16) =
        *reinterpret_cast<const uint4*>(bins + (src * n_rows + r) * 16);
  }
}

// Present-value layout (see SparseBins): one thread per (sparse tile, row),
// i = tile * n_rows + row.  The row's bytes of the tile's features are read
// from the 16-feature tiles (16 bytes per dense tile); bytes of features past
// n_features are padding, not values.
__device__ __forceinline__ void sparse_tile_row(int64_t i, int64_t n_rows, int32_t n_features,
                                                int32_t tile_features, int64_t& row,
                                                int32_t& f_begin, int32_t& f_end) {
  const int64_t t = i / n_rows;
  row = i - t * n_rows;
  f_begin = int32_t(t) * tile_features;
  f_end = f_begin + tile_features < n_features ? f_begin + tile_features : n_features;
}

__global__ void sparse_count_kernel(const uint8_t* __restrict__ bins, int64_t n_rows,
                                    int32_t n_features, int32_t tile_features, int64_t n,
                                    int32_t missing_bin, uint32_t* __restrict__ counts) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x) {
    int64_t r;
    int32_t fb, fe;
    sparse_tile_row(i, n_rows, n_features, tile_features, r, fb, fe);
    uint32_t c = 0;
    for (int32_t d = fb / 16; d * 16 < fe; ++d) {
      const uint4 v = *reinterpret_cast<const uint4*>(bins + (int64_t(d) * n_rows + r) * 16);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int32_t f = d * 16 + k;
        const uint32_t b = (w[k >> 2] >> (8 * (k & 3))) & 0xffu;
        c += (f < fe && int32_t(b) != missing_bin) ? 1u : 0u;
      }
    }
    counts[i] = c;
  }
}

// An entry: the LDS plane word of (feature offset fo, bin b) with ps words per
// feature (see SparseBins).
__device__ __forceinline__ uint16_t sparse_entry(int32_t fo, uint32_t b, uint32_t ps) {
  return uint16_t(uint32_t(fo) * ps + b);
}

__global__ void sparse_fill_kernel(const uint8_t* __restrict__ bins, int64_t n_rows,
                                   int32_t n_features, int32_t tile_features, int64_t n,
                                   int32_t missing_bin, uint32_t ps, const uint32_t* __restrict__ ptr,
                                   uint16_t* __restrict__ entries) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x) {
    int64_t r;
    int32_t fb, fe;
    sparse_tile_row(i, n_rows, n_features, tile_features, r, fb, fe);
    uint32_t o = ptr[i];
    for (int32_t d = fb / 16; d * 16 < fe; ++d) {
      const uint4 v = *reinterpret_cast<const uint4*>(bins + (int64_t(d) * n_rows + r) * 16);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int32_t f = d * 16 + k;
        const uint32_t b = (w[k >> 2] >> (8 * (k & 3))) & 0xffu;
        if (f < fe && int32_t(b) != missing_bin) entries[o++] = sparse_entry(f - fb, b, ps);
      }
    }
  }
}

// 16-bit column copy of a matrix whose missing values need a symbol beside 256
// bins: cols[f * n_rows + r] = the bin of (r, f), kWideMissing for NaN.  A
// thread bins one row of one 16-feature tile (the tile's cuts staged in LDS)
// and stores its 16 symbols, so that for each feature a wavefront stores 64
// adjacent symbols.
__global__ __launch_bounds__(256) void bin_columns16_kernel(const float* __restrict__ values,
                                                            int64_t n_rows, int32_t n_features,
                                                            const int32_t* __restrict__ cut_ptr,
                                                            const float* __restrict__ cut_values,
                                                            uint16_t* __restrict__ cols) {
  __shared__ float s_cuts[16 * kMaxBins];
  __shared__ int s_count[16];
  const int f0 = blockIdx.y * 16;
  if (threadIdx.x < 16) {
    const int f = f0 + int(threadIdx.x);
    s_count[threadIdx.x] = f < n_features ? cut_ptr[f + 1] - cut_ptr[f] : 0;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 16 * kMaxBins; e += blockDim.x) {
    const int jf = e / kMaxBins, b = e % kMaxBins;
    s_cuts[e] = b < s_count[jf] ? cut_values[cut_ptr[f0 + jf] + b] : 0.0f;
  }
  __syncthreads();
  for (int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < n_rows;
       r += int64_t(gridDim.x) * blockDim.x) {
    for (int k = 0; k < 16 && f0 + k < n_features; ++k) {
      const float x = values[r * n_features + f0 + k];
      uint32_t b = uint32_t(kWideMissing);
      if (x == x) {
        const float* c = s_cuts + k * kMaxBins;
        int lo = 0, hi = s_count[k];
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (c[mid] > x) hi = mid; else lo = mid + 1;
        }
        b = uint32_t(lo < s_count[k] ? lo : s_count[k] - 1);
      }
      cols[int64_t(f0 + k) * n_rows + r] = uint16_t(b);
    }
  }
}

// The present-value layout from 16-bit columns (missing: kWideMissing); one
// thread per (sparse tile, row) as sparse_count_kernel / sparse_fill_kernel,
// reading the tile's features of its row from the columns (adjacent threads,
// adjacent rows).
__global__ void sparse_count16_kernel(const uint16_t* __restrict__ cols, int64_t n_rows,
                                      int32_t n_features, int32_t tile_features, int64_t n,
                                      uint32_t* __restrict__ counts) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x) {
    int64_t r;
    int32_t fb, fe;
    sparse_tile_row(i, n_rows, n_features, tile_features, r, fb, fe);
    uint32_t c = 0;
    for (int32_t f = fb; f < fe; ++f) c += cols[int64_t(f) * n_rows + r] != kWideMissing ? 1u : 0u;
    counts[i] = c;
  }
}

__global__ void sparse_fill16_kernel(const uint16_t* __restrict__ cols, int64_t n_rows,
                                     int32_t n_features, int32_t tile_features, int64_t n,
                                     uint32_t ps, const uint32_t* __restrict__ ptr,
                                     uint16_t* __restrict__ entries) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x) {
    int64_t r;
    int32_t fb, fe;
    sparse_tile_row(i, n_rows, n_features, tile_features, r, fb, fe);
    uint32_t o = ptr[i];
    for (int32_t f = fb; f < fe; ++f) {
      const uint32_t b = cols[int64_t(f) * n_rows + r];
      if (b != uint32_t(kWideMissing)) entries[o++] = sparse_entry(f - fb, b, ps);
    }
  }
}

// counts[f][b] += rows of this workgroup's row range whose bin of feature f is
// b, from the column copy.  Workgroup i takes row range i % blocks_per_feature
// of feature i / blocks_per_feature; each wavefront counts into its own 256 LDS
// counters, then the counters go to global memory.
constexpr int kCountThreads = 256;
__global__ __launch_bounds__(kCountThreads) void bin_counts_kernel(
    const uint8_t* __restrict__ cols, int64_t n_rows, int64_t rows_per_block,
    int64_t blocks_per_feature, unsigned int* __restrict__ counts) {
  __shared__ unsigned int c[kCountThreads / 64][256];
  const int wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < (kCountThreads / 64) * 256; i += kCountThreads) (&c[0][0])[i] = 0u;
  __syncthreads();
  const int64_t f = int64_t(blockIdx.x) / blocks_per_feature;
  const uint8_t* col = cols + f * n_rows;
  const int64_t r0 = (int64_t(blockIdx.x) % blocks_per_feature) * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < n_rows ? r0 + rows_per_block : n_rows;
  for (int64_t r = r0 + threadIdx.x; r < r1; r += kCountThreads) atomicAdd(&c[wave][col[r]], 1u);
  __syncthreads();
  for (int b = threadIdx.x; b < 256; b += kCountThreads) {
    unsigned int t = 0;
    for (int w = 0; w < kCountThreads / 64; ++w) t += c[w][b];
    if (t) atomicAdd(&counts[f * 256 + b], t);
  }
}

}  // namespace

void launch_bin_counts(const uint8_t* cols, int64_t n_rows, int32_t n_features,
                       unsigned int* counts, hipStream_t s) {
  if (n_rows <= 0 || n_features <= 0) return;
  launch_fill_u8(reinterpret_cast<uint8_t*>(counts), int64_t(n_features) * 256 * 4, 0, s);
  const int64_t per = 1 << 16;
  const int64_t blocks = (n_rows + per - 1) / per;
  need(blocks * n_features < (int64_t(1) << 31), "bin counts grid too large");
  hipLaunchKernelGGL(bin_counts_kernel, dim3(unsigned(blocks * n_features)), dim3(kCountThreads),
                     0, s, cols, n_rows, per, blocks, counts);
  DP_HIP(hipGetLastError());
}

void launch_tiles_to_rows(const uint8_t* bins, const dp_bin_layout& layout, uint8_t* rows,
                          hipStream_t s) {
  if (layout.n_rows <= 0) return;
  need(layout.tile_width == 16, "row copy needs 16-feature tiles");
  check_pairs(layout);
  hipLaunchKernelGGL(tiles_to_rows_kernel,
                     dim3(grid_for(layout.n_rows * layout.n_tiles, 256, 8192)), dim3(256), 0, s,
                     bins, layout.n_rows, layout.n_tiles, layout.paired_tiles, rows);
  DP_HIP(hipGetLastError());
}

void launch_join_tiles(uint8_t* bins, const dp_bin_layout& layout, hipStream_t s) {
  if (!layout.paired_tiles || layout.n_rows <= 0) return;
  check_pairs(layout);
  const int32_t pairs = __builtin_popcountll(layout.paired_tiles);
  hipLaunchKernelGGL(join_tiles_kernel, dim3(grid_for(layout.n_rows, 256, 4096), pairs),
                     dim3(256), 0, s, bins, layout.n_rows, layout.n_tiles, layout.paired_tiles);
  DP_HIP(hipGetLastError());
}

void launch_tiles_to_columns(const uint8_t* bins, const dp_bin_layout& layout, uint8_t* cols,
                             hipStream_t s) {
  if (layout.n_rows <= 0) return;
  need(layout.tile_width == 16, "column copy needs 16-feature tiles");
  hipLaunchKernelGGL(tiles_to_columns_kernel, dim3(grid_for(layout.n_rows, 256, 4096),
                     layout.n_tiles), dim3(256), 0, s, bins, layout.n_rows, layout.n_features,
                     cols);
  DP_HIP(hipGetLastError());
}


// Row-major present values: counts of (row r, tile t) at r * T + t, from the
// tile-major offsets.
__global__ void sparse_row_counts_kernel(const uint32_t* __restrict__ ptr, int64_t n_rows,
                                         int32_t n_tiles, uint32_t* __restrict__ counts) {
  const int64_t n = n_rows * n_tiles;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x) {
    const int64_t r = i / n_tiles, t = i - r * n_tiles;
    counts[i] = ptr[t * n_rows + r + 1] - ptr[t * n_rows + r];
  }
}

// Copies each (row, tile)'s entries to their row-major place (one thread each).
__global__ void sparse_row_fill_kernel(const uint32_t* __restrict__ ptr,
                                       const uint16_t* __restrict__ entries, int64_t n_rows,
                                       int32_t n_tiles, const uint32_t* __restrict__ rptr,
                                       uint16_t* __restrict__ rentries) {
  const int64_t n = n_rows * n_tiles;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x) {
    const int64_t r = i / n_tiles, t = i - r * n_tiles;
    const uint32_t b = ptr[t * n_rows + r], e = ptr[t * n_rows + r + 1], d = rptr[i];
    for (uint32_t k = 0; k < e - b; ++k) rentries[d + k] = entries[b + k];
  }
}

int32_t sparse_tile_features(int32_t bin_stride) {
  int32_t t = int32_t(kSparseLdsBytes / (int64_t(bin_stride) * 16)) / 16 * 16;
  if (t > 256) t = 256;
  return t < 16 ? 16 : t;
}

namespace {

// The present-value layout of an n_rows x n_features matrix in tiles of
// sparse_tile_features(bin_stride): count(counts, n) writes the present
// values of every (tile, row), fill(ptr, entries, n) writes the entries.
// Built when their share is at most max_density (and the count fits 32-bit
// offsets); returns the share.  Synchronises the stream.
template <class Count, class Fill>
double build_sparse(int64_t N, int32_t n_features, int32_t bin_stride, double max_density,
                    SparseBins& out, hipStream_t s, Count count, Fill fill) {
  const int32_t tf = sparse_tile_features(bin_stride);
  const int32_t T = (n_features + tf - 1) / tf;
  const int64_t n = N * T;
  DeviceBuffer<uint32_t> counts(size_t(n + 1)), ptr(size_t(n + 1));
  launch_fill_u8(reinterpret_cast<uint8_t*>(counts.p + n), sizeof(uint32_t), 0, s);
  count(counts.p, tf, n);
  DP_HIP(hipGetLastError());
  // Exclusive scan over n + 1 counts (the last is 0): ptr[n] is the total.  A
  // 64-bit accumulator catches totals that do not fit 32-bit offsets.
  size_t temp_bytes = 0;
  DP_HIP(rocprim::exclusive_scan(nullptr, temp_bytes, counts.p, ptr.p, 0u, size_t(n + 1),
                                 rocprim::plus<uint32_t>(), s));
  DeviceBuffer<uint8_t> temp(temp_bytes ? temp_bytes : 1);
  DP_HIP(rocprim::exclusive_scan(temp.p, temp_bytes, counts.p, ptr.p, 0u, size_t(n + 1),
                                 rocprim::plus<uint32_t>(), s));
  DeviceBuffer<unsigned long long> total(1);
  launch_fill_u8(reinterpret_cast<uint8_t*>(total.p), sizeof(unsigned long long), 0, s);
  size_t sum_bytes = 0;
  DP_HIP(rocprim::reduce(nullptr, sum_bytes, counts.p, total.p, 0ull, size_t(n),
                         rocprim::plus<unsigned long long>(), s));
  DeviceBuffer<uint8_t> sum_temp(sum_bytes ? sum_bytes : 1);
  DP_HIP(rocprim::reduce(sum_temp.p, sum_bytes, counts.p, total.p, 0ull, size_t(n),
                         rocprim::plus<unsigned long long>(), s));
  unsigned long long nnz = 0;
  DP_HIP(hipMemcpyAsync(&nnz, total.p, sizeof nnz, hipMemcpyDeviceToHost, s));
  DP_HIP(hipStreamSynchronize(s));
  const double density = double(nnz) / (double(N) * double(n_features));
  if (density > max_density || nnz >= (1ull << 32)) return density;
  DeviceBuffer<uint16_t> entries(size_t(nnz + kSparseEntryPad));
  fill(ptr.p, entries.p, tf, n);
  DP_HIP(hipGetLastError());
  // The row-major copy: counts in (row, tile) order, their exclusive scan,
  // then each (row, tile)'s entries copied to its place.
  DeviceBuffer<uint32_t> rptr(size_t(n + 1));
  const dim3 grid(grid_for(n, 256, 16384));
  hipLaunchKernelGGL(sparse_row_counts_kernel, grid, dim3(256), 0, s, ptr.p, N, T, counts.p);
  DP_HIP(hipGetLastError());
  DP_HIP(rocprim::exclusive_scan(temp.p, temp_bytes, counts.p, rptr.p, 0u, size_t(n + 1),
                                 rocprim::plus<uint32_t>(), s));
  DeviceBuffer<uint16_t> rentries(size_t(nnz + kSparseEntryPad));
  hipLaunchKernelGGL(sparse_row_fill_kernel, grid, dim3(256), 0, s, ptr.p, entries.p, N, T,
                     rptr.p, rentries.p);
  DP_HIP(hipGetLastError());
  DP_HIP(hipStreamSynchronize(s));
  out.tile_features = tf;
  out.n_tiles = T;
  out.bin_stride = bin_stride;
  out.nnz = int64_t(nnz);
  out.ptr = std::move(ptr);
  out.entries = std::move(entries);
  out.rptr = std::move(rptr);
  out.rentries = std::move(rentries);
  return density;
}

}  // namespace

double build_sparse_bins(const uint8_t* bins, const dp_bin_layout& layout, int32_t bin_stride,
                         double max_density, SparseBins& out, hipStream_t s) {
  need(layout.tile_width == 16, "present-value layout needs 16-feature tiles");
  need(layout.missing_bin == 255, "present-value layout needs missing values");
  const int64_t N = layout.n_rows;
  const int32_t F = layout.n_features;
  const dim3 grid(grid_for(N * ((F + sparse_tile_features(bin_stride) - 1) /
                                sparse_tile_features(bin_stride)), 256, 16384));
  return build_sparse(
      N, F, bin_stride, max_density, out, s,
      [&](uint32_t* counts, int32_t tf, int64_t n) {
        hipLaunchKernelGGL(sparse_count_kernel, grid, dim3(256), 0, s, bins, N, F, tf, n,
                           layout.missing_bin, counts);
      },
      [&](const uint32_t* ptr, uint16_t* entries, int32_t tf, int64_t n) {
        hipLaunchKernelGGL(sparse_fill_kernel, grid, dim3(256), 0, s, bins, N, F, tf, n,
                           layout.missing_bin, uint32_t(bin_stride + 1), ptr, entries);
      });
}

void build_sparse_bins_wide(const uint16_t* cols, int64_t n_rows, int32_t n_features,
                            int32_t bin_stride, SparseBins& out, hipStream_t s) {
  const int32_t tf = sparse_tile_features(bin_stride);
  const dim3 grid(grid_for(n_rows * ((n_features + tf - 1) / tf), 256, 16384));
  const double density = build_sparse(
      n_rows, n_features, bin_stride, 1.0, out, s,
      [&](uint32_t* counts, int32_t t, int64_t n) {
        hipLaunchKernelGGL(sparse_count16_kernel, grid, dim3(256), 0, s, cols, n_rows,
                           n_features, t, n, counts);
      },
      [&](const uint32_t* ptr, uint16_t* entries, int32_t t, int64_t n) {
        hipLaunchKernelGGL(sparse_fill16_kernel, grid, dim3(256), 0, s, cols, n_rows,
                           n_features, t, n, uint32_t(bin_stride + 1), ptr, entries);
      });
  need(out.n_tiles > 0,
       "matrix has " + std::to_string(int64_t(density * double(n_rows) * double(n_features))) +
           " present values: more than the 2^32 the present-value layout of a matrix with "
           "missing values and 256 bins holds (use max_bin 255 or less)");
}

void launch_bin_columns16(const float* values, int64_t n_rows, int32_t n_features,
                          const int32_t* cut_ptr, const float* cut_values, uint16_t* cols,
                          hipStream_t s) {
  if (n_rows <= 0 || n_features <= 0) return;
  hipLaunchKernelGGL(bin_columns16_kernel, dim3(grid_for(n_rows, 256, 4096), (n_features + 15) / 16),
                     dim3(256), 0, s, values, n_rows, n_features, cut_ptr, cut_values, cols);
  DP_HIP(hipGetLastError());
}

void launch_any_nan(const float* values, int64_t n, int32_t* flag, hipStream_t s) {
  launch_fill_u8(reinterpret_cast<uint8_t*>(flag), 4, 0, s);
  if (n <= 0) return;
  hipLaunchKernelGGL(any_nan_kernel, dim3(grid_for(n, 256, 8192)), dim3(256), 0, s, values, n,
                     flag);
  DP_HIP(hipGetLastError());
}

void launch_copy_matrix(const float* src, int64_t row_stride, int64_t n_rows, int32_t n_features,
                        float missing, float* dst, int32_t* bad, hipStream_t s) {
  launch_fill_u8(reinterpret_cast<uint8_t*>(bad), 4, 0, s);
  const int64_t total = n_rows * n_features;
  if (total <= 0) return;
  hipLaunchKernelGGL(copy_matrix_kernel, dim3(grid_for(total, 256, 16384)), dim3(256), 0, s, src,
                     row_stride, n_rows, n_features, missing, dst, bad);
  DP_HIP(hipGetLastError());
}

void launch_bin_values(const float* values, const dp_bin_layout& layout, const int32_t* cut_ptr,
                       const float* cut_values, uint8_t* bins, hipStream_t s) {
  if (layout.n_rows <= 0) return;
  const int stride = kMaxBins;
  const int rows_per_block = 256 / (layout.tile_width / 16);
  const int gx = grid_for(layout.n_rows, rows_per_block, 4096);
  const size_t lds = size_t(layout.tile_width) * stride * sizeof(float);
  need(layout.tile_width == 16, "binning needs 16-feature tiles");
  hipLaunchKernelGGL(bin_kernel<16>, dim3(gx, layout.n_tiles), dim3(256), lds, s, values,
                     layout.n_rows, layout.n_features, cut_ptr, cut_values, stride,
                     layout.missing_bin, bins);
  DP_HIP(hipGetLastError());
}

void sketch_cuts(dp_workspace_s& ws, const float* values, int64_t n_rows, int32_t n_features,
                 int32_t max_bin, int32_t* cut_ptr, float* cut_values, float* min_values,
                 int32_t* has_missing, hipStream_t s) {
  need(max_bin >= 2 && max_bin <= kMaxBins, "max_bin must be in [2, 256]");
  need(n_rows > 0 && n_features > 0, "empty matrix");
  need(n_rows <= int64_t(UINT32_MAX), "row count exceeds uint32 row ids");
  // Features are sorted in blocks bounded to ~2^31 keys of device scratch.
  int64_t block = (int64_t(1) << 31) / n_rows;
  if (block < 1) block = 1;
  if (block > n_features) block = n_features;
  DeviceBuffer<uint32_t> keys(static_cast<size_t>(block * n_rows)), sorted(static_cast<size_t>(block * n_rows));
  DeviceBuffer<int32_t> counts(static_cast<size_t>(n_features)), flag(1);
  DeviceBuffer<float> cuts(static_cast<size_t>(n_features) * max_bin), mins(static_cast<size_t>(n_features));
  size_t temp_bytes = 0;
  DP_HIP(rocprim::radix_sort_keys(nullptr, temp_bytes, keys.p, sorted.p, size_t(n_rows), 0, 32, s));
  DeviceBuffer<uint8_t> temp(temp_bytes ? temp_bytes : 1);
  launch_fill_u8(reinterpret_cast<uint8_t*>(flag.p), 4, 0, s);
  (void)ws;
  for (int64_t f0 = 0; f0 < n_features; f0 += block) {
    const int32_t fc = int32_t(std::min<int64_t>(block, n_features - f0));
    hipLaunchKernelGGL(keys_kernel, dim3(grid_for(n_rows * fc, 256, 16384)), dim3(256), 0, s,
                       values, n_rows, n_features, int32_t(f0), fc, keys.p);
    DP_HIP(hipGetLastError());
    for (int32_t j = 0; j < fc; ++j) {
      size_t tb = temp_bytes;
      DP_HIP(rocprim::radix_sort_keys(temp.p, tb, keys.p + int64_t(j) * n_rows,
                                      sorted.p + int64_t(j) * n_rows, size_t(n_rows), 0, 32, s));
    }
    hipLaunchKernelGGL(cuts_kernel, dim3(fc), dim3(kCutThreads), 0, s, sorted.p, n_rows,
                       int32_t(f0), max_bin, counts.p, cuts.p, mins.p, flag.p);
    DP_HIP(hipGetLastError());
  }
  std::vector<int32_t> h_counts(static_cast<size_t>(n_features));
  std::vector<float> h_cuts(static_cast<size_t>(n_features) * max_bin);
  DP_HIP(hipMemcpyAsync(h_counts.data(), counts.p, counts.bytes(), hipMemcpyDeviceToHost, s));
  DP_HIP(hipMemcpyAsync(h_cuts.data(), cuts.p, cuts.bytes(), hipMemcpyDeviceToHost, s));
  DP_HIP(hipMemcpyAsync(min_values, mins.p, mins.bytes(), hipMemcpyDeviceToHost, s));
  DP_HIP(hipMemcpyAsync(has_missing, flag.p, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  DP_HIP(hipStreamSynchronize(s));
  cut_ptr[0] = 0;
  for (int32_t f = 0; f < n_features; ++f) {
    const int32_t c = h_counts[size_t(f)];
    need(c >= 1 && c <= max_bin, "cut count out of range");
    std::memcpy(cut_values + cut_ptr[f], h_cuts.data() + int64_t(f) * max_bin,
                sizeof(float) * size_t(c));
    cut_ptr[f + 1] = cut_ptr[f] + c;
  }
}

}  // namespace dp
