// LDS atomic roof: the rate at which one MI355X retires the histogram's LDS
// atomics when nothing else runs (no global loads), for bench.py.
//
// Each workgroup (1024 threads, 64 KiB of LDS laid out as the histogram
// kernel's [bin][g f0..15 | h f0..15] int64 image) runs `rows` steps; at each
// step a lane issues the atomics of 16 (feature, bin) elements, feature
// (step + lane) & 15 and a pseudo-random bin, exactly the histogram kernel's
// addressing.  Modes: 0 = two 64-bit atomics per element (g and h, the
// histogram kernel's exact accumulation), 1 = one 64-bit atomic, 2 = two
// 32-bit atomics, 3 = one 32-bit atomic, 4 = the same loop without LDS work.
//
// Modes 5-9 measure wavefront aggregation of lanes that share a (feature,
// bin).  With the lane rotation, lanes l and l ^ 32 take the same feature at
// every element; in the aggregated modes each lane compares its address with
// lane l ^ 32's (v_permlane32_swap), and when they are equal the lower lane
// adds both lanes' (g, h) -- precomputed once per row -- and the upper lane
// issues nothing.  5 = mode 0 with bins drawn from 16 values (C3's
// integer-valued features: same-address conflicts), 6 = mode 5 aggregated,
// 7 = mode 0 aggregated (random bins: the aggregation's cost alone), 8 = mode
// 0 with 80 % of the elements in bin 0 (C4's zero pixels), 9 = mode 8
// aggregated.
// Not part of the library: built as libdp_roof.so and loaded by bench.py only.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef __attribute__((address_space(3))) unsigned long long lds_u64;
typedef __attribute__((address_space(3))) unsigned int lds_u32;

constexpr int kModes = 10;

__device__ __forceinline__ void add64(lds_u64* p, unsigned long long v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Lane l ^ 32's value of v (the swap's two results hold the other half's).
__device__ __forceinline__ uint32_t xor32(uint32_t v, bool upper) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return upper ? r[0] : r[1];
}

template <int MODE>
__global__ __launch_bounds__(1024) void lds_roof_kernel(int rows, unsigned long long* out) {
  __shared__ unsigned long long h[8192];  // 64 KiB; every offset below is < 65536 bytes
  for (int i = threadIdx.x; i < 8192; i += 1024) h[i] = 0;
  __syncthreads();
  const uint32_t rot = threadIdx.x & 15u;
  const bool upper = (threadIdx.x & 32u) != 0u;
  uint32_t x = 0x9E3779B9u * (blockIdx.x * 1024u + threadIdx.x + 1u);
  lds_u64* p64 = (lds_u64*)h;
  lds_u32* p32 = (lds_u32*)h;
  constexpr bool kAgg = MODE == 6 || MODE == 7 || MODE == 9;
  for (int r = 0; r < rows; ++r) {
    // this row's (g, h) and, for aggregation, the pair's sums (once per row)
    const uint32_t gq = x ^ uint32_t(r), hq = (x >> 7) | 1u;
    unsigned long long gs = gq, hs = hq;
    if (kAgg) {
      gs += xor32(gq, upper);
      hs += xor32(hq, upper);
    }
#pragma unroll
    for (int f = 0; f < 16; ++f) {
      x = x * 1664525u + 1013904223u;
      uint32_t bin = x >> 24;  // 0..255
      if (MODE == 5 || MODE == 6) bin &= 15u;
      if (MODE == 8 || MODE == 9) bin = (x >> 8) % 5u == 0u ? bin : 0u;  // 80 % zeros
      const uint32_t feat = (uint32_t(f) + rot) & 15u;  // 0..15
      const uint32_t slot = bin * 32 + feat;
      if (MODE == 0 || MODE == 5 || MODE == 8) {
        add64(p64 + slot, gq);
        add64(p64 + slot + 16, hq);
      } else if (kAgg) {
        const bool same = xor32(slot, upper) == slot;
        if (!(same && upper)) {
          add64(p64 + slot, same ? gs : (unsigned long long)gq);
          add64(p64 + slot + 16, same ? hs : (unsigned long long)hq);
        }
      } else if (MODE == 1) {
        add64(p64 + slot, x);
      } else if (MODE == 2) {
        __hip_atomic_fetch_add(p32 + bin * 64 + feat, x, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        __hip_atomic_fetch_add(p32 + bin * 64 + 16 + feat, bin, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
      } else if (MODE == 3) {
        __hip_atomic_fetch_add(p32 + bin * 64 + feat, x, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
      } else if (x == 0x12345u) {  // keeps the loop; practically never taken
        p64[bin] = x;
      }
    }
  }
  __syncthreads();
  unsigned long long s = 0;
  for (int i = threadIdx.x; i < 8192; i += 1024) s += h[i];
  out[int64_t(blockIdx.x) * 1024 + threadIdx.x] = s + x;
}

template <int M>
void launch_mode(int mode, int grid, int rows, unsigned long long* o, hipStream_t stream) {
  if constexpr (M < kModes) {
    if (mode == M)
      hipLaunchKernelGGL(lds_roof_kernel<M>, dim3(grid), dim3(1024), 0, stream, rows, o);
    else
      launch_mode<M + 1>(mode, grid, rows, o, stream);
  }
}

}  // namespace

// Times `reps` launches of mode `mode` over grid x 1024 threads x rows x 16
// elements on `stream`; out must hold grid * 1024 words.  Writes the fastest
// launch in milliseconds to *ms.  Returns 0, or a HIP error code.
extern "C" int dp_roof_lds_atomics(int mode, int grid, int rows, int reps, void* out, float* ms,
                                   hipStream_t stream) {
  if (mode < 0 || mode >= kModes || grid < 1 || rows < 1 || reps < 1 || !out || !ms) return -1;
  hipEvent_t a, b;
  hipError_t e = hipEventCreate(&a);
  if (e != hipSuccess) return int(e);
  e = hipEventCreate(&b);
  if (e != hipSuccess) return int(e);
  float best = 1e30f;
  auto* o = static_cast<unsigned long long*>(out);
  for (int it = 0; it < reps && e == hipSuccess; ++it) {
    e = hipEventRecord(a, stream);
    if (e != hipSuccess) break;
    launch_mode<0>(mode, grid, rows, o, stream);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipEventRecord(b, stream);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    float t = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, a, b);
    if (e == hipSuccess && it > 0 && t < best) best = t;  // the first launch warms up
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  if (e != hipSuccess) return int(e);
  *ms = reps > 1 ? best : 0.0f;
  return 0;
}
