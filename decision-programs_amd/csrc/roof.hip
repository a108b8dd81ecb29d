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
// Not part of the library: built as libdp_roof.so and loaded by bench.py only.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef __attribute__((address_space(3))) unsigned long long lds_u64;
typedef __attribute__((address_space(3))) unsigned int lds_u32;

template <int MODE>
__global__ __launch_bounds__(1024) void lds_roof_kernel(int rows, unsigned long long* out) {
  __shared__ unsigned long long h[8192];  // 64 KiB; every offset below is < 65536 bytes
  for (int i = threadIdx.x; i < 8192; i += 1024) h[i] = 0;
  __syncthreads();
  const uint32_t rot = threadIdx.x & 15u;
  uint32_t x = 0x9E3779B9u * (blockIdx.x * 1024u + threadIdx.x + 1u);
  lds_u64* p64 = (lds_u64*)h;
  lds_u32* p32 = (lds_u32*)h;
  for (int r = 0; r < rows; ++r) {
#pragma unroll
    for (int f = 0; f < 16; ++f) {
      x = x * 1664525u + 1013904223u;
      const uint32_t bin = x >> 24;                     // 0..255
      const uint32_t feat = (uint32_t(f) + rot) & 15u;  // 0..15
      if (MODE == 0) {
        __hip_atomic_fetch_add(p64 + bin * 32 + feat, (unsigned long long)x, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        __hip_atomic_fetch_add(p64 + bin * 32 + 16 + feat, (unsigned long long)bin,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      } else if (MODE == 1) {
        __hip_atomic_fetch_add(p64 + bin * 32 + feat, (unsigned long long)x, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
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

}  // namespace

// Times `reps` launches of mode `mode` over grid x 1024 threads x rows x 16
// elements on `stream`; out must hold grid * 1024 words.  Writes the fastest
// launch in milliseconds to *ms.  Returns 0, or a HIP error code.
extern "C" int dp_roof_lds_atomics(int mode, int grid, int rows, int reps, void* out, float* ms,
                                   hipStream_t stream) {
  if (mode < 0 || mode > 4 || grid < 1 || rows < 1 || reps < 1 || !out || !ms) return -1;
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
    switch (mode) {
      case 0: hipLaunchKernelGGL(lds_roof_kernel<0>, dim3(grid), dim3(1024), 0, stream, rows, o); break;
      case 1: hipLaunchKernelGGL(lds_roof_kernel<1>, dim3(grid), dim3(1024), 0, stream, rows, o); break;
      case 2: hipLaunchKernelGGL(lds_roof_kernel<2>, dim3(grid), dim3(1024), 0, stream, rows, o); break;
      case 3: hipLaunchKernelGGL(lds_roof_kernel<3>, dim3(grid), dim3(1024), 0, stream, rows, o); break;
      default: hipLaunchKernelGGL(lds_roof_kernel<4>, dim3(grid), dim3(1024), 0, stream, rows, o); break;
    }
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
