// Allocation cache for the booster's training buffers (see dp_internal.hpp).
//
// Blocks are kept by (device, exact size in 256-byte units).  At most
// kCachedBytes per kind stay cached and blocks above kLargestBlock are never
// cached, so a process that trains many boosters of one configuration reuses
// the same blocks while one-off large buffers still go back to the driver.
// The cache lives until the process ends (no destructor runs at exit, when
// the runtime may already be gone).
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "dp_internal.hpp"

namespace dp {
namespace {

constexpr size_t kCachedBytes = size_t(16) << 30;
constexpr size_t kLargestBlock = size_t(4) << 30;

struct Cache {
  std::mutex m;
  std::map<std::pair<int, size_t>, std::vector<void*>> blocks;
  size_t cached = 0;
};

Cache& device_cache() {
  static Cache* c = new Cache();  // never destroyed
  return *c;
}

Cache& pinned_cache() {
  static Cache* c = new Cache();  // never destroyed
  return *c;
}

size_t rounded(size_t bytes) { return (bytes + 255) & ~size_t(255); }

int current_device() {
  int d = 0;
  DP_HIP(hipGetDevice(&d));
  return d;
}

void* take(Cache& c, int dev, size_t bytes) {
  std::lock_guard<std::mutex> lock(c.m);
  auto it = c.blocks.find({dev, bytes});
  if (it == c.blocks.end() || it->second.empty()) return nullptr;
  void* p = it->second.back();
  it->second.pop_back();
  c.cached -= bytes;
  return p;
}

// Hands every cached block of `dev` back to the driver.
void drain(Cache& c, int dev, bool pinned) {
  std::lock_guard<std::mutex> lock(c.m);
  for (auto it = c.blocks.begin(); it != c.blocks.end();) {
    if (it->first.first != dev) {
      ++it;
      continue;
    }
    for (void* p : it->second) {
      if (pinned) (void)hipHostFree(p);
      else (void)hipFree(p);
      c.cached -= it->first.second;
    }
    it = c.blocks.erase(it);
  }
}

void give(Cache& c, int dev, void* p, size_t bytes, bool pinned) {
  {
    std::lock_guard<std::mutex> lock(c.m);
    if (bytes <= kLargestBlock && c.cached + bytes <= kCachedBytes) {
      c.blocks[{dev, bytes}].push_back(p);
      c.cached += bytes;
      return;
    }
  }
  if (pinned) (void)hipHostFree(p);
  else (void)hipFree(p);
}

}  // namespace

void* device_pool_get(size_t bytes, int* device) {
  bytes = rounded(bytes);
  const int dev = current_device();
  *device = dev;
  if (void* p = take(device_cache(), dev, bytes)) return p;
  void* p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    drain(device_cache(), dev, false);
    DP_HIP(hipMalloc(&p, bytes));
  }
  return p;
}

void device_pool_put(void* p, size_t bytes, int device) {
  if (!p) return;
  give(device_cache(), device, p, rounded(bytes), false);
}

void* pinned_pool_get(size_t bytes) {
  bytes = rounded(bytes);
  if (void* p = take(pinned_cache(), -1, bytes)) return p;
  void* p = nullptr;
  if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
    (void)hipGetLastError();
    drain(pinned_cache(), -1, true);
    DP_HIP(hipHostMalloc(&p, bytes, hipHostMallocDefault));
  }
  return p;
}

void pinned_pool_put(void* p, size_t bytes) {
  if (!p) return;
  give(pinned_cache(), -1, p, rounded(bytes), true);
}

}  // namespace dp
