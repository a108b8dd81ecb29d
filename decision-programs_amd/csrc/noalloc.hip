// Device memory for the entry points that allocate nothing.
//
// dp_evaluate_splits_noalloc (c_api.cpp) keeps its per-(node, feature)
// candidates in the file-scope array below instead of a workspace, so a
// caller that cannot allocate (code under HIP graph capture, a serving loop
// that forbids hipMalloc) can run the split evaluation.  Each GPU the library
// runs on holds its own copy of the array until the process ends.  In host
// code the array's name is only a host-side stand-in: its device address is
// looked up once per device with hipGetSymbolAddress and only that address is
// passed to kernels.
//
// Every call on one GPU shares that GPU's array, and each call overwrites the
// entries it reads (the evaluation writes the candidate of every (node,
// feature) before the selection reads it), so nothing needs clearing between
// calls.  Calls that overlap on one GPU (two streams, two threads) race on it.
#include <mutex>

#include "dp_internal.hpp"

namespace dp {
namespace {

constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_lock;
void* g_address[kMaxDevices] = {};

}  // namespace

void* noalloc_scratch(size_t bytes) {
  need(bytes <= kNoAllocScratchBytes,
       "request of " + std::to_string(bytes) + " scratch bytes exceeds the " +
           std::to_string(kNoAllocScratchBytes) + "-byte device array of the no-allocation entry "
           "points");
  int device = 0;
  DP_HIP(hipGetDevice(&device));
  need(device >= 0 && device < kMaxDevices, "device ordinal beyond the no-allocation table");
  std::lock_guard<std::mutex> hold(g_lock);
  if (!g_address[device]) {
    void* p = nullptr;
    DP_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    need(p != nullptr, "hipGetSymbolAddress returned no address for the scratch array");
    g_address[device] = p;
  }
  return g_address[device];
}

}  // namespace dp
