// Fixed device scratch for the entry points that allocate nothing
// (rvc_conv1d_noalloc): callers under HIP graph capture, in tight serving
// loops or in harnesses that forbid hipMalloc.
//
// `scratch` is a file-scope device array, one copy per GPU that loads this
// library, held until the process ends.  Host code never passes its name to
// a kernel: its device address is looked up once per device, with that
// device current, when an engine is created (noalloc_setup), and every use
// goes through that address.  Every call on one GPU shares that GPU's
// array and it keeps the last call's contents; calls that overlap on one
// GPU (two engines' streams at once) race on it.
#include <mutex>

#include "internal.h"

namespace rvc {

__device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
float* g_ptr[kMaxDevices] = {};
}  // namespace

void noalloc_setup(int device) {
  RVC_CHECK(device >= 0 && device < kMaxDevices, "noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ptr[device]) return;
  int cur = -1;
  RVC_HIP(hipGetDevice(&cur));
  RVC_CHECK(cur == device, "noalloc: setup must run with its device current");
  void* p = nullptr;
  RVC_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  RVC_CHECK(p != nullptr && (reinterpret_cast<uintptr_t>(p) & 255) == 0, "noalloc: scratch address not aligned");
  g_ptr[device] = static_cast<float*>(p);
}

float* noalloc_scratch(int device) {
  RVC_CHECK(device >= 0 && device < kMaxDevices, "noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(g_mu);
  RVC_CHECK(g_ptr[device] != nullptr, "noalloc: scratch of this device was not set up");
  return g_ptr[device];
}

}  // namespace rvc
