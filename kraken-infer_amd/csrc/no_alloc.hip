// The static device scratch behind the allocation-free attention entry point
// (kraken_hip_attention_f32_batched_f16_kv_gated_no_alloc).  Each GPU the
// library runs on holds one copy of `scratch` from code-object load until the
// process ends; its device address is looked up once per device, with that
// device current, when the first context on it is created, and only that
// address is ever handed to kernels or copies.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "context_internal.hpp"

namespace kraken {
namespace {

// In host code this name is only a stand-in for the device symbol, never an
// address: everything below goes through the pointer hipGetSymbolAddress
// returns for the current device.
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

int resolve_no_alloc_scratch(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) {
    return unavailable("HIP backend: device index " + std::to_string(device) +
                       " is past the allocation-free scratch table");
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      return unavailable(std::string("HIP backend: cannot resolve the allocation-free scratch "
                                     "array on device ") +
                         std::to_string(device) + ": " + hipGetErrorString(e));
    }
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return KRAKEN_OK;
}

}  // namespace kraken
