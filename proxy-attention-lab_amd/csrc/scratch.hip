// Library-held scratch memory for the no-allocation entry point
// (pal_paged_attention_decode_noalloc): a file-scope device array, one copy
// per GPU the library runs on, held until the process ends.
//
// In host code `scratch` names a host-side stand-in, not device memory: its
// device address (different on every GPU) is read once per device with
// hipGetSymbolAddress, with that device current, and kept here; host code
// only ever hands out that address.
#include <mutex>

#include "pal_device.h"

namespace pal {

namespace {

__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

}  // namespace

hipError_t scratch_buffer(void** ptr) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return err;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[dev] = p;
  }
  *ptr = g_ptr[dev];
  return hipSuccess;
}

}  // namespace pal
