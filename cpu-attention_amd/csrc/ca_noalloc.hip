// The split-K scratch of ca_decode_noalloc, in a source file of its own that holds
// no kernel: its device code object carries only this array, and HIP loads a code
// object (and reserves its device variables) on a device when something in it is
// first used there, here when decode_noalloc_scratch() first resolves the array
// on that device.  Processes that never call ca_decode_noalloc do not reserve it;
// those that do keep it on each GPU that ran such a call until the process ends.
#include <atomic>
#include <mutex>

#include "ca_device.h"
#include "ca_internal.h"

// A fixed array in device memory, one copy per GPU.  Host code never names it as
// a kernel argument or copy target (on the host the name is only a stand-in for
// the symbol): decode_noalloc_scratch() resolves its device address per GPU, and
// that address is what the decode kernels get.
static __device__ __align__(256) unsigned char scratch[CA_DECODE_NOALLOC_SCRATCH_BYTES];

namespace ca {

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;
}  // namespace

// The current device's copy of `scratch`, looked up once per device (with that
// device current) and remembered.
int decode_noalloc_scratch(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return CA_HIP_ERROR - (int)e;
  if (dev < 0 || dev >= kMaxDevices) return CA_DECLINED;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return CA_HIP_ERROR - (int)e;
      if (!p) return CA_HIP_ERROR;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return CA_OK;
}

}  // namespace ca
