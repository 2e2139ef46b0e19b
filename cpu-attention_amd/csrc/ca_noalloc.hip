// The split-K scratch of ca_decode_noalloc, in a source file of its own that holds
// no kernel: its device code object carries only this array, and HIP loads a code
// object (and reserves its device variables) on a device when something in it is
// first used there, here when decode_noalloc_scratch() first resolves the array
// on that device.  Processes that never call ca_decode_noalloc do not reserve it;
// those that do keep it on each GPU that ran such a call until the process ends.
#include <atomic>
#include <functional>
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
// Per device: an event recorded after the kernels of the last call that used the
// scratch there (none until the first such call), and the mutex that orders the
// calls' wait-launch-record sequences.
hipEvent_t g_last[kMaxDevices];
bool g_has_last[kMaxDevices];
std::mutex g_use_mu[kMaxDevices];
}  // namespace

// The current device's copy of `scratch`, looked up once per device (with that
// device current) and remembered, with the device's ordering event created at the
// same set-up.
int decode_noalloc_scratch(void** ptr, int* device) {
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
      e = hipEventCreateWithFlags(&g_last[dev], hipEventDisableTiming);
      if (e != hipSuccess) return CA_HIP_ERROR - (int)e;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  *device = dev;
  return CA_OK;
}

// Runs launch(), which enqueues the kernels of one call that uses `device`'s
// scratch on `stream`, after every earlier such call's kernels on that device:
// the stream first waits for the event recorded after the previous call (on
// whichever stream it ran), and the event is recorded again after this call.
// The host mutex keeps the wait, the launch and the record of one call together.
// A stream under graph capture neither waits nor records (an event recorded
// outside the capture cannot be waited on inside it): captured calls, and their
// replays, are ordered by the caller.
int decode_noalloc_ordered(int device, hipStream_t stream, const std::function<int()>& launch) {
  std::lock_guard<std::mutex> lock(g_use_mu[device]);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &cap);
  if (e != hipSuccess) return CA_HIP_ERROR - (int)e;
  const bool order = cap == hipStreamCaptureStatusNone;
  if (order && g_has_last[device]) {
    e = hipStreamWaitEvent(stream, g_last[device], 0);
    if (e != hipSuccess) return CA_HIP_ERROR - (int)e;
  }
  const int r = launch();
  if (r != CA_OK || !order) return r;
  e = hipEventRecord(g_last[device], stream);
  if (e != hipSuccess) return CA_HIP_ERROR - (int)e;
  g_has_last[device] = true;
  return CA_OK;
}

}  // namespace ca
