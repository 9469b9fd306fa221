// fagq_device.hip - the per-device gfx950 check shared by the library's
// entry points (libfagq.so) and the measurement probes (libfagq_probe.so).
#include <atomic>
#include <cstring>

#include "fagq.h"
#include "fagq_dispatch.hpp"

namespace fagq {
namespace {
constexpr int kMaxDevices = 64;
}  // namespace

// gfx950 check, done once per device.  The launch-failure test build has no
// device to check.
int device_check() {
#ifdef FAGQ_TEST_LAUNCH_FAILURE
  return FAGQ_OK;
#endif
  static std::atomic<int> cache[kMaxDevices];   // 0 unknown, 1 gfx950, 2 other
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(int)e;
  if (dev < 0 || dev >= kMaxDevices) return FAGQ_E_DEVICE;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return -(int)e;
    c = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
    cache[dev].store(c, std::memory_order_relaxed);
  }
  return c == 1 ? FAGQ_OK : FAGQ_E_DEVICE;
}

}  // namespace fagq
