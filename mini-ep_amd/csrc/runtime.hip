// Host-side runtime helpers of the C ABI: the thread-local last-error
// message and per-device properties.
#include "common.h"

#include <atomic>

namespace mep {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

// Compute-unit count of the current device, looked up once per device and
// kept in a per-device slot (a value the device fixes, so concurrent first
// calls store the same number).  Devices past the table are queried on
// every call.
constexpr int kMaxDevices = 64;
static std::atomic<int> g_cu_count[kMaxDevices];

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < kMaxDevices) {
    const int cached = g_cu_count[dev].load(std::memory_order_relaxed);
    if (cached > 0) return cached;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev >= 0 && dev < kMaxDevices) g_cu_count[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace mep

extern "C" const char* mep_last_error(void) { return mep::g_last_error; }

extern "C" int mep_abi_version(void) { return 4; }
