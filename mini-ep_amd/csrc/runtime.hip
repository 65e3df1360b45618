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

static std::atomic<int> g_giveup_site{0}, g_giveup_polls{0};

GiveupTest giveup_test() {
  return GiveupTest{g_giveup_site.load(std::memory_order_relaxed), g_giveup_polls.load(std::memory_order_relaxed)};
}

}  // namespace mep

extern "C" int mep_test_force_giveup(int32_t site, int32_t polls) {
  mep::clear_error();
  MEP_REQUIRE(site >= MEP_GIVEUP_NONE && site <= MEP_GIVEUP_ROUTED, MEP_ERR_INVALID_ARG,
              "mep_test_force_giveup: unknown site %d", site);
  MEP_REQUIRE(site == MEP_GIVEUP_NONE || polls > 0, MEP_ERR_INVALID_ARG,
              "mep_test_force_giveup: polls must be positive (got %d)", polls);
  mep::g_giveup_polls.store(site == MEP_GIVEUP_NONE ? 0 : polls, std::memory_order_relaxed);
  mep::g_giveup_site.store(site, std::memory_order_relaxed);
  return MEP_OK;
}

extern "C" const char* mep_last_error(void) { return mep::g_last_error; }

extern "C" int mep_abi_version(void) { return 5; }
