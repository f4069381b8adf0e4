// Error reporting, ABI version and device queries shared by every entry point.
#include <cstdarg>
#include <mutex>

#include "common.h"

namespace pmsst {

namespace {
thread_local std::string g_last_error;
constexpr int kMaxDevices = 64;
int g_cus[kMaxDevices] = {0};
std::mutex g_cus_mutex;
}  // namespace

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* kernel) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(PMSST_ELAUNCH, "%s: launch failed: %s", kernel, hipGetErrorString(err));
  }
  return PMSST_OK;
}

// Compute units of the current device (cached per device ordinal).
int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::lock_guard<std::mutex> lock(g_cus_mutex);
  if (g_cus[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
      cus = 256;
    }
    g_cus[dev] = cus;
  }
  return g_cus[dev];
}

}  // namespace pmsst

extern "C" {

const char* pmsst_last_error(void) { return pmsst::g_last_error.c_str(); }

int pmsst_abi_version(void) { return 6; }

}  // extern "C"
