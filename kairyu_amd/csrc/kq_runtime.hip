// Host-side runtime pieces of the C ABI: error reporting, version, device
// probe.  No kernels here.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "kq_common.h"

namespace kq {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return KQ_ELAUNCH;
  }
  return KQ_OK;
}

}  // namespace kq

extern "C" int kq_version(void) { return 100; }

extern "C" const char* kq_last_error(void) { return kq::g_last_error.c_str(); }

extern "C" int kq_device_supported(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
    kq::set_error("hipGetDeviceProperties(%d) failed", device);
    return 0;
  }
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}
