// Library-level entry points: version, error reporting, device admission.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "mx_common.h"

namespace mxl {
static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}
}  // namespace mxl

#define MXL_VERSION 1

extern "C" int mxl_version(void) { return MXL_VERSION; }

extern "C" const char* mxl_last_error(void) { return mxl::g_error; }

// Returns 1 when `device` is a gfx950 (MI355X class) GPU, 0 otherwise, and
// a negative code when the HIP runtime cannot be queried.
extern "C" int mxl_device_supported(int device) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) {
    mxl::set_error("hipGetDeviceProperties(%d): %s", device, hipGetErrorString(e));
    return MXL_EHIP;
  }
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}
