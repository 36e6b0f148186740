// C-ABI plumbing shared by every entry point: the per-thread error message,
// the ABI version and the gfx950 device check.
#include <stdarg.h>
#include <stdio.h>

#include "dsa_common.hpp"

namespace dsa {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DSA_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return DSA_OK;
}

}  // namespace dsa

extern "C" const char *dsa_last_error(void) { return dsa::g_last_error; }

extern "C" int dsa_abi_version(void) { return 100; }

extern "C" int dsa_device_check(int device) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess)
    return dsa::set_error(DSA_ERR_HIP, "hipGetDeviceProperties(%d): %s", device, hipGetErrorString(e));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return dsa::set_error(DSA_ERR_UNSUPPORTED,
                          "device %d is %s; this library is built for gfx950 (MI355X) only",
                          device, prop.gcnArchName);
  return DSA_OK;
}
