// Library-wide entry points: version, error text, device check.
#include <stdarg.h>
#include <stdio.h>

#include "qx_common.h"
#include "qx_status.h"

namespace qx {
static thread_local char g_error[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}
}  // namespace qx

extern "C" {

int qx_version(void) { return QX_LIBRARY_ABI_VERSION; }

const char* qx_last_error(void) { return qx::g_error; }

// 1 when the current device is a gfx950 (MI350/MI355X), 0 otherwise, or a
// negative hipError_t when no device can be queried.
int qx_device_is_gfx950(void) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(int)e;
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return -(int)e;
  const char* arch = prop.gcnArchName;
  return (arch[0] == 'g' && arch[1] == 'f' && arch[2] == 'x' && arch[3] == '9' &&
          arch[4] == '5' && arch[5] == '0')
             ? 1
             : 0;
}

}  // extern "C"
