// Error text for the extern "C" entry points: each returns QX_OK (0),
// QX_EINVAL (-1) after recording a message here, or a positive hipError_t.
#pragma once

#ifndef QX_OK
#define QX_OK 0
#define QX_EINVAL (-1)
#endif

// The ABI version qx_version() reports; equal to QX_ABI_VERSION of
// include/quail_mi355x.h (a CPU test compares the two).
#define QX_LIBRARY_ABI_VERSION 2

namespace qx {
void set_error(const char* fmt, ...);
}

#define QX_CHECK(cond, ...)        \
  do {                             \
    if (!(cond)) {                 \
      qx::set_error(__VA_ARGS__);  \
      return QX_EINVAL;            \
    }                              \
  } while (0)
