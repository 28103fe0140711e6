// Host-side plumbing shared by the C-ABI translation units: error reporting and checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>

#include "../../include/gdn_mi355x.h"

namespace gdn {

// Record a printf-style message as this thread's last error and return `code`.
int set_error(int code, const char* fmt, ...);
// Clear this thread's last error and return GDN_OK.
int clear_error();
// After a kernel launch: turn a pending HIP error into GDN_ELAUNCH.
int check_launch(const char* what);

inline bool aligned(const void* p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }

}  // namespace gdn

#define GDN_REQUIRE(cond, ...)                                  \
  do {                                                          \
    if (!(cond)) return ::gdn::set_error(GDN_EINVAL, __VA_ARGS__); \
  } while (0)
#define GDN_SUPPORT(cond, ...)                                  \
  do {                                                          \
    if (!(cond)) return ::gdn::set_error(GDN_EUNSUP, __VA_ARGS__); \
  } while (0)
