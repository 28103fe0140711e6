// Library-wide C-ABI entry points: version, error string, limits.
#include <stdio.h>
#include <string.h>

#include "gdn_internal.h"

namespace gdn {

static thread_local char g_err[512] = {0};

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int clear_error() {
  g_err[0] = 0;
  return GDN_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(GDN_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return GDN_OK;
}

}  // namespace gdn

extern "C" int gdn_version(void) { return 100; }

extern "C" const char* gdn_last_error(void) { return gdn::g_err; }

extern "C" int gdn_limits(int* head_dim, int* max_group_ratio, int* max_conv_kernel) {
  if (head_dim) *head_dim = 128;
  if (max_group_ratio) *max_group_ratio = 4;
  if (max_conv_kernel) *max_conv_kernel = 8;
  return GDN_OK;
}
