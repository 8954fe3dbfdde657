// Library-level pieces of the C ABI: version and per-thread error text.
#include <stdarg.h>
#include <stdio.h>

#include "odp_internal.h"

static thread_local char g_last_error[512] = "";

void odp_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int odp_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    odp_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return ODP_ERR_HIP;
  }
  return ODP_OK;
}

int odp_check_table(const char* what, const void* problems, const int32_t* work_start,
                    int32_t n_prob, int32_t total_blocks) {
  if (n_prob < 0 || total_blocks < 0) {
    odp_set_error("%s: negative n_prob (%d) or total_blocks (%d)", what, n_prob, total_blocks);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (n_prob > 0 && (problems == nullptr || work_start == nullptr)) {
    odp_set_error("%s: null problem table or work_start", what);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (n_prob == 0 && total_blocks != 0) {
    odp_set_error("%s: total_blocks must be 0 with no problems", what);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  return ODP_OK;
}

extern "C" int odp_abi_version(void) { return ODP_ABI_VERSION; }

extern "C" const char* odp_last_error(void) { return g_last_error; }
