// Library-wide status reporting and version for the fastkernels_amd C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "fk_common.h"

namespace fk {

namespace {
thread_local char g_last_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

// Reports a failed launch (bad configuration, no device, ...) as its hipError_t.
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(static_cast<int>(e), "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return FK_OK;
}

int num_cus() {
  static int cached[64] = {};  // per device; 0 = not yet queried
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;  // MI355X
  }
  if (cached[dev] == 0) {
    hipDeviceProp_t prop;
    int n = 256;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0)
      n = prop.multiProcessorCount;
    (void)hipGetLastError();
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace fk

// 2.0.0: fk_paged_prefill / fk_varlen_prefill gained head_size_v, lse and
// lse_row_stride (1.x had max_seqlen_k added in the middle of both signatures).
// 2.1.0: fk_prefill_split_plan, fk_paged_prefill_ws and fk_varlen_prefill_ws added.
extern "C" int fk_version(void) { return FK_VERSION_MAJOR * 10000 + FK_VERSION_MINOR * 100; }

extern "C" const char* fk_last_error(void) { return fk::g_last_error; }
