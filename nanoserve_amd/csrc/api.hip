// Error reporting and version of libnanoserve_hip.so.
#include "ns_common.h"

namespace ns {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

// Called right after a launch: a launch failure (bad grid, missing code object for this GPU) is
// reported here; faults inside the kernel surface at the caller's next synchronisation.
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return NS_E_HIP_BASE + int(e);
  }
  return NS_OK;
}

}  // namespace ns

extern "C" const char* ns_last_error(void) { return ns::g_err; }

extern "C" const char* ns_version(void) { return "nanoserve_hip gfx950 r1"; }
