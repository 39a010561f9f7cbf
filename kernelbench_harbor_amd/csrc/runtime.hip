// Library-wide C-ABI helpers: version, status strings, launch error capture.
#include <atomic>

#include "kbh_common.h"

namespace kbh {

static std::atomic<int> g_last_hip_error{0};

void set_last_hip_error(int e) { g_last_hip_error.store(e, std::memory_order_relaxed); }

int launch_status() {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return KBH_OK;
  set_last_hip_error((int)e);
  return KBH_ERR_LAUNCH;
}

}  // namespace kbh

extern "C" int kbh_abi_version(void) { return KBH_ABI_VERSION; }

extern "C" int kbh_last_hip_error(void) { return kbh::g_last_hip_error.load(std::memory_order_relaxed); }

extern "C" const char* kbh_status_string(int status) {
  switch (status) {
    case KBH_OK: return "ok";
    case KBH_ERR_NULL: return "a required pointer is NULL";
    case KBH_ERR_SHAPE: return "shape not supported";
    case KBH_ERR_DTYPE: return "dtype not supported";
    case KBH_ERR_WORKSPACE: return "workspace missing or too small";
    case KBH_ERR_ALIGN: return "pointer not 16-byte aligned";
    case KBH_ERR_LAUNCH: return "kernel launch failed";
    case KBH_ERR_SCRATCH_LIMIT:
      return "the call needs more than the library's fixed scratch (use the workspace entry point)";
    default: return "unknown status";
  }
}
