// Library-wide C ABI helpers: status text, HIP error capture, version.
#include <hip/hip_runtime.h>

#include <atomic>

#include "../../include/twilight_hip.h"

namespace tw_host {

static std::atomic<int> g_last_hip_error{0};

int record_hip_error(hipError_t err) {
  g_last_hip_error.store(static_cast<int>(err));
  return TW_EHIP;
}

int check_launch() {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return record_hip_error(err);
  return TW_OK;
}

bool device_memory(const void* p) {
  hipPointerAttribute_t attr;
  if (p == nullptr || hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();  // an unknown pointer is not an error of the launch that follows
    return false;
  }
  return attr.type == hipMemoryTypeDevice;
}

}  // namespace tw_host

extern "C" const char* tw_status_string(int status) {
  switch (status) {
    case TW_OK: return "ok";
    case TW_EINVAL: return "invalid argument (shape, dtype, pointer or flag)";
    case TW_ERANGE: return "index out of range";
    case TW_ENOMEM: return "workspace too small";
    case TW_EHIP: return "HIP runtime error";
    case TW_EUNSUPPORTED: return "unsupported configuration";
    default: return "unknown status";
  }
}

extern "C" int tw_last_hip_error(void) { return tw_host::g_last_hip_error.load(); }

extern "C" int tw_version(void) { return (0 << 16) | 1; }
