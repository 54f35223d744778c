// Library-level C-ABI helpers: version and status strings.
#include "mpk_common.h"

extern "C" int mpk_version(void) { return 1; }

extern "C" const char* mpk_status_string(int status) {
  switch (status) {
    case MPK_OK: return "success";
    case MPK_EINVAL: return "invalid argument (null pointer, negative size or unknown dtype)";
    case MPK_EUNSUPPORTED: return "unsupported shape or variant for the gfx950 kernels";
    case MPK_EALIGN: return "pointer or stride is not 16-byte aligned";
    default: return hipGetErrorString(static_cast<hipError_t>(status));
  }
}

// Device synchronisation helper for callers that do not link the HIP runtime
// themselves (returns the hipError_t of hipDeviceSynchronize as int).
extern "C" int mpk_device_synchronize(void) { return (int)hipDeviceSynchronize(); }
