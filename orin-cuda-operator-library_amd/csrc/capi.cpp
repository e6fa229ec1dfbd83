// Library-wide C ABI helpers (version and status text).
#include <hip/hip_runtime.h>

#include "operatorlib/operatorlib_c.h"

extern "C" int operatorlib_abi_version(void) { return OPERATORLIB_ABI_VERSION; }

extern "C" const char* operatorlib_status_string(int status) {
  return hipGetErrorString(static_cast<hipError_t>(status));
}
