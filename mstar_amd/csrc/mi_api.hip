// Library-level C entry points: status text and ABI version.
#include "mi_common.h"

extern "C" const char* mi_status_string(int status) {
  switch (status) {
    case MI_OK: return "ok";
    case MI_ERR_INVALID: return "invalid argument";
    case MI_ERR_UNSUPPORTED: return "unsupported configuration";
    case MI_ERR_WORKSPACE: return "workspace too small or not planned";
    case MI_ERR_LAUNCH: return "HIP kernel launch failed";
    default: return "unknown status";
  }
}

extern "C" int mi_abi_version(void) { return MI_ABI_VERSION; }
