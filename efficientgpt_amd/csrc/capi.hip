// Library-wide entry points of libegpt_hip.so: ABI version and status strings.
#include "common.h"

extern "C" int egpt_abi_version(void) { return 1; }

extern "C" const char* egpt_status_string(int status) {
  switch (status) {
    case EGPT_OK: return "ok";
    case EGPT_ERR_INVALID: return "invalid argument (pointer, size, stride or alignment)";
    case EGPT_ERR_UNSUPPORTED: return "unsupported shape or dtype";
    case EGPT_ERR_LAUNCH: return "HIP kernel launch failed";
    case EGPT_ERR_WORKSPACE: return "workspace missing or too small";
    default: return "unknown status";
  }
}
