// ABI version and error names of the C entry points.
#include "common.h"

extern "C" int dd_abi_version(void) { return DD_ABI_VERSION; }

extern "C" const char *dd_error_string(int code) {
  switch (code) {
    case DD_OK: return "ok";
    case DD_EINVAL: return "invalid argument";
    case DD_EUNSUPPORTED: return "unsupported shape or dtype";
    case DD_ELAUNCH: return "HIP kernel launch failed";
    case DD_ESCRATCH: return "scratch buffer too small";
    default: return "unknown error";
  }
}
