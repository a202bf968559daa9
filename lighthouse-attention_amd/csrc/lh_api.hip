// Library-level entry points of liblighthouse_hip.so.
#include "lh_common.h"

extern "C" const char* lh_strerror(int rc) {
  switch (rc) {
    case LH_OK: return "ok";
    case LH_ERR_INVALID_ARG: return "invalid argument (size, pointer, stride or alignment)";
    case LH_ERR_DOMAIN: return "geometry outside the reference selection kernel's domain (strict mode)";
    case LH_ERR_LAUNCH: return "HIP kernel launch failed";
    case LH_ERR_UNSUPPORTED: return "shape beyond this build's limits";
    case LH_ERR_RUNTIME: return "a HIP runtime call failed";
    default: return "unknown error";
  }
}

extern "C" int lh_abi_version(void) { return LH_ABI_VERSION; }
