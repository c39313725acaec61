// Library-level entry points of libsmla.so.
#include "smla_internal.h"

extern "C" const char* smla_strerror(int status) {
  switch (status) {
    case SMLA_OK: return "ok";
    case SMLA_E_NULL: return "a required pointer is NULL";
    case SMLA_E_SHAPE: return "a size is non-positive or inconsistent";
    case SMLA_E_DTYPE: return "unsupported element type";
    case SMLA_E_UNSUPPORTED: return "unsupported combination of sizes or types";
    case SMLA_E_WORKSPACE: return "workspace missing or too small";
    case SMLA_E_RANGE: return "scalar argument out of range";
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown smla status";
}

extern "C" int smla_api_version(void) { return SMLA_API_VERSION; }
