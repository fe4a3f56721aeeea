// Library identity and status strings.
#include "common.h"

extern "C" int akas_version(void) { return 100; }  // 0.1.0

extern "C" const char* akas_status_string(int status) {
  switch (status) {
    case AKAS_OK: return "ok";
    case AKAS_ERR_GEOMETRY: return "invalid geometry";
    case AKAS_ERR_NULL: return "null pointer";
    case AKAS_ERR_DTYPE: return "unsupported dtype";
    case AKAS_ERR_LAUNCH: return "kernel launch failed";
    case AKAS_ERR_WORKSPACE: return "workspace missing or too small";
    case AKAS_ERR_SCRATCH: return "problem larger than the static scratch (AKAS_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown status";
  }
}

// Entry points declared in include/akas_fp8.h (kept in step by the ABI test).
extern "C" int akas_abi_count(void) { return 33; }
