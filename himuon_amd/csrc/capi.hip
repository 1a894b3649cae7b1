// Library-level C ABI entry points (version, error strings).
#include "common.h"

extern "C" int himuon_abi_version(void) { return HIMUON_ABI_VERSION; }

extern "C" const char* himuon_error_string(int code) {
  if (code == 0) return "success";
  if (code == HIMUON_EINVAL) return "himuon: invalid argument (shape, dtype, pointer or geometry)";
  if (code == HIMUON_ENOSPC) return "himuon: workspace too small";
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "himuon: unknown error";
}
