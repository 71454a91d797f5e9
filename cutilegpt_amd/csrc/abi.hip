// Library-level entry points of the C ABI: version and status strings.
#include "common.h"

extern "C" int cgpt_version(void) { return CGPT_ABI_VERSION; }

extern "C" const char* cgpt_status_string(int status) {
  switch (status) {
    case CGPT_OK: return "ok";
    case CGPT_EINVAL: return "invalid argument (pointer, size, stride or alignment)";
    case CGPT_EDTYPE: return "unsupported dtype combination";
    case CGPT_ESHAPE: return "shape outside what the kernels support";
    case CGPT_ESCRATCH: return "problem needs more scratch memory than the static buffer holds";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}
