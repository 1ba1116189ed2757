// Library-level C ABI: version and error strings.
#include "common.hpp"

extern "C" const char* umic_version(void) { return "umic-hip 0.1.0 gfx950"; }

extern "C" const char* umic_error_string(int code) {
  switch (code) {
    case UMIC_OK: return "success";
    case UMIC_ERR_INVALID_ARG: return "invalid argument (null pointer, negative size or bad enum)";
    case UMIC_ERR_UNSUPPORTED: return "unsupported shape, stride or alignment";
    case UMIC_ERR_SCRATCH:
      return "shape needs more stream-K scratch than the library's static 64 MiB";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown umic error";
}
