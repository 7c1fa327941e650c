// Library-wide entry points of libg16.so: ABI version and status strings.
#include "g16_common.hpp"

extern "C" int g16_abi_version(void) { return G16_ABI_VERSION; }

extern "C" const char* g16_strerror(int status) {
  switch (status) {
    case G16_OK: return "success";
    case G16_E_SHAPE: return "invalid shape: sizes must be >= 0 and K, N multiples of 8 (or bad threshold)";
    case G16_E_ALIGN: return "pointer not 16-byte aligned";
    case G16_E_NULL: return "required pointer is NULL";
    case G16_E_WORKSPACE: return "workspace missing or too small";
    case G16_E_SPLIT: return "ksplit out of range";
    case G16_E_DTYPE: return "unknown dtype code";
    case G16_E_TOO_LARGE: return "split does not fit the static scratch of the no-allocation entry point";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown g16 status";
}
