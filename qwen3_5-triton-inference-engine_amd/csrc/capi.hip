// Status strings and build information of the C ABI.
#include "wy_common.h"

extern "C" const char *wy_status_string(int code) {
  switch (code) {
    case WY_OK: return "success";
    case WY_E_NULL: return "a required pointer argument is NULL";
    case WY_E_SHAPE: return "a size argument is out of range";
    case WY_E_LAYOUT: return "a stride or alignment the kernel cannot address";
    case WY_E_UNSUPPORTED:
      return "no kernel for this head_dim / group size (built for head_dim 256, 4 query heads per KV head)";
    case WY_E_CAPACITY:
      return "the problem exceeds the fixed capacity of this entry point's static scratch";
    default:
      return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown error";
  }
}

extern "C" const char *wy_build_info(void) { return "wy_attn 0.1 gfx950"; }
