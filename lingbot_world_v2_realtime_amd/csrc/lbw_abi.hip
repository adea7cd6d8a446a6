// Status strings and version of the C-ABI.
#include "lbw_common.h"

extern "C" const char* lbw_status_string(int status) {
  switch (status) {
    case LBW_OK: return "ok";
    case LBW_E_NULL: return "null pointer";
    case LBW_E_SHAPE: return "bad shape";
    case LBW_E_ALIGN: return "misaligned pointer or stride";
    case LBW_E_DEVICE: return "device is not gfx950";
    case LBW_E_LAUNCH: return "kernel launch failed";
    case LBW_E_SEGMENTS: return "bad chunk table";
    default: return "unknown status";
  }
}

extern "C" int lbw_version(void) { return 100; }
