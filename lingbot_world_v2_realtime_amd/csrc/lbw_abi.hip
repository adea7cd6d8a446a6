// Status strings and version of the C-ABI.
#include <atomic>
#include <cstring>

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
    case LBW_E_SCRATCH: return "problem exceeds the fixed scratch array";
    default: return "unknown status";
  }
}

extern "C" int lbw_version(void) { return 100; }

namespace lbw {

// LBW_OK when the current device is a gfx950 (the only target the code objects are built for), else
// LBW_E_DEVICE; the answer is cached per device ordinal. Entry points may run on several host threads at once:
// the cache is atomic (every thread that misses computes and stores the same value).
int check_device() {
  static std::atomic<int> cached[64];   // 0 unknown, 1 gfx950, 2 other (static storage: zero-initialised)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return LBW_E_DEVICE;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return LBW_E_DEVICE;
    v = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v == 1 ? LBW_OK : LBW_E_DEVICE;
}

}  // namespace lbw
