// The per-thread message of the last failure and the status names (lowbit_last_error, lowbit_strerror). Host code
// only: linked into liblowbit_w4.so and into the HIP-free liblowbit_format.so (the host format functions alone).
#include "lowbit_w4.h"
#include "status.hpp"

namespace lowbit {

char* error_buffer() {
  static thread_local char buf[512];
  return buf;
}

}  // namespace lowbit

extern "C" {

const char* lowbit_last_error(void) { return lowbit::error_buffer(); }

const char* lowbit_strerror(int status) {
  switch (status) {
    case LOWBIT_OK: return "ok";
    case LOWBIT_ERR_ARG: return "invalid argument";
    case LOWBIT_ERR_GROUP: return "invalid group size";
    case LOWBIT_ERR_SHAPE: return "shape mismatch";
    case LOWBIT_ERR_ALIGN: return "misaligned pointer";
    case LOWBIT_ERR_ROWS: return "row count out of range";
    case LOWBIT_ERR_VERSION: return "unknown kernel version";
    case LOWBIT_ERR_LAYOUT: return "layout needs K and G multiples of 128";
    case LOWBIT_ERR_TUNING: return "invalid tuning knob";
    case LOWBIT_ERR_HIP: return "HIP error";
    case LOWBIT_ERR_DEVICE: return "unsupported device";
    default: return "unknown status";
  }
}

}  // extern "C"
