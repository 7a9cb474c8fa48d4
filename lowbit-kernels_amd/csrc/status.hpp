// Status codes and the per-thread message of the last failure (lowbit_last_error()).
#pragma once
#include <cstdarg>
#include <cstdio>

namespace lowbit {

char* error_buffer();   // thread-local, 512 bytes

// record a formatted message for the calling thread and return `code`
inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(error_buffer(), 512, fmt, ap);
  va_end(ap);
  return code;
}

inline int ok() {
  error_buffer()[0] = '\0';
  return 0;
}

}  // namespace lowbit
