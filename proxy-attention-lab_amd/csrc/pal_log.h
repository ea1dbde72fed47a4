// Diagnostics shared by the host side of libpal_hip.so: the thread-local
// message of the last failed call (pal_last_error) and an opt-in log.
//
// The log is off unless the environment variable PAL_LOG is set to a
// non-empty value other than "0" when the library first checks it; then
// every entry point writes one line to stderr (the operation, its shapes,
// the launch configuration or the error).  Disabled, PAL_LOG costs one
// predictable branch per call.
#pragma once

#include <cstdarg>

namespace pal {

void set_last_error(const char* msg);
void clear_last_error();
const char* last_error();

bool log_enabled();
void log_write(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

}  // namespace pal

#define PAL_LOG(...)                                 \
  do {                                               \
    if (::pal::log_enabled()) ::pal::log_write(__VA_ARGS__); \
  } while (0)
