// Last-error string and the PAL_LOG stderr log (see pal_log.h).
#include "pal_log.h"

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

namespace pal {

namespace {

thread_local std::string g_last_error;

// 0: not checked yet, 1: off, 2: on
std::atomic<int> g_log_state{0};

}  // namespace

void set_last_error(const char* msg) {
  g_last_error = msg ? msg : "";
  PAL_LOG("error: %s", g_last_error.c_str());
}

void clear_last_error() { g_last_error.clear(); }

const char* last_error() { return g_last_error.c_str(); }

bool log_enabled() {
  int s = g_log_state.load(std::memory_order_relaxed);
  if (s == 0) {
    const char* v = std::getenv("PAL_LOG");
    s = (v && *v && std::strcmp(v, "0") != 0) ? 2 : 1;
    g_log_state.store(s, std::memory_order_relaxed);
  }
  return s == 2;
}

void log_write(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  std::fprintf(stderr, "[pal] %s\n", buf);
}

}  // namespace pal
