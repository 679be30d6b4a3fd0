// Library-wide host helpers: error state, version, launch checks.
#include "fg_common.h"

namespace fg {

static thread_local std::string g_error;

void set_error(const std::string& msg) { g_error = msg; }

int fail(const std::string& msg) {
  g_error = msg;
  return -1;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_error = std::string(what) + ": " + hipGetErrorString(e);
    return -2;
  }
  return 0;
}

}  // namespace fg

extern "C" {

const char* fg_last_error(void) { return fg::g_error.c_str(); }

int fg_version(void) { return 1; }

}  // extern "C"
