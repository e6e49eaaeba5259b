// Error state of the dionw C ABI: one message per calling thread.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

namespace dionw {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buf, sizeof(buf), fmt, args);
  va_end(args);
  g_last_error = buf;
}

int check_launch(const char* what) {
  const hipError_t rc = hipGetLastError();
  if (rc != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(rc));
    return 2;
  }
  return 0;
}

}  // namespace dionw

extern "C" {

const char* dionw_last_error(void) { return dionw::g_last_error.c_str(); }

int dionw_abi_version(void) { return 2; }

}  // extern "C"
