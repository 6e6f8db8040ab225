// Error reporting and launch checks shared by every entry point.
#include "common.h"

#include <string>

namespace qv {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return QV_EHIP;
  }
  return QV_OK;
}

}  // namespace qv

extern "C" const char* qv_last_error(void) { return qv::g_last_error.c_str(); }

extern "C" const char* qv_version(void) { return "qvggt_hip 0.1 (gfx950)"; }
