// Thread-local error state shared by every entry point of the library.
#include <cstdarg>
#include <cstring>

#include "common.h"

namespace kessie {

namespace {
thread_local int g_status = KESSIE_OK;
thread_local char g_message[512] = {0};
}  // namespace

void set_error(int code, const char* fmt, ...) {
  g_status = code;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_message, sizeof(g_message), fmt, ap);
  va_end(ap);
}

void clear_error() {
  g_status = KESSIE_OK;
  g_message[0] = '\0';
}

int last_status() { return g_status; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(KESSIE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return KESSIE_ERR_HIP;
  }
  return KESSIE_OK;
}

}  // namespace kessie

extern "C" int kessie_get_last_error(char* buf, size_t cap) {
  if (buf != nullptr && cap > 0) {
    strncpy(buf, kessie::g_message, cap - 1);
    buf[cap - 1] = '\0';
  }
  return kessie::g_status;
}

extern "C" int kessie_version(void) { return 100; }
