// Library-wide runtime helpers: version and thread-local error messages.
#include "common.h"

#include <string.h>

namespace ssla {

static thread_local char g_last_error[512];

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

hipError_t read_to_host(void *dst, const void *src, size_t bytes, hipStream_t st) {
  constexpr size_t kStage = 4096;
  // one pinned buffer per host thread, kept until the process ends
  static thread_local void *stage = nullptr;
  if (bytes > kStage) return hipErrorInvalidValue;
  if (stage == nullptr) {
    void *p = nullptr;
    const hipError_t e = hipHostMalloc(&p, kStage, hipHostMallocDefault);
    if (e != hipSuccess) return e;
    stage = p;
  }
  hipError_t e = hipMemcpyAsync(stage, src, bytes, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e == hipSuccess) memcpy(dst, stage, bytes);
  return e;
}

}  // namespace ssla

extern "C" int ssla_version(void) { return 100; }

extern "C" const char *ssla_last_error(void) { return ssla::g_last_error; }

extern "C" int ssla_status_read(const int32_t *status, int *value_out, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(status && value_out, "status_read: null pointer");
  int32_t v = 0;
  const hipError_t e = read_to_host(&v, status, sizeof(v), static_cast<hipStream_t>(stream));
  if (e != hipSuccess) {
    set_error("status_read: %s", hipGetErrorString(e));
    return SSLA_ERR_LAUNCH;
  }
  *value_out = v;
  return SSLA_OK;
}
