// Library-level entry points: version, thread-local error string, and the
// small device-memory helpers that let a ctypes caller drive the library
// without any other GPU runtime.
#include <cstdarg>
#include <cstdio>

#include "tq_internal.h"

namespace tq {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

}  // namespace tq

extern "C" {

int tq_version(void) { return 100; /* 0.1.0 */ }

const char* tq_last_error(void) { return tq::g_last_error.c_str(); }

int tq_device_count(int* count) {
  TQ_CHECK_ARG(count != nullptr, "tq_device_count: count is NULL");
  TQ_CHECK_HIP(hipGetDeviceCount(count));
  return TQ_OK;
}

int tq_set_device(int device) {
  TQ_CHECK_HIP(hipSetDevice(device));
  return TQ_OK;
}

int tq_malloc(void** ptr, size_t bytes) {
  TQ_CHECK_ARG(ptr != nullptr, "tq_malloc: ptr is NULL");
  TQ_CHECK_HIP(hipMalloc(ptr, bytes > 0 ? bytes : 1));
  return TQ_OK;
}

int tq_free(void* ptr) {
  if (ptr) TQ_CHECK_HIP(hipFree(ptr));
  return TQ_OK;
}

int tq_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  TQ_CHECK_ARG(dst && src, "tq_memcpy_h2d: null pointer");
  TQ_CHECK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return TQ_OK;
}

int tq_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  TQ_CHECK_ARG(dst && src, "tq_memcpy_d2h: null pointer");
  TQ_CHECK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return TQ_OK;
}

int tq_memset(void* dst, int value, size_t bytes) {
  TQ_CHECK_ARG(dst != nullptr, "tq_memset: dst is NULL");
  TQ_CHECK_HIP(hipMemset(dst, value, bytes));
  return TQ_OK;
}

int tq_sync(void) {
  TQ_CHECK_HIP(hipDeviceSynchronize());
  return TQ_OK;
}

}  // extern "C"
