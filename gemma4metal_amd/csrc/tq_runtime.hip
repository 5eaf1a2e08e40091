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

// Plain streaming read of `bytes` (a multiple of 16): every lane loads 16 B
// per step with grid-stride, XOR-folds the data and writes one word per
// thread so the loads cannot be dropped.  The achievable-bandwidth reference
// measured beside the attention kernel.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ src,
                                                          size_t n16, uint32_t* __restrict__ sink) {
  const size_t stride = static_cast<size_t>(gridDim.x) * 256;
  size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  sink[static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x] = acc;
}

}  // namespace tq

extern "C" {

int tq_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks, void* stream) {
  TQ_CHECK_ARG(src && sink, "tq_stream_read: null pointer");
  TQ_CHECK_ARG(bytes % 16 == 0, "tq_stream_read: bytes must be a multiple of 16");
  TQ_CHECK_ARG(blocks > 0 && blocks <= 65536, "tq_stream_read: blocks must be in [1, 65536]");
  tq::stream_read_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(src), bytes / 16, sink);
  TQ_CHECK_LAUNCH("stream_read_kernel");
  return TQ_OK;
}


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
