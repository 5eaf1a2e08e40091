// Library-level entry points: version, thread-local error string, and the
// small device-memory helpers that let a ctypes caller drive the library
// without any other GPU runtime.
#include <algorithm>
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

__global__ void zero_words_kernel(uint32_t* p, size_t n) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    p[i] = 0u;
}

int zero_async(void* p, size_t bytes, hipStream_t s) {
  TQ_CHECK_ARG(p != nullptr && bytes % 4 == 0, "zero_async: bad buffer");
  const size_t n = bytes / 4;
  const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 1024));
  if (n) zero_words_kernel<<<blocks, 256, 0, s>>>(static_cast<uint32_t*>(p), n);
  TQ_CHECK_LAUNCH("zero_words_kernel");
  return TQ_OK;
}

// Streaming read in the decode-attention kernel's launch geometry: one
// workgroup of NW waves per contiguous slice of the buffer (the split of a
// kv head), each wave reading U 16-byte loads per lane per iteration (U KiB
// per wave, 1 KiB per load instruction, fully coalesced), DEPTH iterations
// in flight ahead of the one being consumed, non-temporal (kNT) or
// default-policy loads.  Loads past the slice are clamped to its last
// element (in bounds; the repeats hit the same cache line).
template <int NW, int U, int DEPTH, bool kNT>
__global__ __launch_bounds__(NW * 64) void stream_tiles_kernel(const uint4* __restrict__ src,
                                                               int64_t n16,
                                                               uint32_t* __restrict__ sink) {
  constexpr int R = DEPTH + 1;          // register buffers
  constexpr int64_t TILE = NW * 64 * U;  // uint4 per workgroup iteration
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t lo = static_cast<int64_t>(blockIdx.x) * per;
  const int64_t hi = lo + per < n16 ? lo + per : n16;
  uint32_t acc = 0;
  if (lo < hi) {
    const int64_t last = hi - 1;
    const int nit = static_cast<int>((hi - lo + TILE - 1) / TILE);
    const uint4* base = src + lo + wv * 64 * U + lane;
    // offset bound of this lane, in 16 B units (a slice holds < 2^31 of them)
    const int lim = static_cast<int>(last - lo) - wv * 64 * U - lane;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4* vbase = reinterpret_cast<const u32x4*>(base);
    u32x4 buf[R][U];
    auto load = [&](u32x4 (&b)[U], int it) {
#pragma unroll
      for (int j = 0; j < U; ++j) {
        int off = it * static_cast<int>(TILE) + j * 64;
        off = off < lim ? off : lim;
        if constexpr (kNT) b[j] = __builtin_nontemporal_load(vbase + off);
        else b[j] = vbase[off];
      }
    };
    auto consume = [&](const u32x4 (&b)[U]) {
#pragma unroll
      for (int j = 0; j < U; ++j) acc ^= b[j].x ^ b[j].y ^ b[j].z ^ b[j].w;
    };
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load(buf[d], d);
    int it = 0;
    for (; it + R <= nit; it += R) {
#pragma unroll
      for (int s = 0; s < R; ++s) {
        if (it + s + DEPTH < nit) load(buf[(s + DEPTH) % R], it + s + DEPTH);
        consume(buf[s]);
      }
    }
#pragma unroll
    for (int s = 0; s < R; ++s) {
      if (it + s < nit) {
        if (it + s + DEPTH < nit) load(buf[(s + DEPTH) % R], it + s + DEPTH);
        consume(buf[s]);
      }
    }
  }
  sink[static_cast<int64_t>(blockIdx.x) * NW * 64 + threadIdx.x] = acc;
}

template <int NW, int U, int DEPTH>
int launch_stream_tiles(const void* src, size_t bytes, uint32_t* sink, int blocks, bool nt,
                        hipStream_t s) {
  if (nt)
    stream_tiles_kernel<NW, U, DEPTH, true><<<blocks, NW * 64, 0, s>>>(
        static_cast<const uint4*>(src), static_cast<int64_t>(bytes / 16), sink);
  else
    stream_tiles_kernel<NW, U, DEPTH, false><<<blocks, NW * 64, 0, s>>>(
        static_cast<const uint4*>(src), static_cast<int64_t>(bytes / 16), sink);
  TQ_CHECK_LAUNCH("stream_tiles_kernel");
  return TQ_OK;
}

template <int NW, int U>
int launch_stream_tiles_u(const void* src, size_t bytes, uint32_t* sink, int blocks, int depth,
                          bool nt, hipStream_t s) {
  switch (depth) {
    case 1: return launch_stream_tiles<NW, U, 1>(src, bytes, sink, blocks, nt, s);
    case 2: return launch_stream_tiles<NW, U, 2>(src, bytes, sink, blocks, nt, s);
    default: return launch_stream_tiles<NW, U, 3>(src, bytes, sink, blocks, nt, s);
  }
}

}  // namespace tq

extern "C" {

int tq_stream_read_tiles(const void* src, size_t bytes, uint32_t* sink, int blocks, int waves,
                         int loads_per_lane, int depth, int nontemporal, void* stream) {
  TQ_CHECK_ARG(src && sink, "tq_stream_read_tiles: null pointer");
  TQ_CHECK_ARG(bytes % 16 == 0 && bytes > 0, "tq_stream_read_tiles: bytes must be a positive multiple of 16");
  TQ_CHECK_ARG(blocks > 0 && blocks <= 65536, "tq_stream_read_tiles: blocks must be in [1, 65536]");
  TQ_CHECK_ARG(depth >= 1 && depth <= 3, "tq_stream_read_tiles: depth must be 1, 2 or 3");
  TQ_CHECK_ARG(bytes / 16 / blocks < (size_t{1} << 30), "tq_stream_read_tiles: slice too large");
  // register budget: the buffers in flight must fit without spilling
  TQ_CHECK_ARG(loads_per_lane * (depth + 1) * 4 <= (waves == 16 ? 72 : 128),
               "tq_stream_read_tiles: loads_per_lane * (depth + 1) too large for %d waves", waves);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool nt = nontemporal != 0;
  if (waves == 8 && loads_per_lane == 4) return tq::launch_stream_tiles_u<8, 4>(src, bytes, sink, blocks, depth, nt, s);
  if (waves == 8 && loads_per_lane == 9) return tq::launch_stream_tiles_u<8, 9>(src, bytes, sink, blocks, depth, nt, s);
  if (waves == 8 && loads_per_lane == 16) return tq::launch_stream_tiles_u<8, 16>(src, bytes, sink, blocks, depth, nt, s);
  if (waves == 4 && loads_per_lane == 9) return tq::launch_stream_tiles_u<4, 9>(src, bytes, sink, blocks, depth, nt, s);
  if (waves == 4 && loads_per_lane == 16) return tq::launch_stream_tiles_u<4, 16>(src, bytes, sink, blocks, depth, nt, s);
  if (waves == 16 && loads_per_lane == 4) return tq::launch_stream_tiles_u<16, 4>(src, bytes, sink, blocks, depth, nt, s);
  if (waves == 16 && loads_per_lane == 9) return tq::launch_stream_tiles_u<16, 9>(src, bytes, sink, blocks, depth, nt, s);
  tq::set_error("tq_stream_read_tiles: (waves, loads_per_lane) must be one of (8,4) (8,9) (8,16) "
                "(4,9) (4,16) (16,4) (16,9)");
  return TQ_ERR_UNSUPPORTED;
}

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
