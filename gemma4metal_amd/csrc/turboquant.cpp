// C++ API of include/turboquant.h over the C ABI of include/tq_c_api.h.
//
// Outputs are allocated here (the reference allocates inside eval_gpu,
// lib/turboquant.cpp:372); the split-K workspace is a zero-filled buffer per
// (device, stream), grown on demand with stream-ordered allocation and
// reused (the kernels return its counters to zero).  sdpa_int4_into also
// takes a caller-owned workspace.
#include "turboquant.h"

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <stdexcept>
#include <utility>

#include "tq_c_api.h"

namespace tq {
// Zero-fills `bytes` (a multiple of 4) at p with a kernel on stream s
// (tq_runtime.hip).
int zero_async(void* p, size_t bytes, hipStream_t s);
}  // namespace tq

namespace turboquant {
namespace {

void check(int status, const char* fn) {
  if (status != TQ_OK)
    throw std::runtime_error(std::string(fn) + ": " + tq_last_error());
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void need(bool cond, const std::string& msg) {
  if (!cond) throw std::invalid_argument(msg);
}

tq_dtype c_dtype(Dtype d) {
  switch (d) {
    case Dtype::float32: return TQ_F32;
    case Dtype::float16: return TQ_F16;
    case Dtype::bfloat16: return TQ_BF16;
    default: throw std::invalid_argument("not a floating-point dtype");
  }
}

bool is_sb(Dtype d) { return d == Dtype::float32 || d == Dtype::float16; }

// Split-K workspaces, one per (device, stream): calls on one stream run in
// order, so they can share one; calls on different streams never do.  A
// workspace that must grow is replaced by a stream-ordered allocation on that
// stream, zero-filled by a kernel on the same stream, and the old buffer is
// released with a stream-ordered free after the calls already queued there:
// nothing synchronises the device, and no buffer is freed while a queued
// kernel may still use it.
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

void* workspace(size_t bytes, size_t* have, StreamOrDevice s) {
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  const hipStream_t stream = static_cast<hipStream_t>(s);
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Workspace& w = g_ws[{dev, stream}];
  if (w.bytes < bytes) {
    // Growing records an allocation, a fill and a free: under stream capture
    // they would become graph nodes, and the graph would own the buffer this
    // map keeps.  Refuse instead of recording them.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    check_hip(hipStreamIsCapturing(stream, &cap), "hipStreamIsCapturing");
    if (cap != hipStreamCaptureStatusNone)
      throw std::runtime_error(
          "turboquant: the split-K workspace of this (device, stream) must grow, but the stream "
          "is being captured; make one eager call of the largest shape on this stream before "
          "capture, pass a workspace (sdpa_int4_into with workspace), or use "
          "tq_sdpa_int4_noalloc");
    const size_t nb = std::max<size_t>(bytes, size_t{1} << 20);
    void* p = nullptr;
    check_hip(hipMallocAsync(&p, nb, stream), "hipMallocAsync");
    check(tq::zero_async(p, nb, stream), "workspace zero-fill");
    if (w.ptr) check_hip(hipFreeAsync(w.ptr, stream), "hipFreeAsync");
    w.ptr = p;
    w.bytes = nb;
  }
  *have = w.bytes;
  return w.ptr;
}

// The four codebooks back to back in one device buffer + their sizes.
struct Codebooks {
  array buf;
  int sizes[4];
};

Codebooks concat_codebooks(const array& c1, const array& c2, const array& c3, const array& c4,
                           int width, StreamOrDevice s) {
  Codebooks cb;
  const array* cs[4] = {&c1, &c2, &c3, &c4};
  int64_t total = 0;
  for (int i = 0; i < 4; ++i) {
    need(cs[i]->dtype() == Dtype::float32, "codebooks must be float32");
    cb.sizes[i] = static_cast<int>(cs[i]->size() / width);
    total += cs[i]->size();
  }
  cb.buf = array::empty({total}, Dtype::float32);
  size_t off = 0;
  for (int i = 0; i < 4; ++i) {
    check_hip(hipMemcpyAsync(static_cast<char*>(cb.buf.data()) + off, cs[i]->data(),
                             cs[i]->nbytes(), hipMemcpyDeviceToDevice,
                             static_cast<hipStream_t>(s)),
              "hipMemcpyAsync");
    off += cs[i]->nbytes();
  }
  return cb;
}

}  // namespace

size_t dtype_size(Dtype d) {
  switch (d) {
    case Dtype::float16:
    case Dtype::bfloat16: return 2;
    case Dtype::uint8: return 1;
    default: return 4;
  }
}

int64_t array::size() const {
  int64_t n = 1;
  for (int64_t d : shape_) n *= d;
  return n;
}

array array::empty(std::vector<int64_t> shape, Dtype dtype) {
  array a;
  a.shape_ = std::move(shape);
  a.dtype_ = dtype;
  void* p = nullptr;
  check_hip(hipMalloc(&p, std::max<size_t>(a.nbytes(), 1)), "hipMalloc");
  a.owner_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
  a.ptr_ = p;
  return a;
}

array array::borrow(void* data, std::vector<int64_t> shape, Dtype dtype) {
  array a;
  a.ptr_ = data;
  a.shape_ = std::move(shape);
  a.dtype_ = dtype;
  return a;
}

array array::from_host(const void* host, std::vector<int64_t> shape, Dtype dtype) {
  array a = empty(std::move(shape), dtype);
  check_hip(hipMemcpy(a.ptr_, host, a.nbytes(), hipMemcpyHostToDevice), "hipMemcpy");
  return a;
}

array array::reshape(std::vector<int64_t> shape) const {
  array a = *this;
  a.shape_ = std::move(shape);
  need(a.size() == size(), "reshape: element count differs");
  return a;
}

void array::to_host(void* host) const {
  check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
  check_hip(hipMemcpy(host, ptr_, nbytes(), hipMemcpyDeviceToHost), "hipMemcpy");
}

void synchronize(StreamOrDevice s) {
  check_hip(hipStreamSynchronize(static_cast<hipStream_t>(s)), "hipStreamSynchronize");
}

void set_metallib_path(const std::string&) {}

// ---------------------------------------------------------------------------

size_t sdpa_int4_workspace_size(int batch, int num_heads, int num_kv_heads, int head_dim,
                                int max_kv_len) {
  return tq_sdpa_int4_workspace_size(batch, num_heads, num_kv_heads, head_dim, max_kv_len);
}

void sdpa_int4_into(array& out, const array& queries, const array& k_quant, const array& k_scales,
                    const array& k_biases, const array& v_quant, const array& v_scales,
                    const array& v_biases, int gqa_factor, float scale, int sliding_window,
                    int kv_len, StreamOrDevice s) {
  sdpa_int4_into(out, queries, k_quant, k_scales, k_biases, v_quant, v_scales, v_biases,
                 gqa_factor, scale, sliding_window, kv_len, nullptr, 0, s);
}

void sdpa_int4_into(array& out, const array& queries, const array& k_quant, const array& k_scales,
                    const array& k_biases, const array& v_quant, const array& v_scales,
                    const array& v_biases, int gqa_factor, float scale, int sliding_window,
                    int kv_len, void* workspace_ptr, size_t workspace_bytes, StreamOrDevice s) {
  need(queries.ndim() == 2, "queries must be (num_heads, head_dim)");
  need(k_quant.ndim() == 3 && v_quant.shape() == k_quant.shape(),
       "k_quant / v_quant must be (num_kv_heads, N, head_dim/8)");
  need(is_sb(k_scales.dtype()), "scales must be float32 or float16");
  const int Hq = static_cast<int>(queries.shape(0)), D = static_cast<int>(queries.shape(1));
  const int Hkv = static_cast<int>(k_quant.shape(0)), cap = static_cast<int>(k_quant.shape(1));
  need(k_quant.shape(2) == D / 8, "k_quant last dim must be head_dim / 8");
  for (const array* a : {&k_scales, &k_biases, &v_scales, &v_biases})
    need(a->shape() == std::vector<int64_t>{Hkv, cap, D / 64} && a->dtype() == k_scales.dtype(),
         "scales / biases must be (num_kv_heads, N, head_dim/64) of one dtype");
  need(out.shape() == std::vector<int64_t>{Hq, D} && out.dtype() == Dtype::float32,
       "out must be (num_heads, head_dim) float32");
  const int n = kv_len < 0 ? cap : kv_len;
  size_t have = workspace_bytes;
  void* ws = workspace_ptr;
  if (!ws) ws = workspace(tq_sdpa_int4_workspace_size(1, Hq, Hkv, D, n), &have, s);
  check(tq_sdpa_int4(queries.data(), c_dtype(queries.dtype()),
                     static_cast<const uint32_t*>(k_quant.data()), k_scales.data(),
                     k_biases.data(), static_cast<const uint32_t*>(v_quant.data()),
                     v_scales.data(), v_biases.data(), c_dtype(k_scales.dtype()),
                     static_cast<float*>(out.data()), Hq, Hkv, D, n, cap, gqa_factor, scale,
                     sliding_window, ws, have, s),
        "sdpa_int4");
}

array sdpa_int4(const array& queries, const array& k_quant, const array& k_scales,
                const array& k_biases, const array& v_quant, const array& v_scales,
                const array& v_biases, int gqa_factor, float scale, int sliding_window,
                StreamOrDevice s) {
  need(queries.ndim() == 2, "queries must be (num_heads, head_dim)");
  array out = array::empty({queries.shape(0), queries.shape(1)}, Dtype::float32);
  sdpa_int4_into(out, queries, k_quant, k_scales, k_biases, v_quant, v_scales, v_biases,
                 gqa_factor, scale, sliding_window, -1, s);
  return out;
}

array sdpa_int4_ragged(const array& queries, const array& k_quant, const array& k_scales,
                       const array& k_biases, const array& v_quant, const array& v_scales,
                       const array& v_biases, const array& seq_lens, int gqa_factor, float scale,
                       int sliding_window, const array& windows, StreamOrDevice s) {
  need(queries.ndim() == 3 && k_quant.ndim() == 4, "queries (B, Hq, D), caches (B, Hkv, cap, .)");
  const int B = static_cast<int>(queries.shape(0)), Hq = static_cast<int>(queries.shape(1));
  const int D = static_cast<int>(queries.shape(2));
  const int Hkv = static_cast<int>(k_quant.shape(1)), cap = static_cast<int>(k_quant.shape(2));
  need(seq_lens.dtype() == Dtype::int32 && seq_lens.size() == B, "seq_lens must be int32 (B)");
  need(is_sb(k_scales.dtype()), "scales must be float32 or float16");
  array out = array::empty({B, Hq, D}, Dtype::float32);
  size_t have = 0;
  void* ws = workspace(tq_sdpa_int4_workspace_size(B, Hq, Hkv, D, cap), &have, s);
  check(tq_sdpa_int4_ragged(queries.data(), c_dtype(queries.dtype()),
                            static_cast<const uint32_t*>(k_quant.data()), k_scales.data(),
                            k_biases.data(), static_cast<const uint32_t*>(v_quant.data()),
                            v_scales.data(), v_biases.data(), c_dtype(k_scales.dtype()),
                            static_cast<float*>(out.data()), B, Hq, Hkv, D, cap,
                            static_cast<const int32_t*>(seq_lens.data()),
                            windows.size() > 0 && windows.data()
                                ? static_cast<const int32_t*>(windows.data())
                                : nullptr,
                            cap, gqa_factor, scale, sliding_window, ws, have, s),
        "sdpa_int4_ragged");
  return out;
}

array sdpa_int4_prefill(const array& queries, const array& k_quant, const array& k_scales,
                        const array& k_biases, const array& v_quant, const array& v_scales,
                        const array& v_biases, int n_prior, int gqa_factor, float scale,
                        int sliding_window, StreamOrDevice s) {
  need(queries.ndim() == 3 && k_quant.ndim() == 3, "queries (n_new, Hq, D), caches (Hkv, cap, .)");
  const int S = static_cast<int>(queries.shape(0)), Hq = static_cast<int>(queries.shape(1));
  const int D = static_cast<int>(queries.shape(2));
  const int Hkv = static_cast<int>(k_quant.shape(0)), cap = static_cast<int>(k_quant.shape(1));
  need(is_sb(k_scales.dtype()), "scales must be float32 or float16");
  array out = array::empty({S, Hq, D}, Dtype::float32);
  size_t have = 0;
  void* ws = workspace(tq_sdpa_int4_workspace_size(S > 0 ? S : 1, Hq, Hkv, D, n_prior + S), &have, s);
  check(tq_sdpa_int4_prefill(queries.data(), c_dtype(queries.dtype()),
                             static_cast<const uint32_t*>(k_quant.data()), k_scales.data(),
                             k_biases.data(), static_cast<const uint32_t*>(v_quant.data()),
                             v_scales.data(), v_biases.data(), c_dtype(k_scales.dtype()),
                             static_cast<float*>(out.data()), Hq, Hkv, D, n_prior, S, cap,
                             gqa_factor, scale, sliding_window, ws, have, s),
        "sdpa_int4_prefill");
  return out;
}

std::vector<array> quantize(const array& x, int group_size, int bits, Dtype scale_dtype,
                            StreamOrDevice s) {
  need(x.ndim() >= 1, "x must have a last axis");
  need(is_sb(scale_dtype), "scale_dtype must be float16 or float32");
  const int64_t D = x.shape(-1);
  std::vector<int64_t> lead(x.shape().begin(), x.shape().end() - 1);
  auto with = [&](int64_t last) {
    std::vector<int64_t> sh = lead;
    sh.push_back(last);
    return sh;
  };
  array wq = array::empty(with(D / 8), Dtype::uint32);
  array sc = array::empty(with(D / 64), scale_dtype);
  array bi = array::empty(with(D / 64), scale_dtype);
  const int64_t rows = D > 0 ? x.size() / D : 0;
  check(tq_quantize_int4(x.data(), c_dtype(x.dtype()), rows, static_cast<int>(D), group_size,
                         bits, TQ_QUANT_MLX, static_cast<uint32_t*>(wq.data()), sc.data(),
                         bi.data(), c_dtype(scale_dtype), s),
        "quantize");
  return {wq, sc, bi};
}

array dequantize(const array& w, const array& scales, const array& biases, int group_size,
                 int bits, StreamOrDevice s) {
  need(group_size == 64 && bits == 4, "only group_size 64, bits 4");
  const int64_t D = w.shape(-1) * 8;
  std::vector<int64_t> sh(w.shape().begin(), w.shape().end() - 1);
  sh.push_back(D);
  array out = array::empty(sh, Dtype::float32);
  check(tq_dequantize_int4(static_cast<const uint32_t*>(w.data()), scales.data(), biases.data(),
                           c_dtype(scales.dtype()), w.size() / w.shape(-1), static_cast<int>(D),
                           static_cast<float*>(out.data()), s),
        "dequantize");
  return out;
}

namespace {
using AppendFn = int (*)(const void*, const void*, tq_dtype, uint32_t*, void*, void*, uint32_t*,
                         void*, void*, tq_dtype, int, int, int, int, const int32_t*, int,
                         tq_quant_mode, void*);
void append_common(AppendFn fn, const char* what, const array& k_new, const array& v_new,
                   array& k_quant, array& k_scales, array& k_biases, array& v_quant,
                   array& v_scales, array& v_biases, const array& positions, StreamOrDevice s) {
  need(k_new.ndim() == 4 && v_new.shape() == k_new.shape(), "k_new / v_new must be (B, Hkv, T, D)");
  need(k_quant.ndim() == 4, "caches must be (B, Hkv, capacity, .)");
  need(positions.dtype() == Dtype::int32, "positions must be int32");
  check(fn(k_new.data(), v_new.data(), c_dtype(k_new.dtype()),
           static_cast<uint32_t*>(k_quant.data()), k_scales.data(), k_biases.data(),
           static_cast<uint32_t*>(v_quant.data()), v_scales.data(), v_biases.data(),
           c_dtype(k_scales.dtype()), static_cast<int>(k_new.shape(0)),
           static_cast<int>(k_new.shape(1)), static_cast<int>(k_new.shape(3)),
           static_cast<int>(k_quant.shape(2)), static_cast<const int32_t*>(positions.data()),
           static_cast<int>(k_new.shape(2)), TQ_QUANT_MLX, s),
        what);
}
}  // namespace

void kv_append_int4(const array& k_new, const array& v_new, array& k_quant, array& k_scales,
                    array& k_biases, array& v_quant, array& v_scales, array& v_biases,
                    const array& positions, StreamOrDevice s) {
  append_common(tq_kv_append_int4, "kv_append_int4", k_new, v_new, k_quant, k_scales, k_biases,
                v_quant, v_scales, v_biases, positions, s);
}

void kv_append_int4_ring(const array& k_new, const array& v_new, array& k_quant,
                         array& k_scales, array& k_biases, array& v_quant, array& v_scales,
                         array& v_biases, const array& positions, StreamOrDevice s) {
  append_common(tq_kv_append_int4_ring, "kv_append_int4_ring", k_new, v_new, k_quant, k_scales,
                k_biases, v_quant, v_scales, v_biases, positions, s);
}

// ---------------------------------------------------------------------------
// PolarQuant

std::vector<array> polar_quantize(const array& vectors, const array& precondition,
                                  const array& cb_l1, const array& cb_l2, const array& cb_l3,
                                  const array& cb_l4, int block_size, StreamOrDevice s) {
  need(vectors.ndim() == 2 && vectors.dtype() == Dtype::float32, "vectors must be (N, D) float32");
  const int64_t N = vectors.shape(0), D = vectors.shape(1), nb = N * (D / 16);
  Codebooks cb = concat_codebooks(cb_l1, cb_l2, cb_l3, cb_l4, 1, s);
  array i1 = array::empty({nb * 8}, Dtype::uint8), i2 = array::empty({nb * 4}, Dtype::uint8);
  array i3 = array::empty({nb * 2}, Dtype::uint8), i4 = array::empty({nb}, Dtype::uint8);
  array r = array::empty({nb}, Dtype::float16);
  check(tq_polar_quantize(static_cast<const float*>(vectors.data()),
                          static_cast<const float*>(precondition.data()),
                          static_cast<const float*>(cb.buf.data()), cb.sizes, N,
                          static_cast<int>(D), block_size, static_cast<uint8_t*>(i1.data()),
                          static_cast<uint8_t*>(i2.data()), static_cast<uint8_t*>(i3.data()),
                          static_cast<uint8_t*>(i4.data()), static_cast<uint16_t*>(r.data()), s),
        "polar_quantize");
  return {i1, i2, i3, i4, r};
}

std::vector<array> polar_quantize_packed(const array& vectors, const array& precondition,
                                         const array& cb_l1, const array& cb_l2,
                                         const array& cb_l3, const array& cb_l4, int block_size,
                                         StreamOrDevice s) {
  need(vectors.ndim() == 2 && vectors.dtype() == Dtype::float32, "vectors must be (N, D) float32");
  const int64_t N = vectors.shape(0), D = vectors.shape(1), nb = N * (D / 16);
  Codebooks cb = concat_codebooks(cb_l1, cb_l2, cb_l3, cb_l4, 1, s);
  array p1 = array::empty({nb}, Dtype::uint32), p2 = array::empty({nb}, Dtype::uint8);
  array p3 = array::empty({nb}, Dtype::uint8), p4 = array::empty({nb}, Dtype::uint8);
  array r = array::empty({nb}, Dtype::float16);
  check(tq_polar_quantize_packed(
            static_cast<const float*>(vectors.data()), static_cast<const float*>(precondition.data()),
            static_cast<const float*>(cb.buf.data()), cb.sizes, N, static_cast<int>(D), block_size,
            static_cast<uint32_t*>(p1.data()), static_cast<uint8_t*>(p2.data()),
            static_cast<uint8_t*>(p3.data()), static_cast<uint8_t*>(p4.data()),
            static_cast<uint16_t*>(r.data()), s),
        "polar_quantize_packed");
  return {p1, p2, p3, p4, r};
}

namespace {
array dequant_unpacked(const array& i1, const array& i2, const array& i3, const array& i4,
                       const array& radii, const float* P, const array& c1, const array& c2,
                       const array& c3, const array& c4, int64_t D, int block_size,
                       StreamOrDevice s, const char* fn) {
  const int64_t N = radii.size() * 16 / D;
  Codebooks cb = concat_codebooks(c1, c2, c3, c4, 1, s);
  array out = array::empty({N, D}, Dtype::float32);
  check(tq_polar_dequantize(static_cast<const uint8_t*>(i1.data()),
                            static_cast<const uint8_t*>(i2.data()),
                            static_cast<const uint8_t*>(i3.data()),
                            static_cast<const uint8_t*>(i4.data()),
                            static_cast<const uint16_t*>(radii.data()), P,
                            static_cast<const float*>(cb.buf.data()), cb.sizes, N,
                            static_cast<int>(D), block_size, static_cast<float*>(out.data()), s),
        fn);
  return out;
}

array dequant_packed(const array& p1, const array& p2, const array& p3, const array& p4,
                     const array& radii, const array& c1, const array& c2, const array& c3,
                     const array& c4, bool cs, int64_t D, int block_size, StreamOrDevice s,
                     const char* fn) {
  const int64_t N = radii.size() * 16 / D;
  Codebooks cb = concat_codebooks(c1, c2, c3, c4, cs ? 2 : 1, s);
  array out = array::empty({N, D}, Dtype::float32);
  const float* buf = static_cast<const float*>(cb.buf.data());
  check(tq_polar_dequantize_packed(static_cast<const uint32_t*>(p1.data()),
                                   static_cast<const uint8_t*>(p2.data()),
                                   static_cast<const uint8_t*>(p3.data()),
                                   static_cast<const uint8_t*>(p4.data()),
                                   static_cast<const uint16_t*>(radii.data()), cs ? nullptr : buf,
                                   cs ? buf : nullptr, cb.sizes, N, static_cast<int>(D),
                                   block_size, static_cast<float*>(out.data()), s),
        fn);
  return out;
}
}  // namespace

array polar_dequantize(const array& indices_l1, const array& indices_l2, const array& indices_l3,
                       const array& indices_l4, const array& radii, const array& precondition,
                       const array& cb_l1, const array& cb_l2, const array& cb_l3,
                       const array& cb_l4, int block_size, StreamOrDevice s) {
  return dequant_unpacked(indices_l1, indices_l2, indices_l3, indices_l4, radii,
                          static_cast<const float*>(precondition.data()), cb_l1, cb_l2, cb_l3,
                          cb_l4, precondition.shape(0), block_size, s, "polar_dequantize");
}

array polar_dequantize_fast(const array& indices_l1, const array& indices_l2,
                            const array& indices_l3, const array& indices_l4, const array& radii,
                            const array& cb_l1, const array& cb_l2, const array& cb_l3,
                            const array& cb_l4, int D, int block_size, StreamOrDevice s) {
  return dequant_unpacked(indices_l1, indices_l2, indices_l3, indices_l4, radii, nullptr, cb_l1,
                          cb_l2, cb_l3, cb_l4, D, block_size, s, "polar_dequantize_fast");
}

array polar_dequantize_packed(const array& packed_l1, const array& packed_l2,
                              const array& packed_l3, const array& packed_l4, const array& radii,
                              const array& cb_l1, const array& cb_l2, const array& cb_l3,
                              const array& cb_l4, int D, int block_size, StreamOrDevice s) {
  return dequant_packed(packed_l1, packed_l2, packed_l3, packed_l4, radii, cb_l1, cb_l2, cb_l3,
                        cb_l4, false, D, block_size, s, "polar_dequantize_packed");
}

array polar_dequantize_packed_fast(const array& packed_l1, const array& packed_l2,
                                   const array& packed_l3, const array& packed_l4,
                                   const array& radii, const array& cs_l1, const array& cs_l2,
                                   const array& cs_l3, const array& cs_l4, int D, int block_size,
                                   StreamOrDevice s) {
  return dequant_packed(packed_l1, packed_l2, packed_l3, packed_l4, radii, cs_l1, cs_l2, cs_l3,
                        cs_l4, true, D, block_size, s, "polar_dequantize_packed_fast");
}

array compressed_score(const array& queries, const array& indices_l1, const array& indices_l2,
                       const array& indices_l3, const array& indices_l4, const array& radii,
                       const array& cb_l1, const array& cb_l2, const array& cb_l3,
                       const array& cb_l4, int N, int block_size, float scale, StreamOrDevice s) {
  need(queries.ndim() == 2 && queries.dtype() == Dtype::float32, "queries must be (Nq, D) float32");
  const int Nq = static_cast<int>(queries.shape(0)), D = static_cast<int>(queries.shape(1));
  Codebooks cb = concat_codebooks(cb_l1, cb_l2, cb_l3, cb_l4, 1, s);
  array out = array::empty({Nq, N}, Dtype::float32);
  check(tq_compressed_score(static_cast<const float*>(queries.data()), Nq,
                            static_cast<const uint8_t*>(indices_l1.data()),
                            static_cast<const uint8_t*>(indices_l2.data()),
                            static_cast<const uint8_t*>(indices_l3.data()),
                            static_cast<const uint8_t*>(indices_l4.data()),
                            static_cast<const uint16_t*>(radii.data()),
                            static_cast<const float*>(cb.buf.data()), cb.sizes, Nq, N, D,
                            block_size, scale, static_cast<float*>(out.data()), s),
        "compressed_score");
  return out;
}

array compressed_sdpa(const array& queries, const array& indices_l1, const array& indices_l2,
                      const array& indices_l3, const array& indices_l4, const array& radii,
                      const array& cb_l1, const array& cb_l2, const array& cb_l3,
                      const array& cb_l4, const array& values, int block_size, float scale,
                      StreamOrDevice s) {
  need(queries.ndim() == 2 && values.ndim() == 2, "queries (Nq, D), values (Nq * N, D)");
  const int Nq = static_cast<int>(queries.shape(0)), D = static_cast<int>(queries.shape(1));
  const int N = static_cast<int>(values.shape(0) / Nq);
  Codebooks cb = concat_codebooks(cb_l1, cb_l2, cb_l3, cb_l4, 1, s);
  array out = array::empty({Nq, D}, Dtype::float32);
  size_t have = 0;
  void* ws = workspace(tq_compressed_sdpa_workspace_size(Nq, Nq, D, N), &have, s);
  check(tq_compressed_sdpa(static_cast<const float*>(queries.data()), Nq,
                           static_cast<const uint8_t*>(indices_l1.data()),
                           static_cast<const uint8_t*>(indices_l2.data()),
                           static_cast<const uint8_t*>(indices_l3.data()),
                           static_cast<const uint8_t*>(indices_l4.data()),
                           static_cast<const uint16_t*>(radii.data()),
                           static_cast<const float*>(cb.buf.data()), cb.sizes,
                           static_cast<const float*>(values.data()), Nq, N, D, block_size, scale,
                           static_cast<float*>(out.data()), ws, have, s),
        "compressed_sdpa");
  return out;
}

}  // namespace turboquant
