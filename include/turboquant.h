// turboquant.h -- C++ API of libturboquant_hip.so with the names, argument
// order and defaults of the reference's lib/turboquant.h, so that a caller
// such as engine/gemma4_multilayer.cpp:280-282 keeps its call expressions.
//
// `array` stands in for mlx::core::array on this path: a device tensor with
// a shape and a dtype, either owning its HIP allocation (outputs, which the
// reference also allocates inside eval_gpu, lib/turboquant.cpp:372) or
// borrowing caller memory.  Calls are stream-ordered on the HIP stream passed
// as StreamOrDevice (nullptr = the null stream) and asynchronous, like MLX's
// lazy evaluation until eval(); errors throw std::runtime_error, as the
// reference's primitives do (lib/turboquant.cpp:363-365).  The C ABI these
// functions call is include/tq_c_api.h.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace turboquant {

enum class Dtype : int {
  float32 = 0,   // TQ_F32
  float16 = 1,   // TQ_F16
  bfloat16 = 2,  // TQ_BF16
  uint32 = 16,
  uint8 = 17,
  int32 = 18,
};
size_t dtype_size(Dtype d);

using StreamOrDevice = void*;  // hipStream_t; nullptr = null stream

class array {
 public:
  array() = default;
  // Owning device allocation (uninitialised).
  static array empty(std::vector<int64_t> shape, Dtype dtype);
  // Borrowed device memory (the caller keeps it alive).
  static array borrow(void* data, std::vector<int64_t> shape, Dtype dtype);
  // Owning copy of host data.
  static array from_host(const void* host, std::vector<int64_t> shape, Dtype dtype);

  void* data() { return ptr_; }
  const void* data() const { return ptr_; }
  Dtype dtype() const { return dtype_; }
  const std::vector<int64_t>& shape() const { return shape_; }
  int64_t shape(int dim) const { return shape_.at(dim < 0 ? dim + ndim() : dim); }
  int ndim() const { return static_cast<int>(shape_.size()); }
  int64_t size() const;
  size_t nbytes() const { return static_cast<size_t>(size()) * dtype_size(dtype_); }
  bool valid() const { return ptr_ != nullptr || size() == 0; }
  // Same memory, new shape (element count must match).
  array reshape(std::vector<int64_t> shape) const;
  // Synchronous copy to host (waits for the device).
  void to_host(void* host) const;

 private:
  std::shared_ptr<void> owner_;
  void* ptr_ = nullptr;
  std::vector<int64_t> shape_;
  Dtype dtype_ = Dtype::float32;
};

// Blocks until all work queued on the stream is done (MLX's eval()).
void synchronize(StreamOrDevice s = {});

// ---- fused int4 decode attention (lib/turboquant.h:196-207) -----------------
// queries (num_heads, head_dim) f32|f16|bf16; k_quant/v_quant (num_kv_heads,
// N, head_dim/8) uint32; scales/biases (num_kv_heads, N, head_dim/64) f32|f16.
// Returns (num_heads, head_dim) f32.  head_dim in {128, 256, 512}.
array sdpa_int4(const array& queries, const array& k_quant, const array& k_scales,
                const array& k_biases, const array& v_quant, const array& v_scales,
                const array& v_biases, int gqa_factor, float scale = 1.0f,
                int sliding_window = 0, StreamOrDevice s = {});

// The same into a caller-owned output, over rows [0, kv_len) of caches whose
// row stride is k_quant.shape(1) (kv_len < 0: all rows).  The split-K
// workspace is the library's buffer for the calling (device, stream); it
// grows with stream-ordered allocations, so under stream (graph) capture a
// call that would grow it throws: make one eager call of the largest shape on
// that stream first, or use the overload below.
void sdpa_int4_into(array& out, const array& queries, const array& k_quant,
                    const array& k_scales, const array& k_biases, const array& v_quant,
                    const array& v_scales, const array& v_biases, int gqa_factor,
                    float scale = 1.0f, int sliding_window = 0, int kv_len = -1,
                    StreamOrDevice s = {});

// The same with a caller-owned split-K workspace of workspace_bytes (at
// least sdpa_int4_workspace_size(1, ...), zero-filled once before first use;
// the kernels leave it zeroed).  Calls that may run concurrently need
// separate workspaces.  Allocates nothing.
void sdpa_int4_into(array& out, const array& queries, const array& k_quant,
                    const array& k_scales, const array& k_biases, const array& v_quant,
                    const array& v_scales, const array& v_biases, int gqa_factor, float scale,
                    int sliding_window, int kv_len, void* workspace, size_t workspace_bytes,
                    StreamOrDevice s = {});

// Workspace bytes of a decode call (tq_sdpa_int4_workspace_size).
size_t sdpa_int4_workspace_size(int batch, int num_heads, int num_kv_heads, int head_dim,
                                int max_kv_len);

// Batched ragged decode: queries (B, num_heads, head_dim), caches (B,
// num_kv_heads, capacity, .), seq_lens / windows int32 (B) device arrays
// (windows may be an empty array: sliding_window for all).
array sdpa_int4_ragged(const array& queries, const array& k_quant, const array& k_scales,
                       const array& k_biases, const array& v_quant, const array& v_scales,
                       const array& v_biases, const array& seq_lens, int gqa_factor,
                       float scale = 1.0f, int sliding_window = 0, const array& windows = {},
                       StreamOrDevice s = {});

// Multi-query (prefill) attention of the engine's fallback path
// (engine/gemma4_multilayer.cpp:343-364): queries (n_new, num_heads,
// head_dim) at positions n_prior .. n_prior+n_new-1 over rows
// [0, n_prior + n_new) of caches (num_kv_heads, capacity, .) that already
// hold the new rows; causal, and sliding_window > 0 limits each query to its
// last sliding_window keys.  Returns (n_new, num_heads, head_dim) f32.
array sdpa_int4_prefill(const array& queries, const array& k_quant, const array& k_scales,
                        const array& k_biases, const array& v_quant, const array& v_scales,
                        const array& v_biases, int n_prior, int gqa_factor, float scale = 1.0f,
                        int sliding_window = 0, StreamOrDevice s = {});

// ---- quantize / append (MLX quantize(x, 64, 4) at
// engine/gemma4_multilayer.cpp:228-229) --------------------------------------
// Returns {w_q uint32 (..., D/8), scales (..., D/64), biases (..., D/64)} with
// scales/biases in scale_dtype (float16 or float32).
std::vector<array> quantize(const array& x, int group_size = 64, int bits = 4,
                            Dtype scale_dtype = Dtype::float16, StreamOrDevice s = {});
array dequantize(const array& w, const array& scales, const array& biases, int group_size = 64,
                 int bits = 4, StreamOrDevice s = {});
// In-place append of k_new / v_new (B, Hkv, T, D) at rows positions[b] ..
// positions[b]+T-1 of (B, Hkv, capacity, .) caches (replaces the
// concatenate of engine/gemma4_multilayer.cpp:230-240).
void kv_append_int4(const array& k_new, const array& v_new, array& k_quant, array& k_scales,
                    array& k_biases, array& v_quant, array& v_scales, array& v_biases,
                    const array& positions, StreamOrDevice s = {});
// The same into rings of capacity rows (sliding-window eviction): token t
// goes to row (positions[b] + t) mod capacity, positions[b] = tokens seen.
void kv_append_int4_ring(const array& k_new, const array& v_new, array& k_quant,
                         array& k_scales, array& k_biases, array& v_quant, array& v_scales,
                         array& v_biases, const array& positions, StreamOrDevice s = {});

// ---- PolarQuant (lib/turboquant.h:52-165) -----------------------------------
// Reference layouts: 16-value blocks, 4 levels, codebooks per level.
std::vector<array> polar_quantize(const array& vectors, const array& precondition,
                                  const array& cb_l1, const array& cb_l2, const array& cb_l3,
                                  const array& cb_l4, int block_size = 16, StreamOrDevice s = {});
array polar_dequantize(const array& indices_l1, const array& indices_l2,
                       const array& indices_l3, const array& indices_l4, const array& radii,
                       const array& precondition, const array& cb_l1, const array& cb_l2,
                       const array& cb_l3, const array& cb_l4, int block_size = 16,
                       StreamOrDevice s = {});
std::vector<array> polar_quantize_packed(const array& vectors, const array& precondition,
                                         const array& cb_l1, const array& cb_l2,
                                         const array& cb_l3, const array& cb_l4,
                                         int block_size = 16, StreamOrDevice s = {});
array polar_dequantize_packed(const array& packed_l1, const array& packed_l2,
                              const array& packed_l3, const array& packed_l4,
                              const array& radii, const array& cb_l1, const array& cb_l2,
                              const array& cb_l3, const array& cb_l4, int D, int block_size = 16,
                              StreamOrDevice s = {});
array polar_dequantize_packed_fast(const array& packed_l1, const array& packed_l2,
                                   const array& packed_l3, const array& packed_l4,
                                   const array& radii, const array& cs_l1, const array& cs_l2,
                                   const array& cs_l3, const array& cs_l4, int D,
                                   int block_size = 16, StreamOrDevice s = {});
array compressed_sdpa(const array& queries, const array& indices_l1, const array& indices_l2,
                      const array& indices_l3, const array& indices_l4, const array& radii,
                      const array& cb_l1, const array& cb_l2, const array& cb_l3,
                      const array& cb_l4, const array& values, int block_size = 16,
                      float scale = 0.0884f, StreamOrDevice s = {});
array polar_dequantize_fast(const array& indices_l1, const array& indices_l2,
                            const array& indices_l3, const array& indices_l4, const array& radii,
                            const array& cb_l1, const array& cb_l2, const array& cb_l3,
                            const array& cb_l4, int D, int block_size = 16,
                            StreamOrDevice s = {});
array compressed_score(const array& queries, const array& indices_l1, const array& indices_l2,
                       const array& indices_l3, const array& indices_l4, const array& radii,
                       const array& cb_l1, const array& cb_l2, const array& cb_l3,
                       const array& cb_l4, int N, int block_size = 16, float scale = 0.0884f,
                       StreamOrDevice s = {});

// lib/turboquant.h:209: the Metal library path.  The HIP kernels are linked
// into the shared library, so the path is accepted and not used.
void set_metallib_path(const std::string& path);

}  // namespace turboquant
