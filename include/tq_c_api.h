/*
 * tq_c_api.h -- C ABI of the MI355X (gfx950) int4-KV decode-attention library
 * libturboquant_hip.so.
 *
 * Plain pointers and sizes only; every call is stream-ordered and asynchronous
 * on `stream` (a hipStream_t passed as void*, NULL = the null stream).  Callers
 * own every device buffer, including outputs and the split-K workspace: no
 * entry point allocates.  Every function returns a tq_status; on failure
 * tq_last_error() returns a message for the calling thread.
 *
 * Layouts (MLX affine int4, group size 64, lib/turboquant.h:196-201):
 *   quant   uint32 [.., rows, D/8]   8 nibbles per word, element i at bits [4i, 4i+4)
 *   scales  f16|f32 [.., rows, D/64] per-group scale
 *   biases  f16|f32 [.., rows, D/64] per-group bias; value = scale*nibble + bias
 * A KV cache of one sequence is [Hkv, capacity, .]; a batched cache is
 * [B, Hkv, capacity, .].  Rows [0, kv_len) of each head are valid.
 */
#ifndef TQ_C_API_H
#define TQ_C_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  TQ_OK = 0,
  TQ_ERR_INVALID = 1,     /* bad argument: null pointer, shape, dtype, alignment */
  TQ_ERR_UNSUPPORTED = 2, /* valid but not implemented (e.g. head_dim not in {128,256,512}) */
  TQ_ERR_HIP = 3,         /* a HIP runtime call failed */
  TQ_ERR_WORKSPACE = 4    /* workspace too small */
} tq_status;

typedef enum { TQ_F32 = 0, TQ_F16 = 1, TQ_BF16 = 2 } tq_dtype;

/* Quantization rule. TQ_QUANT_MLX reproduces MLX quantize(x, 64, 4)
 * (engine/gemma4_multilayer.cpp:228-229); TQ_QUANT_MINMAX is the literal
 * scale=(max-min)/15, bias=min rule. */
typedef enum { TQ_QUANT_MLX = 0, TQ_QUANT_MINMAX = 1 } tq_quant_mode;

/* ---- library / runtime --------------------------------------------------- */
int tq_version(void);                        /* 10000*major + 100*minor + patch */
const char* tq_last_error(void);             /* thread-local, never NULL */
int tq_device_count(int* count);
int tq_set_device(int device);
int tq_malloc(void** ptr, size_t bytes);
int tq_free(void* ptr);
int tq_memcpy_h2d(void* dst, const void* src, size_t bytes);
int tq_memcpy_d2h(void* dst, const void* src, size_t bytes);
int tq_memset(void* dst, int value, size_t bytes);
int tq_sync(void);

/* Measurement utility (no counterpart in the reference): a plain streaming
 * read of `bytes` (multiple of 16) by `blocks` x 256 threads, XOR-folded into
 * sink[blocks * 256].  The achievable-HBM-bandwidth reference for the
 * attention kernel's roofline. */
int tq_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks, void* stream);

/* ---- fused int4 decode attention ------------------------------------------
 * Replaces turboquant::sdpa_int4 (lib/turboquant.h:196-207,
 * lib/turboquant.cpp:367-417).  out[h] = softmax(scale * q[h] . K^T) V over
 * the dequantized rows of kv head h / gqa_factor; key ki is skipped when
 * sliding_window > 0 and kv_len-1-ki >= sliding_window
 * (lib/turboquant.metal:779); an empty key set gives 0 (:886).
 *   q        [num_heads, head_dim] in q_dtype (f32, f16 or bf16)
 *   out      [num_heads, head_dim] f32
 *   head_dim in {128, 256, 512}; num_heads == num_kv_heads * gqa_factor
 *   kv_capacity >= kv_len is the row stride of each head (== kv_len for a
 *   tight [Hkv, N, .] tensor as in the reference).
 * workspace: >= tq_sdpa_int4_workspace_size(...) bytes, zero-filled once
 * before first use.  Its first 256 KiB hold split counters that every call
 * returns to zero, so one workspace may serve calls of any shape one after
 * another on a stream; calls that run concurrently need separate workspaces.
 * batch * num_heads must not exceed 65536. */
size_t tq_sdpa_int4_workspace_size(int batch, int num_heads, int num_kv_heads,
                                   int head_dim, int max_kv_len);
int tq_sdpa_int4(const void* q, tq_dtype q_dtype,
                 const uint32_t* k_quant, const void* k_scales, const void* k_biases,
                 const uint32_t* v_quant, const void* v_scales, const void* v_biases,
                 tq_dtype sb_dtype, float* out,
                 int num_heads, int num_kv_heads, int head_dim, int kv_len, int kv_capacity,
                 int gqa_factor, float scale, int sliding_window,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Batched ragged decode: sequence b attends rows [0, seq_lens[b]) of its cache
 * under window windows[b] (windows == NULL -> sliding_window for all).
 * seq_lens / windows are DEVICE int32 arrays of length batch; max_kv_len must
 * bound every seq_lens[b] (it sizes the launch grid).
 *   q [batch, num_heads, head_dim]; caches [batch, num_kv_heads, kv_capacity, .];
 *   out [batch, num_heads, head_dim] f32.
 * The reference has no batch dimension (lib/turboquant.cpp:392,400); this is
 * the same operator applied per sequence. */
int tq_sdpa_int4_ragged(const void* q, tq_dtype q_dtype,
                        const uint32_t* k_quant, const void* k_scales, const void* k_biases,
                        const uint32_t* v_quant, const void* v_scales, const void* v_biases,
                        tq_dtype sb_dtype, float* out,
                        int batch, int num_heads, int num_kv_heads, int head_dim,
                        int kv_capacity, const int32_t* seq_lens, const int32_t* windows,
                        int max_kv_len, int gqa_factor, float scale, int sliding_window,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ---- quantize / append ----------------------------------------------------
 * tq_quantize_int4 replaces MLX quantize(x, 64, 4) as called at
 * engine/gemma4_multilayer.cpp:228-229: rows x dim values of x (x_dtype) ->
 * w_q [rows, dim/8] uint32 + scales/biases [rows, dim/64] in sb_dtype (the
 * float32 scale/bias used for the nibbles, cast round-to-nearest-even).
 * dim must be a multiple of 64 and at most 4096; group_size must be 64, bits 4. */
int tq_quantize_int4(const void* x, tq_dtype x_dtype, int64_t rows, int dim,
                     int group_size, int bits, tq_quant_mode mode,
                     uint32_t* w_q, void* scales, void* biases, tq_dtype sb_dtype,
                     void* stream);

/* tq_kv_append_int4 replaces the quantize + concatenate append of
 * engine/gemma4_multilayer.cpp:228-240 with an in-place write: k_new / v_new
 * [batch, num_kv_heads, n_new, head_dim] are quantized and stored at rows
 * positions[b] .. positions[b]+n_new-1 of the [batch, num_kv_heads,
 * kv_capacity, .] caches.  positions is a DEVICE int32 array; rows that
 * would fall outside [0, kv_capacity) are not written. */
int tq_kv_append_int4(const void* k_new, const void* v_new, tq_dtype x_dtype,
                      uint32_t* k_quant, void* k_scales, void* k_biases,
                      uint32_t* v_quant, void* v_scales, void* v_biases, tq_dtype sb_dtype,
                      int batch, int num_kv_heads, int head_dim, int kv_capacity,
                      const int32_t* positions, int n_new, tq_quant_mode mode,
                      void* stream);

/* Dequantize rows (for the engine's prefill fallback,
 * engine/gemma4_multilayer.cpp:307-308): out[r, d] = s*nibble + b as f32. */
int tq_dequantize_int4(const uint32_t* w_q, const void* scales, const void* biases,
                       tq_dtype sb_dtype, int64_t rows, int dim, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TQ_C_API_H */
