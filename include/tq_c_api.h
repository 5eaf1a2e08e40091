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

/* Measurement utility (no counterpart in the reference): a streaming read in
 * the decode-attention kernel's geometry -- `blocks` workgroups of `waves`
 * wave64s, workgroup b reading the b-th contiguous slice of `bytes`, each
 * lane issuing `loads_per_lane` 16-byte loads per iteration with `depth`
 * iterations in flight, non-temporal when `nontemporal` != 0.  sink holds
 * blocks * waves * 64 words.  (waves, loads_per_lane) is one of (8,4) (8,9)
 * (8,16) (4,9) (4,16) (16,4) (16,9); depth is 1, 2 or 3. */
int tq_stream_read_tiles(const void* src, size_t bytes, uint32_t* sink, int blocks, int waves,
                         int loads_per_lane, int depth, int nontemporal, void* stream);

/* ---- fused int4 decode attention ------------------------------------------
 * Replaces turboquant::sdpa_int4 (lib/turboquant.h:196-207,
 * lib/turboquant.cpp:367-417).  out[h] = softmax(scale * q[h] . K^T) V over
 * the dequantized rows of kv head h / gqa_factor; key ki is skipped when
 * sliding_window > 0 and kv_len-1-ki >= sliding_window
 * (lib/turboquant.metal:779); an empty key set gives 0 (:886).
 *   q        [num_heads, head_dim] in q_dtype (f32, f16 or bf16), 16-byte
 *            aligned (as k_quant and v_quant)
 *   out      [num_heads, head_dim] f32
 *   head_dim in {128, 256, 512}; num_heads == num_kv_heads * gqa_factor
 *   kv_capacity >= kv_len is the row stride of each head (== kv_len for a
 *   tight [Hkv, N, .] tensor as in the reference).
 * workspace: >= tq_sdpa_int4_workspace_size(...) bytes, 16-byte aligned,
 * zero-filled once before first use.  Its first 256 KiB hold split counters that every call
 * returns to zero, so one workspace may serve calls of any shape one after
 * another on a stream; calls that run concurrently need separate workspaces.
 * batch * num_heads must not exceed 65536. */
size_t tq_sdpa_int4_workspace_size(int batch, int num_heads, int num_kv_heads,
                                   int head_dim, int max_kv_len);

/* tq_sdpa_int4 without a caller workspace.  No counterpart in the reference:
 * for callers that cannot allocate (HIP graph capture, allocation-free
 * serving loops).  The split-K workspace is a library-owned static device
 * array of 8 MiB per GPU (held until the process ends), which covers every
 * single-sequence decode shape under the default split planner; a shape
 * that would need more returns TQ_ERR_UNSUPPORTED before any GPU work.
 * Allocates nothing.  All calls on one GPU share its array: calls that
 * overlap on one GPU (concurrent streams, or graphs replayed concurrently)
 * race.  Arguments as tq_sdpa_int4. */
int tq_sdpa_int4_noalloc(const void* q, tq_dtype q_dtype,
                         const uint32_t* k_quant, const void* k_scales, const void* k_biases,
                         const uint32_t* v_quant, const void* v_scales, const void* v_biases,
                         tq_dtype sb_dtype, float* out, int num_heads, int num_kv_heads,
                         int head_dim, int kv_len, int kv_capacity, int gqa_factor, float scale,
                         int sliding_window, void* stream);

/* Planning query (no counterpart in the reference, whose eval_gpu picks a
 * kernel by name at lib/turboquant.cpp:376-379): the kernel a call with
 * these arguments launches and its split plan, with no GPU work.  mode 0 =
 * tq_sdpa_int4 (max_kv_len = kv_len), 1 = tq_sdpa_int4_ragged, 2 =
 * tq_sdpa_int4_prefill (batch = n_new, max_kv_len = n_prior + n_new).
 * *splits = workgroups per sequence along the keys (grid x), *chunk_keys =
 * keys per split; the kernel's name is written to kernel[kernel_bytes].
 * The cache capacity is taken as max_kv_len: caches of fewer than 32 rows
 * run the VALU kernel (the matrix-core kernel reads 32-row blocks). */
int tq_sdpa_int4_plan(int mode, int batch, int num_heads, int num_kv_heads, int head_dim,
                      int max_kv_len, tq_dtype sb_dtype, int sliding_window, int* splits,
                      int* chunk_keys, char* kernel, size_t kernel_bytes);

/* Re-reads the kernel-choice switches from the environment (no counterpart
 * in the reference).  They are read once per process otherwise:
 * TQ_SDPA_IMPL=valu, TQ_SDPA_CHUNK=<keys>, TQ_PREFILL_IMPL=splitk,
 * TQ_PREFILL_WS=0, TQ_HC_IMPL=1.  For tests and measurement; calls that run
 * while it executes see the old or the new values. */
int tq_reload_options(void);
int tq_sdpa_int4(const void* q, tq_dtype q_dtype,
                 const uint32_t* k_quant, const void* k_scales, const void* k_biases,
                 const uint32_t* v_quant, const void* v_scales, const void* v_biases,
                 tq_dtype sb_dtype, float* out,
                 int num_heads, int num_kv_heads, int head_dim, int kv_len, int kv_capacity,
                 int gqa_factor, float scale, int sliding_window,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Batched ragged decode: sequence b attends rows [0, seq_lens[b]) of its cache
 * under window windows[b] (windows == NULL -> sliding_window for all).
 * seq_lens / windows are DEVICE int32 arrays of length batch; max_kv_len
 * (<= kv_capacity) sizes the launch grid, and a seq_lens[b] above it is
 * clamped to it (a ring cache passes tokens seen, see
 * tq_kv_append_int4_ring).
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

/* Multi-query (prefill) attention over one cache: the n_new queries
 * q [n_new, num_heads, head_dim] at positions n_prior .. n_prior+n_new-1
 * attend rows [0, n_prior + n_new) of the [num_kv_heads, kv_capacity, .]
 * caches, which must already hold the new rows.  Query i sees key j iff
 * j <= n_prior + i and, for sliding_window > 0, n_prior + i - j <
 * sliding_window: the mask of the reference's prefill fallback
 * (engine/gemma4_multilayer.cpp:343-364, dequantize + masked
 * scaled_dot_product_attention).  out [n_new, num_heads, head_dim] f32.
 * Workspace: tq_sdpa_int4_workspace_size(n_new, num_heads, num_kv_heads,
 * head_dim, n_prior + n_new) bytes (zero-filled once, as for decode). */
int tq_sdpa_int4_prefill(const void* q, tq_dtype q_dtype,
                         const uint32_t* k_quant, const void* k_scales, const void* k_biases,
                         const uint32_t* v_quant, const void* v_scales, const void* v_biases,
                         tq_dtype sb_dtype, float* out,
                         int num_heads, int num_kv_heads, int head_dim,
                         int n_prior, int n_new, int kv_capacity,
                         int gqa_factor, float scale, int sliding_window,
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

/* tq_kv_append_int4_ring: the same quantize-and-store into a ring of
 * kv_capacity rows per (sequence, kv head), the window eviction of a
 * sliding-attention layer (the reference instead trims with `slice`,
 * engine/gemma4_multilayer.cpp:243-248).  positions[b] >= 0 is the number of
 * tokens sequence b has seen; token t of the append goes to row
 * (positions[b] + t) mod kv_capacity, and of an append longer than the ring
 * only its last kv_capacity tokens are stored.  The ring then holds exactly
 * the keys the reference window rule keeps (lib/turboquant.metal:779) when
 * kv_capacity equals the window; attend with tq_sdpa_int4_ragged, seq_lens =
 * tokens seen, max_kv_len = kv_capacity (lengths are clamped to it) and
 * window 0 -- attention does not depend on the order of the keys. */
int tq_kv_append_int4_ring(const void* k_new, const void* v_new, tq_dtype x_dtype,
                           uint32_t* k_quant, void* k_scales, void* k_biases,
                           uint32_t* v_quant, void* v_scales, void* v_biases, tq_dtype sb_dtype,
                           int batch, int num_kv_heads, int head_dim, int kv_capacity,
                           const int32_t* positions, int n_new, tq_quant_mode mode,
                           void* stream);

/* Dequantize rows (for the engine's prefill fallback,
 * engine/gemma4_multilayer.cpp:307-308): out[r, d] = s*nibble + b as f32. */
int tq_dequantize_int4(const uint32_t* w_q, const void* scales, const void* biases,
                       tq_dtype sb_dtype, int64_t rows, int dim, float* out, void* stream);

/* ---- PolarQuant, reference layouts (16-value blocks, 4 levels) -------------
 * Codebooks: `codebooks` is a DEVICE float array holding the level 1..4
 * codebooks back to back (angles, radians); `n_codebook` a HOST int[4] with
 * their sizes.  Level 1 angles are atan2 wrapped to [0, 2pi), levels 2-4 are
 * in [0, pi/2]; each angle becomes the index of the nearest entry under
 * |theta - c| (first minimum wins, lib/turboquant.metal:38-42).  Sizes: <= 256
 * per level unpacked; <= 16 (level 1) and <= 4 (levels 2-4) packed.
 * Blocks are the n_vectors * dim / 16 consecutive 16-value slices of the
 * (rotated) vectors, in row-major order.  block_size must be 16 (the
 * reference kernels hard-code it, lib/turboquant.metal:25-27). */

/* Replaces turboquant::polar_quantize (lib/turboquant.h:52-60,
 * lib/turboquant.cpp:97-110; kernel lib/turboquant.metal:8-98).  x [n, dim]
 * f32; precondition [dim, dim] f32 (y = x P^T) or NULL when x is already
 * rotated.  Outputs idx_l1 u8 [nb*8], idx_l2 [nb*4], idx_l3 [nb*2],
 * idx_l4 [nb], radii f16 bits [nb]. */
int tq_polar_quantize(const float* x, const float* precondition, const float* codebooks,
                      const int* n_codebook, int64_t n_vectors, int dim, int block_size,
                      uint8_t* idx_l1, uint8_t* idx_l2, uint8_t* idx_l3, uint8_t* idx_l4,
                      uint16_t* radii, void* stream);

/* Replaces turboquant::polar_quantize_packed (lib/turboquant.h:77-82,
 * lib/turboquant.cpp:255-272; kernel lib/turboquant.metal:501-600): per
 * block one u32 (level-1 index j at bits 4j), one u8 each for levels 2, 3, 4
 * (index j at bits 2j), one f16 radius. */
int tq_polar_quantize_packed(const float* x, const float* precondition, const float* codebooks,
                             const int* n_codebook, int64_t n_vectors, int dim, int block_size,
                             uint32_t* packed_l1, uint8_t* packed_l2, uint8_t* packed_l3,
                             uint8_t* packed_l4, uint16_t* radii, void* stream);

/* Replaces turboquant::polar_dequantize (precondition != NULL: x = y P,
 * lib/turboquant.cpp:112-123) and polar_dequantize_fast (precondition ==
 * NULL: y only, lib/turboquant.cpp:191-200); kernel
 * lib/turboquant.metal:100-164.  out [n_vectors, dim] f32. */
int tq_polar_dequantize(const uint8_t* idx_l1, const uint8_t* idx_l2, const uint8_t* idx_l3,
                        const uint8_t* idx_l4, const uint16_t* radii, const float* precondition,
                        const float* codebooks, const int* n_codebook, int64_t n_vectors, int dim,
                        int block_size, float* out, void* stream);

/* Replaces polar_dequantize_packed (cs_tables == NULL: cos/sin of the
 * codebook angles, lib/turboquant.cpp:274-282, kernel
 * lib/turboquant.metal:602-653) and polar_dequantize_packed_fast (cs_tables =
 * DEVICE float (cos, sin) pairs laid out like the codebooks,
 * lib/turboquant.cpp:312-320, kernel :655-704).  Output y (no
 * preconditioner), as the reference. */
int tq_polar_dequantize_packed(const uint32_t* packed_l1, const uint8_t* packed_l2,
                               const uint8_t* packed_l3, const uint8_t* packed_l4,
                               const uint16_t* radii, const float* codebooks,
                               const float* cs_tables, const int* n_codebook, int64_t n_vectors,
                               int dim, int block_size, float* out, void* stream);

/* Replaces turboquant::compressed_score (lib/turboquant.h:157-165,
 * lib/turboquant.cpp:323-359; kernel tq_score_shared,
 * lib/turboquant.metal:424-499): scores[h, n] = sum_d scale q[h, d]
 * khat[(h / gqa) * n_keys + n, d] for q [num_heads, dim] f32 (preconditioned),
 * keys of num_kv_heads heads x n_keys; gqa = num_heads / num_kv_heads (the
 * reference is gqa = 1).  dim in {64, 128, 256}. scores [num_heads, n_keys]. */
int tq_compressed_score(const float* q, int num_heads, const uint8_t* idx_l1, const uint8_t* idx_l2,
                        const uint8_t* idx_l3, const uint8_t* idx_l4, const uint16_t* radii,
                        const float* codebooks, const int* n_codebook, int num_kv_heads,
                        int n_keys, int dim, int block_size, float scale, float* scores,
                        void* stream);
/* The same over the packed layout (no reference counterpart: the reference
 * scores only unpacked keys). */
int tq_compressed_score_packed(const float* q, int num_heads, const uint32_t* packed_l1,
                               const uint8_t* packed_l2, const uint8_t* packed_l3,
                               const uint8_t* packed_l4, const uint16_t* radii,
                               const float* codebooks, const int* n_codebook, int num_kv_heads,
                               int n_keys, int dim, int block_size, float scale, float* scores,
                               void* stream);

/* Replaces turboquant::compressed_sdpa (lib/turboquant.h:127-143,
 * lib/turboquant.cpp:125-188; kernel sdpa_tq_sequential,
 * lib/turboquant.metal:166-224): out[h] = sum_n softmax(scores[h])_n
 * values[(h / gqa) * n_keys + n] / (l + 1e-8) semantics of :222, values
 * [num_kv_heads * n_keys, dim] f32.  Split-K: workspace as tq_sdpa_int4
 * (zero-filled once, its first 256 KiB are counters that calls return to
 * zero). */
size_t tq_compressed_sdpa_workspace_size(int num_heads, int num_kv_heads, int dim, int max_n_keys);
int tq_compressed_sdpa(const float* q, int num_heads, const uint8_t* idx_l1, const uint8_t* idx_l2,
                       const uint8_t* idx_l3, const uint8_t* idx_l4, const uint16_t* radii,
                       const float* codebooks, const int* n_codebook, const float* values,
                       int num_kv_heads, int n_keys, int dim, int block_size, float scale,
                       float* out, void* workspace, size_t workspace_bytes, void* stream);

/* ---- 7-level PolarQuant + QJL ("polar7"; D = 128) ---------------------------
 * No reference kernel: the same polar recursion as polar_quantize over one
 * 128-value block (7 levels; level-1 angles 4-bit, levels 2-7 2-bit) plus
 * the QJL residual sketch the reference README describes (README.md:11,176).
 * Per vector (row of a [.., capacity, .] cache):
 *   angles u32 [12]: words 0-7 level 1 (pair j at word j/8, bits 4(j%8)),
 *     words 8-9 level 2 (pair j at word 8 + j/16, bits 2(j%16)), word 10
 *     level 3 (bits 2j), word 11 levels 4 (bits 2j), 5 (16+2j), 6 (24+2j),
 *     7 (28-29);
 *   norms u32: fp16 radius (bits 0-15) | fp16 ||r|| (bits 16-31);
 *   qjl u32 [4]: bit i of word i/32 = [(S r)_i >= 0], r = y - yhat.
 * codebooks: DEVICE float[20] = level-1 codebook [16] then the levels 2-7
 * codebook [4]; cs_tables: DEVICE float[40] = their (cos, sin) pairs (the
 * decoder's tables; the encoder's residual uses the same values).
 * sketch: DEVICE S [128][128] f32. */
int tq_polar7_encode(const float* x, const float* precondition, const float* sketch,
                     const float* codebooks, const float* cs_tables, int64_t n_vectors,
                     uint32_t* angles, uint32_t* norms, uint32_t* qjl, void* stream);
/* Encode k_new [batch, num_kv_heads, n_new, 128] f32 into rows
 * positions[b] .. positions[b] + n_new - 1 of the [batch, num_kv_heads,
 * kv_capacity, .] caches (rows outside [0, kv_capacity) are not written). */
int tq_polar7_kv_append(const float* k_new, const float* precondition, const float* sketch,
                        const float* codebooks, const float* cs_tables, uint32_t* angles,
                        uint32_t* norms, uint32_t* qjl, int batch, int num_kv_heads,
                        int kv_capacity, const int32_t* positions, int n_new, void* stream);
/* y = x P^T for rows of 128 (the query rotation q' = P q), and the query
 * sketch S q' (utilities; tq_polar7_prepare_query does both). */
int tq_polar_rotate(const float* x, const float* precondition, int64_t rows, int dim, float* y,
                    void* stream);
int tq_qjl_query(const float* q_rot, const float* sketch, int num_heads, float* q_sketch,
                 void* stream);

/* Query side of a decode step: q [num_heads, 128] f32 -> q' = P q
 * (precondition NULL: q' = q), S q', and the per-head tables the score
 * kernels read, TQ_POLAR7_QTAB floats per head in q_tables (16-byte
 * aligned): [64][16] level-1 table q'[2j] cos c_k + q'[2j+1] sin c_k,
 * [16][256] QJL byte table (sum of (S q')_{8 pos + i} over the set bits i),
 * then sum(S q') as the sum of four floats, and padding.  q_rot / q_sketch
 * ([num_heads, 128]) are optional copies of q' and S q' (NULL: not
 * written). */
#define TQ_POLAR7_QTAB 5136
int tq_polar7_prepare_query(const float* q, const float* precondition, const float* sketch,
                            const float* cs_tables, int num_heads, float* q_tables, float* q_rot,
                            float* q_sketch, void* stream);
/* No counterpart in the reference (QJL is this build's addition, README.md:
 * 11,176): sketch_precondition [128][128] = S P (S when precondition is
 * NULL), computed once per codec. */
int tq_polar7_sketch_precondition(const float* precondition, const float* sketch,
                                  float* sketch_precondition, void* stream);
/* The same tables as tq_polar7_prepare_query from S P in place of S: S q'
 * is then (S P) q, a product of q independent of q', so the tables of a
 * head are built in four parts of 32 rows each, without a second product
 * pass (no counterpart in the reference, as above). */
int tq_polar7_prepare_query_sp(const float* q, const float* precondition,
                               const float* sketch_precondition, const float* cs_tables,
                               int num_heads, float* q_tables, float* q_rot, float* q_sketch,
                               void* stream);
/* scores[h, n] = scale * (<q'_h, yhat_n> + sqrt(pi/2)/128 * ||r_n|| *
 * <S q'_h, sign(S r_n)>) over rows [0, kv_len) of kv head h / gqa. */
int tq_polar7_score(const float* q_tables, const uint32_t* angles, const uint32_t* norms,
                    const uint32_t* qjl, const float* cs_tables, int num_heads, int num_kv_heads,
                    int kv_len, int kv_capacity, float scale, float* scores, void* stream);
/* The same scores straight from q [num_heads, 128] f32: each workgroup
 * builds the query tables of its heads (as tq_polar7_prepare_query_sp) in
 * its prologue, one launch in all (no counterpart in the reference, as
 * above; compressed_score, lib/turboquant.h:157-165, also scores from the
 * preconditioned query in one launch). */
int tq_polar7_score_q(const float* q, const float* precondition, const float* sketch_precondition,
                      const float* cs_tables, const uint32_t* angles, const uint32_t* norms,
                      const uint32_t* qjl, int num_heads, int num_kv_heads, int kv_len,
                      int kv_capacity, float scale, float* scores, void* stream);
/* Decode attention over those scores (window rule and empty-set rule of
 * tq_sdpa_int4) with int4 V [num_kv_heads, kv_capacity, 16] + scale/bias
 * [.., 2] in sb_dtype; out [num_heads, 128] f32.  Workspace as
 * tq_sdpa_int4. */
size_t tq_polar7_sdpa_workspace_size(int num_heads, int num_kv_heads, int max_kv_len);
int tq_polar7_sdpa_int4v(const float* q_tables, const uint32_t* angles,
                         const uint32_t* norms, const uint32_t* qjl, const float* cs_tables,
                         const uint32_t* v_quant, const void* v_scales, const void* v_biases,
                         tq_dtype sb_dtype, float* out, int num_heads, int num_kv_heads,
                         int kv_len, int kv_capacity, float scale, int sliding_window,
                         void* workspace, size_t workspace_bytes, void* stream);
/* The same attention straight from q [num_heads, 128] f32: each workgroup
 * builds the query tables of its heads (as tq_polar7_prepare_query_sp, from
 * precondition P -- NULL: q' = q -- and sketch_precondition = S P) in its
 * prologue, so a decode step is one launch.  No counterpart in the
 * reference (polar7 and QJL are this build's, README.md:11,176). */
int tq_polar7_sdpa_int4v_q(const float* q, const float* precondition,
                           const float* sketch_precondition, const float* cs_tables,
                           const uint32_t* angles, const uint32_t* norms, const uint32_t* qjl,
                           const uint32_t* v_quant, const void* v_scales, const void* v_biases,
                           tq_dtype sb_dtype, float* out, int num_heads, int num_kv_heads,
                           int kv_len, int kv_capacity, float scale, int sliding_window,
                           void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TQ_C_API_H */
