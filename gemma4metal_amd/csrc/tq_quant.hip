// Affine int4 quantize / in-place KV append / dequantize for gfx950.
//
// One lane owns one output word (8 consecutive elements); the 8 lanes of a
// 64-element group find the group min/max with three xor exchanges, so a wave
// quantizes 8 groups per instruction stream with 16-32 B coalesced loads and a
// 4 B store per lane.  All arithmetic is IEEE float32 in the order of the MLX
// rule (no contraction: there is no a*b+c in it), with rint = v_rndne_f32 and
// correctly rounded division, so the nibbles are bit-identical to MLX
// quantize(x, 64, 4) (engine/gemma4_multilayer.cpp:228-229).
#include "tq_internal.h"

namespace tq {
namespace {

struct QuantJob {
  const void* x;
  uint32_t* wq;
  void* s;
  void* b;
};

struct QuantParams {
  QuantJob job[2];      // [0] = K (or the only tensor), [1] = V
  int x_dtype;
  int64_t rows;         // input rows per job
  int dim;
  int mode;             // tq_quant_mode
  const int32_t* pos;   // append: per-sequence start row (device); nullptr = identity
  int heads;            // append: kv heads per sequence
  int n_new;            // append: rows per (sequence, head)
  int cap;              // append: cache capacity (row stride per head)
  int ring;             // append: rows (pos[b] + t) mod cap, last cap rows of n_new only
};

__device__ __forceinline__ void load8(const void* x, int dtype, int64_t off, float v[8]) {
  if (dtype == TQ_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + off);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + off);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = w[i] & 0xFFFFu, hi = w[i] >> 16;
      if (dtype == TQ_F16) {
        v[2 * i] = __half2float(__ushort_as_half(lo));
        v[2 * i + 1] = __half2float(__ushort_as_half(hi));
      } else {
        v[2 * i] = bf16_to_f32(lo);
        v[2 * i + 1] = bf16_to_f32(hi);
      }
    }
  }
}

template <typename SB>
__global__ __launch_bounds__(256) void quantize_int4_kernel(QuantParams p) {
  // every argument in one batch of scalar loads (one memory round trip),
  // the job picked by a select rather than a load indexed by blockIdx.y
  asm volatile("" ::"s"(p.job[0].x), "s"(p.job[0].wq), "s"(p.job[0].s), "s"(p.job[0].b),
               "s"(p.job[1].x), "s"(p.job[1].wq), "s"(p.job[1].s), "s"(p.job[1].b),
               "s"(p.x_dtype), "s"(p.rows), "s"(p.dim), "s"(p.mode), "s"(p.pos), "s"(p.heads),
               "s"(p.n_new), "s"(p.cap), "s"(p.ring));
  const QuantJob J = blockIdx.y ? p.job[1] : p.job[0];
  const int wpr = p.dim >> 3;  // words per row
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = gid / wpr;
  const int w = static_cast<int>(gid - row * wpr);
  if (row >= p.rows) return;  // whole 8-lane groups leave together (wpr % 8 == 0)

  float v[8];
  load8(J.x, p.x_dtype, row * p.dim + static_cast<int64_t>(w) * 8, v);

  float mx = v[0], mn = v[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    mx = fmaxf(mx, v[i]);
    mn = fminf(mn, v[i]);
  }
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) {
    mx = fmaxf(mx, shfl_xor_f(mx, off));
    mn = fminf(mn, shfl_xor_f(mn, off));
  }

  const float n_bins = 15.0f, eps = 1e-7f;
  float d = (mx - mn) / n_bins;
  float scale = d < eps ? eps : d;
  float bias;
  if (p.mode == TQ_QUANT_MLX) {
    const bool side = fabsf(mn) > fabsf(mx);
    scale = side ? scale : -scale;
    const float edge = side ? mn : mx;
    const float q0 = __builtin_rintf(edge / scale);
    bias = 0.0f;
    if (q0 != 0.0f) {
      scale = edge / q0;
      bias = edge;
    }
  } else {
    bias = mn;
  }

  uint32_t word = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float q = __builtin_rintf((v[k] - bias) / scale);
    q = q < 0.0f ? 0.0f : (q > n_bins ? n_bins : q);
    word |= static_cast<uint32_t>(q) << (4 * k);
  }

  int64_t drow = row;
  if (p.pos != nullptr) {
    // input row = ((b * heads + h) * n_new + t) -> cache row (b*heads+h)*cap + pos[b] + t
    const int64_t bh = row / p.n_new;
    const int t = static_cast<int>(row - bh * p.n_new);
    const int64_t b = bh / p.heads;
    int dst = p.pos[b] + t;
    if (p.ring) {
      // a ring keeps the newest cap rows: older rows of this append would
      // land on the same slots, so they are not written at all
      if (p.pos[b] < 0 || t < p.n_new - p.cap) return;
      dst %= p.cap;
    }
    if (dst < 0 || dst >= p.cap) return;
    drow = bh * p.cap + dst;
  }
  J.wq[drow * wpr + w] = word;
  if ((w & 7) == 0) {
    const int ng = p.dim >> 6;
    static_cast<SB*>(J.s)[drow * ng + (w >> 3)] = f32_to_sb<SB>(scale);
    static_cast<SB*>(J.b)[drow * ng + (w >> 3)] = f32_to_sb<SB>(bias);
  }
}

template <typename SB>
__global__ __launch_bounds__(256) void dequantize_int4_kernel(const uint32_t* wq, const SB* s,
                                                              const SB* b, int64_t rows,
                                                              int dim, float* out) {
  const int wpr = dim >> 3;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= rows * wpr) return;
  const int64_t row = gid / wpr;
  const int w = static_cast<int>(gid - row * wpr);
  const uint32_t word = wq[gid];
  const int g = (w * 8) >> 6;
  const float sc = sb_to_f32<SB>(s[row * (dim >> 6) + g]);
  const float bi = sb_to_f32<SB>(b[row * (dim >> 6) + g]);
  float4 o0, o1;
  o0.x = sc * static_cast<float>(word & 0xF) + bi;
  o0.y = sc * static_cast<float>((word >> 4) & 0xF) + bi;
  o0.z = sc * static_cast<float>((word >> 8) & 0xF) + bi;
  o0.w = sc * static_cast<float>((word >> 12) & 0xF) + bi;
  o1.x = sc * static_cast<float>((word >> 16) & 0xF) + bi;
  o1.y = sc * static_cast<float>((word >> 20) & 0xF) + bi;
  o1.z = sc * static_cast<float>((word >> 24) & 0xF) + bi;
  o1.w = sc * static_cast<float>(word >> 28) + bi;
  float4* o = reinterpret_cast<float4*>(out + gid * 8);
  o[0] = o0;
  o[1] = o1;
}

int check_align(const void* p, size_t a, const char* what) {
  if (reinterpret_cast<uintptr_t>(p) % a != 0) {
    set_error("%s must be %zu-byte aligned", what, a);
    return TQ_ERR_INVALID;
  }
  return TQ_OK;
}

int launch_quantize(const QuantParams& p, int jobs, int sb_dtype, hipStream_t stream) {
  const int64_t lanes = p.rows * (p.dim / 8);
  if (lanes == 0) return TQ_OK;
  const int64_t blocks = (lanes + 255) / 256;
  if (blocks > 0x7FFFFFFF) {
    set_error("quantize: too many rows");
    return TQ_ERR_INVALID;
  }
  dim3 grid(static_cast<unsigned>(blocks), jobs);
  if (sb_dtype == TQ_F16)
    quantize_int4_kernel<__half><<<grid, 256, 0, stream>>>(p);
  else
    quantize_int4_kernel<float><<<grid, 256, 0, stream>>>(p);
  TQ_CHECK_LAUNCH("quantize_int4_kernel");
  return TQ_OK;
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" int tq_quantize_int4(const void* x, tq_dtype x_dtype, int64_t rows, int dim,
                                int group_size, int bits, tq_quant_mode mode, uint32_t* w_q,
                                void* scales, void* biases, tq_dtype sb_dtype, void* stream) {
  clear_error();
  TQ_CHECK_ARG(group_size == 64 && bits == 4,
               "tq_quantize_int4: only group_size=64, bits=4 (got %d, %d)", group_size, bits);
  TQ_CHECK_ARG(valid_dtype(x_dtype), "tq_quantize_int4: bad x_dtype %d", (int)x_dtype);
  TQ_CHECK_ARG(sb_dtype == TQ_F16 || sb_dtype == TQ_F32,
               "tq_quantize_int4: sb_dtype must be f16 or f32");
  TQ_CHECK_ARG(mode == TQ_QUANT_MLX || mode == TQ_QUANT_MINMAX, "tq_quantize_int4: bad mode");
  TQ_CHECK_ARG(dim > 0 && dim % 64 == 0 && dim <= 4096,
               "tq_quantize_int4: dim must be a positive multiple of 64 <= 4096 (got %d)", dim);
  TQ_CHECK_ARG(rows >= 0, "tq_quantize_int4: rows < 0");
  if (rows == 0) return TQ_OK;
  TQ_CHECK_ARG(x && w_q && scales && biases, "tq_quantize_int4: null pointer");
  if (int r = check_align(x, 16, "x")) return r;
  QuantParams p{};
  p.job[0] = {x, w_q, scales, biases};
  p.x_dtype = x_dtype;
  p.rows = rows;
  p.dim = dim;
  p.mode = mode;
  return launch_quantize(p, 1, sb_dtype, static_cast<hipStream_t>(stream));
}

namespace {
int kv_append(const void* k_new, const void* v_new, tq_dtype x_dtype, uint32_t* k_quant,
              void* k_scales, void* k_biases, uint32_t* v_quant, void* v_scales, void* v_biases,
              tq_dtype sb_dtype, int batch, int num_kv_heads, int head_dim, int kv_capacity,
              const int32_t* positions, int n_new, tq_quant_mode mode, int ring, void* stream,
              const char* fn) {
  clear_error();
  TQ_CHECK_ARG(valid_dtype(x_dtype), "%s: bad x_dtype", fn);
  TQ_CHECK_ARG(sb_dtype == TQ_F16 || sb_dtype == TQ_F32,
               "%s: sb_dtype must be f16 or f32", fn);
  TQ_CHECK_ARG(mode == TQ_QUANT_MLX || mode == TQ_QUANT_MINMAX, "%s: bad mode", fn);
  TQ_CHECK_ARG(head_dim > 0 && head_dim % 64 == 0 && head_dim <= 4096,
               "%s: head_dim must be a multiple of 64 <= 4096", fn);
  TQ_CHECK_ARG(batch >= 0 && num_kv_heads > 0 && n_new >= 0 && kv_capacity > 0,
               "%s: bad sizes", fn);
  if (batch == 0 || n_new == 0) return TQ_OK;
  TQ_CHECK_ARG(k_new && v_new && k_quant && k_scales && k_biases && v_quant && v_scales &&
                   v_biases && positions,
               "%s: null pointer", fn);
  if (int r = check_align(k_new, 16, "k_new")) return r;
  if (int r = check_align(v_new, 16, "v_new")) return r;
  QuantParams p{};
  p.job[0] = {k_new, k_quant, k_scales, k_biases};
  p.job[1] = {v_new, v_quant, v_scales, v_biases};
  p.x_dtype = x_dtype;
  p.rows = static_cast<int64_t>(batch) * num_kv_heads * n_new;
  p.dim = head_dim;
  p.mode = mode;
  p.pos = positions;
  p.heads = num_kv_heads;
  p.n_new = n_new;
  p.cap = kv_capacity;
  p.ring = ring;
  return launch_quantize(p, 2, sb_dtype, static_cast<hipStream_t>(stream));
}
}  // namespace

extern "C" int tq_kv_append_int4(const void* k_new, const void* v_new, tq_dtype x_dtype,
                                 uint32_t* k_quant, void* k_scales, void* k_biases,
                                 uint32_t* v_quant, void* v_scales, void* v_biases,
                                 tq_dtype sb_dtype, int batch, int num_kv_heads, int head_dim,
                                 int kv_capacity, const int32_t* positions, int n_new,
                                 tq_quant_mode mode, void* stream) {
  return kv_append(k_new, v_new, x_dtype, k_quant, k_scales, k_biases, v_quant, v_scales,
                   v_biases, sb_dtype, batch, num_kv_heads, head_dim, kv_capacity, positions,
                   n_new, mode, 0, stream, "tq_kv_append_int4");
}

extern "C" int tq_kv_append_int4_ring(const void* k_new, const void* v_new, tq_dtype x_dtype,
                                      uint32_t* k_quant, void* k_scales, void* k_biases,
                                      uint32_t* v_quant, void* v_scales, void* v_biases,
                                      tq_dtype sb_dtype, int batch, int num_kv_heads,
                                      int head_dim, int kv_capacity, const int32_t* positions,
                                      int n_new, tq_quant_mode mode, void* stream) {
  return kv_append(k_new, v_new, x_dtype, k_quant, k_scales, k_biases, v_quant, v_scales,
                   v_biases, sb_dtype, batch, num_kv_heads, head_dim, kv_capacity, positions,
                   n_new, mode, 1, stream, "tq_kv_append_int4_ring");
}

extern "C" int tq_dequantize_int4(const uint32_t* w_q, const void* scales, const void* biases,
                                  tq_dtype sb_dtype, int64_t rows, int dim, float* out,
                                  void* stream) {
  clear_error();
  TQ_CHECK_ARG(sb_dtype == TQ_F16 || sb_dtype == TQ_F32, "tq_dequantize_int4: bad sb_dtype");
  TQ_CHECK_ARG(dim > 0 && dim % 64 == 0, "tq_dequantize_int4: dim must be a multiple of 64");
  TQ_CHECK_ARG(rows >= 0, "tq_dequantize_int4: rows < 0");
  if (rows == 0) return TQ_OK;
  TQ_CHECK_ARG(w_q && scales && biases && out, "tq_dequantize_int4: null pointer");
  if (int r = check_align(out, 16, "out")) return r;
  const int64_t lanes = rows * (dim / 8);
  const unsigned blocks = static_cast<unsigned>((lanes + 255) / 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (sb_dtype == TQ_F16)
    dequantize_int4_kernel<__half><<<blocks, 256, 0, s>>>(
        w_q, static_cast<const __half*>(scales), static_cast<const __half*>(biases), rows, dim, out);
  else
    dequantize_int4_kernel<float><<<blocks, 256, 0, s>>>(
        w_q, static_cast<const float*>(scales), static_cast<const float*>(biases), rows, dim, out);
  TQ_CHECK_LAUNCH("dequantize_int4_kernel");
  return TQ_OK;
}
