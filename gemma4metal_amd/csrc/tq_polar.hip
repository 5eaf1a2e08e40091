// PolarQuant / QJL on gfx950: encoders, decoders, compressed-key scores and
// compressed-key decode attention (replaces lib/turboquant.metal:8-224,
// 424-704 and the primitives of lib/turboquant.cpp:11-359).
//
// Two key layouts:
//  * the reference layouts: 16-value blocks, 4 levels, indices unpacked (one
//    u8 per angle, lib/turboquant.cpp:105-109) or packed (u32 + 3 u8 per
//    block, lib/turboquant.metal:501-600), one fp16 radius per block, and
//    caller-supplied codebooks;
//  * the 7-level layout ("polar7"): one 128-value block
//    per vector -- 64 level-1 angles (4 bits) and 63 angles of levels 2-7
//    (2 bits) in 12 words, the fp16 radius and the fp16 norm of the QJL
//    residual in one word, and the 128 sign bits of the QJL residual sketch
//    in 4 words.
//
// The encoders reproduce the float32 oracle bit for bit: atan2, square roots
// and the rotation / sketch dot products are a fixed sequence of IEEE fp32
// operations (correctly rounded division and square root, FMA contraction
// off), so every index decision and sketch bit is reproducible.
//
// Scores and attention run one key per lane.  The polar7 score uses two
// per-head LDS tables built in the workgroup prologue: the q'-premultiplied
// level-1 table t1[j][k] = q'[2j] cos c_k + q'[2j+1] sin c_k (a level-1 angle
// costs one gather instead of a cos/sin pair and 2 FMAs per head), and the
// QJL byte table tq[pos][byte] = sum of (S q')_i over the set bits of the
// byte (the 128-bit sign dot costs 16 gathers).  Levels 7..2 are decoded
// top-down with a 4-entry (cos, sin) table.  V is accumulated with lanes
// owning dimensions; workgroups merge through the shared split-K
// finalisation of the int4 kernels.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "tq_sdpa_common.h"

namespace tq {
namespace {

// float32 constants of the deterministic atan2 (same values as the oracle)
constexpr float kPi = 0x1.921fb6p+1f;
constexpr float kPi2 = 0x1.921fb6p+0f;
constexpr float kPi4 = 0x1.921fb6p-1f;
constexpr float kTwoPi = 0x1.921fb6p+2f;
constexpr float kTanPi8 = 0x1.a8279ap-2f;
// (-1)^k / (2k+1), k = 1..10
constexpr float kAtanC[10] = {-0x1.555556p-2f, 0x1.99999ap-3f, -0x1.24924ap-3f, 0x1.c71c72p-4f,
                              -0x1.745d18p-4f, 0x1.3b13b2p-4f, -0x1.111112p-4f, 0x1.e1e1e2p-5f,
                              -0x1.af286cp-5f, 0x1.861862p-5f};
constexpr float kLog2e = 1.4426950408889634f;
// sqrt(pi/2) / m
constexpr float kQjlCoef = 0.009791516697777346f;
constexpr int kP7Words = 12;
// query heads per workgroup of the polar7 kernels (tables: 20 KB of LDS per head)
constexpr int kP7MaxG = 2;

// atan2(y, x) in (-pi, pi]: |t| = min/max of |x|, |y|, reduced with
// atan(t) = pi/4 + atan((t-1)/(t+1)) above tan(pi/8), then the Taylor series
// of atan to u^21; octant and sign fix-ups as atan2 (signed zeros included).
__device__ __forceinline__ float atan2_det(float y, float x) {
#pragma clang fp contract(off)
  const float ax = fabsf(x), ay = fabsf(y);
  const float mx = fmaxf(ax, ay), mn = fminf(ax, ay);
  const float t = mx > 0.0f ? mn / mx : 0.0f;
  const bool big = t > kTanPi8;
  const float u = big ? (t - 1.0f) / (t + 1.0f) : t;
  const float s = u * u;
  float p = kAtanC[9];
#pragma unroll
  for (int k = 8; k >= 0; --k) {
    p = p * s;
    p = p + kAtanC[k];
  }
  float r = s * p;
  r = u * r;
  float a = u + r;
  if (big) a = kPi4 + a;
  if (ay > ax) a = kPi2 - a;
  if (__float_as_uint(x) >> 31) a = kPi - a;
  if (__float_as_uint(y) >> 31) a = -a;
  return a;
}

// nearest codebook entry under |theta - c|, first minimum wins
// (lib/turboquant.metal:38-42)
__device__ __forceinline__ int nearest_idx(float th, const float* cb, int n) {
#pragma clang fp contract(off)
  float best = 1e10f;
  int idx = 0;
  for (int c = 0; c < n; ++c) {
    const float d = fabsf(th - cb[c]);
    if (d < best) {
      best = d;
      idx = c;
    }
  }
  return idx;
}

__device__ __forceinline__ float pair_radius(float a, float b) {
#pragma clang fp contract(off)
  const float aa = a * a;
  const float bb = b * b;
  return sqrtf(aa + bb);
}

__device__ __forceinline__ float h2f_lo(uint32_t w) {
  return __half2float(__ushort_as_half(static_cast<uint16_t>(w & 0xFFFFu)));
}
__device__ __forceinline__ float h2f_hi(uint32_t w) {
  return __half2float(__ushort_as_half(static_cast<uint16_t>(w >> 16)));
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float wave_max_f(float v) { return wave_max_dpp(v); }
__device__ __forceinline__ float wave_sum_f(float v) { return group_sum<64>(v); }

// ============================================================================
// Reference layouts: 16-value blocks, 4 levels
// ============================================================================

struct Enc16Params {
  const float* x;
  const float* P;  // D x D preconditioner or null (x already rotated)
  int64_t n;       // vectors
  int D;
  int rows;        // vectors per workgroup
  const float* cb; // concatenated codebooks of levels 1..4
  int ncb[4];
  int cb_off[4];
  uint8_t *i1, *i2, *i3, *i4;  // unpacked outputs
  uint32_t* p1;                 // packed outputs
  uint8_t *p2, *p3, *p4;
  uint16_t* radii;
};

// One workgroup per `rows` vectors: the tile is rotated in LDS (y = x P^T,
// y_i accumulated d = 0..D-1 with separately rounded products and sums),
// then one thread encodes each 16-value block.
template <bool kPacked>
__global__ __launch_bounds__(256) void polar_encode16_kernel(Enc16Params p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) float smem[];
  const int D = p.D, R = p.rows;
  float* cbs = smem;       // [4][256]
  float* xs = smem + 1024; // [R][D]
  float* ys = xs + R * D;  // [R][D]
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
  const int rows = static_cast<int>(min(static_cast<int64_t>(R), p.n - row0));
  for (int i = threadIdx.x; i < 1024; i += 256) {
    const int l = i >> 8, c = i & 255;
    cbs[i] = c < p.ncb[l] ? p.cb[p.cb_off[l] + c] : 0.0f;
  }
  for (int i = threadIdx.x; i < rows * D; i += 256) xs[i] = p.x[row0 * D + i];
  __syncthreads();
  const float* y = xs;
  if (p.P) {
    for (int o = threadIdx.x; o < rows * D; o += 256) {
      const int r = o / D, i = o - r * D;
      const float* pr = p.P + static_cast<int64_t>(i) * D;
      const float* xr = xs + r * D;
      float acc = 0.0f;
      for (int d = 0; d < D; ++d) acc = acc + xr[d] * pr[d];
      ys[o] = acc;
    }
    __syncthreads();
    y = ys;
  }
  const int nb = D / 16;
  for (int blk = threadIdx.x; blk < rows * nb; blk += 256) {
    float r[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) r[j] = y[blk * 16 + j];
    int k1[8], k2[4], k3[2], k4;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float a = r[2 * j], b = r[2 * j + 1];
      float th = atan2_det(b, a);
      if (th < 0.0f) th = th + kTwoPi;
      k1[j] = nearest_idx(th, cbs, p.ncb[0]);
      r[j] = pair_radius(a, b);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = r[2 * j], b = r[2 * j + 1];
      k2[j] = nearest_idx(atan2_det(b, a), cbs + 256, p.ncb[1]);
      r[j] = pair_radius(a, b);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float a = r[2 * j], b = r[2 * j + 1];
      k3[j] = nearest_idx(atan2_det(b, a), cbs + 512, p.ncb[2]);
      r[j] = pair_radius(a, b);
    }
    k4 = nearest_idx(atan2_det(r[1], r[0]), cbs + 768, p.ncb[3]);
    const float rad = pair_radius(r[0], r[1]);
    const int64_t gb = row0 * nb + blk;
    if constexpr (kPacked) {
      uint32_t w1 = 0, w2 = 0, w3 = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) w1 |= (static_cast<uint32_t>(k1[j]) & 0xFu) << (4 * j);
#pragma unroll
      for (int j = 0; j < 4; ++j) w2 |= (static_cast<uint32_t>(k2[j]) & 0x3u) << (2 * j);
#pragma unroll
      for (int j = 0; j < 2; ++j) w3 |= (static_cast<uint32_t>(k3[j]) & 0x3u) << (2 * j);
      p.p1[gb] = w1;
      p.p2[gb] = static_cast<uint8_t>(w2);
      p.p3[gb] = static_cast<uint8_t>(w3);
      p.p4[gb] = static_cast<uint8_t>(k4 & 0x3);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) p.i1[gb * 8 + j] = static_cast<uint8_t>(k1[j]);
#pragma unroll
      for (int j = 0; j < 4; ++j) p.i2[gb * 4 + j] = static_cast<uint8_t>(k2[j]);
#pragma unroll
      for (int j = 0; j < 2; ++j) p.i3[gb * 2 + j] = static_cast<uint8_t>(k3[j]);
      p.i4[gb] = static_cast<uint8_t>(k4);
    }
    p.radii[gb] = __half_as_ushort(__float2half_rn(rad));
  }
}

struct Keys16 {
  const uint8_t *i1, *i2, *i3, *i4;  // unpacked indices
  const uint32_t* p1;                 // packed indices
  const uint8_t *p2, *p3, *p4;
  const uint16_t* radii;
};

// indices of one 16-value block
template <bool kPacked>
__device__ __forceinline__ void load_block_idx(const Keys16& k, int64_t gb, int k1[8], int k2[4],
                                               int k3[2], int& k4) {
  if constexpr (kPacked) {
    const uint32_t w = k.p1[gb], b2 = k.p2[gb], b3 = k.p3[gb];
#pragma unroll
    for (int j = 0; j < 8; ++j) k1[j] = (w >> (4 * j)) & 0xF;
#pragma unroll
    for (int j = 0; j < 4; ++j) k2[j] = (b2 >> (2 * j)) & 0x3;
#pragma unroll
    for (int j = 0; j < 2; ++j) k3[j] = (b3 >> (2 * j)) & 0x3;
    k4 = k.p4[gb] & 0x3;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) k1[j] = k.i1[gb * 8 + j];
#pragma unroll
    for (int j = 0; j < 4; ++j) k2[j] = k.i2[gb * 4 + j];
#pragma unroll
    for (int j = 0; j < 2; ++j) k3[j] = k.i3[gb * 2 + j];
    k4 = k.i4[gb];
  }
}

// Top-down decode of one block with the (cos, sin) tables cst[level][256]
// (lib/turboquant.metal:100-164).
__device__ __forceinline__ void decode_block16(const float2* cst, float rad, const int k1[8],
                                               const int k2[4], const int k3[2], int k4,
                                               float v[16]) {
  float a[2], b[4], c[8];
  {
    const float2 cs = cst[768 + k4];
    a[0] = rad * cs.x;
    a[1] = rad * cs.y;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float2 cs = cst[512 + k3[j]];
    b[2 * j] = a[j] * cs.x;
    b[2 * j + 1] = a[j] * cs.y;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float2 cs = cst[256 + k2[j]];
    c[2 * j] = b[j] * cs.x;
    c[2 * j + 1] = b[j] * cs.y;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float2 cs = cst[k1[j]];
    v[2 * j] = c[j] * cs.x;
    v[2 * j + 1] = c[j] * cs.y;
  }
}

// (cos, sin) tables of the four levels in LDS: from the caller's tables when
// given (the reference's "_fast" variants), else cos/sin of the codebook
// angles (zero beyond each codebook's size, so any u8 index stays in range).
struct CsSource {
  const float* cb;   // concatenated codebooks, or null
  const float* cs;   // concatenated (cos, sin) pairs, or null
  int ncb[4];
  int off[4];
};

template <int NT>
__device__ __forceinline__ void fill_cs_tables(float2* cst, const CsSource& s) {
  for (int i = threadIdx.x; i < 1024; i += NT) {
    const int l = i >> 8, c = i & 255;
    float2 v = make_float2(0.0f, 0.0f);
    if (c < s.ncb[l]) {
      if (s.cs) {
        v = make_float2(s.cs[2 * (s.off[l] + c)], s.cs[2 * (s.off[l] + c) + 1]);
      } else {
        const float th = s.cb[s.off[l] + c];
        v = make_float2(cosf(th), sinf(th));
      }
    }
    cst[i] = v;
  }
}

struct Dec16Params {
  Keys16 k;
  CsSource src;
  const float* P;  // x = y P when non-null
  float* out;
  int64_t n;
  int D;
  int rows;
};

template <bool kPacked>
__global__ __launch_bounds__(256) void polar_decode16_kernel(Dec16Params p) {
  extern __shared__ __align__(16) float smem[];
  float2* cst = reinterpret_cast<float2*>(smem);  // [4][256]
  float* ys = smem + 2048;                        // [R][D]
  fill_cs_tables<256>(cst, p.src);
  __syncthreads();
  const int R = p.rows, D = p.D, nb = D / 16;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
  const int rows = static_cast<int>(min(static_cast<int64_t>(R), p.n - row0));
  for (int blk = threadIdx.x; blk < rows * nb; blk += 256) {
    const int64_t gb = row0 * nb + blk;
    int k1[8], k2[4], k3[2], k4;
    load_block_idx<kPacked>(p.k, gb, k1, k2, k3, k4);
    const float rad = __half2float(__ushort_as_half(p.k.radii[gb]));
    float v[16];
    decode_block16(cst, rad, k1, k2, k3, k4, v);
    float* dst = p.P ? ys + blk * 16 : p.out + gb * 16;
#pragma unroll
    for (int j = 0; j < 16; j += 4)
      *reinterpret_cast<float4*>(dst + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
  }
  if (p.P) {
    __syncthreads();
    for (int o = threadIdx.x; o < rows * D; o += 256) {
      const int r = o / D, d = o - r * D;
      const float* yr = ys + r * D;
      float acc = 0.0f;
      for (int i = 0; i < D; ++i) acc = fmaf(yr[i], p.P[static_cast<int64_t>(i) * D + d], acc);
      p.out[(row0 + r) * D + d] = acc;
    }
  }
}

// ---- reference scores and attention (keys [kv head][n][D/16 blocks]) -------

struct Attn16 {
  Keys16 k;
  CsSource src;
  const float* q;       // [Hq][D] f32
  const float* values;  // [Hkv][n][D] f32 (attention only)
  float* scores;        // [Hq][n] (score only)
  int D;
  float qscale;         // multiplies q (scale, or scale*log2e for attention)
};

// scores of key t of kv head kvh for G heads (q pre-scaled in LDS, [G][D])
template <int D, int G, bool kPacked>
__device__ __forceinline__ void score16(const Attn16& a, const float2* cst, const float* qs,
                                        int64_t keyrow, float s[G]) {
  constexpr int NB = D / 16;
#pragma unroll
  for (int g = 0; g < G; ++g) s[g] = 0.0f;
  for (int blk = 0; blk < NB; ++blk) {
    const int64_t gb = keyrow * NB + blk;
    int k1[8], k2[4], k3[2], k4;
    load_block_idx<kPacked>(a.k, gb, k1, k2, k3, k4);
    const float rad = __half2float(__ushort_as_half(a.k.radii[gb]));
    float v[16];
    decode_block16(cst, rad, k1, k2, k3, k4, v);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float4* q4 = reinterpret_cast<const float4*>(qs + g * D + blk * 16);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 qv = q4[j];
        s[g] = fmaf(qv.x, v[4 * j], s[g]);
        s[g] = fmaf(qv.y, v[4 * j + 1], s[g]);
        s[g] = fmaf(qv.z, v[4 * j + 2], s[g]);
        s[g] = fmaf(qv.w, v[4 * j + 3], s[g]);
      }
    }
  }
}

// tq_score_shared (lib/turboquant.metal:424-499) + GQA: one key per thread,
// 1024 keys per workgroup, grid (key blocks, kv heads * head subgroups).
template <int D, int G, bool kPacked>
__global__ __launch_bounds__(256) void polar16_score_kernel(Attn16 a, int n, int gqa, int n_sub) {
  __shared__ float2 cst[1024];
  __shared__ __align__(16) float qs[G * D];
  const int hy = blockIdx.y, kvh = hy / n_sub, sub = hy - (hy / n_sub) * n_sub;
  const int h0 = kvh * gqa + sub * G;
  fill_cs_tables<256>(cst, a.src);
  for (int i = threadIdx.x; i < G * D; i += 256) qs[i] = a.qscale * a.q[static_cast<int64_t>(h0) * D + i];
  __syncthreads();
  for (int t = blockIdx.x * 1024 + threadIdx.x; t < min(n, (blockIdx.x + 1) * 1024); t += 256) {
    float s[G];
    score16<D, G, kPacked>(a, cst, qs, static_cast<int64_t>(kvh) * n + t, s);
#pragma unroll
    for (int g = 0; g < G; ++g) a.scores[static_cast<int64_t>(h0 + g) * n + t] = s[g];
  }
}

// sdpa_tq_sequential (lib/turboquant.metal:166-224) as split-K flash decoding
// + GQA: 64-key tiles per wave (one key per lane), fp32 V with lanes owning
// dimensions, output acc / (l + 1e-8).
template <int D, int G, bool kPacked>
__global__ __launch_bounds__(256) void polar16_sdpa_kernel(SdpaParams p, Attn16 a) {
  pin_args(p);
  constexpr int NW = 4, VE = D / 64;
  __shared__ float2 cst[1024];
  __shared__ __align__(16) float qs[G * D];
  using Fin = Finalize<G, D, NW>;
  __shared__ __align__(16) float arena[Fin::kArena];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hy = blockIdx.y, split = blockIdx.x;
  const int kvh = hy / p.n_sub, sub = hy - kvh * p.n_sub;
  const int h0 = kvh * p.gqa + sub * G;
  const SplitRange rg = split_range(p, 0, split);
  if (split >= rg.S) return;
  fill_cs_tables<256>(cst, a.src);
  for (int i = threadIdx.x; i < G * D; i += 256) qs[i] = a.qscale * a.q[static_cast<int64_t>(h0) * D + i];
  __syncthreads();

  float m_run[G], l_run[G], acc[G][VE];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < VE; ++e) acc[g][e] = 0.0f;
  }
  const int64_t rowbase = static_cast<int64_t>(kvh) * p.cap;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  for (int tb = rg.t_begin + wv * 64; tb < rg.t_end; tb += NW * 64) {
    const bool valid = tb + lane < rg.t_end;
    const int t = min(tb + lane, rg.t_end - 1);
    float s[G], pw[G];
    score16<D, G, kPacked>(a, cst, qs, rowbase + t, s);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float sv = valid ? s[g] : -INFINITY;
      const float m_new = fmaxf(m_run[g], wave_max_f(sv));
      if (m_new > m_run[g]) {  // wave-uniform
        const float f = merge_factor(m_run[g], m_new);
        l_run[g] *= f;
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[g][e] *= f;
        m_run[g] = m_new;
      }
      pw[g] = valid ? fast_exp2(sv - m_run[g]) : 0.0f;
      l_run[g] += pw[g];
    }
    const int nk = min(64, rg.t_end - tb);
    for (int kk = 0; kk < nk; ++kk) {
      const float* vr = a.values + (rowbase + tb + kk) * D + lane;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pw[g]), kk));
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[g][e] = fmaf(pg, vr[64 * e], acc[g][e]);
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int e = 0; e < VE; ++e) Fin::o(arena, wave, g)[lane + 64 * e] = acc[g][e];
    const float ls = wave_sum_f(l_run[g]);
    if (lane == 0) {
      Fin::m(arena, wave)[g] = m_run[g];
      Fin::l(arena, wave)[g] = ls;
    }
  }
  Fin::run(p, arena, h0, rg.S, split, hy);
}

// ============================================================================
// polar7 layout: 7 levels over one 128-value block + QJL
// ============================================================================

struct P7EncParams {
  const float* x;    // [rows][128]
  const float* P;    // [128][128] or null
  const float* S;    // [128][128] QJL sketch matrix
  const float* cb;   // cb1[16] then cb2[4]
  const float* cs;   // cs1[16][2] then cs2[4][2]
  int64_t n;
  // append mapping (positions != null): x is [B][Hkv][n_new][128], outputs are
  // [B][Hkv][cap][.] and row t of (b, h) goes to positions[b] + t
  const int32_t* positions;
  int n_new, cap, Hkv;
  uint32_t* angles;  // [.][12]
  uint32_t* norms;   // [.]   fp16 radius | fp16 ||r|| << 16
  uint32_t* qjl;     // [.][4]
};

// One wave per vector: lane l holds y[2l], y[2l+1]; level k pairs come from
// lanes 2j, 2j+1 of level k-1.  Grid-stride over vectors.
__global__ __launch_bounds__(256) void polar7_encode_kernel(P7EncParams p) {
#pragma clang fp contract(off)
  __shared__ float cb[20];
  __shared__ float2 cs[20];
  __shared__ float xs[4][128];
  __shared__ float rs[4][128];
  if (threadIdx.x < 20) {
    cb[threadIdx.x] = p.cb[threadIdx.x];
    cs[threadIdx.x] = make_float2(p.cs[2 * threadIdx.x], p.cs[2 * threadIdx.x + 1]);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wave; row < p.n;
       row += static_cast<int64_t>(gridDim.x) * 4) {
    int64_t orow = row;
    if (p.positions) {
      const int64_t bh = row / p.n_new;
      const int t = static_cast<int>(row - bh * p.n_new);
      const int64_t pos = static_cast<int64_t>(p.positions[bh / p.Hkv]) + t;
      if (pos < 0 || pos >= p.cap) continue;  // wave-uniform
      orow = bh * p.cap + pos;
    }
    const float2 xv = reinterpret_cast<const float2*>(p.x + row * 128)[lane];
    float y0 = xv.x, y1 = xv.y;
    if (p.P) {
      xs[wave][2 * lane] = xv.x;
      xs[wave][2 * lane + 1] = xv.y;
      wave_lds_sync();
      const float* pa = p.P + (2 * lane) * 128;
      const float* pb = pa + 128;
      float acc0 = 0.0f, acc1 = 0.0f;
      for (int d = 0; d < 128; d += 4) {
        const float4 a4 = *reinterpret_cast<const float4*>(pa + d);
        const float4 b4 = *reinterpret_cast<const float4*>(pb + d);
        const float x0 = xs[wave][d], x1 = xs[wave][d + 1], x2 = xs[wave][d + 2], x3 = xs[wave][d + 3];
        acc0 = acc0 + x0 * a4.x; acc0 = acc0 + x1 * a4.y; acc0 = acc0 + x2 * a4.z; acc0 = acc0 + x3 * a4.w;
        acc1 = acc1 + x0 * b4.x; acc1 = acc1 + x1 * b4.y; acc1 = acc1 + x2 * b4.z; acc1 = acc1 + x3 * b4.w;
      }
      y0 = acc0;
      y1 = acc1;
    }
    // ---- encode: level 1 (4-bit, wrapped to [0, 2pi)), levels 2..7 (2-bit)
    int idx[7];
    float r;
    {
      float th = atan2_det(y1, y0);
      if (th < 0.0f) th = th + kTwoPi;
      idx[0] = nearest_idx(th, cb, 16);
      r = pair_radius(y0, y1);
    }
#pragma unroll
    for (int lv = 1; lv < 7; ++lv) {
      const float a = __shfl(r, (2 * lane) & 63, 64);
      const float b = __shfl(r, (2 * lane + 1) & 63, 64);
      idx[lv] = nearest_idx(atan2_det(b, a), cb + 16, 4);
      r = pair_radius(a, b);
    }
    const float R = __shfl(r, 0, 64);
    const __half R16 = __float2half_rn(R);
    // ---- decode top-down (the stored bits): child = parent * cos|sin
    float v = __half2float(R16);
#pragma unroll
    for (int lv = 6; lv >= 1; --lv) {
      const float pv = __shfl(v, lane >> 1, 64);
      const int pi = __shfl(idx[lv], lane >> 1, 64);
      const float2 c = cs[16 + pi];
      v = (lane & 1) ? pv * c.y : pv * c.x;
    }
    const float2 c1 = cs[idx[0]];
    const float yh0 = v * c1.x, yh1 = v * c1.y;
    const float r0 = y0 - yh0, r1 = y1 - yh1;
    float nrm = r0 * r0;
    const float q1 = r1 * r1;
    nrm = nrm + q1;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) nrm = nrm + shfl_xor_f(nrm, off);
    const __half rn16 = __float2half_rn(sqrtf(nrm));
    // ---- QJL sketch: rows lane and lane + 64 of S r
    rs[wave][2 * lane] = r0;
    rs[wave][2 * lane + 1] = r1;
    wave_lds_sync();
    const float* sa = p.S + lane * 128;
    const float* sb = sa + 64 * 128;
    float ka = 0.0f, kb = 0.0f;
    for (int d = 0; d < 128; d += 4) {
      const float4 a4 = *reinterpret_cast<const float4*>(sa + d);
      const float4 b4 = *reinterpret_cast<const float4*>(sb + d);
      const float e0 = rs[wave][d], e1 = rs[wave][d + 1], e2 = rs[wave][d + 2], e3 = rs[wave][d + 3];
      ka = ka + e0 * a4.x; ka = ka + e1 * a4.y; ka = ka + e2 * a4.z; ka = ka + e3 * a4.w;
      kb = kb + e0 * b4.x; kb = kb + e1 * b4.y; kb = kb + e2 * b4.z; kb = kb + e3 * b4.w;
    }
    const uint64_t ba = __ballot(ka >= 0.0f);
    const uint64_t bb = __ballot(kb >= 0.0f);
    // ---- pack: lanes 0-7 level-1 words, 8-9 level-2, 10 level 3, 11 levels 4-7
    uint32_t wa = 0, wb = 0, wc = 0, wd = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      wa |= (static_cast<uint32_t>(__shfl(idx[0], (8 * lane + i) & 63, 64)) & 0xFu) << (4 * i);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      wb |= (static_cast<uint32_t>(__shfl(idx[1], (16 * (lane - 8) + i) & 63, 64)) & 0x3u) << (2 * i);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      wc |= (static_cast<uint32_t>(__builtin_amdgcn_readlane(idx[2], i)) & 0x3u) << (2 * i);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      wd |= (static_cast<uint32_t>(__builtin_amdgcn_readlane(idx[3], i)) & 0x3u) << (2 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      wd |= (static_cast<uint32_t>(__builtin_amdgcn_readlane(idx[4], i)) & 0x3u) << (16 + 2 * i);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      wd |= (static_cast<uint32_t>(__builtin_amdgcn_readlane(idx[5], i)) & 0x3u) << (24 + 2 * i);
    wd |= (static_cast<uint32_t>(__builtin_amdgcn_readlane(idx[6], 0)) & 0x3u) << 28;
    const uint32_t w = lane < 8 ? wa : (lane < 10 ? wb : (lane == 10 ? wc : wd));
    if (lane < kP7Words) p.angles[orow * kP7Words + lane] = w;
    if (lane < 4) {
      const uint64_t bits = lane < 2 ? ba : bb;
      p.qjl[orow * 4 + lane] = static_cast<uint32_t>(bits >> (32 * (lane & 1)));
    }
    if (lane == 0)
      p.norms[orow] = static_cast<uint32_t>(__half_as_ushort(R16)) |
                      (static_cast<uint32_t>(__half_as_ushort(rn16)) << 16);
  }
}

// y = x P^T for rows of 128 (the query rotation q' = P q); fp32, any order.
__global__ __launch_bounds__(128) void rotate128_kernel(const float* x, const float* P, float* y,
                                                        int rows) {
  __shared__ float xs[128];
  const int r = blockIdx.x, i = threadIdx.x;
  xs[i] = x[static_cast<int64_t>(r) * 128 + i];
  __syncthreads();
  const float* pr = P + i * 128;
  float acc = 0.0f;
  for (int d = 0; d < 128; d += 4) {
    const float4 a = *reinterpret_cast<const float4*>(pr + d);
    acc = fmaf(xs[d], a.x, acc);
    acc = fmaf(xs[d + 1], a.y, acc);
    acc = fmaf(xs[d + 2], a.z, acc);
    acc = fmaf(xs[d + 3], a.w, acc);
  }
  y[static_cast<int64_t>(r) * 128 + i] = acc;
}

// ---- polar7 scores ------------------------------------------------------------

// Per-head query tables written by polar7_prepare_kernel or
// polar7_prepare_sp_kernel, kP7QTab floats per head: t1 [64][16] (level 1:
// q'[2j] cos c1_k + q'[2j+1] sin c1_k), tq [16][256] (QJL: sum of
// (S q')_{8 pos + i} over the set bits i of a byte), then U = sum of S q'
// as the sum of four floats (partial sums, or U and three zeros) and
// padding to a 16-byte multiple.
constexpr int kP7QTab = 1024 + 4096 + 16;

struct P7Keys {
  const float* qtab;      // [Hq][kP7QTab]
  // attention straight from q (build_p7_tables): q [Hq][128], P [128][128]
  // (null: q' = q) and S P [128][128]; null otherwise
  const float* q;
  const float* P;
  const float* SP;
  const float* cs;        // cs1[16][2] then cs2[4][2]
  const uint32_t* angles; // [Hkv][cap][12]
  const uint32_t* norms;  // [Hkv][cap]
  const uint32_t* qjl;    // [Hkv][cap][4]
  float* scores;          // [Hq][n] (score only)
};

// Per-workgroup LDS tables (unscaled; the score scale multiplies each key's
// total):
//   t1[g][j][c] = q'[2j] cos c1_c + q'[2j+1] sin c1_c  (level 1, per head)
//   tq[g][pos][b] = sum of (S q')_{8 pos + i} over the set bits i of b
//   t2[kp | k0 << 2 | k1 << 4] = the four grandchild factors of a level pair
//     with code kp whose child pairs have codes k0, k1:
//     (cos_p cos_0, cos_p sin_0, sin_p cos_1, sin_p sin_1) -- two levels of
//     the top-down decode per lookup (levels 7-6, 5-4, 3-2).
// The G heads' entries of t1 and tq are adjacent, so one 8-byte LDS read
// (G = 2) serves both heads of a lookup.
template <int G>
struct P7Tables {
  float t1[64][16][G];  // [row (rotated, see p7_t1_row)][codeword][head]
  float tq[16][256][G];  // [QJL byte position][byte value][head]
  float4 t2[64];
  float U[G];
};

// LDS row of level-1 row 16 qt + jj (pair jj of quarter qt): the rows are
// rotated within each group of four, to 16 qt + (jj & ~3) + ((jj + qt) & 3).
// The four lanes of a key read row jj of their quarters in one instruction.
// At G = 1 (64 B rows) the rotation puts those rows into four different
// 16-bank groups; at G = 2 a row covers all banks and it changes nothing.
__device__ __forceinline__ int p7_t1_row(int row) {
  const int qt = row >> 4, jj = row & 15;
  return (row & ~15) | (jj & ~3) | ((jj + qt) & 3);
}

// Copies the query tables of heads h0 .. h0+G-1 into LDS and builds the
// combined two-level table t2[kp | k0 << 2 | k1 << 4] = (cos_p cos_0,
// cos_p sin_0, sin_p cos_1, sin_p sin_1) of the levels 2-7 codebook: the
// four grandchild factors of a pair with code kp whose child pairs have
// codes k0, k1 (two levels of the top-down decode per lookup).
// `after_loads()` runs once the tables' loads are issued (the caller's first
// key loads go there, behind them).  All NT threads call it; it ends with a
// barrier.
template <int G, int NT, typename AfterLoads>
__device__ __forceinline__ void load_p7_tables(P7Tables<G>& T, const P7Keys& k, int h0, AfterLoads&& after_loads) {
  constexpr int kVec = kP7QTab / 4;
  // every 16-byte load first (one memory round trip), then the LDS stores:
  // a load-then-store loop would wait a round trip per iteration
  constexpr int NV = (G * kVec + NT - 1) / NT;
  const float4* src = reinterpret_cast<const float4*>(k.qtab + static_cast<int64_t>(h0) * kP7QTab);
  float4 vv[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = min(static_cast<int>(threadIdx.x) + j * NT, G * kVec - 1);  // clamped; dropped below
    vv[j] = src[i];  // head h0 + i / kVec, entry i % kVec: the G heads' tables are adjacent
  }
  // the level-pair factors of lane (kp, k0, k1) of the first wave, loaded
  // with the tables
  const int kp = threadIdx.x & 3, k0 = (threadIdx.x >> 2) & 3, k1 = (threadIdx.x >> 4) & 3;
  const float* c2 = k.cs + 32;  // (cos, sin) pairs; 4-byte alignment only
  const float2 cpp = make_float2(c2[2 * kp], c2[2 * kp + 1]), c0p = make_float2(c2[2 * k0], c2[2 * k0 + 1]),
               c1p = make_float2(c2[2 * k1], c2[2 * k1 + 1]);
  // the caller's first key loads go out behind the tables' (which are
  // needed first)
  after_loads();
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = static_cast<int>(threadIdx.x) + j * NT;
    if (i >= G * kVec) break;
    const int g = i / kVec, r = i - (i / kVec) * kVec;
    const float4 v = vv[j];
    const float f[4] = {v.x, v.y, v.z, v.w};
    if (r < 256) {
      const int row = p7_t1_row(r >> 2), c0 = 4 * (r & 3);
#pragma unroll
      for (int k = 0; k < 4; ++k) T.t1[row][c0 + k][g] = f[k];
    } else if (r < 1280) {
      const int e = 4 * (r - 256), pos = e >> 8, b0 = e & 255;
#pragma unroll
      for (int k = 0; k < 4; ++k) T.tq[pos][b0 + k][g] = f[k];
    }
    else if (r == 1280) T.U[g] = (v.x + v.y) + (v.z + v.w);
  }
  if (threadIdx.x < 64)
    T.t2[threadIdx.x] = make_float4(cpp.x * c0p.x, cpp.x * c0p.y, cpp.y * c1p.x, cpp.y * c1p.y);
  __syncthreads();
}

// The tables of load_p7_tables built in the workgroup from q, P and S P
// (the work of polar7_prepare_sp_kernel, for the G heads of this workgroup
// only): q' = P q (q' = q without P) and u = S q' = (S P) q, then t1, tq, U
// and t2.  Every wave takes 256 / (NT / 64) of the 256 rows of [P; S P] in
// passes of 8 rows: lane (row 8 r + l / 8, j = l % 8) loads float4 columns
// 8c + j, c = 0..3, so each load instruction reads 8 whole 128-byte lines,
// and the 8 lanes of a row finish its dot products with a DPP butterfly.
// All NT threads call it; it ends with a barrier.
template <int G, int NT>
__device__ __forceinline__ void build_p7_tables(P7Tables<G>& T, const P7Keys& k, int h0) {
  static_assert(NT == 512 || NT == 1024, "8 or 16 waves cover the rows of [P; S P]");
  constexpr int RPW = 256 / (NT / 64), NPS = RPW / 8;  // rows per wave, passes
  __shared__ __attribute__((aligned(16))) float xs[G][128];
  __shared__ float qp[G][128], us[G][128], csl[40];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int j = lane & 7, rs = lane >> 3;
  // rows RPW w .. of [P; S P]; without P the waves of the P rows read S P
  // as well and drop the sums
  const bool is_p = wave * RPW < 128;
  const float* mat = (is_p && k.P) ? k.P : k.SP;
  const int row0 = (wave * RPW) & 127;
  float4 a[NPS][4];
#pragma unroll
  for (int r = 0; r < NPS; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      a[r][c] = *reinterpret_cast<const float4*>(mat + (row0 + 8 * r + rs) * 128 + 4 * (8 * c + j));
  if (t < G * 128) xs[t >> 7][t & 127] = k.q[static_cast<int64_t>(h0) * 128 + t];
  if (t < 40) csl[t] = k.cs[t];
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float4 x[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) x[c] = *reinterpret_cast<const float4*>(&xs[g][4 * (8 * c + j)]);
#pragma unroll
    for (int r = 0; r < NPS; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc = fmaf(a[r][c].x, x[c].x, acc);
        acc = fmaf(a[r][c].y, x[c].y, acc);
        acc = fmaf(a[r][c].z, x[c].z, acc);
        acc = fmaf(a[r][c].w, x[c].w, acc);
      }
      acc = group_sum<8>(acc);
      const int row = row0 + 8 * r + rs;
      if (j == 0) {
        if (!is_p) us[g][row] = acc;
        else qp[g][row] = k.P ? acc : xs[g][row];
      }
    }
  }
  __syncthreads();
  // level-1 table t1[row(jj)][c][g] = q'[2 jj] cos c + q'[2 jj + 1] sin c
  for (int e = t; e < 64 * 16 * G; e += NT) {
    const int g = e % G, c = (e / G) & 15, jj = e / (16 * G);
    T.t1[p7_t1_row(jj)][c][g] = qp[g][2 * jj] * csl[2 * c] + qp[g][2 * jj + 1] * csl[2 * c + 1];
  }
  // QJL byte table tq[pos][16 hi + lo][g]: the set bits of lo over u rows
  // 8 pos .. + 3, of hi over rows 8 pos + 4 .. + 7
  for (int e = t; e < 16 * 16 * G; e += NT) {
    const int g = e % G, lo = (e / G) & 15, pos = e / (16 * G);
    const float* uu = &us[g][8 * pos];
    float slo = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) slo += ((lo >> i) & 1) ? uu[i] : 0.0f;
    const float u4 = uu[4], u5 = uu[5], u6 = uu[6], u7 = uu[7];
#pragma unroll
    for (int hi = 0; hi < 16; ++hi) {
      float sum = slo;
      if (hi & 1) sum += u4;
      if (hi & 2) sum += u5;
      if (hi & 4) sum += u6;
      if (hi & 8) sum += u7;
      T.tq[pos][16 * hi + lo][g] = sum;
    }
  }
  if (t < 64) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float sum = wave_sum_f(us[g][t] + us[g][t + 64]);
      if (t == 0) T.U[g] = sum;
    }
  }
  if (t >= 64 && t < 128) {
    const int i = t - 64;
    const int kp = i & 3, k0 = (i >> 2) & 3, k1 = i >> 4;
    const float* c2 = csl + 32;
    const float cp = c2[2 * kp], sp = c2[2 * kp + 1];
    T.t2[i] = make_float4(cp * c2[2 * k0], cp * c2[2 * k0 + 1], sp * c2[2 * k1], sp * c2[2 * k1 + 1]);
  }
  __syncthreads();
}

// q' = P q (or q), u = S q', and the tables of one head.  Grid (heads,
// kP7PrepParts): the workgroups of a head each recompute q' and u (two
// 128 x 128 products, two threads per output) and write their share of the
// tables.  P and S are staged in LDS with coalesced loads (consecutive
// threads, consecutive 16 B: a workgroup load instruction covers 4 KB),
// all issued before the first wait; rows are padded to kPrepRS floats.
// (Loading each thread's own half row straight into registers made every
// load instruction touch 64 separate lines.)
constexpr int kP7PrepParts = 4;
constexpr int kPrepRS = 132;
__global__ __launch_bounds__(256) void polar7_prepare_kernel(const float* q, const float* P,
                                                             const float* S, const float* cs,
                                                             float* qtab, float* q_rot,
                                                             float* q_sketch) {
  __shared__ __attribute__((aligned(16))) float mat[2][128 * kPrepRS];  // P, S
  __shared__ float xs[128], qp[128], u[128], csl[40];
  const int h = blockIdx.x, part = blockIdx.y, t = threadIdx.x;
  const int i = t >> 1, half = t & 1;  // output row, half of its dot product
  {
    // float4 f = 256 c + t of a matrix: row f / 32, columns 4 (f % 32) .. + 3
    const float4* P4 = reinterpret_cast<const float4*>(P ? P : S);
    const float4* S4 = reinterpret_cast<const float4*>(S);
    float4 pv[16], sv[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      pv[c] = P4[256 * c + t];
      sv[c] = S4[256 * c + t];
    }
    if (t < 128) xs[t] = q[static_cast<int64_t>(h) * 128 + t];
    if (t < 40) csl[t] = cs[t];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int f = 256 * c + t, at = (f >> 5) * kPrepRS + 4 * (f & 31);
      *reinterpret_cast<float4*>(&mat[0][at]) = pv[c];
      *reinterpret_cast<float4*>(&mat[1][at]) = sv[c];
    }
  }
  __syncthreads();
  const float* prow = &mat[0][i * kPrepRS + 64 * half];
  const float* srow = &mat[1][i * kPrepRS + 64 * half];
  float acc = 0.0f;
  if (P) {
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const float4 a = *reinterpret_cast<const float4*>(prow + 4 * c);
      const float* x = xs + 64 * half + 4 * c;
      acc = fmaf(x[0], a.x, acc);
      acc = fmaf(x[1], a.y, acc);
      acc = fmaf(x[2], a.z, acc);
      acc = fmaf(x[3], a.w, acc);
    }
  } else {
    acc = half == 0 ? xs[i] : 0.0f;
  }
  acc = group_sum<2>(acc);
  if (half == 0) {
    qp[i] = acc;
    if (q_rot && part == 0) q_rot[static_cast<int64_t>(h) * 128 + i] = acc;
  }
  __syncthreads();
  float us = 0.0f;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const float4 a = *reinterpret_cast<const float4*>(srow + 4 * c);
    const float* x = qp + 64 * half + 4 * c;
    us = fmaf(x[0], a.x, us);
    us = fmaf(x[1], a.y, us);
    us = fmaf(x[2], a.z, us);
    us = fmaf(x[3], a.w, us);
  }
  us = group_sum<2>(us);
  if (half == 0) {
    u[i] = us;
    if (q_sketch && part == 0) q_sketch[static_cast<int64_t>(h) * 128 + i] = us;
  }
  __syncthreads();
  float* out = qtab + static_cast<int64_t>(h) * kP7QTab;
  constexpr int kT1 = 1024 / kP7PrepParts, kTq = 4096 / kP7PrepParts;
  for (int e = kT1 * part + t; e < kT1 * (part + 1); e += 256) {
    const int j = e >> 4, c = e & 15;
    out[e] = qp[2 * j] * csl[2 * c] + qp[2 * j + 1] * csl[2 * c + 1];
  }
  for (int e = kTq * part + t; e < kTq * (part + 1); e += 256) {
    const int pos = e >> 8, bits = e & 255;
    float sum = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; ++b) sum += ((bits >> b) & 1) ? u[8 * pos + b] : 0.0f;
    out[1024 + e] = sum;
  }
  if (part == 0 && t < 64) {
    const float sum = wave_sum_f(u[t] + u[t + 64]);
    if (t < 16) out[5120 + t] = t == 0 ? sum : 0.0f;
  }
}

// SP = S P (S when P is null): grid 128 rows x 128 threads; thread j reads
// column j of P, so each k is one coalesced row of P.
__global__ __launch_bounds__(128) void polar7_sp_kernel(const float* P, const float* S, float* SP) {
  const int i = blockIdx.x, j = threadIdx.x;
  const float* srow = S + i * 128;
  float acc = 0.0f;
  if (P) {
#pragma unroll 8
    for (int k = 0; k < 128; ++k) acc = fmaf(srow[k], P[k * 128 + j], acc);
  } else {
    acc = srow[j];
  }
  SP[i * 128 + j] = acc;
}

// The tables of polar7_prepare_kernel from q, P and SP = S P: u = S q' =
// SP q, so q' and u are independent products of q.  Part `part` of a head
// computes rows 32 part .. + 31 of both (its share of the tables needs no
// others: level-1 pairs 16 part .. + 15, QJL bytes 4 part .. + 3), staging
// just those rows of P and SP (32 KB) in LDS, and writes the partial sum
// of its u rows to float 5120 + part.
constexpr int kPrepRows = 128 / kP7PrepParts;
__global__ __launch_bounds__(256) void polar7_prepare_sp_kernel(const float* q, const float* P,
                                                                const float* SP, const float* cs,
                                                                float* qtab, float* q_rot,
                                                                float* q_sketch) {
  __shared__ __attribute__((aligned(16))) float mat[2][kPrepRows * kPrepRS];  // rows of P, SP
  __shared__ float xs[128], qp[128], u[128], csl[40];
  const int h = blockIdx.x, part = blockIdx.y, t = threadIdx.x;
  const int r0 = kPrepRows * part;
  {
    // float4 f = 256 c + t of the 32-row slab: row f / 32, columns 4 (f % 32) .. + 3
    const float4* P4 = reinterpret_cast<const float4*>((P ? P : SP) + r0 * 128);
    const float4* S4 = reinterpret_cast<const float4*>(SP + r0 * 128);
    float4 pv[4], sv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      pv[c] = P4[256 * c + t];
      sv[c] = S4[256 * c + t];
    }
    if (t < 128) xs[t] = q[static_cast<int64_t>(h) * 128 + t];
    if (t < 40) csl[t] = cs[t];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int f = 256 * c + t, at = (f >> 5) * kPrepRS + 4 * (f & 31);
      *reinterpret_cast<float4*>(&mat[0][at]) = pv[c];
      *reinterpret_cast<float4*>(&mat[1][at]) = sv[c];
    }
  }
  __syncthreads();
  // outputs o = 0..31: q' row r0 + o; o = 32..63: u row r0 + o - 32; four
  // threads per output, 32 elements each
  const int o = t >> 2, qr = t & 3;
  const float* row = &mat[o >> 5][(o & 31) * kPrepRS + 32 * qr];
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float4 a = *reinterpret_cast<const float4*>(row + 4 * c);
    const float* x = xs + 32 * qr + 4 * c;
    acc = fmaf(x[0], a.x, acc);
    acc = fmaf(x[1], a.y, acc);
    acc = fmaf(x[2], a.z, acc);
    acc = fmaf(x[3], a.w, acc);
  }
  if (o < 32 && !P) acc = qr == 0 ? xs[r0 + o] : 0.0f;
  acc = group_sum<4>(acc);
  if (qr == 0) {
    const int r = r0 + (o & 31);
    if (o < 32) {
      qp[r] = acc;
      if (q_rot) q_rot[static_cast<int64_t>(h) * 128 + r] = acc;
    } else {
      u[r] = acc;
      if (q_sketch) q_sketch[static_cast<int64_t>(h) * 128 + r] = acc;
    }
  }
  __syncthreads();
  float* out = qtab + static_cast<int64_t>(h) * kP7QTab;
  constexpr int kT1 = 1024 / kP7PrepParts, kTq = 4096 / kP7PrepParts;
  for (int e = kT1 * part + t; e < kT1 * (part + 1); e += 256) {
    const int j = e >> 4, c = e & 15;
    out[e] = qp[2 * j] * csl[2 * c] + qp[2 * j + 1] * csl[2 * c + 1];
  }
  for (int e = kTq * part + t; e < kTq * (part + 1); e += 256) {
    const int pos = e >> 8, bits = e & 255;
    float sum = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; ++b) sum += ((bits >> b) & 1) ? u[8 * pos + b] : 0.0f;
    out[1024 + e] = sum;
  }
  if (t < 64) {
    const float sum = wave_sum_f(t < kPrepRows ? u[r0 + t] : 0.0f);
    if (t == 0) out[5120 + part] = sum;
    if (part == 0 && t >= kP7PrepParts && t < 16) out[5120 + t] = 0.0f;
  }
}

typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

struct P7Quarter {
  uint32_t l1[2];  // level-1 angle words 2qt, 2qt+1
  uint32_t l2;     // level-2 word 8 + qt/2
  uint32_t w10, w11;
  uint32_t qj;     // QJL word qt
  uint32_t nrm;
};

// Row pointers of the key arrays at a wave-uniform first row; the lanes add
// 32-bit row offsets (scalar base + vector offset addressing).
struct P7Rows {
  const uint32_t* ang;
  const uint32_t* nrm;
  const uint32_t* qjl;
};

__device__ __forceinline__ P7Rows p7_rows(const P7Keys& k, int64_t row0) {
  return P7Rows{k.angles + row0 * kP7Words, k.norms + row0, k.qjl + row0 * 4};
}

template <typename T>
__device__ __forceinline__ T nt_at(const void* base, uint32_t byte_off) {
  return __builtin_nontemporal_load(
      reinterpret_cast<const T*>(static_cast<const char*>(base) + byte_off));
}

__device__ __forceinline__ void load_p7_quarter(const P7Rows& R, uint32_t off, int qt, P7Quarter& Q) {
  const uint32_t a = off * (kP7Words * 4);
  const u32x2v l1 = nt_at<u32x2v>(R.ang, a + 8 * qt);
  Q.l1[0] = l1.x;
  Q.l1[1] = l1.y;
  Q.l2 = nt_at<uint32_t>(R.ang, a + 32 + 4 * (qt >> 1));
  const u32x2v hi = nt_at<u32x2v>(R.ang, a + 40);
  Q.w10 = hi.x;
  Q.w11 = hi.y;
  Q.qj = nt_at<uint32_t>(R.qjl, off * 16 + 4 * qt);
  Q.nrm = nt_at<uint32_t>(R.nrm, off * 4);
}

// Quarter qt's part of the score of one key for the G heads of the tables;
// the four quarters (lanes 4m .. 4m+3) sum to
// sc * (sum_j r1_j t1[j][n_j] + coef ||r|| (2 sum tq - U)).
template <int G>
__device__ __forceinline__ void p7_quarter_score(const P7Tables<G>& T, const P7Quarter& Q, int qt,
                                                 float sc, float out[G]) {
  const uint32_t w11 = Q.w11, w10 = Q.w10;
  // the top pair's factor: one float of the entry per quarter lane
  const float ta_q = reinterpret_cast<const float*>(&T.t2[((w11 >> 28) & 3u) | ((w11 >> 22) & 0x3Cu)])[qt];
  const float4 tb = T.t2[((w11 >> (16 + 2 * qt)) & 3u) | (((w11 >> (4 * qt)) & 15u) << 2)];
  float4 tc[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii)
    tc[ii] = T.t2[((w10 >> (8 * qt + 2 * ii)) & 3u) | (((Q.l2 >> (16 * (qt & 1) + 4 * ii)) & 15u) << 2)];
  float qa[G], acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    qa[g] = 0.0f;
    acc[g] = 0.0f;
  }
  // byte addresses: lane base + (index << 2), constant parts in the
  // instruction's offset field
  constexpr int kE = 4 * G;  // bytes of one table entry (G heads)
  const char* tqb = reinterpret_cast<const char*>(&T.tq[0][0][0]) + qt * (4 * 256 * kE);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t byte = __builtin_amdgcn_ubfe(Q.qj, 8 * b, 8);
    const float* e = reinterpret_cast<const float*>(tqb + b * (256 * kE) + byte * kE);
#pragma unroll
    for (int g = 0; g < G; ++g) qa[g] += e[g];
  }
  const float R = h2f_lo(Q.nrm), rn = h2f_hi(Q.nrm);
  const float r5 = R * ta_q;
  const float r3[4] = {r5 * tb.x, r5 * tb.y, r5 * tb.z, r5 * tb.w};
  // rotated level-1 rows (p7_t1_row): row jj of quarter qt is at
  // 16 qt + (jj & ~3) + ((jj + qt) & 3)
  const char* t1b = reinterpret_cast<const char*>(&T.t1[0][0][0]) + qt * (16 * 16 * kE);
  const char* t1r[4];  // rotated row base of pair jj with jj % 4 == e
#pragma unroll
  for (int e = 0; e < 4; ++e) t1r[e] = t1b + static_cast<uint32_t>((e + qt) & 3) * (16 * kE);
  // entry offsets nibble * kE (at most 15 * 16 = 240) pre-scaled into bytes:
  // byte b of lo[w] / hi[w] is the low / high nibble of byte b of word w
  // times kE, so each lookup address is one add of a selected byte
  constexpr int kSh = kE == 4 ? 2 : (kE == 8 ? 3 : 4);
  constexpr uint32_t kMask = 0x0F0F0F0Fu << kSh;
  uint32_t lo[2], hi[2];
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    lo[w] = (Q.l1[w] << kSh) & kMask;
    hi[w] = (Q.l1[w] >> (4 - kSh)) & kMask;
    // opaque: otherwise each byte select is folded back into a shift and a
    // mask of the raw word (two instructions per lookup instead of none)
    asm("" : "+v"(lo[w]), "+v"(hi[w]));
  }
  // all 16 level-1 entries first (one aligned G-float read each, ds_read_b64
  // at G = 2 with the constant in its offset field), then the products
  typedef float vGf __attribute__((ext_vector_type(G)));
  vGf ents[16];
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) {
    const int ii = jj >> 2, e = jj & 3, n = jj % 8;
    const uint32_t src = (n & 1) ? hi[jj >> 3] : lo[jj >> 3];
    const uint32_t off = (src >> (8 * (n >> 1))) & 0xFFu;
    ents[jj] = *reinterpret_cast<const vGf*>(t1r[e] + ii * (4 * 16 * kE) + off);
  }
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const float r1[4] = {r3[ii] * tc[ii].x, r3[ii] * tc[ii].y, r3[ii] * tc[ii].z, r3[ii] * tc[ii].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int g = 0; g < G; ++g) acc[g] = fmaf(r1[e], ents[4 * ii + e][g], acc[g]);
    }
  }
  const float cr = kQjlCoef * rn;
#pragma unroll
  for (int g = 0; g < G; ++g) out[g] = sc * fmaf(cr, 2.0f * qa[g] - (qt == 0 ? T.U[g] : 0.0f), acc[g]);
}

// Full scores in all four lanes of each key.
template <int G>
__device__ __forceinline__ void quarter_sum(float s[G]) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    s[g] = group_sum<4>(s[g]);  // DPP quad permutes: (a + b) + (c + d)
  }
}

// Scores only (compressed_score over polar7 keys): four lanes per key, NT / 4
// keys per pass of an NT-thread workgroup, NP passes per workgroup; the next
// pass's words are loaded while the current pass is scored.  Grid (key
// blocks, kv heads * head subgroups).
// FUSED: the query tables are built in the prologue from q, P and S P
// (build_p7_tables) instead of read from k.qtab.
template <int G, int NT, int NP, bool FUSED = false>
__global__ __launch_bounds__(NT) void polar7_score_kernel(P7Keys k, int n, int cap, int gqa,
                                                          int n_sub, float scale) {
  constexpr int KPP = NT / 4, KPW = NP * KPP;  // keys per pass, per workgroup
  __shared__ P7Tables<G> T;
  const int hy = blockIdx.y, kvh = hy / n_sub, sub = hy - (hy / n_sub) * n_sub;
  const int h0 = kvh * gqa + sub * G;
  const int qt = threadIdx.x & 3, key = threadIdx.x >> 2;  // key of a pass
  const int t0 = blockIdx.x * KPW + key;
  const int last = n - 1;
  const int64_t rowbase = static_cast<int64_t>(kvh) * cap;
  const int npass = min(NP, (n - blockIdx.x * KPW + KPP - 1) / KPP);
  // rows of this workgroup: rowbase + blockIdx.x * KPW + (0 .. lim)
  const P7Rows R = p7_rows(k, rowbase + blockIdx.x * KPW);
  const uint32_t lim = static_cast<uint32_t>(last - blockIdx.x * KPW);
  __shared__ int s_done[NT / 64];  // passes done, per wave (issue pacing)
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  if (lane == 0) s_done[wv] = 0;  // published by the tables' barrier
  P7Quarter A, B;
  auto first = [&]() { load_p7_quarter(R, min(static_cast<uint32_t>(key), lim), qt, A); };
  if constexpr (FUSED) {
    first();
    build_p7_tables<G, NT>(T, k, h0);
  } else {
    load_p7_tables<G, NT>(T, k, h0, first);
  }
  auto pass = [&](const P7Quarter& Q, int r) {
    float s[G];
    p7_quarter_score<G>(T, Q, qt, scale, s);
    quarter_sum<G>(s);
    const int t = t0 + KPP * r;
    if (qt < G && t < n) {
      float v = s[0];
#pragma unroll
      for (int g = 1; g < G; ++g) v = qt == g ? s[g] : v;
      k.scores[static_cast<int64_t>(h0 + qt) * n + t] = v;
    }
  };
  // the four waves of a SIMD kept level (see pace_waves)
  pace_waves<NT / 64>(s_done, wv, lane, 0);
  for (int r = 0; r < npass; r += 2) {
    load_p7_quarter(R, min(static_cast<uint32_t>(key + KPP * (r + 1)), lim), qt, B);
    pass(A, r);
    pace_waves<NT / 64>(s_done, wv, lane, r + 1);
    load_p7_quarter(R, min(static_cast<uint32_t>(key + KPP * (r + 2)), lim), qt, A);
    if (r + 1 < npass) {
      pass(B, r + 1);
      pace_waves<NT / 64>(s_done, wv, lane, r + 2);
    }
  }
}

template <typename SB>
__device__ __forceinline__ float2 sb_pair(const uint32_t* w);
template <>
__device__ __forceinline__ float2 sb_pair<__half>(const uint32_t* w) {
  return make_float2(h2f_lo(w[0]), h2f_hi(w[0]));
}
template <>
__device__ __forceinline__ float2 sb_pair<float>(const uint32_t* w) {
  return make_float2(__uint_as_float(w[0]), __uint_as_float(w[1]));
}

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// K slot of tile key t (0..63) in the P.V operands: key 32 kb + 4 j + c is
// slot 32 kb + 8 c + j (lane group c of the B operand holds slots 8c .. 8c+7).
__device__ __forceinline__ int p7_slot(int t) { return (t & 32) | ((t & 3) << 3) | ((t >> 2) & 7); }

// polar7 attention: polar7 + QJL scores, softmax, int4 V (group 64,
// scale/bias SB), split-K.  Per 64-key tile of a wave:
//  - scores: four lanes per key (quarter qt = lane & 3) over four sub-tiles
//    of 16 keys; the key words are loaded one tile ahead, the V words of a
//    tile before its scores (which hide their latency);
//  - the weights p and the tile's V scale / bias go to LDS in K-slot order;
//  - P.V on v_mfma_f32_16x16x32_bf16, two blocks of 32 keys: A = (128 +
//    nibble) as bf16 for 16 V words x 32 keys (lane: word lane % 16 of keys
//    32 kb + 4 j + lane / 16, one v_perm + and-or per two nibbles), B = the
//    bf16 hi / lo split of p * s_v (~16 bits) in columns (head, quant group).
//    bf16 keeps fp32's exponent range, so no scale of V can overflow it.
//    The 128 offset (128 * sum(hi + lo)) and the bias term sum(p * b_v) are
//    accumulated per column and removed at the end.
// Waves per polar7 attention workgroup: eight, two per SIMD at one workgroup
// per CU, sharing the workgroup's staged query tables.
constexpr int kP7Waves = 8;

// FUSED: the query tables are built in the prologue from q, P and S P
// (build_p7_tables) instead of read from k.qtab.
template <int G, typename SB, int NW, bool FUSED = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void polar7_sdpa_kernel(SdpaParams p, P7Keys k) {
  pin_args(p);
  asm volatile("" ::"s"(k.qtab), "s"(k.cs), "s"(k.angles), "s"(k.norms), "s"(k.qjl));
  constexpr int D = 128;
  __shared__ P7Tables<G> T;
  using Fin = Finalize<G, D, NW>;
  __shared__ __align__(16) float arena[Fin::kArena];
  __shared__ float p_lds[NW][G][64];   // [wave][head][slot]
  __shared__ float sv_lds[NW][2][64];  // [wave][quant group][slot] V scale
  __shared__ float bv_lds[NW][2][64];  // V bias
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hy = blockIdx.y, split = blockIdx.x;
  const int kvh = hy / p.n_sub, sub = hy - kvh * p.n_sub;
  const int h0 = kvh * p.gqa + sub * G;
  const SplitRange rg = split_range(p, 0, split);
  if (split >= rg.S) return;
  const int64_t rowbase = static_cast<int64_t>(kvh) * p.cap;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int base0 = rg.t_begin + wv * 64;
  const int last = rg.t_end - 1;
  const int ntile = base0 < rg.t_end ? (rg.t_end - base0 + NW * 64 - 1) / (NW * 64) : 0;
  constexpr int SBW = sizeof(SB) / 2;  // words of one row's two scales (or biases)
  const int qt = lane & 3, kq = lane >> 2;  // scoring: quarter, key of the sub-tile
  const int vm = lane & 15, vc = lane >> 4;  // P.V: V word / B column, K-slot group
  const int cg = (vm >> 1) % G, cgr = vm & 1;  // this lane's B column (head, quant group)
  const int my_slot = p7_slot(lane);

  // Key words of sub-tile u (keys 16 u + (lane >> 2)) of the current tile;
  // once scored, each sub-tile's registers receive the next tile's words.
  P7Quarter key[4];
  auto load_sub = [&](P7Quarter& Q, int tb, int u) {
    const P7Rows R = p7_rows(k, rowbase + tb);
    load_p7_quarter(R, min(static_cast<uint32_t>(16 * u + kq), static_cast<uint32_t>(last - tb)), qt, Q);
  };
  auto first = [&]() {
    if (ntile > 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u) load_sub(key[u], base0, u);
    }
  };
  __shared__ int s_done[NW];  // tiles processed, per wave (issue pacing)
  if (lane == 0) s_done[wave] = 0;  // published by the tables' barrier
  if constexpr (FUSED) {
    first();
    build_p7_tables<G, NW * 64>(T, k, h0);
  } else {
    load_p7_tables<G, NW * 64>(T, k, h0, first);
  }

  float m_run[G], l_run[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.0f;
  }
  float wsum = 0.0f, bacc = 0.0f;  // this lane's column: sum(hi + lo), sum(p * b_v)
  v4f cv[8];                       // [2 * byte + nibble half]
#pragma unroll
  for (int f = 0; f < 8; ++f) cv[f] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // bf16 magic of (128 + nibble), in a VGPR so each A word is one and-or
  uint32_t magic = 0x43004300u;
  asm volatile("" : "+v"(magic));

  // tile at tb; tn = first key of the next tile (clamped into the split)
  auto process = [&](int tb, int tn) {
    const uint32_t lim = static_cast<uint32_t>(last - tb);
    const uint32_t* vrow = p.vq + (rowbase + tb) * 16;
    uint32_t vw[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t key = min(static_cast<uint32_t>(32 * kb + 4 * j + vc), lim);
        vw[kb][j] = nt_at<uint32_t>(vrow, key * 64 + vm * 4);
      }
    const uint32_t kl = min(static_cast<uint32_t>(lane), lim);
    const void* vsrow = static_cast<const uint32_t*>(p.vs) + (rowbase + tb) * SBW;
    const void* vbrow = static_cast<const uint32_t*>(p.vb) + (rowbase + tb) * SBW;
    uint32_t vsw[SBW], vbw[SBW];
#pragma unroll
    for (int i = 0; i < SBW; ++i) {
      vsw[i] = nt_at<uint32_t>(vsrow, (kl * SBW + i) * 4);
      vbw[i] = nt_at<uint32_t>(vbrow, (kl * SBW + i) * 4);
    }
    float s[4][G];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      p7_quarter_score<G>(T, key[u], qt, p.scale_log2, s[u]);
      load_sub(key[u], tn, u);
      quarter_sum<G>(s[u]);
      const bool valid = tb + 16 * u + kq < rg.t_end;
#pragma unroll
      for (int g = 0; g < G; ++g) s[u][g] = valid ? s[u][g] : -INFINITY;
    }
    __builtin_amdgcn_sched_barrier(0);
    // online softmax (log2 domain); a raised max rescales this lane's column
    float fac = 1.0f;
    bool raised = false;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mt = fmaxf(fmaxf(s[0][g], s[1][g]), fmaxf(s[2][g], s[3][g]));
      const float m_new = fmaxf(m_run[g], wave_max_f(mt));
      if (m_new > m_run[g]) {  // wave-uniform
        const float f = merge_factor(m_run[g], m_new);
        l_run[g] *= f;
        fac = cg == g ? f : fac;
        m_run[g] = m_new;
        raised = true;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float pw = s[u][g] == -INFINITY ? 0.0f : fast_exp2(s[u][g] - m_run[g]);
        if (qt == 0) {
          l_run[g] += pw;
          p_lds[wave][g][p7_slot(16 * u + kq)] = pw;
        }
      }
    }
    if (raised) {
      wsum *= fac;
      bacc *= fac;
#pragma unroll
      for (int f = 0; f < 8; ++f) cv[f] *= fac;
    }
    const float2 sc2 = sb_pair<SB>(vsw), bi2 = sb_pair<SB>(vbw);
    sv_lds[wave][0][my_slot] = sc2.x;
    sv_lds[wave][1][my_slot] = sc2.y;
    bv_lds[wave][0][my_slot] = bi2.x;
    bv_lds[wave][1][my_slot] = bi2.y;
    wave_lds_sync();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int s0 = 32 * kb + 8 * vc;
      const float4 pa = *reinterpret_cast<const float4*>(&p_lds[wave][cg][s0]);
      const float4 pb = *reinterpret_cast<const float4*>(&p_lds[wave][cg][s0 + 4]);
      const float4 sa = *reinterpret_cast<const float4*>(&sv_lds[wave][cgr][s0]);
      const float4 sb = *reinterpret_cast<const float4*>(&sv_lds[wave][cgr][s0 + 4]);
      const float4 ba = *reinterpret_cast<const float4*>(&bv_lds[wave][cgr][s0]);
      const float4 bb = *reinterpret_cast<const float4*>(&bv_lds[wave][cgr][s0 + 4]);
      const float pj[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
      const float sj[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
      const float bj[8] = {ba.x, ba.y, ba.z, ba.w, bb.x, bb.y, bb.z, bb.w};
      // weights in bf16 pairs (slots 2k, 2k + 1: one B operand word): hi and
      // lo = w - hi, each pair by one packed conversion; the weight sum of
      // the 128 offset takes a word per v_dot2 with (1, 1)
      uint32_t bh[4], bl[4];
      const v2bf ones = __builtin_bit_cast(v2bf, 0x3F803F80u);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float w0 = pj[2 * k] * sj[2 * k], w1 = pj[2 * k + 1] * sj[2 * k + 1];
        uint32_t hb = __builtin_bit_cast(uint32_t, v2bf{static_cast<__bf16>(w0), static_cast<__bf16>(w1)});
        asm("" : "+v"(hb));  // h0, h1 from the packed word
        const float h0 = __uint_as_float(hb << 16), h1 = __uint_as_float(hb & 0xFFFF0000u);
        const uint32_t lb =
            __builtin_bit_cast(uint32_t, v2bf{static_cast<__bf16>(w0 - h0), static_cast<__bf16>(w1 - h1)});
        bh[k] = hb;
        bl[k] = lb;
        wsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, hb), ones, wsum, false);
        wsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, lb), ones, wsum, false);
        bacc = fmaf(pj[2 * k], bj[2 * k], bacc);
        bacc = fmaf(pj[2 * k + 1], bj[2 * k + 1], bacc);
      }
      const v8bf bhi = __builtin_bit_cast(v8bf, u32x4v{bh[0], bh[1], bh[2], bh[3]});
      const v8bf blo = __builtin_bit_cast(v8bf, u32x4v{bl[0], bl[1], bl[2], bl[3]});
#pragma unroll
      for (int by = 0; by < 4; ++by) {
        // byte `by` of the words of slots 2r, 2r+1 -> the two 16-bit halves
        const uint32_t sel = static_cast<uint32_t>(by) | (0x0Cu << 8) |
                             (static_cast<uint32_t>(4 + by) << 16) | (0x0Cu << 24);
        uint32_t alo[4], ahi[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t x = __builtin_amdgcn_perm(vw[kb][2 * r + 1], vw[kb][2 * r], sel);
          alo[r] = (x & 0x000F000Fu) | magic;
          ahi[r] = ((x >> 4) & 0x000F000Fu) | magic;
        }
        const v8bf a_lo = __builtin_bit_cast(v8bf, u32x4v{alo[0], alo[1], alo[2], alo[3]});
        const v8bf a_hi = __builtin_bit_cast(v8bf, u32x4v{ahi[0], ahi[1], ahi[2], ahi[3]});
        cv[2 * by] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, bhi, cv[2 * by], 0, 0, 0);
        cv[2 * by + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, bhi, cv[2 * by + 1], 0, 0, 0);
        cv[2 * by] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, blo, cv[2 * by], 0, 0, 0);
        cv[2 * by + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, blo, cv[2 * by + 1], 0, 0, 0);
      }
    }
    wave_lds_sync();
  };

  // the two waves of a SIMD kept level: the one behind issues first (its
  // priority raised), so they end their tiles together rather than ~4.5 us
  // apart, the later one alone on the SIMD
  pace_waves<NW>(s_done, wv, lane, 0);
  for (int it = 0; it < ntile; ++it) {
    const int tb = base0 + it * NW * 64;
    process(tb, min(tb + NW * 64, last));
    pace_waves<NW>(s_done, wv, lane, it + 1);
  }

  // columns: sum the four K-slot groups; lane (vm, vc) holds V words
  // 4 vc + i (dims 8 (4 vc + i) + 2 byte + half) of column vm, and the words
  // of quant group cgr are those with vc >> 1 == cgr
  wsum = xor16_sum(wsum);
  wsum = xor32_sum(wsum);
  bacc = xor16_sum(bacc);
  bacc = xor32_sum(bacc);
  float ls[G];
#pragma unroll
  for (int g = 0; g < G; ++g) ls[g] = wave_sum_f(l_run[g]);
  if (vm < 2 * G && (vc >> 1) == cgr) {
    float* o = Fin::o(arena, wave, cg);
    const float off = bacc - 128.0f * wsum;
#pragma unroll
    for (int f = 0; f < 8; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[8 * (4 * vc + i) + f] = cv[f][i] + off;
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      Fin::m(arena, wave)[g] = m_run[g];
      Fin::l(arena, wave)[g] = ls[g];
    }
  }
  Fin::run(p, arena, h0, rg.S, split, hy);
}

// ---- host helpers -----------------------------------------------------------------

// query heads per workgroup of the polar kernels (LDS tables scale with it)
int polar_subgroup(int gqa, int max_g) {
  for (int g : {4, 2}) if (g <= max_g && gqa % g == 0) return g;
  return 1;
}

// keys per workgroup: about one workgroup per CU, multiples of 256 keys.
// Every workgroup first stages its query tables (~52 KB at GQA 2) in LDS;
// at four workgroups per CU (72 KB of keys per workgroup at 32k) that fixed
// cost is paid four times as often: the polar7 attention kernel measured
// 51.7 us at four per CU, 45.0 us at one.
int polar_chunk(int L, int64_t groups) {
  const int64_t floor_c = (static_cast<int64_t>(L) + kMaxSplits - 1) / kMaxSplits;
  const int64_t want = (static_cast<int64_t>(L) * groups + target_wgs() - 1) / target_wgs();
  int64_t c = (want + 255) / 256 * 256;
  c = std::max<int64_t>({c, int64_t{256}, floor_c});
  return static_cast<int>(std::min<int64_t>(c, 1 << 30));
}

int polar_splits_bound(int L, int64_t groups) {
  if (L <= 0) return 1;
  const int64_t by_len = (static_cast<int64_t>(L) + 255) / 256;
  const int64_t by_wgs = (target_wgs() + groups - 1) / groups;
  return static_cast<int>(std::max<int64_t>(1, std::min({by_len, by_wgs, int64_t{kMaxSplits}})));
}

int check_codebooks(const float* cb, const int* ncb, int max_first, int max_rest, CsSource& s,
                     const char* fn) {
  TQ_CHECK_ARG(ncb != nullptr, "%s: n_codebook is NULL", fn);
  int off = 0;
  for (int l = 0; l < 4; ++l) {
    const int mx = l == 0 ? max_first : max_rest;
    TQ_CHECK_ARG(ncb[l] >= 1 && ncb[l] <= mx, "%s: codebook %d size %d not in [1, %d]", fn, l + 1,
                 ncb[l], mx);
    s.ncb[l] = ncb[l];
    s.off[l] = off;
    off += ncb[l];
  }
  s.cb = cb;
  return TQ_OK;
}

}  // namespace
}  // namespace tq

using namespace tq;

// ============================================================================
// C ABI
// ============================================================================

namespace {

int encode16_common(const float* x, const float* P, const float* codebooks, const int* n_codebook,
                    int64_t n, int D, int block_size, bool packed, uint8_t* i1, uint8_t* i2,
                    uint8_t* i3, uint8_t* i4, uint32_t* p1, uint8_t* p2, uint8_t* p3, uint8_t* p4,
                    uint16_t* radii, void* stream, const char* fn) {
  if (block_size != 16) {
    set_error("%s: block_size must be 16 (the reference kernels hard-code it)", fn);
    return TQ_ERR_UNSUPPORTED;
  }
  TQ_CHECK_ARG(D >= 16 && D <= 2048 && D % 16 == 0, "%s: dim must be a multiple of 16 in [16, 2048]", fn);
  TQ_CHECK_ARG(n >= 0, "%s: n_vectors must be >= 0", fn);
  TQ_CHECK_ARG(x && codebooks && radii, "%s: null pointer", fn);
  CsSource s{};
  const int st = check_codebooks(codebooks, n_codebook, packed ? 16 : 256, packed ? 4 : 256, s, fn);
  if (st != TQ_OK) return st;
  if (packed) TQ_CHECK_ARG(p1 && p2 && p3 && p4, "%s: null output", fn);
  else TQ_CHECK_ARG(i1 && i2 && i3 && i4, "%s: null output", fn);
  if (n == 0) return TQ_OK;
  Enc16Params p{};
  p.x = x; p.P = P; p.n = n; p.D = D;
  p.rows = std::max(1, 2048 / D);
  p.cb = codebooks;
  for (int l = 0; l < 4; ++l) { p.ncb[l] = s.ncb[l]; p.cb_off[l] = s.off[l]; }
  p.i1 = i1; p.i2 = i2; p.i3 = i3; p.i4 = i4;
  p.p1 = p1; p.p2 = p2; p.p3 = p3; p.p4 = p4;
  p.radii = radii;
  const int64_t grid = (n + p.rows - 1) / p.rows;
  TQ_CHECK_ARG(grid <= (int64_t{1} << 31) - 1, "%s: too many vectors", fn);
  const size_t shm = sizeof(float) * (1024 + 2 * static_cast<size_t>(p.rows) * D);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (packed) polar_encode16_kernel<true><<<static_cast<unsigned>(grid), 256, shm, hs>>>(p);
  else polar_encode16_kernel<false><<<static_cast<unsigned>(grid), 256, shm, hs>>>(p);
  TQ_CHECK_LAUNCH("polar_encode16_kernel");
  return TQ_OK;
}

int decode16_common(const Keys16& k, const float* P, const float* codebooks, const float* cs_tables,
                    const int* n_codebook, int64_t n, int D, int block_size, bool packed, float* out,
                    void* stream, const char* fn) {
  if (block_size != 16) {
    set_error("%s: block_size must be 16 (the reference kernels hard-code it)", fn);
    return TQ_ERR_UNSUPPORTED;
  }
  TQ_CHECK_ARG(D >= 16 && D <= 2048 && D % 16 == 0, "%s: dim must be a multiple of 16 in [16, 2048]", fn);
  TQ_CHECK_ARG(n >= 0 && out && k.radii, "%s: null pointer or negative n", fn);
  TQ_CHECK_ARG(codebooks || cs_tables, "%s: codebooks or cos/sin tables required", fn);
  Dec16Params p{};
  const int st = check_codebooks(codebooks, n_codebook, packed ? 16 : 256, packed ? 4 : 256, p.src, fn);
  if (st != TQ_OK) return st;
  p.src.cs = cs_tables;
  p.k = k;
  p.P = P;
  p.out = out;
  p.n = n;
  p.D = D;
  p.rows = std::max(1, 2048 / D);
  if (n == 0) return TQ_OK;
  const int64_t grid = (n + p.rows - 1) / p.rows;
  const size_t shm = sizeof(float) * (2048 + static_cast<size_t>(p.rows) * D);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (packed) polar_decode16_kernel<true><<<static_cast<unsigned>(grid), 256, shm, hs>>>(p);
  else polar_decode16_kernel<false><<<static_cast<unsigned>(grid), 256, shm, hs>>>(p);
  TQ_CHECK_LAUNCH("polar_decode16_kernel");
  return TQ_OK;
}

template <int D, int G, bool kPacked>
void launch_score16(const Attn16& a, int n, int gqa, int n_sub, dim3 grid, hipStream_t s) {
  polar16_score_kernel<D, G, kPacked><<<grid, 256, 0, s>>>(a, n, gqa, n_sub);
}

template <int D, bool kPacked>
int dispatch_score16_g(int G, const Attn16& a, int n, int gqa, int n_sub, dim3 grid, hipStream_t s) {
  switch (G) {
    case 1: launch_score16<D, 1, kPacked>(a, n, gqa, n_sub, grid, s); break;
    case 2: launch_score16<D, 2, kPacked>(a, n, gqa, n_sub, grid, s); break;
    default: launch_score16<D, 4, kPacked>(a, n, gqa, n_sub, grid, s); break;
  }
  TQ_CHECK_LAUNCH("polar16_score_kernel");
  return TQ_OK;
}

template <int D, bool kPacked>
int dispatch_sdpa16_g(int G, const SdpaParams& p, const Attn16& a, dim3 grid, hipStream_t s) {
  switch (G) {
    case 1: polar16_sdpa_kernel<D, 1, kPacked><<<grid, 256, 0, s>>>(p, a); break;
    case 2: polar16_sdpa_kernel<D, 2, kPacked><<<grid, 256, 0, s>>>(p, a); break;
    default: polar16_sdpa_kernel<D, 4, kPacked><<<grid, 256, 0, s>>>(p, a); break;
  }
  TQ_CHECK_LAUNCH("polar16_sdpa_kernel");
  return TQ_OK;
}

int attn16_setup(Attn16& a, const float* q, const uint8_t* i1, const uint8_t* i2, const uint8_t* i3,
                 const uint8_t* i4, const uint32_t* p1, const uint8_t* p2, const uint8_t* p3,
                 const uint8_t* p4, const uint16_t* radii, const float* codebooks,
                 const int* n_codebook, bool packed, int Hq, int Hkv, int n, int D, int block_size,
                 const char* fn) {
  if (block_size != 16) {
    set_error("%s: block_size must be 16 (the reference kernels hard-code it)", fn);
    return TQ_ERR_UNSUPPORTED;
  }
  if (D != 64 && D != 128 && D != 256) {
    set_error("%s: dim must be 64, 128 or 256 (got %d)", fn, D);
    return TQ_ERR_UNSUPPORTED;
  }
  TQ_CHECK_ARG(Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "%s: num_heads must be a multiple of num_kv_heads", fn);
  TQ_CHECK_ARG(n >= 0, "%s: n_keys must be >= 0", fn);
  TQ_CHECK_ARG(q && radii && codebooks, "%s: null pointer", fn);
  if (packed) TQ_CHECK_ARG(p1 && p2 && p3 && p4, "%s: null index array", fn);
  else TQ_CHECK_ARG(i1 && i2 && i3 && i4, "%s: null index array", fn);
  a = Attn16{};
  const int st = check_codebooks(codebooks, n_codebook, packed ? 16 : 256, packed ? 4 : 256, a.src, fn);
  if (st != TQ_OK) return st;
  a.k.i1 = i1; a.k.i2 = i2; a.k.i3 = i3; a.k.i4 = i4;
  a.k.p1 = p1; a.k.p2 = p2; a.k.p3 = p3; a.k.p4 = p4;
  a.k.radii = radii;
  a.q = q;
  a.D = D;
  return TQ_OK;
}

int score16_common(Attn16& a, int Hq, int Hkv, int n, float scale, float* scores, bool packed,
                   void* stream, const char* fn) {
  TQ_CHECK_ARG(scores != nullptr, "%s: scores is NULL", fn);
  TQ_CHECK_ARG(std::isfinite(scale), "%s: scale must be finite", fn);
  if (n == 0) return TQ_OK;
  const int gqa = Hq / Hkv, G = polar_subgroup(gqa, 4), n_sub = gqa / G;
  a.scores = scores;
  a.qscale = scale;
  TQ_CHECK_ARG(Hkv * n_sub <= 65535, "%s: too many heads", fn);
  dim3 grid((n + 1023) / 1024, Hkv * n_sub);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (a.D) {
    case 64: return packed ? dispatch_score16_g<64, true>(G, a, n, gqa, n_sub, grid, s)
                           : dispatch_score16_g<64, false>(G, a, n, gqa, n_sub, grid, s);
    case 128: return packed ? dispatch_score16_g<128, true>(G, a, n, gqa, n_sub, grid, s)
                            : dispatch_score16_g<128, false>(G, a, n, gqa, n_sub, grid, s);
    default: return packed ? dispatch_score16_g<256, true>(G, a, n, gqa, n_sub, grid, s)
                           : dispatch_score16_g<256, false>(G, a, n, gqa, n_sub, grid, s);
  }
}

size_t polar_ws_size(int Hq, int Hkv, int D, int max_len, int max_g) {
  const int gqa = Hq / Hkv, G = polar_subgroup(gqa, max_g);
  const int64_t groups = static_cast<int64_t>(Hkv) * (gqa / G);
  return ws_layout(1, Hq, D, polar_splits_bound(max_len, groups)).total;
}

// common split-K set-up of the polar attention kernels
int polar_sdpa_params(SdpaParams& p, int Hq, int Hkv, int D, int n, int cap, float scale, int window,
                      float denom_eps, int max_g, float* out, void* workspace, size_t ws_bytes,
                      dim3& grid, int& G, const char* fn) {
  TQ_CHECK_ARG(out != nullptr, "%s: out is NULL", fn);
  TQ_CHECK_ARG(std::isfinite(scale), "%s: scale must be finite", fn);
  TQ_CHECK_ARG(window >= 0, "%s: sliding_window must be >= 0", fn);
  TQ_CHECK_ARG(n >= 0 && cap >= 1 && n <= cap, "%s: need 0 <= kv_len <= kv_capacity", fn);
  TQ_CHECK_ARG(Hq <= kMaxCounters, "%s: too many heads", fn);
  const int gqa = Hq / Hkv;
  G = polar_subgroup(gqa, max_g);
  const int n_sub = gqa / G;
  const int64_t groups = static_cast<int64_t>(Hkv) * n_sub;
  const int eff = window > 0 ? std::min(n, window) : n;
  const int chunk = polar_chunk(eff, groups);
  const int max_splits = polar_splits_bound(eff, groups);
  const WsLayout wl = ws_layout(1, Hq, D, max_splits);
  // the split partials are addressed with 32-bit byte offsets
  TQ_CHECK_ARG(wl.total - wl.o_off < (size_t{1} << 31), "%s: split-K partials exceed 2 GiB", fn);
  if (max_splits > 1 && (!workspace || ws_bytes < wl.total)) {
    set_error("%s: workspace of %zu bytes needed (got %zu)", fn, wl.total, ws_bytes);
    return TQ_ERR_WORKSPACE;
  }
  TQ_CHECK_ARG(Hkv * n_sub <= 65535, "%s: too many heads", fn);
  p = SdpaParams{};
  p.out = out;
  char* ws = static_cast<char*>(workspace);
  p.ws_cnt = ws ? reinterpret_cast<int*>(ws + wl.cnt_off) : nullptr;
  p.ws_ml = ws ? reinterpret_cast<float*>(ws + wl.ml_off) : nullptr;
  p.ws_o = ws ? reinterpret_cast<float*>(ws + wl.o_off) : nullptr;
  p.Hq = Hq; p.Hkv = Hkv; p.cap = cap; p.gqa = gqa; p.n_sub = n_sub;
  p.n = n; p.n_clamp = n; p.window = window;
  p.scale_log2 = scale * kLog2e;
  p.chunk = chunk;
  p.max_splits = max_splits;
  p.denom_eps = denom_eps;
  grid = dim3(max_splits, Hkv * n_sub, 1);
  p.cnt_stride = counter_stride(Hq);
  return TQ_OK;
}

int p7_keys_setup(P7Keys& k, const float* q_tables, const uint32_t* angles, const uint32_t* norms,
                  const uint32_t* qjl, const float* cs_tables, int Hq, int Hkv, const char* fn) {
  TQ_CHECK_ARG(q_tables && angles && norms && qjl && cs_tables, "%s: null pointer", fn);
  TQ_CHECK_ARG(Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "%s: num_heads must be a multiple of num_kv_heads", fn);
  TQ_CHECK_ARG(reinterpret_cast<uintptr_t>(angles) % 16 == 0 && reinterpret_cast<uintptr_t>(qjl) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(q_tables) % 16 == 0,
               "%s: angles / qjl / q_tables must be 16-byte aligned", fn);
  k = P7Keys{};
  k.qtab = q_tables; k.cs = cs_tables;
  k.angles = angles; k.norms = norms; k.qjl = qjl;
  return TQ_OK;
}

}  // namespace

extern "C" {

int tq_polar_quantize(const float* x, const float* precondition, const float* codebooks,
                      const int* n_codebook, int64_t n_vectors, int dim, int block_size,
                      uint8_t* idx_l1, uint8_t* idx_l2, uint8_t* idx_l3, uint8_t* idx_l4,
                      uint16_t* radii, void* stream) {
  return encode16_common(x, precondition, codebooks, n_codebook, n_vectors, dim, block_size, false,
                         idx_l1, idx_l2, idx_l3, idx_l4, nullptr, nullptr, nullptr, nullptr, radii,
                         stream, "tq_polar_quantize");
}

int tq_polar_quantize_packed(const float* x, const float* precondition, const float* codebooks,
                             const int* n_codebook, int64_t n_vectors, int dim, int block_size,
                             uint32_t* packed_l1, uint8_t* packed_l2, uint8_t* packed_l3,
                             uint8_t* packed_l4, uint16_t* radii, void* stream) {
  return encode16_common(x, precondition, codebooks, n_codebook, n_vectors, dim, block_size, true,
                         nullptr, nullptr, nullptr, nullptr, packed_l1, packed_l2, packed_l3,
                         packed_l4, radii, stream, "tq_polar_quantize_packed");
}

int tq_polar_dequantize(const uint8_t* idx_l1, const uint8_t* idx_l2, const uint8_t* idx_l3,
                        const uint8_t* idx_l4, const uint16_t* radii, const float* precondition,
                        const float* codebooks, const int* n_codebook, int64_t n_vectors, int dim,
                        int block_size, float* out, void* stream) {
  Keys16 k{};
  k.i1 = idx_l1; k.i2 = idx_l2; k.i3 = idx_l3; k.i4 = idx_l4; k.radii = radii;
  TQ_CHECK_ARG(idx_l1 && idx_l2 && idx_l3 && idx_l4, "tq_polar_dequantize: null index array");
  return decode16_common(k, precondition, codebooks, nullptr, n_codebook, n_vectors, dim, block_size,
                         false, out, stream, "tq_polar_dequantize");
}

int tq_polar_dequantize_packed(const uint32_t* packed_l1, const uint8_t* packed_l2,
                               const uint8_t* packed_l3, const uint8_t* packed_l4,
                               const uint16_t* radii, const float* codebooks,
                               const float* cs_tables, const int* n_codebook, int64_t n_vectors,
                               int dim, int block_size, float* out, void* stream) {
  Keys16 k{};
  k.p1 = packed_l1; k.p2 = packed_l2; k.p3 = packed_l3; k.p4 = packed_l4; k.radii = radii;
  TQ_CHECK_ARG(packed_l1 && packed_l2 && packed_l3 && packed_l4,
               "tq_polar_dequantize_packed: null index array");
  return decode16_common(k, nullptr, codebooks, cs_tables, n_codebook, n_vectors, dim, block_size,
                         true, out, stream, "tq_polar_dequantize_packed");
}

int tq_compressed_score(const float* q, int num_heads, const uint8_t* idx_l1, const uint8_t* idx_l2,
                        const uint8_t* idx_l3, const uint8_t* idx_l4, const uint16_t* radii,
                        const float* codebooks, const int* n_codebook, int num_kv_heads,
                        int n_keys, int dim, int block_size, float scale, float* scores,
                        void* stream) {
  const char* fn = "tq_compressed_score";
  Attn16 a;
  int st = attn16_setup(a, q, idx_l1, idx_l2, idx_l3, idx_l4, nullptr, nullptr, nullptr, nullptr,
                        radii, codebooks, n_codebook, false, num_heads, num_kv_heads, n_keys, dim,
                        block_size, fn);
  if (st != TQ_OK) return st;
  return score16_common(a, num_heads, num_kv_heads, n_keys, scale, scores, false, stream, fn);
}

int tq_compressed_score_packed(const float* q, int num_heads, const uint32_t* packed_l1,
                               const uint8_t* packed_l2, const uint8_t* packed_l3,
                               const uint8_t* packed_l4, const uint16_t* radii,
                               const float* codebooks, const int* n_codebook, int num_kv_heads,
                               int n_keys, int dim, int block_size, float scale, float* scores,
                               void* stream) {
  const char* fn = "tq_compressed_score_packed";
  Attn16 a;
  int st = attn16_setup(a, q, nullptr, nullptr, nullptr, nullptr, packed_l1, packed_l2, packed_l3,
                        packed_l4, radii, codebooks, n_codebook, true, num_heads, num_kv_heads,
                        n_keys, dim, block_size, fn);
  if (st != TQ_OK) return st;
  return score16_common(a, num_heads, num_kv_heads, n_keys, scale, scores, true, stream, fn);
}

size_t tq_compressed_sdpa_workspace_size(int num_heads, int num_kv_heads, int dim, int max_n_keys) {
  if (num_kv_heads < 1 || num_heads < num_kv_heads || max_n_keys < 0 || dim < 1) return 0;
  return polar_ws_size(num_heads, num_kv_heads, dim, max_n_keys, 4);
}

int tq_compressed_sdpa(const float* q, int num_heads, const uint8_t* idx_l1, const uint8_t* idx_l2,
                       const uint8_t* idx_l3, const uint8_t* idx_l4, const uint16_t* radii,
                       const float* codebooks, const int* n_codebook, const float* values,
                       int num_kv_heads, int n_keys, int dim, int block_size, float scale,
                       float* out, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "tq_compressed_sdpa";
  Attn16 a;
  int st = attn16_setup(a, q, idx_l1, idx_l2, idx_l3, idx_l4, nullptr, nullptr, nullptr, nullptr,
                        radii, codebooks, n_codebook, false, num_heads, num_kv_heads, n_keys, dim,
                        block_size, fn);
  if (st != TQ_OK) return st;
  TQ_CHECK_ARG(values != nullptr, "%s: values is NULL", fn);
  SdpaParams p;
  dim3 grid;
  int G = 1;
  st = polar_sdpa_params(p, num_heads, num_kv_heads, dim, n_keys, std::max(n_keys, 1), scale, 0,
                         1e-8f, 4, out, workspace, workspace_bytes, grid, G, fn);
  if (st != TQ_OK) return st;
  a.values = values;
  a.qscale = scale * kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dim) {
    case 64: return dispatch_sdpa16_g<64, false>(G, p, a, grid, s);
    case 128: return dispatch_sdpa16_g<128, false>(G, p, a, grid, s);
    default: return dispatch_sdpa16_g<256, false>(G, p, a, grid, s);
  }
}

int tq_polar_rotate(const float* x, const float* precondition, int64_t rows, int dim, float* y,
                    void* stream) {
  TQ_CHECK_ARG(x && precondition && y, "tq_polar_rotate: null pointer");
  if (dim != 128) {
    set_error("tq_polar_rotate: dim must be 128 (got %d)", dim);
    return TQ_ERR_UNSUPPORTED;
  }
  TQ_CHECK_ARG(rows >= 0 && rows <= 0x7FFFFFFF, "tq_polar_rotate: bad rows");
  if (rows == 0) return TQ_OK;
  rotate128_kernel<<<static_cast<unsigned>(rows), 128, 0, static_cast<hipStream_t>(stream)>>>(
      x, precondition, y, static_cast<int>(rows));
  TQ_CHECK_LAUNCH("rotate128_kernel");
  return TQ_OK;
}

int tq_qjl_query(const float* q_rot, const float* sketch, int num_heads, float* q_sketch,
                 void* stream) {
  // S q' per head: the same product as the rotation with S in place of P
  TQ_CHECK_ARG(q_rot && sketch && q_sketch && num_heads >= 0, "tq_qjl_query: bad argument");
  if (num_heads == 0) return TQ_OK;
  rotate128_kernel<<<num_heads, 128, 0, static_cast<hipStream_t>(stream)>>>(q_rot, sketch, q_sketch,
                                                                             num_heads);
  TQ_CHECK_LAUNCH("rotate128_kernel");
  return TQ_OK;
}

int tq_polar7_encode(const float* x, const float* precondition, const float* sketch,
                     const float* codebooks, const float* cs_tables, int64_t n_vectors,
                     uint32_t* angles, uint32_t* norms, uint32_t* qjl, void* stream) {
  const char* fn = "tq_polar7_encode";
  TQ_CHECK_ARG(x && sketch && codebooks && cs_tables && angles && norms && qjl, "%s: null pointer", fn);
  TQ_CHECK_ARG(n_vectors >= 0, "%s: n_vectors must be >= 0", fn);
  if (n_vectors == 0) return TQ_OK;
  P7EncParams p{};
  p.x = x; p.P = precondition; p.S = sketch; p.cb = codebooks; p.cs = cs_tables;
  p.n = n_vectors;
  p.angles = angles; p.norms = norms; p.qjl = qjl;
  const int64_t grid = std::min<int64_t>((n_vectors + 3) / 4, 8192);
  polar7_encode_kernel<<<static_cast<unsigned>(grid), 256, 0, static_cast<hipStream_t>(stream)>>>(p);
  TQ_CHECK_LAUNCH("polar7_encode_kernel");
  return TQ_OK;
}

int tq_polar7_kv_append(const float* k_new, const float* precondition, const float* sketch,
                        const float* codebooks, const float* cs_tables, uint32_t* angles,
                        uint32_t* norms, uint32_t* qjl, int batch, int num_kv_heads,
                        int kv_capacity, const int32_t* positions, int n_new, void* stream) {
  const char* fn = "tq_polar7_kv_append";
  TQ_CHECK_ARG(k_new && sketch && codebooks && cs_tables && angles && norms && qjl && positions,
               "%s: null pointer", fn);
  TQ_CHECK_ARG(batch >= 1 && num_kv_heads >= 1 && kv_capacity >= 1 && n_new >= 0,
               "%s: bad shape", fn);
  if (n_new == 0) return TQ_OK;
  P7EncParams p{};
  p.x = k_new; p.P = precondition; p.S = sketch; p.cb = codebooks; p.cs = cs_tables;
  p.n = static_cast<int64_t>(batch) * num_kv_heads * n_new;
  p.positions = positions; p.n_new = n_new; p.cap = kv_capacity; p.Hkv = num_kv_heads;
  p.angles = angles; p.norms = norms; p.qjl = qjl;
  const int64_t grid = std::min<int64_t>((p.n + 3) / 4, 8192);
  polar7_encode_kernel<<<static_cast<unsigned>(grid), 256, 0, static_cast<hipStream_t>(stream)>>>(p);
  TQ_CHECK_LAUNCH("polar7_encode_kernel");
  return TQ_OK;
}

int tq_polar7_prepare_query(const float* q, const float* precondition, const float* sketch,
                            const float* cs_tables, int num_heads, float* q_tables, float* q_rot,
                            float* q_sketch, void* stream) {
  const char* fn = "tq_polar7_prepare_query";
  TQ_CHECK_ARG(q && sketch && cs_tables && q_tables, "%s: null pointer", fn);
  TQ_CHECK_ARG(num_heads >= 0 && num_heads <= 65535, "%s: bad num_heads", fn);
  TQ_CHECK_ARG(reinterpret_cast<uintptr_t>(q_tables) % 16 == 0, "%s: q_tables must be 16-byte aligned", fn);
  if (num_heads == 0) return TQ_OK;
  polar7_prepare_kernel<<<dim3(num_heads, kP7PrepParts), 256, 0, static_cast<hipStream_t>(stream)>>>(
      q, precondition, sketch, cs_tables, q_tables, q_rot, q_sketch);
  TQ_CHECK_LAUNCH("polar7_prepare_kernel");
  return TQ_OK;
}

int tq_polar7_sketch_precondition(const float* precondition, const float* sketch,
                                  float* sketch_precondition, void* stream) {
  const char* fn = "tq_polar7_sketch_precondition";
  TQ_CHECK_ARG(sketch && sketch_precondition, "%s: null pointer", fn);
  polar7_sp_kernel<<<128, 128, 0, static_cast<hipStream_t>(stream)>>>(precondition, sketch,
                                                                      sketch_precondition);
  TQ_CHECK_LAUNCH("polar7_sp_kernel");
  return TQ_OK;
}

int tq_polar7_prepare_query_sp(const float* q, const float* precondition,
                               const float* sketch_precondition, const float* cs_tables,
                               int num_heads, float* q_tables, float* q_rot, float* q_sketch,
                               void* stream) {
  const char* fn = "tq_polar7_prepare_query_sp";
  TQ_CHECK_ARG(q && sketch_precondition && cs_tables && q_tables, "%s: null pointer", fn);
  TQ_CHECK_ARG(num_heads >= 0 && num_heads <= 65535, "%s: bad num_heads", fn);
  TQ_CHECK_ARG(reinterpret_cast<uintptr_t>(q_tables) % 16 == 0, "%s: q_tables must be 16-byte aligned", fn);
  if (num_heads == 0) return TQ_OK;
  polar7_prepare_sp_kernel<<<dim3(num_heads, kP7PrepParts), 256, 0, static_cast<hipStream_t>(stream)>>>(
      q, precondition, sketch_precondition, cs_tables, q_tables, q_rot, q_sketch);
  TQ_CHECK_LAUNCH("polar7_prepare_sp_kernel");
  return TQ_OK;
}

int tq_polar7_score(const float* q_tables, const uint32_t* angles, const uint32_t* norms,
                    const uint32_t* qjl, const float* cs_tables, int num_heads, int num_kv_heads,
                    int kv_len, int kv_capacity, float scale, float* scores, void* stream) {
  const char* fn = "tq_polar7_score";
  P7Keys k;
  int st = p7_keys_setup(k, q_tables, angles, norms, qjl, cs_tables, num_heads, num_kv_heads, fn);
  if (st != TQ_OK) return st;
  TQ_CHECK_ARG(kv_len >= 0 && kv_capacity >= 1 && kv_len <= kv_capacity, "%s: bad kv_len", fn);
  TQ_CHECK_ARG(std::isfinite(scale), "%s: scale must be finite", fn);
  if (kv_len == 0) return TQ_OK;  // nothing to write (scores may be NULL)
  TQ_CHECK_ARG(scores != nullptr, "%s: scores is NULL", fn);
  k.scores = scores;
  const int gqa = num_heads / num_kv_heads, G = polar_subgroup(gqa, kP7MaxG), n_sub = gqa / G;
  TQ_CHECK_ARG(num_kv_heads * n_sub <= 65535, "%s: too many heads", fn);
  // 1024 threads (four waves per SIMD) in 8 passes, 2048 keys per workgroup:
  // the staged query tables are paid once per 2048 keys
  constexpr int NT = 1024, NP = 8, KPW = NP * NT / 4;
  dim3 grid((kv_len + KPW - 1) / KPW, num_kv_heads * n_sub);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (G == 1) polar7_score_kernel<1, NT, NP><<<grid, NT, 0, s>>>(k, kv_len, kv_capacity, gqa, n_sub, scale);
  else polar7_score_kernel<2, NT, NP><<<grid, NT, 0, s>>>(k, kv_len, kv_capacity, gqa, n_sub, scale);
  TQ_CHECK_LAUNCH("polar7_score_kernel");
  return TQ_OK;
}

int tq_polar7_score_q(const float* q, const float* precondition, const float* sketch_precondition,
                      const float* cs_tables, const uint32_t* angles, const uint32_t* norms,
                      const uint32_t* qjl, int num_heads, int num_kv_heads, int kv_len,
                      int kv_capacity, float scale, float* scores, void* stream) {
  const char* fn = "tq_polar7_score_q";
  TQ_CHECK_ARG(q && sketch_precondition && cs_tables && angles && norms && qjl, "%s: null pointer", fn);
  TQ_CHECK_ARG(num_kv_heads >= 1 && num_heads >= num_kv_heads && num_heads % num_kv_heads == 0,
               "%s: num_heads must be a multiple of num_kv_heads", fn);
  TQ_CHECK_ARG(reinterpret_cast<uintptr_t>(angles) % 16 == 0 && reinterpret_cast<uintptr_t>(qjl) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(sketch_precondition) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(precondition) % 16 == 0,
               "%s: angles / qjl / precondition / sketch_precondition must be 16-byte aligned", fn);
  TQ_CHECK_ARG(kv_len >= 0 && kv_capacity >= 1 && kv_len <= kv_capacity, "%s: bad kv_len", fn);
  TQ_CHECK_ARG(std::isfinite(scale), "%s: scale must be finite", fn);
  if (kv_len == 0) return TQ_OK;  // nothing to write (scores may be NULL)
  TQ_CHECK_ARG(scores != nullptr, "%s: scores is NULL", fn);
  P7Keys k{};
  k.cs = cs_tables;
  k.angles = angles; k.norms = norms; k.qjl = qjl;
  k.q = q; k.P = precondition; k.SP = sketch_precondition;
  k.scores = scores;
  const int gqa = num_heads / num_kv_heads, G = polar_subgroup(gqa, kP7MaxG), n_sub = gqa / G;
  TQ_CHECK_ARG(num_kv_heads * n_sub <= 65535, "%s: too many heads", fn);
  constexpr int NT = 1024, NP = 8, KPW = NP * NT / 4;
  dim3 grid((kv_len + KPW - 1) / KPW, num_kv_heads * n_sub);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (G == 1) polar7_score_kernel<1, NT, NP, true><<<grid, NT, 0, s>>>(k, kv_len, kv_capacity, gqa, n_sub, scale);
  else polar7_score_kernel<2, NT, NP, true><<<grid, NT, 0, s>>>(k, kv_len, kv_capacity, gqa, n_sub, scale);
  TQ_CHECK_LAUNCH("polar7_score_kernel (fused query tables)");
  return TQ_OK;
}

size_t tq_polar7_sdpa_workspace_size(int num_heads, int num_kv_heads, int max_kv_len) {
  if (num_kv_heads < 1 || num_heads < num_kv_heads || max_kv_len < 0) return 0;
  return polar_ws_size(num_heads, num_kv_heads, 128, max_kv_len, kP7MaxG);
}

int tq_polar7_sdpa_int4v(const float* q_tables, const uint32_t* angles,
                         const uint32_t* norms, const uint32_t* qjl, const float* cs_tables,
                         const uint32_t* v_quant, const void* v_scales, const void* v_biases,
                         tq_dtype sb_dtype, float* out, int num_heads, int num_kv_heads,
                         int kv_len, int kv_capacity, float scale, int sliding_window,
                         void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "tq_polar7_sdpa_int4v";
  P7Keys k;
  int st = p7_keys_setup(k, q_tables, angles, norms, qjl, cs_tables, num_heads, num_kv_heads, fn);
  if (st != TQ_OK) return st;
  TQ_CHECK_ARG(v_quant && v_scales && v_biases, "%s: null V pointer", fn);
  TQ_CHECK_ARG(sb_dtype == TQ_F16 || sb_dtype == TQ_F32, "%s: sb_dtype must be f16 or f32", fn);
  SdpaParams p;
  dim3 grid;
  int G = 1;
  st = polar_sdpa_params(p, num_heads, num_kv_heads, 128, kv_len, kv_capacity, scale, sliding_window,
                         0.0f, kP7MaxG, out, workspace, workspace_bytes, grid, G, fn);
  if (st != TQ_OK) return st;
  p.vq = v_quant; p.vs = v_scales; p.vb = v_biases;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool f16 = sb_dtype == TQ_F16;
  constexpr int NW = kP7Waves, NT = kP7Waves * 64;
  if (f16) {
    if (G == 1) polar7_sdpa_kernel<1, __half, NW><<<grid, NT, 0, s>>>(p, k);
    else polar7_sdpa_kernel<2, __half, NW><<<grid, NT, 0, s>>>(p, k);
  } else {
    if (G == 1) polar7_sdpa_kernel<1, float, NW><<<grid, NT, 0, s>>>(p, k);
    else polar7_sdpa_kernel<2, float, NW><<<grid, NT, 0, s>>>(p, k);
  }
  TQ_CHECK_LAUNCH("polar7_sdpa_kernel");
  return TQ_OK;
}

int tq_polar7_sdpa_int4v_q(const float* q, const float* precondition,
                           const float* sketch_precondition, const float* cs_tables,
                           const uint32_t* angles, const uint32_t* norms, const uint32_t* qjl,
                           const uint32_t* v_quant, const void* v_scales, const void* v_biases,
                           tq_dtype sb_dtype, float* out, int num_heads, int num_kv_heads,
                           int kv_len, int kv_capacity, float scale, int sliding_window,
                           void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "tq_polar7_sdpa_int4v_q";
  TQ_CHECK_ARG(q && sketch_precondition && cs_tables && angles && norms && qjl, "%s: null pointer", fn);
  TQ_CHECK_ARG(num_kv_heads >= 1 && num_heads >= num_kv_heads && num_heads % num_kv_heads == 0,
               "%s: num_heads must be a multiple of num_kv_heads", fn);
  TQ_CHECK_ARG(reinterpret_cast<uintptr_t>(angles) % 16 == 0 && reinterpret_cast<uintptr_t>(qjl) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(sketch_precondition) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(precondition) % 16 == 0,
               "%s: angles / qjl / precondition / sketch_precondition must be 16-byte aligned", fn);
  TQ_CHECK_ARG(v_quant && v_scales && v_biases, "%s: null V pointer", fn);
  TQ_CHECK_ARG(sb_dtype == TQ_F16 || sb_dtype == TQ_F32, "%s: sb_dtype must be f16 or f32", fn);
  P7Keys k{};
  k.cs = cs_tables;
  k.angles = angles; k.norms = norms; k.qjl = qjl;
  k.q = q; k.P = precondition; k.SP = sketch_precondition;
  SdpaParams p;
  dim3 grid;
  int G = 1;
  int st = polar_sdpa_params(p, num_heads, num_kv_heads, 128, kv_len, kv_capacity, scale, sliding_window,
                             0.0f, kP7MaxG, out, workspace, workspace_bytes, grid, G, fn);
  if (st != TQ_OK) return st;
  p.vq = v_quant; p.vs = v_scales; p.vb = v_biases;
  hipStream_t s = static_cast<hipStream_t>(stream);
  constexpr int NW = kP7Waves, NT = kP7Waves * 64;
  if (sb_dtype == TQ_F16) {
    if (G == 1) polar7_sdpa_kernel<1, __half, NW, true><<<grid, NT, 0, s>>>(p, k);
    else polar7_sdpa_kernel<2, __half, NW, true><<<grid, NT, 0, s>>>(p, k);
  } else {
    if (G == 1) polar7_sdpa_kernel<1, float, NW, true><<<grid, NT, 0, s>>>(p, k);
    else polar7_sdpa_kernel<2, float, NW, true><<<grid, NT, 0, s>>>(p, k);
  }
  TQ_CHECK_LAUNCH("polar7_sdpa_kernel (fused query tables)");
  return TQ_OK;
}

}  // extern "C"
