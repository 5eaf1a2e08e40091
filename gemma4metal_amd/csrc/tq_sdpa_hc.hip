// Decode attention at head_dim 512 with eight query heads per kv head (Gemma
// global layers, GQA 8: engine/gemma4_multilayer.cpp:3,49-51), on the matrix
// cores with the query heads as MFMA columns.
//
// Same contract, split and finalisation as the kernels of tq_sdpa.hip and
// tq_sdpa_mfma.hip (replaces sdpa_int4_vector<512>, lib/turboquant.metal:
// 723-889, 898-903).  That kernel fills its 16 columns with (head, quant
// group) pairs, which at D = 512 leaves room for 2 heads, so a kv head needs
// 4 workgroups that each unpack the same K/V.  Here one workgroup takes all
// 8 heads of a kv head, so every K/V byte is unpacked once:
//
// K . q  -- per pair of quant groups (2P, 2P + 1): v_mfma_i32_16x16x64_i8
//   with A = 16 keys x (32 nibbles of group 2P | 32 of group 2P + 1) and a
//   block-diagonal B: columns 0-7 the q of the 8 heads over group 2P's dims,
//   columns 8-15 over group 2P + 1's, zero elsewhere; two such products
//   (dims 0-31, 32-63 of each group) accumulate into one C.  q is three
//   signed base-256 digits of round(q * 2^F), so C[key][column] is the exact
//   integer dot of one group.  A lane adds s_g * dot_g + b_g * sum(q * 2^F
//   over g) for its column's group; one cross-lane add (column n and n ^ 8)
//   and one multiply by 2^-F then give the score of head n % 8 in both
//   columns.
// P . V  -- v_mfma_f32_16x16x32_bf16 per block of 16 V words (2 quant
//   groups): A = (128 + nibble) as bf16 of 16 words x 32 keys (v_perm_b32 +
//   and-or), B = the bf16 hi / lo split of p * s_v in columns (head, group of
//   the block), column head + 8 g' taking the block's second group.  bf16
//   keeps fp32's exponent range, so no V scale overflows the weights.  The
//   128 offset (128 * sum of the weights) and the bias term sum(p * b_v) are
//   kept per (column, block) and removed at the end.
//
// Lane roles (l = lane, m = l % 16, c = l / 16):
//   K A-operand of product h of pair P: key 16 tile + m, words
//   8 (2P + c / 2) + 4 (c % 2) + 2h and + 1 (one 16-byte load per pair);
//   scores: C rows 4c .. 4c+3 of column m, i.e. keys 16 tile + 4c + i of
//   head m % 8;  V slot j of lane group c: key 16 (j / 4) + 4c + j % 4 (the
//   key whose weight this lane computed as C[4c + j % 4] of tile j / 4);
//   V A-operand row m of block blk: word 16 blk + m.
// Four waves, one per SIMD (the P.V accumulators of 8 heads x 512 dims take
// 128 registers); loads double-buffered one 32-key iteration ahead.
#include "tq_sdpa_common.h"

namespace tq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

constexpr int kHcWaves = 4;
constexpr int kHcD = 512;
constexpr int kHcG = 8;    // query heads per workgroup
constexpr int kHcNG = 8;   // quant groups per row
constexpr int kHcRB = 256; // bytes per packed row

struct HcBuf {
  uint32_t kw[2][16];  // [tile][4 P + 2 h + e]: word 8 (2P + c/2) + 4 (c%2) + 2h + e of key 16 tile + m
  uint32_t vw[8][4];   // [slot][blk]: word 16 blk + m of the slot's key
  u32x4 sc[2][1];      // scales of array c for keys 2m, 2m+1 (8 fp16 each)
};

// Loads of the 32 keys at t0 (rows clamped to `last`, the uniform limit
// `lim` = last - t0 >= 0), non-temporal, uniform base + 32-bit lane offset:
// K words, the scale arrays and the V words, as separate parts.
// K words: one 16-byte load per (tile, pair P): lane group c takes words
// 16 P + 4c .. + 3 of its key (group 2P + c / 2, half c % 2 of it), so the 4
// lane groups of a row read its 64 bytes of the pair contiguously.
__device__ __forceinline__ void hc_load_kw_pair(uint32_t (&kw)[2][16], const char* kq, int t0, int lim, int m,
                                                int c, int P) {
  const char* kb = kq + static_cast<int64_t>(t0) * kHcRB;
#pragma unroll
  for (int tile = 0; tile < 2; ++tile) {
    const uint32_t off = static_cast<uint32_t>(min(16 * tile + m, lim)) * kHcRB + 16 * c;
    const u32x4 u = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kb + off + 64 * P));
    kw[tile][4 * P] = u.x;
    kw[tile][4 * P + 1] = u.y;
    kw[tile][4 * P + 2] = u.z;
    kw[tile][4 * P + 3] = u.w;
  }
}

__device__ __forceinline__ void hc_load_kw(uint32_t (&kw)[2][16], const char* kq, int t0, int lim, int m, int c) {
#pragma unroll
  for (int P = 0; P < 4; ++P) hc_load_kw_pair(kw, kq, t0, lim, m, c, P);
}

// Scale array of lane group c (k scale, k bias, v scale, v bias) for keys
// 2m, 2m + 1: 8 groups per key, fp16 (4 words per key) or fp32 (8 words).
template <bool F32>
__device__ __forceinline__ void hc_load_sc(u32x4 (&scw)[2][F32 ? 2 : 1], const char* sc, int t0, int lim,
                                           int m) {
  constexpr int RB = F32 ? 32 : 16;  // scale bytes per key
  const char* sb = sc + static_cast<int64_t>(t0) * RB;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint32_t off = static_cast<uint32_t>(min(2 * m + e, lim)) * RB;
#pragma unroll
    for (int h = 0; h < RB / 16; ++h)
      scw[e][h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(sb + off + 16 * h));
  }
}

__device__ __forceinline__ void hc_load_k(uint32_t (&kw)[2][16], u32x4 (&scw)[2][1], const char* kq,
                                          const char* sc, int t0, int lim, int m, int c) {
  hc_load_kw(kw, kq, t0, lim, m, c);
  hc_load_sc<false>(scw, sc, t0, lim, m);
}

__device__ __forceinline__ void hc_load_v(uint32_t (&vw)[8][4], const char* vq, int t0, int lim, int m,
                                          int c) {
  const char* vb = vq + static_cast<int64_t>(t0) * kHcRB;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t off = static_cast<uint32_t>(min(16 * (j >> 2) + 4 * c + (j & 3), lim)) * kHcRB + m * 4;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
      vw[j][blk] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(vb + off + 64 * blk));
  }
}

// V words for the wave-specialised kernel: one 16-byte load per (tile T,
// block blk): lane (m = 4 qd + i, c) loads words 16 blk + 4 qd .. + 3 of key
// 16 T + 4c + i, so a quad of lanes reads 4 keys x 16 contiguous bytes.
// hc_quad_transpose then gives lane i of the quad word 16 blk + 4 qd + i of
// keys 16 T + 4c + 0 .. 3: the slots 4T .. 4T + 3 of hc_load_v's layout.
__device__ __forceinline__ void hc_load_v4_blk(u32x4 (&vr)[2][4], const char* vq, int t0, int lim, int m, int c,
                                               int blk) {
  const char* vb = vq + static_cast<int64_t>(t0) * kHcRB;
#pragma unroll
  for (int T = 0; T < 2; ++T) {
    const uint32_t off = static_cast<uint32_t>(min(16 * T + 4 * c + (m & 3), lim)) * kHcRB + 16 * (m >> 2);
    vr[T][blk] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vb + off + 64 * blk));
  }
}

__device__ __forceinline__ void hc_load_v4(u32x4 (&vr)[2][4], const char* vq, int t0, int lim, int m, int c) {
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) hc_load_v4_blk(vr, vq, t0, lim, m, c, blk);
}

// 4 x 4 transpose of dwords inside each quad of lanes: lane i of the quad
// returns R[i] of lanes 0 .. 3.  Two butterfly stages on DPP quad_perm
// (lane ^ 2, then lane ^ 1), each exchanging one bit of the register index
// with the same bit of the lane index.
__device__ __forceinline__ u32x4 hc_quad_transpose(u32x4 R, int lane) {
  const bool i1 = (lane & 2) != 0, i0 = (lane & 1) != 0;
  uint32_t U[4], W[4];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const uint32_t X = i1 ? R[x] : R[2 + x];
    const uint32_t Y = static_cast<uint32_t>(
        __builtin_amdgcn_mov_dpp(static_cast<int>(X), 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    U[x] = i1 ? Y : R[x];
    U[2 + x] = i1 ? R[2 + x] : Y;
  }
#pragma unroll
  for (int y = 0; y < 4; y += 2) {
    const uint32_t X = i0 ? U[y] : U[y + 1];
    const uint32_t Y = static_cast<uint32_t>(
        __builtin_amdgcn_mov_dpp(static_cast<int>(X), 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    W[y] = i0 ? Y : U[y];
    W[y + 1] = i0 ? U[y + 1] : Y;
  }
  return u32x4{W[0], W[1], W[2], W[3]};
}

__device__ __forceinline__ void hc_load(HcBuf& B, const char* kq, const char* vq, const char* sc,
                                        int t0, int lim, int m, int c) {
  hc_load_k(B.kw, B.sc, kq, sc, t0, lim, m, c);
  hc_load_v(B.vw, vq, t0, lim, m, c);
}

__device__ __forceinline__ float hc_half(uint32_t w, int hi) {
  return __half2float(__ushort_as_half(static_cast<uint16_t>(hi ? (w >> 16) : (w & 0xFFFFu))));
}

// Prologue of both kernels: the workgroup's q (8 heads x 512, one contiguous
// block) as 21-bit fixed point per head, scattered into the block-diagonal B
// images of the K.q products (bq_lds, whose off-diagonal blocks are zeroed
// here), with the per-(head, group) sums of the fixed-point q (sh_qhat) and
// the per-head exponent F (sh_F).  Thread t takes the 8-element chunks
// t + kNT i: a wave's 64 chunks are the 512 dims of one head, so the head's
// maximum is a wave reduction, and a chunk is one word (8 dims) of one quant
// group, whose three base-256 digits fill two whole dwords of one lane's B
// operand each.
template <int kNT>
struct HcQ {
  static constexpr int NCH = kHcG * kHcD / 8 / kNT;  // chunks per thread
  u32x4 raw[NCH][2];                                 // 8 elements (fp32: both vectors)
};

template <int kNT>
__device__ __forceinline__ void hc_q_load(HcQ<kNT>& Q, const SdpaParams& p, int64_t qbase) {
  const int qsz = p.q_dtype == TQ_F32 ? 4 : 2;
  const char* qb = static_cast<const char*>(p.q) + qbase * qsz;
  const bool al16 = (reinterpret_cast<uintptr_t>(qb) & 15) == 0;  // uniform
#pragma unroll
  for (int i = 0; i < HcQ<kNT>::NCH; ++i) {
    const char* src = qb + static_cast<int64_t>(threadIdx.x + kNT * i) * 8 * qsz;
    if (al16) {
      Q.raw[i][0] = *reinterpret_cast<const u32x4*>(src);
      Q.raw[i][1] = qsz == 4 ? *reinterpret_cast<const u32x4*>(src + 16) : Q.raw[i][0];
    } else if (qsz == 4) {
      const uint32_t* s32 = reinterpret_cast<const uint32_t*>(src);
      Q.raw[i][0] = u32x4{s32[0], s32[1], s32[2], s32[3]};
      Q.raw[i][1] = u32x4{s32[4], s32[5], s32[6], s32[7]};
    } else {
      const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src);
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = static_cast<uint32_t>(s16[2 * j]) | (static_cast<uint32_t>(s16[2 * j + 1]) << 16);
      Q.raw[i][0] = u32x4{w[0], w[1], w[2], w[3]};
      Q.raw[i][1] = Q.raw[i][0];
    }
  }
}

// Exact int32 sum over aligned groups of 8 lanes (DPP butterfly in the row).
__device__ __forceinline__ int group8_sum_i(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // lane ^ 1
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // lane ^ 2
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // half-row mirror
  return v;
}

// Ends with a barrier.
template <int kNT>
__device__ __forceinline__ void hc_q_build(const HcQ<kNT>& Q, const SdpaParams& p, uint4 (&bq_lds)[3][kHcNG][64],
                                           float (&sh_qhat)[kHcG][kHcNG], int (&sh_F)[kHcG], int lane) {
  constexpr int NG = kHcNG;
  {
    // the off-diagonal blocks of the B images stay zero: lane 16c + n of an
    // image is nonzero only where column n takes the group of lane group c
    // ((n >= 8) == (c >= 2)); the two sets are disjoint, so no barrier
    // separates these stores from the digit stores below
    uint4* z = &bq_lds[0][0][0];
    for (int i = threadIdx.x; i < 3 * NG * 32; i += kNT) {
      const int cz = (i >> 3) & 3, nz = (i & 7) + ((cz >> 1) ? 0 : 8);
      z[(i >> 5) * 64 + 16 * cz + nz] = uint4{0u, 0u, 0u, 0u};
    }
  }
  uint8_t* bq_bytes = reinterpret_cast<uint8_t*>(&bq_lds[0][0][0]);
  // this lane's chunk: word w of quant group g; in the products of pair
  // g / 2 it is loaded by lane group cc = w / 4 + 2 (g % 2) as product
  // hf = (w / 2) % 2, vector elements 2 (w % 2) (even dims) and + 1 (odd
  // dims), byte (d % 8) / 2 -- the order in which the unpack spreads a
  // word's nibbles
  const int g = lane >> 3, w = lane & 7;
  const int cc = (w >> 2) + 2 * (g & 1), hf = (w >> 1) & 1, e = w & 1;
#pragma unroll
  for (int i = 0; i < HcQ<kNT>::NCH; ++i) {
    const int head = static_cast<int>((threadIdx.x + kNT * i) >> 6);
    float qv[8];
    float mx = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      float f;
      if (p.q_dtype == TQ_F32) {
        f = __uint_as_float(Q.raw[i][t >> 2][t & 3]);
      } else {
        const uint32_t wd = Q.raw[i][0][t >> 1];
        const uint32_t h16 = (t & 1) ? (wd >> 16) : (wd & 0xFFFFu);
        f = p.q_dtype == TQ_F16 ? __half2float(__ushort_as_half(static_cast<uint16_t>(h16)))
                                : __uint_as_float(h16 << 16);
      }
      qv[t] = f * p.scale_log2;
      mx = fmaxf(mx, fabsf(qv[t]));
    }
    mx = wave_max_dpp(mx);
    int ex = 0;
    if (mx > 0.0f) frexpf(mx, &ex);  // mx < 2^ex
    // |round(q * 2^F)| <= 2^21: the top base-256 digit is then within
    // [-32, 32], and a group's dot sum_d nibble_d * X_d (|.| <= 64 * 15 *
    // 2^21 < 2^31) is exact in int32
    const int F = 21 - ex;
    const float up = ldexpf(1.0f, F);
    uint32_t ev[3] = {0u, 0u, 0u}, od[3] = {0u, 0u, 0u};
    int xs = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int X = static_cast<int>(__builtin_rintf(qv[t] * up));
      xs += X;
      const int d0 = static_cast<int8_t>(X & 0xFF);
      const int X1 = (X - d0) >> 8;
      const int d1 = static_cast<int8_t>(X1 & 0xFF);
      const int d2 = (X1 - d1) >> 8;
      const int sh = 8 * (t >> 1);
      uint32_t* dst = (t & 1) ? od : ev;
      dst[0] |= static_cast<uint32_t>(d0 & 0xFF) << sh;
      dst[1] |= static_cast<uint32_t>(d1 & 0xFF) << sh;
      dst[2] |= static_cast<uint32_t>(d2 & 0xFF) << sh;
    }
    const int ln = 16 * cc + head + 8 * (g & 1);
    const int o = (((g >> 1) * 2 + hf) * 64 + ln) * 16 + 8 * e;
#pragma unroll
    for (int dg = 0; dg < 3; ++dg)
      *reinterpret_cast<u32x2*>(bq_bytes + o + dg * NG * 64 * 16) = u32x2{ev[dg], od[dg]};
    // per (head, quant group) sum of the fixed-point q over the group's 8
    // lanes, exact: 64 * 2^21 < 2^31
    xs = group8_sum_i(xs);
    if (w == 0) sh_qhat[head][g] = static_cast<float>(xs) * ldexpf(1.0f, -F);
    if (lane == 0) sh_F[head] = F;
  }
  __syncthreads();
}

__global__ __launch_bounds__(kHcWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void sdpa_int4_hc_kernel(SdpaParams p) {
  pin_args(p);
  constexpr int NW = kHcWaves, D = kHcD, G = kHcG, NG = kHcNG;
  constexpr int kNT = NW * 64;
  constexpr int kIter = 32 * NW;          // keys per workgroup iteration

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = lane & 15, c = lane >> 4;
  const int hh = m & 7;                   // this lane's head (column m)
  const int b = blockIdx.z, hy = blockIdx.y, split = blockIdx.x;
  const int kvh = hy / p.n_sub, sub = hy - kvh * p.n_sub;
  const int h0 = kvh * p.gqa + sub * G;

  const SplitRange rg = split_range(p, b, split);
  if (split >= rg.S) return;
  const int t_end = rg.t_end;

  using Fin = Finalize<G, D, NW>;
  __shared__ __attribute__((aligned(16))) float arena[Fin::kArena];
  __shared__ uint4 bq_lds[3][NG][64];           // K MFMA B operands [digit][2 pair + half][lane]
  __shared__ uint32_t sc_lds[NW][4][NG][16];    // [wave][array][group][key pair] fp16 x 2
  __shared__ float sh_qhat[G][NG];
  __shared__ int sh_F[G];

  const int64_t row0 = (static_cast<int64_t>(cache_batch(p, b)) * p.Hkv + kvh) * p.cap;
  const char* kq_rows = reinterpret_cast<const char*>(p.kq + row0 * (D / 8));
  const char* vq_rows = reinterpret_cast<const char*>(p.vq + row0 * (D / 8));
  // lane group c loads scale array c: k scale, k bias, v scale, v bias
  const void* sc_base = c == 0 ? p.ks : (c == 1 ? p.kb : (c == 2 ? p.vs : p.vb));
  const char* sc_rows = static_cast<const char*>(sc_base) + row0 * 16;

  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int base0 = rg.t_begin + wv * 32;
  const int nit = base0 < t_end ? (t_end - base0 + kIter - 1) / kIter : 0;
  const int last = t_end - 1;
  const int safe_last = max(last, 0);

  // q first, then the first iteration's K/V, which stay in flight through
  // the prologue
  HcQ<kNT> Q;
  hc_q_load<kNT>(Q, p, (static_cast<int64_t>(b) * p.Hq + h0) * D);
  __builtin_amdgcn_sched_barrier(0);
  HcBuf bufA, bufB;
  {
    const int t0 = min(base0, safe_last);
    hc_load(bufA, kq_rows, vq_rows, sc_rows, t0, safe_last - t0, m, c);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- prologue: q of the 8 heads as 21-bit fixed point, B images in LDS --
  hc_q_build<kNT>(Q, p, bq_lds, sh_qhat, sh_F, lane);
  const float sf = ldexpf(1.0f, -sh_F[hh]);
  // q sums of this lane's column: head hh, group 2P + m / 8 of pair P
  float qh[NG / 2];
#pragma unroll
  for (int P = 0; P < NG / 2; ++P) qh[P] = sh_qhat[hh][2 * P + (m >> 3)] * ldexpf(1.0f, sh_F[hh]);

  // ---- main loop ----------------------------------------------------------
  float m_run = -INFINITY, l_run = 0.0f;
  float wsum[4], bacc[4];  // per V block: sum of the weights, sum of p * b_v
  v4f cv[4][8];            // [blk][2 byte + nibble half]
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    wsum[blk] = 0.0f;
    bacc[blk] = 0.0f;
#pragma unroll
    for (int f = 0; f < 8; ++f) cv[blk][f] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  }
  uint32_t magic = 0x43004300u;  // bf16 of (128 + nibble)
  asm volatile("" : "+v"(magic));
  const v4i zero4 = v4i{0, 0, 0, 0};

  auto process = [&](const HcBuf& B, int t0) {
    // scales -> LDS [array][group][key pair]
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const uint32_t a0 = B.sc[0][0][g >> 1], a1 = B.sc[1][0][g >> 1];
      sc_lds[wv][c][g][m] = (g & 1) ? ((a0 >> 16) | (a1 & 0xFFFF0000u)) : ((a0 & 0xFFFFu) | (a1 << 16));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // K . q per pair of quant groups, both 16-key tiles: this lane sums its
    // column's groups (2P + m / 8)
    float sc[2][4];
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[tile][i] = 0.0f;
    auto bop = [&](int dg, int j) {
      const uint4 u = bq_lds[dg][j][lane];
      return v4i{static_cast<int>(u.x), static_cast<int>(u.y), static_cast<int>(u.z), static_cast<int>(u.w)};
    };
    auto aop = [&](uint32_t w0, uint32_t w1) {
      return v4i{static_cast<int>(w0 & 0x0F0F0F0Fu), static_cast<int>((w0 >> 4) & 0x0F0F0F0Fu),
                 static_cast<int>(w1 & 0x0F0F0F0Fu), static_cast<int>((w1 >> 4) & 0x0F0F0F0Fu)};
    };
#pragma unroll
    for (int P = 0; P < NG / 2; ++P) {
      const v4i b00 = bop(0, 2 * P), b01 = bop(0, 2 * P + 1);
      const v4i b10 = bop(1, 2 * P), b11 = bop(1, 2 * P + 1);
      const v4i b20 = bop(2, 2 * P), b21 = bop(2, 2 * P + 1);
      const int gl = 2 * P + (m >> 3);
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        const v4i a0 = aop(B.kw[tile][4 * P], B.kw[tile][4 * P + 1]);
        const v4i a1 = aop(B.kw[tile][4 * P + 2], B.kw[tile][4 * P + 3]);
        v4i acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b00, zero4, 0, 0, 0);
        v4i acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b10, zero4, 0, 0, 0);
        v4i acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b20, zero4, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b01, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b11, acc1, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b21, acc2, 0, 0, 0);
        const uint2 ks = *reinterpret_cast<const uint2*>(&sc_lds[wv][0][gl][8 * tile + 2 * c]);
        const uint2 kb = *reinterpret_cast<const uint2*>(&sc_lds[wv][1][gl][8 * tile + 2 * c]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // the three digits' products, exact in int32 (two shift-adds)
          const float dot = static_cast<float>((acc2[i] << 16) + ((acc1[i] << 8) + acc0[i]));
          const uint32_t ksw = (i >> 1) ? ks.y : ks.x, kbw = (i >> 1) ? kb.y : kb.x;
          sc[tile][i] = fmaf(dot, hc_half(ksw, i & 1), fmaf(hc_half(kbw, i & 1), qh[P], sc[tile][i]));
        }
      }
    }
    // column n holds the even groups of head n % 8 for n < 8, the odd ones
    // for n >= 8: add lane m ^ 8 of the same 16-lane row (DPP row rotate 8)
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sc[tile][i] = sf * (sc[tile][i] + __int_as_float(__builtin_amdgcn_mov_dpp(
                                               __float_as_int(sc[tile][i]), 0x128, 0xF, 0xF, false)));
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (t0 + 16 * tile + 4 * c + i >= t_end) sc[tile][i] = -INFINITY;

    // online softmax over the 32 keys, per head (column)
    float mt = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                     fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
    mt = xor16_max(mt);
    mt = xor32_max(mt);
    const float m_new = fmaxf(m_run, mt);
    if (t0 == base0) {
      m_run = m_new;  // first batch: nothing accumulated yet
    } else if (__any(m_new > m_run + kLazyMax)) {
      const float f = (m_new == m_run) ? 1.0f : merge_factor(m_run, m_new);
      l_run *= f;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        wsum[blk] *= f;
        bacc[blk] *= f;
#pragma unroll
        for (int ff = 0; ff < 8; ++ff) cv[blk][ff] *= f;
      }
      m_run = m_new;
    }
    float pw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float sj = sc[j >> 2][j & 3];
      pw[j] = sj == -INFINITY ? 0.0f : fast_exp2(sj - m_run);
      l_run += pw[j];
    }

    // P . V per block of 16 V words (quant groups 2 blk, 2 blk + 1)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int gv = 2 * blk + (m >> 3);
      const uint2 vs0 = *reinterpret_cast<const uint2*>(&sc_lds[wv][2][gv][2 * c]);
      const uint2 vs1 = *reinterpret_cast<const uint2*>(&sc_lds[wv][2][gv][8 + 2 * c]);
      const uint2 vb0 = *reinterpret_cast<const uint2*>(&sc_lds[wv][3][gv][2 * c]);
      const uint2 vb1 = *reinterpret_cast<const uint2*>(&sc_lds[wv][3][gv][8 + 2 * c]);
      const uint32_t vsw[4] = {vs0.x, vs0.y, vs1.x, vs1.y};
      const uint32_t vbw[4] = {vb0.x, vb0.y, vb1.x, vb1.y};
      __bf16 hi[8], lo[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float w = pw[j] * hc_half(vsw[j >> 1], j & 1);
        hi[j] = static_cast<__bf16>(w);
        const float hf = static_cast<float>(hi[j]);
        lo[j] = static_cast<__bf16>(w - hf);
        wsum[blk] += hf + static_cast<float>(lo[j]);
        bacc[blk] = fmaf(pw[j], hc_half(vbw[j >> 1], j & 1), bacc[blk]);
      }
      const v8bf bhi = v8bf{hi[0], hi[1], hi[2], hi[3], hi[4], hi[5], hi[6], hi[7]};
      const v8bf blo = v8bf{lo[0], lo[1], lo[2], lo[3], lo[4], lo[5], lo[6], lo[7]};
#pragma unroll
      for (int by = 0; by < 4; ++by) {
        const uint32_t sel = static_cast<uint32_t>(by) | (0x0Cu << 8) |
                             (static_cast<uint32_t>(4 + by) << 16) | (0x0Cu << 24);
        uint32_t alo[4], ahi[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t x = __builtin_amdgcn_perm(B.vw[2 * r + 1][blk], B.vw[2 * r][blk], sel);
          alo[r] = (x & 0x000F000Fu) | magic;
          ahi[r] = ((x >> 4) & 0x000F000Fu) | magic;
        }
        const v8bf a_lo = __builtin_bit_cast(v8bf, u32x4{alo[0], alo[1], alo[2], alo[3]});
        const v8bf a_hi = __builtin_bit_cast(v8bf, u32x4{ahi[0], ahi[1], ahi[2], ahi[3]});
        cv[blk][2 * by] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, bhi, cv[blk][2 * by], 0, 0, 0);
        cv[blk][2 * by + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, bhi, cv[blk][2 * by + 1], 0, 0, 0);
        cv[blk][2 * by] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, blo, cv[blk][2 * by], 0, 0, 0);
        cv[blk][2 * by + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, blo, cv[blk][2 * by + 1], 0, 0, 0);
      }
    }
  };

  auto load_next = [&](HcBuf& B, int t0) {
    const int tc = min(t0, last);
    hc_load(B, kq_rows, vq_rows, sc_rows, tc, last - tc, m, c);
  };

  for (int it = 0; it < nit; it += 2) {
    load_next(bufB, base0 + (it + 1) * kIter);
    __builtin_amdgcn_sched_barrier(0);
    process(bufA, base0 + it * kIter);
    __builtin_amdgcn_sched_barrier(0);
    load_next(bufA, base0 + (it + 2) * kIter);
    __builtin_amdgcn_sched_barrier(0);
    if (it + 1 < nit) process(bufB, base0 + (it + 1) * kIter);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- per-wave result into the finalisation arena --------------------------
  // lane (m, c) holds V words 16 blk + 4c + i of column m; the column's
  // group in block blk is 2 blk + m / 8, the words' group 2 blk + c / 2
  float l_sum = xor16_sum(l_run);
  l_sum = xor32_sum(l_sum);
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    wsum[blk] = xor16_sum(wsum[blk]);
    wsum[blk] = xor32_sum(wsum[blk]);
    bacc[blk] = xor16_sum(bacc[blk]);
    bacc[blk] = xor32_sum(bacc[blk]);
  }
  if ((c >> 1) == (m >> 3)) {
    float* o = Fin::o(arena, wave, hh);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const float off = bacc[blk] - 128.0f * wsum[blk];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // dims 8 (16 blk + 4c + i) + f, f = 0..7: two 16-byte stores
        float4* dst = reinterpret_cast<float4*>(o + 8 * (16 * blk + 4 * c + i));
        dst[0] = make_float4(cv[blk][0][i] + off, cv[blk][1][i] + off, cv[blk][2][i] + off, cv[blk][3][i] + off);
        dst[1] = make_float4(cv[blk][4][i] + off, cv[blk][5][i] + off, cv[blk][6][i] + off, cv[blk][7][i] + off);
      }
    }
  }
  if (c == 0 && m < 8) {
    Fin::m(arena, wave)[hh] = m_run;
    Fin::l(arena, wave)[hh] = l_sum;
  }
  Fin::run(p, arena, static_cast<int64_t>(b) * p.Hq + h0, rg.S, split, b * p.Hq + hy);
}

// ---- wave-specialised variant ---------------------------------------------
// The kernel above runs one wave per SIMD: every wave does both products of
// its keys, and at 1,500 instructions per 32 keys with nothing to hide its
// stalls, it is bound by issue, not HBM.  Here eight waves (two per SIMD)
// split the work of four 32-key streams:
//   producer s (waves 0-3): loads the K words and the four scale arrays of
//     stream s, computes K . q and the online softmax, and builds the P . V
//     B operands (bf16 hi / lo of p * s_v per block) plus the offset and bias
//     sums, staged in LDS (two slots, by iteration parity);
//   consumer s (waves 4-7): loads the V words of stream s, builds the A
//     operands and runs the 64 P . V products, one iteration behind.
// One barrier per step orders a slot's writes before its reads and the
// reads before its reuse two steps later.  Each role runs as its own code
// path (no buffer lives across a join of the two), through the same number
// of barriers: every wave runs the same even number of steps, and blocks
// past a stream's end are masked.  The accumulators of the consumer (128)
// and the doubled buffers of either role fit 256 registers, two waves per
// SIMD.
constexpr int kHs = 4;  // key streams (producer / consumer pairs)

// F32: fp32 scale/bias (8 words per key in each array instead of 4); the
// producer's scale registers and LDS stage double, nothing else changes.
template <bool F32>
__global__ __launch_bounds__(2 * kHs * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sdpa_int4_hc2_kernel(SdpaParams p) {
  pin_args(p);
  constexpr int NS = kHs, NWV = 2 * kHs, D = kHcD, G = kHcG, NG = kHcNG;
  constexpr int kNT = NWV * 64;
  constexpr int kIter = 32 * NS;   // keys per workgroup iteration

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = lane & 15, c = lane >> 4;
  const int hh = m & 7;  // this lane's head (column m)
  const int b = blockIdx.z, hy = blockIdx.y, split = blockIdx.x;
  const int kvh = hy / p.n_sub, sub = hy - kvh * p.n_sub;
  const int h0 = kvh * p.gqa + sub * G;

  const SplitRange rg = split_range(p, b, split);
  if (split >= rg.S) return;
  const int t_end = rg.t_end;

  // the P . V operand slots during the loop; after it, the streams' partial
  // outputs [stream][head][D + 4] (rows padded by 16 bytes, so the 8 heads'
  // rows start in different LDS banks)
  constexpr int kPvWords = 2 * NS * 4 * 2 * 64 * 4;  // [slot][stream][blk][hi/lo][lane] x uint4
  constexpr int kRow = D + 4;
  constexpr int kOWords = NS * G * kRow;
  constexpr int kArenaWords = kOWords > kPvWords ? kOWords : kPvWords;
  __shared__ __attribute__((aligned(16))) float arena[kArenaWords];
  __shared__ float ml_lds[2][NS][G];          // per stream: running max, sum of weights
  uint4* pv_lds = reinterpret_cast<uint4*>(arena);
  __shared__ uint4 bq_lds[3][NG][64];         // K MFMA B operands [digit][2 pair + half][lane]
  // [stream][array][group][key pair] fp16 x 2, or [..][key] fp32
  constexpr int SK = F32 ? 32 : 16;
  __shared__ __attribute__((aligned(16))) uint32_t sc_lds[NS][4][NG][SK];
  __shared__ float f_lds[2][NS][16];          // rescale factor per column, by slot
  __shared__ float off_lds[NS][4][16];        // final offset per (block, column)
  __shared__ float sh_qhat[G][NG];
  __shared__ int sh_F[G];

  const int64_t row0 = (static_cast<int64_t>(cache_batch(p, b)) * p.Hkv + kvh) * p.cap;
  const char* kq_rows = reinterpret_cast<const char*>(p.kq + row0 * (D / 8));
  const char* vq_rows = reinterpret_cast<const char*>(p.vq + row0 * (D / 8));
  const void* sc_base = c == 0 ? p.ks : (c == 1 ? p.kb : (c == 2 ? p.vs : p.vb));
  const char* sc_rows = static_cast<const char*>(sc_base) + row0 * (F32 ? 32 : 16);

  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const bool producer = wv < NS;
  const int s = producer ? wv : wv - NS;  // key stream
  const int base0 = rg.t_begin + s * 32;
  // steps of every wave: the iterations of stream 0 (the longest), rounded
  // up to even (the loops below take two per trip)
  const int nit0 = (t_end - rg.t_begin + kIter - 1) / kIter;
  const int NI = nit0 + (nit0 & 1);
  const int last = t_end - 1;
  const int safe_last = max(last, 0);
  auto tclamp = [&](int t0) { return min(t0, safe_last); };

  const int64_t qbase = (static_cast<int64_t>(b) * p.Hq + h0) * D;
  const v4i zero4 = v4i{0, 0, 0, 0};

  if (producer) {
    // ======================= producer: K . q, softmax, B operands ===========
    HcQ<kNT> Q;
    hc_q_load<kNT>(Q, p, qbase);
    __builtin_amdgcn_sched_barrier(0);
    constexpr int SW = F32 ? 2 : 1;  // 16-byte scale vectors per key
    uint32_t kA[2][16], kB[2][16];
    u32x4 sA[2][SW], sB[2][SW];
    auto load_k = [&](uint32_t (&kw)[2][16], u32x4 (&scw)[2][SW], int t0) {
      const int tc = tclamp(t0);
      hc_load_kw(kw, kq_rows, tc, safe_last - tc, m, c);
      hc_load_sc<F32>(scw, sc_rows, tc, safe_last - tc, m);
    };
    load_k(kA, sA, base0);
    __builtin_amdgcn_sched_barrier(0);
    hc_q_build<kNT>(Q, p, bq_lds, sh_qhat, sh_F, lane);
    const float sf = ldexpf(1.0f, -sh_F[hh]);
    float qh[NG / 2];
#pragma unroll
    for (int P = 0; P < NG / 2; ++P) qh[P] = sh_qhat[hh][2 * P + (m >> 3)] * ldexpf(1.0f, sh_F[hh]);

    float m_run = -INFINITY, l_run = 0.0f;
    float wsum[4], bacc[4];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) wsum[blk] = bacc[blk] = 0.0f;

    // One step: this step's products, with the next step's K and scale
    // loads issued among them (scales first, then the K loads of two pairs
    // after each even pair), so the wave never stalls on a burst of loads
    // after the barrier.
    auto produce = [&](const uint32_t (&kw)[2][16], const u32x4 (&scw)[2][SW], int st, uint32_t (&nk)[2][16],
                       u32x4 (&ns)[2][SW]) {
      const int t0 = base0 + st * kIter, slot = st & 1;
      const int tn = tclamp(t0 + kIter);
      // scales -> LDS [array][group][key pair] (fp16) or [..][key] (fp32)
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if constexpr (F32) {
          *reinterpret_cast<u32x2*>(&sc_lds[s][c][g][2 * m]) = u32x2{scw[0][g >> 2][g & 3], scw[1][g >> 2][g & 3]};
        } else {
          const uint32_t a0 = scw[0][0][g >> 1], a1 = scw[1][0][g >> 1];
          sc_lds[s][c][g][m] = (g & 1) ? ((a0 >> 16) | (a1 & 0xFFFF0000u)) : ((a0 & 0xFFFFu) | (a1 << 16));
        }
      }
      // the scale arrays' entries of keys k0 .. k0 + 3 (k0 % 4 == 0) of
      // group g, as fp32
      auto scale4 = [&](int a, int g, int k0) -> v4f {
        if constexpr (F32) {
          return *reinterpret_cast<const v4f*>(&sc_lds[s][a][g][k0]);
        } else {
          const uint2 u = *reinterpret_cast<const uint2*>(&sc_lds[s][a][g][k0 >> 1]);
          return v4f{hc_half(u.x, 0), hc_half(u.x, 1), hc_half(u.y, 0), hc_half(u.y, 1)};
        }
      };
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      __builtin_amdgcn_sched_barrier(0);
      hc_load_sc<F32>(ns, sc_rows, tn, safe_last - tn, m);
      __builtin_amdgcn_sched_barrier(0);

      // K . q per pair of quant groups (as in the kernel above)
      float sc[2][4];
#pragma unroll
      for (int tile = 0; tile < 2; ++tile)
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[tile][i] = 0.0f;
      auto bop = [&](int dg, int j) {
        const uint4 u = bq_lds[dg][j][lane];
        return v4i{static_cast<int>(u.x), static_cast<int>(u.y), static_cast<int>(u.z), static_cast<int>(u.w)};
      };
      auto aop = [&](uint32_t w0, uint32_t w1) {
        return v4i{static_cast<int>(w0 & 0x0F0F0F0Fu), static_cast<int>((w0 >> 4) & 0x0F0F0F0Fu),
                   static_cast<int>(w1 & 0x0F0F0F0Fu), static_cast<int>((w1 >> 4) & 0x0F0F0F0Fu)};
      };
#pragma unroll
      for (int P = 0; P < NG / 2; ++P) {
        const v4i b00 = bop(0, 2 * P), b01 = bop(0, 2 * P + 1);
        const v4i b10 = bop(1, 2 * P), b11 = bop(1, 2 * P + 1);
        const v4i b20 = bop(2, 2 * P), b21 = bop(2, 2 * P + 1);
        const int gl = 2 * P + (m >> 3);
#pragma unroll
        for (int tile = 0; tile < 2; ++tile) {
          const v4i a0 = aop(kw[tile][4 * P], kw[tile][4 * P + 1]);
          const v4i a1 = aop(kw[tile][4 * P + 2], kw[tile][4 * P + 3]);
          v4i acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b00, zero4, 0, 0, 0);
          v4i acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b10, zero4, 0, 0, 0);
          v4i acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b20, zero4, 0, 0, 0);
          acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b01, acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b11, acc1, 0, 0, 0);
          acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b21, acc2, 0, 0, 0);
          const v4f ks = scale4(0, gl, 16 * tile + 4 * c), kb = scale4(1, gl, 16 * tile + 4 * c);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // two shift-adds (the compiler's add3 form takes three instructions)
            int lo01 = (acc1[i] << 8) + acc0[i];
            asm("" : "+v"(lo01));
            const float dot = static_cast<float>((acc2[i] << 16) + lo01);
            sc[tile][i] = fmaf(dot, ks[i], fmaf(kb[i], qh[P], sc[tile][i]));
          }
        }
        // pairs 2P', 2P' + 1 together: the two 64-byte halves of each
        // 128-byte line go out in one batch (apart, the non-temporal line
        // was fetched twice: 1.16x the algorithmic bytes)
        if ((P & 1) == 0) {
          __builtin_amdgcn_sched_barrier(0);
          hc_load_kw_pair(nk, kq_rows, tn, safe_last - tn, m, c, P);
          hc_load_kw_pair(nk, kq_rows, tn, safe_last - tn, m, c, P + 1);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int tile = 0; tile < 2; ++tile)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sc[tile][i] = sf * (sc[tile][i] + __int_as_float(__builtin_amdgcn_mov_dpp(
                                                 __float_as_int(sc[tile][i]), 0x128, 0xF, 0xF, false)));
      // keys from t_end on: only the last step of a stream reaches them
      if (t0 + 32 > t_end) {  // uniform
#pragma unroll
        for (int tile = 0; tile < 2; ++tile)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (t0 + 16 * tile + 4 * c + i >= t_end) sc[tile][i] = -INFINITY;
      }

      // online softmax (lazy rescale); the factor goes to the consumer
      float mt = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                       fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
      mt = xor16_max(mt);
      mt = xor32_max(mt);
      const float m_new = fmaxf(m_run, mt);
      float f = 1.0f;
      if (st == 0) {
        m_run = m_new;  // first batch: nothing accumulated yet
      } else if (__any(m_new > m_run + kLazyMax)) {
        f = (m_new == m_run) ? 1.0f : merge_factor(m_run, m_new);
        l_run *= f;
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
          wsum[blk] *= f;
          bacc[blk] *= f;
        }
        m_run = m_new;
      }
      if (c == 0) f_lds[slot][s][m] = f;
      // (every stream runs the steps of the longest one, so a stream's steps
      // can all lie past t_end: m_run is then -inf, and masked scores need
      // the explicit 0)
      float pw[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sj = sc[j >> 2][j & 3];
        pw[j] = sj == -INFINITY ? 0.0f : fast_exp2(sj - m_run);
        l_run += pw[j];
      }

      // B operands of the P . V products per block of 16 V words
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const int gv = 2 * blk + (m >> 3);
        // slot j: key 16 (j / 4) + 4c + j % 4
        const v4f vs[2] = {scale4(2, gv, 4 * c), scale4(2, gv, 16 + 4 * c)};
        const v4f vb[2] = {scale4(3, gv, 4 * c), scale4(3, gv, 16 + 4 * c)};
        // weights in bf16 pairs (slots 2k, 2k + 1: one B operand word): hi
        // and lo = w - hi, each pair by one packed conversion; the weight
        // sum of the 128 offset takes a word per v_dot2 with (1, 1); the
        // fp16 scales convert inside the multiplies (fma with + 0)
        uint32_t bh[4], bl[4];
        const v2bf ones = __builtin_bit_cast(v2bf, 0x3F803F80u);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int j = 2 * k;
          const float w0 = fmaf(pw[j], vs[j >> 2][j & 3], 0.0f);
          const float w1 = fmaf(pw[j + 1], vs[(j + 1) >> 2][(j + 1) & 3], 0.0f);
          uint32_t hb = __builtin_bit_cast(uint32_t, v2bf{static_cast<__bf16>(w0), static_cast<__bf16>(w1)});
          asm("" : "+v"(hb));  // h0, h1 from the packed word
          const float h0 = __uint_as_float(hb << 16), h1 = __uint_as_float(hb & 0xFFFF0000u);
          const uint32_t lb =
              __builtin_bit_cast(uint32_t, v2bf{static_cast<__bf16>(w0 - h0), static_cast<__bf16>(w1 - h1)});
          bh[k] = hb;
          bl[k] = lb;
          wsum[blk] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, hb), ones, wsum[blk], false);
          wsum[blk] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, lb), ones, wsum[blk], false);
          bacc[blk] = fmaf(pw[j], vb[j >> 2][j & 3], bacc[blk]);
          bacc[blk] = fmaf(pw[j + 1], vb[(j + 1) >> 2][(j + 1) & 3], bacc[blk]);
        }
        uint4* dst = pv_lds + (((slot * NS + s) * 4 + blk) * 2) * 64 + lane;
        dst[0] = uint4{bh[0], bh[1], bh[2], bh[3]};
        dst[64] = uint4{bl[0], bl[1], bl[2], bl[3]};
      }
    };

    for (int st = 0; st < NI; st += 2) {
      produce(kA, sA, st, kB, sB);
      __syncthreads();
      produce(kB, sB, st + 1, kA, sA);
      __syncthreads();
    }
    // per-column results, published by the barrier that ends the consumers'
    // last step: (m, l) and the offsets of the weight sums
    float l_sum = xor16_sum(l_run);
    l_sum = xor32_sum(l_sum);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      wsum[blk] = xor16_sum(wsum[blk]);
      wsum[blk] = xor32_sum(wsum[blk]);
      bacc[blk] = xor16_sum(bacc[blk]);
      bacc[blk] = xor32_sum(bacc[blk]);
      if (c == 0) off_lds[s][blk][m] = bacc[blk] - 128.0f * wsum[blk];
    }
    if (c == 0 && m < 8) {
      ml_lds[0][s][hh] = m_run;
      ml_lds[1][s][hh] = l_sum;
    }
    __syncthreads();  // the consumers' last step
  } else {
    // ======================= consumer: P . V ================================
    // the first V loads go out before the q image is built (after them, the
    // V stream started ~2 us late: global layer 24.8 -> 24.2 us)
    u32x4 vA[2][4], vB[2][4];
    HcQ<kNT> Q;
    hc_q_load<kNT>(Q, p, qbase);
    __builtin_amdgcn_sched_barrier(0);
    hc_load_v4(vA, vq_rows, tclamp(base0), safe_last - tclamp(base0), m, c);
    __builtin_amdgcn_sched_barrier(0);
    hc_q_build<kNT>(Q, p, bq_lds, sh_qhat, sh_F, lane);

    v4f cv[4][8];  // [blk][2 byte + nibble half]
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int ff = 0; ff < 8; ++ff) cv[blk][ff] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t magic = 0x43004300u;  // bf16 of (128 + nibble)
    asm volatile("" : "+v"(magic));

    // One step: this step's products, with the next step's V loads issued
    // among them (four after each even block).
    auto consume = [&](const u32x4 (&vr)[2][4], int st, u32x4 (&nx)[2][4]) {
      const int tn = tclamp(base0 + (st + 1) * kIter);
      const int slot = st & 1;
      const float f = f_lds[slot][s][m];
      if (__any(f != 1.0f)) {
#pragma unroll
        for (int blk = 0; blk < 4; ++blk)
#pragma unroll
          for (int ff = 0; ff < 8; ++ff) cv[blk][ff] *= f;
      }
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        // slot j = 4T + i: word 16 blk + m of key 16 T + 4c + i
        uint32_t vw[8];
#pragma unroll
        for (int T = 0; T < 2; ++T) {
          const u32x4 t = hc_quad_transpose(vr[T][blk], lane);
#pragma unroll
          for (int i = 0; i < 4; ++i) vw[4 * T + i] = t[i];
        }
        if ((blk & 1) == 0) {  // both halves of each 128-byte line at once
          __builtin_amdgcn_sched_barrier(0);
          hc_load_v4_blk(nx, vq_rows, tn, safe_last - tn, m, c, blk);
          hc_load_v4_blk(nx, vq_rows, tn, safe_last - tn, m, c, blk + 1);
          __builtin_amdgcn_sched_barrier(0);
        }
        const uint4* src = pv_lds + (((slot * NS + s) * 4 + blk) * 2) * 64 + lane;
        const v8bf bhi = __builtin_bit_cast(v8bf, src[0]);
        const v8bf blo = __builtin_bit_cast(v8bf, src[64]);
#pragma unroll
        for (int by = 0; by < 4; ++by) {
          const uint32_t sel = static_cast<uint32_t>(by) | (0x0Cu << 8) |
                               (static_cast<uint32_t>(4 + by) << 16) | (0x0Cu << 24);
          uint32_t alo[4], ahi[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t x = __builtin_amdgcn_perm(vw[2 * r + 1], vw[2 * r], sel);
            alo[r] = (x & 0x000F000Fu) | magic;
            ahi[r] = ((x >> 4) & 0x000F000Fu) | magic;
          }
          const v8bf a_lo = __builtin_bit_cast(v8bf, u32x4{alo[0], alo[1], alo[2], alo[3]});
          const v8bf a_hi = __builtin_bit_cast(v8bf, u32x4{ahi[0], ahi[1], ahi[2], ahi[3]});
          cv[blk][2 * by] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, bhi, cv[blk][2 * by], 0, 0, 0);
          cv[blk][2 * by + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, bhi, cv[blk][2 * by + 1], 0, 0, 0);
          cv[blk][2 * by] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, blo, cv[blk][2 * by], 0, 0, 0);
          cv[blk][2 * by + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, blo, cv[blk][2 * by + 1], 0, 0, 0);
        }
      }
    };

    __syncthreads();  // the producers' step 0
    for (int st = 0; st < NI; st += 2) {
      consume(vA, st, vB);
      __syncthreads();
      consume(vB, st + 1, vA);
      __syncthreads();
    }
    // the operand slots are dead (every consumer passed its last step) and
    // the producers' offsets visible: the stream's partial into its rows.
    // lane (m, c) holds V words 16 blk + 4c + i of column m; the column's
    // group in block blk is 2 blk + m / 8, the words' group 2 blk + c / 2
    if ((c >> 1) == (m >> 3)) {
      float* o = arena + (s * G + hh) * kRow;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const float off = off_lds[s][blk][m];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // dims 8 (16 blk + 4c + i) + ff, ff = 0..7: two 16-byte stores
          float4* dst = reinterpret_cast<float4*>(o + 8 * (16 * blk + 4 * c + i));
          dst[0] = make_float4(cv[blk][0][i] + off, cv[blk][1][i] + off, cv[blk][2][i] + off, cv[blk][3][i] + off);
          dst[1] = make_float4(cv[blk][4][i] + off, cv[blk][5][i] + off, cv[blk][6][i] + off, cv[blk][7][i] + off);
        }
      }
    }
  }
  __syncthreads();

  // ---- the four streams combined, four dims per thread ---------------------
  // The split's partial (or, for a single split, the output) of the 8 heads;
  // the partials are merged by merge_splits_kernel after this kernel.
  constexpr int D4 = D / 4;
  for (int i = threadIdx.x; i < G * D4; i += kNT) {
    const int h = i / D4, d4 = i - h * D4;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NS; ++w) M = fmaxf(M, ml_lds[0][w][h]);
    v4f O = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < NS; ++w) {
      const float f = merge_factor(ml_lds[0][w][h], M);
      O += f * *reinterpret_cast<const v4f*>(arena + (w * G + h) * kRow + 4 * d4);
      L = fmaf(ml_lds[1][w][h], f, L);
    }
    const int64_t row = static_cast<int64_t>(b) * p.Hq + h0 + h;
    if (rg.S == 1) {
      const v4f r = v4f{normalise(O[0], L, p.denom_eps), normalise(O[1], L, p.denom_eps),
                        normalise(O[2], L, p.denom_eps), normalise(O[3], L, p.denom_eps)};
      float* dst = p.out + row * D + 4 * d4;
      if ((reinterpret_cast<uintptr_t>(p.out) & 15) == 0) {  // uniform
        *reinterpret_cast<v4f*>(dst) = r;
      } else {
        dst[0] = r[0]; dst[1] = r[1]; dst[2] = r[2]; dst[3] = r[3];
      }
    } else {
      // read once, by the merge kernel: streaming (non-temporal) stores
      const int64_t slot = row * p.max_splits + split;
      __builtin_nontemporal_store(O, reinterpret_cast<v4f*>(p.ws_o + slot * D + 4 * d4));
      if (d4 == 0) {
        __builtin_nontemporal_store(M, p.ws_ml + slot * 2);
        __builtin_nontemporal_store(L, p.ws_ml + slot * 2 + 1);
      }
    }
  }
}

// Merge of split partials written with ext_merge = 1.  A wave takes four
// outputs (four dims each), sixteen lanes per output; a lane takes splits
// sl, sl + 16, ...: four at a time, each group's (m, l) and O partials
// loaded together (one memory round trip per 64 splits), folded into the
// lane's running (m, l, O), then the 16 lanes merge by shuffles.  The
// partials come from an earlier kernel, so plain loads see them.  Grid
// (ceil(Hq * D / 4 / 16), batch).
__global__ __launch_bounds__(256) void merge_splits_kernel(SdpaParams p, int D) {
  pin_args(p);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sl = lane & 15;
  const int D4 = D / 4;
  const int o0 = (blockIdx.x * 4 + wave) * 4;  // first output of this wave
  const int b = blockIdx.y;
  if (o0 >= p.Hq * D4) return;                 // whole waves (Hq * D4 % 4 == 0)
  const SplitRange rg = split_range(p, b, 0);
  const int S = rg.S;
  if (S == 1) return;                          // written by the attention kernel
  const int o = o0 + (lane >> 4);
  const int h = o / D4, d4 = o - h * D4;
  const int64_t head = static_cast<int64_t>(b) * p.Hq + h;
  const float* ml = p.ws_ml + head * p.max_splits * 2;
  const float* po = p.ws_o + head * p.max_splits * D + 4 * d4;
  float M = -INFINITY, L = 0.0f;
  float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int s0 = 0; s0 < S; s0 += 64) {
    float mk[4], lk[4];
    float4 ok[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int sp = min(s0 + sl + 16 * k, S - 1);  // clamped; dropped below
      mk[k] = ml[2 * sp];
      lk[k] = ml[2 * sp + 1];
      ok[k] = *reinterpret_cast<const float4*>(po + static_cast<int64_t>(sp) * D);
    }
    float Mn = M;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (s0 + sl + 16 * k >= S) mk[k] = -INFINITY;
      Mn = fmaxf(Mn, mk[k]);
    }
    const float fr = merge_factor(M, Mn);
    L *= fr;
    O.x *= fr; O.y *= fr; O.z *= fr; O.w *= fr;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float f = merge_factor(mk[k], Mn);
      L = fmaf(lk[k], f, L);
      O.x = fmaf(ok[k].x, f, O.x);
      O.y = fmaf(ok[k].y, f, O.y);
      O.z = fmaf(ok[k].z, f, O.z);
      O.w = fmaf(ok[k].w, f, O.w);
    }
    M = Mn;
  }
  // the 16 lanes of an output: DPP butterflies within the row
  const float Mall = row16_max(M);
  const float f = merge_factor(M, Mall);
  L = group_sum<16>(L * f);
  O.x = group_sum<16>(O.x * f);
  O.y = group_sum<16>(O.y * f);
  O.z = group_sum<16>(O.z * f);
  O.w = group_sum<16>(O.w * f);
  if (sl == 0) {
    float* out = p.out + head * D + 4 * d4;
    out[0] = normalise(O.x, L, p.denom_eps);
    out[1] = normalise(O.y, L, p.denom_eps);
    out[2] = normalise(O.z, L, p.denom_eps);
    out[3] = normalise(O.w, L, p.denom_eps);
  }
}

}  // namespace

int launch_merge_splits(const SdpaParams& p, int D, int batch, hipStream_t s) {
  const int outs = p.Hq * D / 4;
  merge_splits_kernel<<<dim3((outs + 15) / 16, batch), 256, 0, s>>>(p, D);
  TQ_CHECK_LAUNCH("merge_splits_kernel");
  return TQ_OK;
}

// fp16 scale/bias on either kernel; fp32 on the wave-specialised one
bool hc_serves(int sb_dtype) {
  return sb_dtype == TQ_F16 || (sb_dtype == TQ_F32 && !options().hc_one);
}

int launch_sdpa_hc(const SdpaParams& p, int sb_dtype, dim3 grid, hipStream_t s) {
  // TQ_HC_IMPL=1 selects the one-wave-per-SIMD kernel (fp16 scale/bias)
  if (!hc_serves(sb_dtype)) {
    set_error("sdpa_int4: the heads-as-columns kernel does not serve this scale/bias dtype");
    return TQ_ERR_INVALID;
  }
  if (options().hc_one) {
    sdpa_int4_hc_kernel<<<grid, kHcWaves * 64, 0, s>>>(p);
    TQ_CHECK_LAUNCH("sdpa_int4_hc_kernel");
  } else if (sb_dtype == TQ_F32) {
    sdpa_int4_hc2_kernel<true><<<grid, 2 * kHs * 64, 0, s>>>(p);
    TQ_CHECK_LAUNCH("sdpa_int4_hc2_kernel<true>");
  } else {
    sdpa_int4_hc2_kernel<false><<<grid, 2 * kHs * 64, 0, s>>>(p);
    TQ_CHECK_LAUNCH("sdpa_int4_hc2_kernel<false>");
  }
  return TQ_OK;
}

}  // namespace tq
