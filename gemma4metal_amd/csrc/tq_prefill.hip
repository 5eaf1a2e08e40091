// Multi-query (prefill) attention over the int4 cache with K/V tiles shared
// by a workgroup's 64 (query, head) rows -- the engine's prefill fallback
// (engine/gemma4_multilayer.cpp:343-364: dequantize, then masked
// scaled_dot_product_attention), for head_dim 128 / 256 / 512.
//
// A workgroup takes all gqa heads of one kv head for 64 / gqa consecutive
// queries (16 rows per wave) and streams the union of their key ranges in
// tiles of 32 keys.  Each tile is dequantized once into LDS:
//   K as fp16 hi / lo rows [key][dim], V transposed as bf16 hi / lo [dim][slot]
// (value = s * nibble + b in fp32, split into a rounded high part and the
// rounded remainder).  V^T slot 8c + 4h + j holds key 16h + 4c + j, so the
// eight keys lane group c weights (below) are one 16 B read.
// Per tile and wave, on the matrix cores (l = lane, m = l % 16, c = l / 16):
//   S^T = K q^T   v_mfma_f32_16x16x32_f16, A = 16 keys x 32 dims of K, B =
//                 32 dims x 16 rows of q (hi / lo in registers); the three
//                 products hi*hi + hi*lo + lo*hi keep ~22 bits.  Lane l then
//                 holds scores of keys 16 tile + 4c + i for row m.
//   O^T += V^T P^T  v_mfma_f32_16x16x32_bf16, A = 16 dims x 32 keys of V^T,
//                 B = the bf16 hi / lo split of the weights: key slot j of
//                 lane group c is key 16 (j / 4) + 4c + j % 4 -- exactly the
//                 scores lane l already holds, so no exchange is needed.  Lane
//                 l accumulates dims 16 blk + 4c + i of row m.
// The online softmax state (max, denominator) of row m lives in the lanes of
// column m; each row has its own causal / window limit.
#include "tq_sdpa_common.h"

#include <type_traits>

namespace tq {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfRows = 16 * kPfWaves;  // (query, head) rows per workgroup
constexpr int kPfKeys = 32;             // keys per tile

template <int D>
struct PfGeom {
  static constexpr int W = D / 8;                     // packed words per row
  static constexpr int KSTR = D + 8;                  // K rows in LDS (halves; 16 B pad)
  static constexpr int KPT = kPfKeys * W / kPfThreads;  // keys per thread in the dequant
  // V^T rows in LDS (halves): 16 B aligned for the 8-slot reads; a 16-row
  // read phase at this stride (20 dwords) covers all 64 banks once
  static constexpr int VSTR = kPfKeys + 8;
  static constexpr int CH = D / 32;                   // K.q k-steps of 32 dims
  static constexpr int DB = D / 16;                   // 16-dim output blocks
  static_assert(KPT == 2 || KPT == 4 || KPT == 8, "D");
  // D = 512: each lane loads one scale and one bias value of a tile per
  // tensor, and the dequantization takes the ones its keys need from the
  // lanes that hold them (ds_bpermute): 4 loads and registers instead of 32
  // while the tile's words are in flight
  static constexpr bool LANE_SB = D == 512;
  static constexpr int NS = LANE_SB ? 1 : KPT;
  static_assert(!LANE_SB || (W == 64 && KPT == 8 && kPfThreads == 256), "lane roles of the D = 512 scales");
};

// Raw int4 words and the scale / bias (fp16 bits, or fp32 with F32) of
// this thread's keys of one tile (with LANE_SB: one value of the wave's).
template <int D, bool F32>
struct PfRaw {
  using SB = typename std::conditional<F32, float, uint16_t>::type;
  uint32_t kw[PfGeom<D>::KPT], vw[PfGeom<D>::KPT];
  SB ks[PfGeom<D>::NS], kb[PfGeom<D>::NS], vs[PfGeom<D>::NS], vb[PfGeom<D>::NS];
};

// The 32-bit value v of lane src of the wave.
__device__ __forceinline__ uint32_t pf_from_lane(uint32_t v, int src) {
  return static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src << 2, static_cast<int>(v)));
}

// The key (0 .. 31 within the tile) held by V^T slot s.
__device__ __forceinline__ int pf_vkey(int s) { return 16 * ((s >> 2) & 1) + 4 * (s >> 3) + (s & 3); }

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ float sbf(uint16_t h) { return h2f(h); }
__device__ __forceinline__ float sbf(float x) { return x; }

// K and V use different thread roles (word w, keys k0 .. k0 + KPT - 1 for
// K, V^T slots k0 .. k0 + KPT - 1 for V): K's lanes run along the words of a
// key (its LDS rows are key-major), V's along the slots of a word (V^T rows
// are dim-major), so that both LDS stores of a 16-lane phase land in
// distinct banks.
// Dequantization of one tile's raw words (this thread's keys) into the LDS
// images: K as fp16 hi / lo rows, V^T as bf16 hi / lo (value s * n + b in
// fp32, then its rounded high part and the rounded remainder).
// Nibbles of a word as floats: the low and high nibble of each byte are
// masked into bytes of their own and converted by byte (v_cvt_f32_ubyte0-3),
// so no nibble needs a shift of its own.  Element i of the word is bits 4i.
__device__ __forceinline__ void pf_nibbles(uint32_t wd, float (&n)[8]) {
  uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
  // opaque: otherwise each byte conversion is folded back into a shift and
  // a mask of the raw word
  asm("" : "+v"(lo), "+v"(hi));
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    n[2 * b] = static_cast<float>((lo >> (8 * b)) & 0xFFu);
    n[2 * b + 1] = static_cast<float>((hi >> (8 * b)) & 0xFFu);
  }
}

// The fp16 remainders x0 - h0, x1 - h1 of a pair whose fp16 high parts are
// packed in hp, as a packed fp16 pair: one mixed-precision fma each (fp16
// source, fp32 addend, fp16 result into the low / high half).  The
// remainder is exact in fp32 and rounded once, to fp16.
__device__ __forceinline__ uint32_t pf_rem_pair(uint32_t hp, float x0, float x1) {
  uint32_t r;
  asm volatile(
      "v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mixhi_f16 %0, %1, -1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "=&v"(r)
      : "v"(hp), "v"(x0), "v"(x1));
  return r;
}

template <int D, bool F32>
__device__ __forceinline__ void pf_dequant(const PfRaw<D, F32>& raw, _Float16* khi, _Float16* klo, __bf16* vthi,
                                           __bf16* vtlo, int w, int kb0, int wv, int kv0) {
  using Gm = PfGeom<D>;
  constexpr int KSTR = Gm::KSTR, VSTR = Gm::VSTR, KPT = Gm::KPT;
  typedef _Float16 v2h __attribute__((ext_vector_type(2)));
  // scale and bias of this thread's K keys and V slots
  float kS[KPT], kB[KPT], vS[KPT], vB[KPT];
  if constexpr (Gm::LANE_SB) {
    // lane s holds K key kb0 + s / 8 of group s % 8, and V key s % 32 of
    // group wv / 8 (lanes 0-31 and 32-63 hold the wave's two V groups)
    const int lane = threadIdx.x & 63;
    uint32_t kp = 0, vp = 0;
    if constexpr (!F32) {
      kp = static_cast<uint32_t>(raw.ks[0]) | (static_cast<uint32_t>(raw.kb[0]) << 16);
      vp = static_cast<uint32_t>(raw.vs[0]) | (static_cast<uint32_t>(raw.vb[0]) << 16);
    }
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      const int sk = (e << 3) | (lane >> 3);
      const int sv = (lane & 32) | (4 * (lane & 3) + (e & 3) + 16 * (e >> 2));
      if constexpr (F32) {
        kS[e] = __uint_as_float(pf_from_lane(__float_as_uint(raw.ks[0]), sk));
        kB[e] = __uint_as_float(pf_from_lane(__float_as_uint(raw.kb[0]), sk));
        vS[e] = __uint_as_float(pf_from_lane(__float_as_uint(raw.vs[0]), sv));
        vB[e] = __uint_as_float(pf_from_lane(__float_as_uint(raw.vb[0]), sv));
      } else {
        const uint32_t kx = pf_from_lane(kp, sk), vx = pf_from_lane(vp, sv);
        kS[e] = h2f(static_cast<uint16_t>(kx & 0xFFFFu));
        kB[e] = h2f(static_cast<uint16_t>(kx >> 16));
        vS[e] = h2f(static_cast<uint16_t>(vx & 0xFFFFu));
        vB[e] = h2f(static_cast<uint16_t>(vx >> 16));
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      kS[e] = sbf(raw.ks[e]);
      kB[e] = sbf(raw.kb[e]);
      vS[e] = sbf(raw.vs[e]);
      vB[e] = sbf(raw.vb[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < KPT; ++e) {
    const int key = kb0 + e;
    const float ks = kS[e], kbias = kB[e];
    float n[8];
    pf_nibbles(raw.kw[e], n);
    u32x4 kh, kl;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float x0 = fmaf(ks, n[2 * q], kbias), x1 = fmaf(ks, n[2 * q + 1], kbias);
      const uint32_t hp = __builtin_bit_cast(uint32_t, v2h{static_cast<_Float16>(x0), static_cast<_Float16>(x1)});
      kh[q] = hp;
      kl[q] = pf_rem_pair(hp, x0, x1);
    }
    *reinterpret_cast<u32x4*>(&khi[key * KSTR + 8 * w]) = kh;
    *reinterpret_cast<u32x4*>(&klo[key * KSTR + 8 * w]) = kl;
  }
  // V^T: the KPT slots of one dim are adjacent -- one 4 / 8 / 16 B store each;
  // the bf16 high and low parts of a key pair each take one packed conversion
  typedef __bf16 vkpt __attribute__((ext_vector_type(KPT)));
  typedef __bf16 v2bf_t __attribute__((ext_vector_type(2)));
  float nv[KPT][8];
#pragma unroll
  for (int e = 0; e < KPT; ++e) pf_nibbles(raw.vw[e], nv[e]);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    vkpt vh, vl;
#pragma unroll
    for (int e = 0; e < KPT; e += 2) {
      const float x0 = fmaf(vS[e], nv[e][j], vB[e]);
      const float x1 = fmaf(vS[e + 1], nv[e + 1][j], vB[e + 1]);
      const v2bf_t h = v2bf_t{static_cast<__bf16>(x0), static_cast<__bf16>(x1)};
      const uint32_t hb = __builtin_bit_cast(uint32_t, h);
      const float h0 = __uint_as_float(hb << 16), h1 = __uint_as_float(hb & 0xFFFF0000u);
      const v2bf_t l = v2bf_t{static_cast<__bf16>(x0 - h0), static_cast<__bf16>(x1 - h1)};
      vh[e] = h[0];
      vh[e + 1] = h[1];
      vl[e] = l[0];
      vl[e + 1] = l[1];
    }
    *reinterpret_cast<vkpt*>(&vthi[(8 * wv + j) * VSTR + kv0]) = vh;
    *reinterpret_cast<vkpt*>(&vtlo[(8 * wv + j) * VSTR + kv0]) = vl;
  }
}

template <int D, bool F32>
__device__ __forceinline__ void pf_load(PfRaw<D, F32>& R, const SdpaParams& p, int64_t row0, int t0,
                                        int last, int wk, int kk0, int wv, int kv0) {
  using Gm = PfGeom<D>;
  using SB = typename PfRaw<D, F32>::SB;
  const SB* ks = static_cast<const SB*>(p.ks);
  const SB* kb = static_cast<const SB*>(p.kb);
  const SB* vs = static_cast<const SB*>(p.vs);
  const SB* vb = static_cast<const SB*>(p.vb);
#pragma unroll
  for (int e = 0; e < Gm::KPT; ++e) {
    const int64_t rk = row0 + min(t0 + kk0 + e, last);
    // slots kv0 .. kv0 + KPT - 1 hold keys vkey(kv0) + e % 4 + 16 (e / 4)
    const int64_t rv = row0 + min(t0 + pf_vkey(kv0) + (e & 3) + 16 * (e >> 2), last);
    R.kw[e] = __builtin_nontemporal_load(p.kq + rk * Gm::W + wk);
    R.vw[e] = __builtin_nontemporal_load(p.vq + rv * Gm::W + wv);
    if constexpr (!Gm::LANE_SB) {
      R.ks[e] = ks[rk * (D / 64) + (wk >> 3)];
      R.kb[e] = kb[rk * (D / 64) + (wk >> 3)];
      R.vs[e] = vs[rv * (D / 64) + (wv >> 3)];
      R.vb[e] = vb[rv * (D / 64) + (wv >> 3)];
    }
  }
  if constexpr (Gm::LANE_SB) {
    // K key kk0 + lane / 8 (the wave's keys) of group lane % 8; V key
    // lane % 32 of group wv / 8
    const int lane = threadIdx.x & 63;
    const int64_t rk = row0 + min(t0 + kk0 + (lane >> 3), last);
    const int64_t rv = row0 + min(t0 + (lane & 31), last);
    R.ks[0] = ks[rk * (D / 64) + (lane & 7)];
    R.kb[0] = kb[rk * (D / 64) + (lane & 7)];
    R.vs[0] = vs[rv * (D / 64) + (wv >> 3)];
    R.vb[0] = vb[rv * (D / 64) + (wv >> 3)];
  }
}

// D = 512: one wave per SIMD (q hi / lo and the O^T accumulators take 256
// registers), 145 KB of LDS.  With one wave per SIMD nothing hides LDS
// latency: the products' operands are read four k-steps / blocks ahead,
// which the scale / bias lane sharing (LANE_SB) leaves registers for.
template <int D, bool F32>
__global__ __launch_bounds__(kPfThreads)
__attribute__((amdgpu_waves_per_eu(D == 512 ? 1 : 2, D == 512 ? 1 : 2)))
void prefill_int4_kernel(SdpaParams p) {
  pin_args(p);
  using Gm = PfGeom<D>;
  constexpr int W = Gm::W, KSTR = Gm::KSTR, VSTR = Gm::VSTR, CH = Gm::CH, DB = Gm::DB;
  constexpr int KPT = Gm::KPT;
  __shared__ __attribute__((aligned(16))) _Float16 khi[kPfKeys * KSTR], klo[kPfKeys * KSTR];
  __shared__ __attribute__((aligned(16))) __bf16 vthi[D * VSTR], vtlo[D * VSTR];
  static_assert(CH % 4 == 0 && DB % 4 == 0, "reads are issued four k-steps / blocks ahead");

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = lane & 15, c = lane >> 4;
  const int kvh = blockIdx.y;
  const int gqa = p.gqa;
  const int qpw = kPfRows / gqa;          // queries per workgroup
  const int q0 = blockIdx.x * qpw;        // first query of this workgroup
  const int q_last = min(q0 + qpw, p.nq) - 1;
  // this lane's row (column m of the wave): query q0 + r / gqa, head r % gqa
  const int r = 16 * wave + m;
  const int qo = r / gqa, ho = r - qo * gqa;
  const bool row_ok = q0 + qo <= q_last;
  const int qi = min(q0 + qo, q_last);
  const int pos = p.n + qi;               // absolute position of the query
  const int W_ = p.window;
  const int lo = W_ > 0 ? max(0, p.n + q0 + 1 - W_) : 0;  // union of the rows' key ranges
  const int hi = p.n + q_last + 1;
  const int last = hi - 1;
  const int ntile = (hi - lo + kPfKeys - 1) / kPfKeys;
  const int64_t row0 = static_cast<int64_t>(kvh) * p.cap;
  const int64_t qrow = static_cast<int64_t>(qi) * p.Hq + kvh * gqa + ho;

  // ---- q of this lane's row: dims 32 ch + 8c .. +7, fp16 hi / lo ----------
  v8h qh[CH], ql[CH];
#pragma unroll
  for (int ch = 0; ch < CH; ++ch) {
    float f[8];
    const int64_t e0 = qrow * D + 32 * ch + 8 * c;
    if (p.q_dtype == TQ_F32) {
      const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + e0);
      const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + e0 + 4);
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else {
      const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.q) + e0);
      const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t a = wd[i] & 0xFFFFu, b = wd[i] >> 16;
        f[2 * i] = p.q_dtype == TQ_F16 ? h2f(a) : __uint_as_float(static_cast<uint32_t>(a) << 16);
        f[2 * i + 1] = p.q_dtype == TQ_F16 ? h2f(b) : __uint_as_float(static_cast<uint32_t>(b) << 16);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = f[i] * p.scale_log2;
      const _Float16 h = static_cast<_Float16>(x);
      qh[ch][i] = h;
      ql[ch][i] = static_cast<_Float16>(x - static_cast<float>(h));
    }
  }

  // dequant roles: word w of keys kb0 .. kb0 + KPT - 1 of a tile (K), word
  // wv of V^T slots kv0 .. (V)
  constexpr int KB = kPfKeys / KPT;  // key blocks per tile
  const int w = threadIdx.x % W, kb0 = (threadIdx.x / W) * KPT;
  const int wv = threadIdx.x / KB, kv0 = (threadIdx.x % KB) * KPT;
  // raw words of the tiles in flight: two (tiles it + 1 and it + 2 load
  // while tile it is computed), one at D = 512 (registers)
  constexpr int NB = D == 512 ? 1 : 2;
  PfRaw<D, F32> rawA, rawB;
  pf_load<D, F32>(rawA, p, row0, lo, last, w, kb0, wv, kv0);
  if constexpr (NB == 2) pf_load<D, F32>(rawB, p, row0, min(lo + kPfKeys, last), last, w, kb0, wv, kv0);

  float m_run = -INFINITY, l_run = 0.0f;
  v4f o[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b) o[b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  auto tile = [&](PfRaw<D, F32>& raw, int it) {
    const int t0 = lo + it * kPfKeys;
    __syncthreads();  // every wave is done with the previous tile's LDS
    // ---- dequantize this thread's K / V words into LDS ----------------------
    pf_dequant<D, F32>(raw, khi, klo, vthi, vtlo, w, kb0, wv, kv0);
    __syncthreads();
    // the words of tile it + NB go into this buffer while tiles it .. run
    pf_load<D, F32>(raw, p, row0, min(t0 + NB * kPfKeys, last), last, w, kb0, wv, kv0);

    // ---- S^T = K q^T: two 16-key halves -----------------------------------
    float sc[8];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      // K reads of four k-steps issued ahead of their products
#pragma unroll
      for (int c0 = 0; c0 < CH; c0 += 4) {
        v8h ah[4], al[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int off = (16 * half + m) * KSTR + 32 * (c0 + j) + 8 * c;
          ah[j] = *reinterpret_cast<const v8h*>(&khi[off]);
          al[j] = *reinterpret_cast<const v8h*>(&klo[off]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j], qh[c0 + j], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j], ql[c0 + j], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[j], qh[c0 + j], acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + 16 * half + 4 * c + i;
        const bool keep = row_ok && t <= last && t <= pos && (W_ == 0 || pos - t < W_);
        sc[4 * half + i] = keep ? acc[i] : -INFINITY;
      }
    }

    // ---- online softmax (log2 domain) for row m --------------------------
    float mt = sc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) mt = fmaxf(mt, sc[j]);
    mt = xor16_max(mt);
    mt = xor32_max(mt);
    const float m_new = fmaxf(m_run, mt);
    if (it == 0) {
      m_run = m_new;  // first tile: nothing accumulated yet
    } else if (__any(m_new > m_run + kLazyMax)) {
      const float f = (m_new == m_run) ? 1.0f : merge_factor(m_run, m_new);
      l_run *= f;
#pragma unroll
      for (int b = 0; b < DB; ++b) o[b] *= f;
      m_run = m_new;
    }
    __bf16 ph[8], pl[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float pw = sc[j] == -INFINITY ? 0.0f : fast_exp2(sc[j] - m_run);
      l_run += pw;
      ph[j] = static_cast<__bf16>(pw);
      pl[j] = static_cast<__bf16>(pw - static_cast<float>(ph[j]));
    }
    const v8bf bh = v8bf{ph[0], ph[1], ph[2], ph[3], ph[4], ph[5], ph[6], ph[7]};
    const v8bf bl = v8bf{pl[0], pl[1], pl[2], pl[3], pl[4], pl[5], pl[6], pl[7]};

    // ---- O^T += V^T P^T ------------------------------------------------------
    // four blocks' V^T reads issued ahead of their products (the compiler
    // otherwise keeps one block's reads in flight)
#pragma unroll
    for (int b0 = 0; b0 < DB; b0 += 4) {
      v8bf ah[4], al[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int off = (16 * (b0 + j) + m) * VSTR + 8 * c;
        ah[j] = *reinterpret_cast<const v8bf*>(&vthi[off]);
        al[j] = *reinterpret_cast<const v8bf*>(&vtlo[off]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int b = b0 + j;
        o[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[j], bh, o[b], 0, 0, 0);
        o[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[j], bl, o[b], 0, 0, 0);
        o[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[j], bh, o[b], 0, 0, 0);
      }
    }
  };
  if constexpr (NB == 2) {
    for (int it = 0; it < ntile; it += 2) {
      tile(rawA, it);
      if (it + 1 < ntile) tile(rawB, it + 1);
    }
  } else {
    for (int it = 0; it < ntile; ++it) tile(rawA, it);
  }

  // ---- normalise and store row m: dims 16 b + 4c + i -------------------------
  float l_sum = xor16_sum(l_run);
  l_sum = xor32_sum(l_sum);
  if (row_ok) {
    float* out = p.out + qrow * D;
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) out[16 * b + 4 * c + i] = normalise(o[b][i], l_sum, 0.0f);
  }
}

// ---- wave-specialised variant (D = 128, 256) ------------------------------
// The kernel above has every wave dequantize its share of a tile, wait at a
// barrier, then run its matrix-core products: at one workgroup per CU the
// two phases never overlap.  Here eight waves (two per SIMD) split them:
// loader waves 0-3 dequantize tile st + 1 into one of two LDS image slots
// while compute waves 4-7 run tile st from the other; one barrier per step.
// Both roles pass the same number of barriers (an even number of steps;
// a step past the last tile dequantizes clamped rows, whose scores the
// mask drops).  Two slots take 146 KB at D = 256, so D = 512 keeps the
// kernel above.
template <int D, bool F32>
__global__ __launch_bounds__(2 * kPfThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_int4_ws_kernel(SdpaParams p) {
  pin_args(p);
  using Gm = PfGeom<D>;
  constexpr int W = Gm::W, KSTR = Gm::KSTR, VSTR = Gm::VSTR, CH = Gm::CH, DB = Gm::DB;
  constexpr int KPT = Gm::KPT;
  constexpr int KI = kPfKeys * KSTR, VI = D * VSTR;  // halves per K / V^T image
  static_assert(CH % 4 == 0 && DB % 4 == 0, "reads are issued four k-steps / blocks ahead");
  __shared__ __attribute__((aligned(16))) _Float16 khi[2][KI], klo[2][KI];
  __shared__ __attribute__((aligned(16))) __bf16 vthi[2][VI], vtlo[2][VI];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const bool loader = wave < kPfWaves;
  const int m = lane & 15, c = lane >> 4;
  const int kvh = blockIdx.y;
  const int gqa = p.gqa;
  const int qpw = kPfRows / gqa;          // queries per workgroup
  const int q0 = blockIdx.x * qpw;        // first query of this workgroup
  const int q_last = min(q0 + qpw, p.nq) - 1;
  const int W_ = p.window;
  const int lo = W_ > 0 ? max(0, p.n + q0 + 1 - W_) : 0;  // union of the rows' key ranges
  const int hi = p.n + q_last + 1;
  const int last = hi - 1;
  const int ntile = (hi - lo + kPfKeys - 1) / kPfKeys;
  const int nt2 = ntile + (ntile & 1);
  const int64_t row0 = static_cast<int64_t>(kvh) * p.cap;

  if (loader) {
    // ================= loaders: raw words -> LDS images ======================
    const int tid = threadIdx.x;
    constexpr int KB = kPfKeys / KPT;
    const int w = tid % W, kb0 = (tid / W) * KPT;
    const int wv = tid / KB, kv0 = (tid % KB) * KPT;
    PfRaw<D, F32> rawA, rawB;
    pf_load<D, F32>(rawA, p, row0, lo, last, w, kb0, wv, kv0);
    for (int st = 0; st < nt2; st += 2) {
      pf_load<D, F32>(rawB, p, row0, min(lo + (st + 1) * kPfKeys, last), last, w, kb0, wv, kv0);
      pf_dequant<D, F32>(rawA, khi[0], klo[0], vthi[0], vtlo[0], w, kb0, wv, kv0);
      __syncthreads();
      pf_load<D, F32>(rawA, p, row0, min(lo + (st + 2) * kPfKeys, last), last, w, kb0, wv, kv0);
      pf_dequant<D, F32>(rawB, khi[1], klo[1], vthi[1], vtlo[1], w, kb0, wv, kv0);
      __syncthreads();
    }
    __syncthreads();  // the compute waves' last tile
    return;
  }

  // =================== compute waves: S^T, softmax, O^T ======================
  // the compute waves bind each step: they win issue over the loader waves
  // sharing their SIMDs
  __builtin_amdgcn_s_setprio(3);
  // this lane's row (column m of its wave): query q0 + r / gqa, head r % gqa
  const int r = 16 * (wave - kPfWaves) + m;
  const int qo = r / gqa, ho = r - qo * gqa;
  const bool row_ok = q0 + qo <= q_last;
  const int qi = min(q0 + qo, q_last);
  const int pos = p.n + qi;               // absolute position of the query
  const int64_t qrow = static_cast<int64_t>(qi) * p.Hq + kvh * gqa + ho;

  // q of this lane's row: dims 32 ch + 8c .. +7, fp16 hi / lo
  v8h qh[CH], ql[CH];
#pragma unroll
  for (int ch = 0; ch < CH; ++ch) {
    float f[8];
    const int64_t e0 = qrow * D + 32 * ch + 8 * c;
    if (p.q_dtype == TQ_F32) {
      const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + e0);
      const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + e0 + 4);
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else {
      const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.q) + e0);
      const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t a = wd[i] & 0xFFFFu, b = wd[i] >> 16;
        f[2 * i] = p.q_dtype == TQ_F16 ? h2f(a) : __uint_as_float(static_cast<uint32_t>(a) << 16);
        f[2 * i + 1] = p.q_dtype == TQ_F16 ? h2f(b) : __uint_as_float(static_cast<uint32_t>(b) << 16);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = f[i] * p.scale_log2;
      const _Float16 h = static_cast<_Float16>(x);
      qh[ch][i] = h;
      ql[ch][i] = static_cast<_Float16>(x - static_cast<float>(h));
    }
  }

  float m_run = -INFINITY, l_run = 0.0f;
  v4f o[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b) o[b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  auto tile = [&](const _Float16* kh_, const _Float16* kl_, const __bf16* vh_, const __bf16* vl_, int it) {
    const int t0 = lo + it * kPfKeys;
    // ---- S^T = K q^T: two 16-key halves -----------------------------------
    float sc[8];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      // K reads of four k-steps issued ahead of their products
#pragma unroll
      for (int c0 = 0; c0 < CH; c0 += 4) {
        v8h ah[4], al[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int off = (16 * half + m) * KSTR + 32 * (c0 + j) + 8 * c;
          ah[j] = *reinterpret_cast<const v8h*>(&kh_[off]);
          al[j] = *reinterpret_cast<const v8h*>(&kl_[off]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j], qh[c0 + j], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j], ql[c0 + j], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[j], qh[c0 + j], acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + 16 * half + 4 * c + i;
        const bool keep = row_ok && t <= last && t <= pos && (W_ == 0 || pos - t < W_);
        sc[4 * half + i] = keep ? acc[i] : -INFINITY;
      }
    }
    // ---- online softmax (log2 domain) for row m --------------------------
    float mt = sc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) mt = fmaxf(mt, sc[j]);
    mt = xor16_max(mt);
    mt = xor32_max(mt);
    const float m_new = fmaxf(m_run, mt);
    if (it == 0) {
      m_run = m_new;  // first tile: nothing accumulated yet
    } else if (__any(m_new > m_run + kLazyMax)) {
      const float f = (m_new == m_run) ? 1.0f : merge_factor(m_run, m_new);
      l_run *= f;
#pragma unroll
      for (int b = 0; b < DB; ++b) o[b] *= f;
      m_run = m_new;
    }
    __bf16 ph[8], pl[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float pw = sc[j] == -INFINITY ? 0.0f : fast_exp2(sc[j] - m_run);
      l_run += pw;
      ph[j] = static_cast<__bf16>(pw);
      pl[j] = static_cast<__bf16>(pw - static_cast<float>(ph[j]));
    }
    const v8bf bh = v8bf{ph[0], ph[1], ph[2], ph[3], ph[4], ph[5], ph[6], ph[7]};
    const v8bf bl = v8bf{pl[0], pl[1], pl[2], pl[3], pl[4], pl[5], pl[6], pl[7]};
    // ---- O^T += V^T P^T ------------------------------------------------------
    // four blocks' V^T reads issued ahead of their products (the compiler
    // otherwise keeps one block's reads in flight)
#pragma unroll
    for (int b0 = 0; b0 < DB; b0 += 4) {
      v8bf ah[4], al[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int off = (16 * (b0 + j) + m) * VSTR + 8 * c;
        ah[j] = *reinterpret_cast<const v8bf*>(&vh_[off]);
        al[j] = *reinterpret_cast<const v8bf*>(&vl_[off]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int b = b0 + j;
        o[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[j], bh, o[b], 0, 0, 0);
        o[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[j], bl, o[b], 0, 0, 0);
        o[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[j], bh, o[b], 0, 0, 0);
      }
    }
  };

  __syncthreads();  // tile 0 is in slot 0
  for (int st = 0; st < nt2; st += 2) {
    tile(khi[0], klo[0], vthi[0], vtlo[0], st);
    __syncthreads();
    tile(khi[1], klo[1], vthi[1], vtlo[1], st + 1);
    __syncthreads();
  }

  // ---- normalise and store row m: dims 16 b + 4c + i -------------------------
  float l_sum = xor16_sum(l_run);
  l_sum = xor32_sum(l_sum);
  if (row_ok) {
    float* out = p.out + qrow * D;
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) out[16 * b + 4 * c + i] = normalise(o[b][i], l_sum, 0.0f);
  }
}

template <bool F32>
void launch_tiles(const SdpaParams& p, int D, bool ws, dim3 grid, hipStream_t s) {
  if (D == 128 && ws) prefill_int4_ws_kernel<128, F32><<<grid, 2 * kPfThreads, 0, s>>>(p);
  else if (D == 256 && ws) prefill_int4_ws_kernel<256, F32><<<grid, 2 * kPfThreads, 0, s>>>(p);
  else if (D == 128) prefill_int4_kernel<128, F32><<<grid, kPfThreads, 0, s>>>(p);
  else if (D == 256) prefill_int4_kernel<256, F32><<<grid, kPfThreads, 0, s>>>(p);
  else prefill_int4_kernel<512, F32><<<grid, kPfThreads, 0, s>>>(p);
}

}  // namespace

// Returns -1 when the tile kernel does not serve the shape (the caller then
// runs the split-K decode kernels in prefill mode).
bool prefill_tiles_serve(int D, int sb_dtype, int gqa) {
  if ((sb_dtype != TQ_F16 && sb_dtype != TQ_F32) || (D != 128 && D != 256 && D != 512)) return false;
  return gqa >= 1 && gqa <= kPfRows && kPfRows % gqa == 0;
}

int launch_prefill_tiles(const SdpaParams& p, int D, int sb_dtype, hipStream_t s) {
  if (!prefill_tiles_serve(D, sb_dtype, p.gqa)) return -1;
  const int qpw = kPfRows / p.gqa;
  dim3 grid((p.nq + qpw - 1) / qpw, p.Hkv);
  // TQ_PREFILL_WS=0 selects the one-role kernel at D 128 / 256
  const bool ws = options().prefill_ws;
  if (sb_dtype == TQ_F32) launch_tiles<true>(p, D, ws, grid, s);
  else launch_tiles<false>(p, D, ws, grid, s);
  TQ_CHECK_LAUNCH("prefill_int4_kernel");
  return TQ_OK;
}

}  // namespace tq
