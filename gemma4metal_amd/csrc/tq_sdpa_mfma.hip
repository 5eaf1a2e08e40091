// Fused int4-KV decode attention on the CDNA4 matrix cores (gfx950).
//
// Same contract, work split and finalisation as the VALU kernel in
// tq_sdpa.hip (replaces sdpa_int4_vector, lib/turboquant.metal:723-889); the
// difference is where the multiply-accumulates run.  Each wave64 consumes 32
// keys per iteration:
//
// K . q  -- v_mfma_i32_16x16x64_i8.  A = 16 keys x 64 dims of nibbles as int8
//   (two ANDs and a shift split a word into 8 int8 lanes), B = q as three
//   signed base-256 digits of round(q * 2^F) (22-bit fixed point per head) in
//   16 columns (head h, quant group g); each B column is zero outside its
//   group's dims, so C[key][(h,g)] is the exact integer partial dot of group g.
//   The fp32 score is sum_g s_g * 2^-F * dot_g + b_g * sum(q over g), the
//   (h,g) columns being folded with a DPP butterfly.
// P . V  -- v_mfma_f32_16x16x32_bf16.  A = 16 dims x 32 keys, built by
//   v_perm_b32 gathering one byte of two keys' words and an and-or with the
//   bf16 magic 0x4300 (128 + nibble); B = the softmax weights p*s_v split
//   into bf16 hi + lo parts (~16 bits), again in (h,g) columns.  bf16 keeps
//   fp32's exponent range, so no V scale can overflow the weights.  The 128
//   offset is removed at the end from the running sum of the weights.
//
// Lane roles (l = lane, m = l % 16, c = l / 16; layouts checked on hardware):
//   A rows / B cols / C cols = m;  k-slot j of lane-group c is k = 8c + j
//   (bf16) or 16c + 4v + byte (i8);  C rows held by lane-group c: 4c .. 4c+3.
//   Key of V slot j in lane-group c: r0 + 16*(j/4) + 4c + (j%4) (r0 = first
//   row of the iteration's 32-row block), which is the
//   K tile (j/4), C row 4c + (j%4): the softmax weights are produced by the
//   K MFMAs exactly in the lanes and slots the V MFMAs consume them from.
//
// Scale/bias of 32 keys are staged through 1 KB of LDS per wave, transposed
// to [array][group][key] so each lane reads its 8 values with two 8 B reads.
// Loads are double-buffered one iteration (9 KB per wave) ahead.
#include <type_traits>

#include "tq_sdpa_common.h"

namespace tq {
namespace {

// Waves per workgroup: 8 = two waves per SIMD at one workgroup per CU.
constexpr int kMfmaWaves = 8;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

template <int D, int G, bool F32>
struct MGeom {
  static constexpr int NG = D / 64;     // quant groups per row
  static constexpr int COLS = G * NG;   // used MFMA columns
  static constexpr int KW = D / 32;     // K words per lane per key (D/8 bytes)
  static constexpr int KM = D / 64;     // int8 MFMAs per 16-key tile (2 words each)
  static constexpr int VW = D / 128;    // V words per lane per key
  // V split: at D = 512 a pair of waves takes the same keys, each wave
  // accumulating half of every lane's V words (registers for two buffers
  // and the accumulators then fit two waves per SIMD)
  static constexpr int VS = D == 512 ? 2 : 1;
  static constexpr int VWH = VW / VS;   // V words per lane per key of one wave
  static constexpr int VM = 8 * VWH;    // P.V accumulator tiles of one wave
  // 32-bit words of one key's scales (or biases): fp16 pairs, or fp32
  static constexpr int SCW = F32 ? NG : NG / 2;
  // Packed columns: with at most 8 (head, group) columns, the two 16-key
  // tiles of an iteration share one K accumulator (tile 0 in columns 0-7,
  // tile 1 in columns 8-15), and the P.V weights' bf16 hi and lo parts go
  // to columns n and n + 8 of one product (one product per A tile instead
  // of two).  Every score-epilogue lane then holds a used column.
  static constexpr bool PACK = COLS <= 8 && VS == 1;
  static_assert(COLS <= 16, "more than 16 (head, group) columns");
  static_assert(D == 128 || D == 256 || D == 512, "D");
};

template <int D, bool F32>
struct IterBuf {
  uint32_t kw[2][D / 32];   // [tile][word] K slice of key (r0 + 16*tile + m)
  uint32_t vw[8][D / 128 / (D == 512 ? 2 : 1)];  // [slot][word] this wave's V words of key(slot)
  uint32_t sc[2][F32 ? D / 64 : D / 128];  // scales of keys (r0 + 2k, r0 + 2k + 1) of array l/16
};

// Per-lane byte offsets inside one 32-key block, from its first row: K row
// m (tile 0; tile 1 adds 16 rows), V row 4c (slot j adds 16 * (j / 4) +
// j % 4 rows), and this lane's scale key pair.  Constant over the stream:
// an iteration moves the uniform block base only.
struct LaneOffs {
  uint32_t k, v, s;
};

// One streamed load: non-temporal when kNT (single sequences: ~7% more HBM
// throughput than default-policy loads at 256k keys), default policy
// otherwise (batched ragged launches read 8% faster with it).
template <bool kNT, typename T>
__device__ __forceinline__ T stream_load(const T* p) {
  if constexpr (kNT) return __builtin_nontemporal_load(p);
  else return *p;
}

// Loads of the 32-row block starting at row `r0` (uniform): each load is
// the block's base (scalar registers) plus a constant lane offset and an
// immediate row offset, so an iteration spends no vector instructions on
// addresses.  The caller keeps rows r0 .. r0 + 31 inside the cache
// (block_row).  In three parts, in the order the products consume them:
// 0 = scales and K, 1 = V slots 0-3, 2 = V slots 4-7.
template <int PART, int D, int G, bool F32, bool kNT>
__device__ __forceinline__ void load_part(IterBuf<D, F32>& B, const uint32_t* kq_row0,
                                          const uint32_t* vq_row0, const uint32_t* sc_arr,
                                          const LaneOffs& lo, int r0) {
  using Gm = MGeom<D, G, F32>;
  constexpr uint32_t RB = D / 2;  // bytes per packed row
  // (uniform base + zero-extended lane offset, then the constant row offset
  // as a separate addition: the form the compiler folds into the
  // instruction's scalar base, vector offset and immediate)
  if constexpr (PART == 0) {
    const char* sb = reinterpret_cast<const char*>(sc_arr + static_cast<int64_t>(r0) * Gm::SCW) + lo.s;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const char* a = sb + e * (Gm::SCW * 4);
      if constexpr (Gm::SCW >= 4) {
#pragma unroll
        for (int w = 0; w < Gm::SCW; w += 4) {
          const u32x4 u = stream_load<kNT>(reinterpret_cast<const u32x4*>(a + 4 * w));
          B.sc[e][w] = u.x; B.sc[e][w + 1] = u.y; B.sc[e][w + 2] = u.z; B.sc[e][w + 3] = u.w;
        }
      } else if constexpr (Gm::SCW == 2) {
        const u32x2 u = stream_load<kNT>(reinterpret_cast<const u32x2*>(a));
        B.sc[e][0] = u.x; B.sc[e][1] = u.y;
      } else {
        B.sc[e][0] = stream_load<kNT>(reinterpret_cast<const uint32_t*>(a));
      }
    }
    const char* kb = reinterpret_cast<const char*>(kq_row0 + static_cast<int64_t>(r0) * (D / 8)) + lo.k;
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
#pragma unroll
      for (int w = 0; w < Gm::KW; w += 4) {
        const u32x4 u = stream_load<kNT>(reinterpret_cast<const u32x4*>(kb + (tile * 16 * RB + w * 4)));
        B.kw[tile][w] = u.x; B.kw[tile][w + 1] = u.y; B.kw[tile][w + 2] = u.z; B.kw[tile][w + 3] = u.w;
      }
    }
  } else {
    const char* vb = reinterpret_cast<const char*>(vq_row0 + static_cast<int64_t>(r0) * (D / 8)) + lo.v;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = 4 * (PART - 1) + jj;
      const char* a = vb + (16 * (j >> 2) + (j & 3)) * RB;
      if constexpr (Gm::VWH == 4) {
        const u32x4 u = stream_load<kNT>(reinterpret_cast<const u32x4*>(a));
        B.vw[j][0] = u.x; B.vw[j][1] = u.y; B.vw[j][2] = u.z; B.vw[j][3] = u.w;
      } else if constexpr (Gm::VWH == 2) {
        const u32x2 u = stream_load<kNT>(reinterpret_cast<const u32x2*>(a));
        B.vw[j][0] = u.x; B.vw[j][1] = u.y;
      } else {
        B.vw[j][0] = stream_load<kNT>(reinterpret_cast<const uint32_t*>(a));
      }
    }
  }
}

template <int D, int G, bool F32, bool kNT>
__device__ __forceinline__ void load_iter(IterBuf<D, F32>& B, const uint32_t* kq_row0,
                                          const uint32_t* vq_row0, const uint32_t* sc_arr,
                                          const LaneOffs& lo, int r0) {
  load_part<0, D, G, F32, kNT>(B, kq_row0, vq_row0, sc_arr, lo, r0);
  load_part<1, D, G, F32, kNT>(B, kq_row0, vq_row0, sc_arr, lo, r0);
  load_part<2, D, G, F32, kNT>(B, kq_row0, vq_row0, sc_arr, lo, r0);
}

__device__ __forceinline__ float half_lo(uint32_t w) {
  return __half2float(__ushort_as_half(static_cast<uint16_t>(w & 0xFFFFu)));
}
__device__ __forceinline__ float half_hi(uint32_t w) {
  return __half2float(__ushort_as_half(static_cast<uint16_t>(w >> 16)));
}

// D = 512: 4-wave workgroups at one wave per SIMD (VGPRs + AGPRs for the
// doubled K buffers and scales).
// kQG: prefill with query groups -- the G column sets are G / p.pq heads x
// p.pq consecutive queries, each column with its own causal / window limit.
// Decode and single-query prefill use kQG = false.
// kStreamNT: non-temporal K/V loads (see stream_load).
// F32: fp32 scale/bias (the reference's cache dtype); fp16 otherwise.
template <int D, int G, int NW, bool kQG, bool kStreamNT, bool F32>
__global__ __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(D == 512 ? 1 : 2, D == 512 ? 1 : 2)))
void sdpa_int4_mfma_kernel(SdpaParams p) {
  constexpr int kNT = NW * 64;       // threads per workgroup
  using Gm = MGeom<D, G, F32>;
  constexpr int kIter = 32 * (NW / Gm::VS);  // keys per workgroup iteration
  constexpr int NG = Gm::NG, COLS = Gm::COLS, KM = Gm::KM, VW = Gm::VW, VM = Gm::VM;
  constexpr int VS = Gm::VS, VWH = Gm::VWH;
  constexpr bool PACK = Gm::PACK;
  constexpr int NTB = PACK ? 2 : 1;      // B-operand images of the K products
  constexpr int SKP = F32 ? 32 : 16;     // staged scale slots per (array, group)
  constexpr int NWK = NW / VS;       // waves per key stream
  constexpr int RW = D / 8;
  // K.q B image: word (k, i, n, ccl) = ((k * KM + i) * QCOL + n) * QCC + ccl
  // holds the 16 k-slots of digit k, MFMA i, column n, for the ccl-th lane
  // group whose dims lie in column n's quant group (D 128: lane groups 2g,
  // 2g + 1; D 256: g; D 512: g / 2, zero for the MFMAs of the other group).
  constexpr int QCOL = PACK ? 8 : 16;
  constexpr int QCC = D == 128 ? 2 : 1;
  constexpr int QWORDS = 3 * KM * QCOL * QCC;
  constexpr int NCH = (G * D + 511) / 512;  // 8-element q chunks per lane

  pin_args(p);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = lane & 15, c = lane >> 4;  // A row / B,C column; lane group
  // This lane's (head, group) column, and with packed columns the key tile
  // of its scores (tile T's keys in C columns 8T .. 8T + 7) and the weight
  // part it feeds the P.V products (0: bf16 hi, 1: bf16 lo).
  const int n = PACK ? (m & 7) : m;
  const int T = PACK ? (m >> 3) : 0;
  const int hn = n / NG, gn = n - (n / NG) * NG;
  const bool col_used = n < COLS;
  int b = blockIdx.z, hy = blockIdx.y, split = blockIdx.x;
  // Longest-first ragged order: batched launches only (single-sequence and
  // grouped-prefill launches never set lpt).
  if constexpr (!kQG && !kStreamNT) {
    if (p.lpt) {
      int chunk = p.chunk;
      const bool job = ragged_job(p, b, hy, split, chunk);
      // Every lane computes the same job; read back as wave-uniform values
      // so that the split range, the key offsets and the load addresses
      // derived from them stay in scalar registers.
      if (!__builtin_amdgcn_readfirstlane(job)) return;
      b = __builtin_amdgcn_readfirstlane(b);
      hy = __builtin_amdgcn_readfirstlane(hy);
      split = __builtin_amdgcn_readfirstlane(split);
      p.chunk = __builtin_amdgcn_readfirstlane(chunk);  // this launch's chunk, chosen from the lengths
    }
  }
  const int kvh = hy / p.n_sub, sub = hy - kvh * p.n_sub;
  // The G column sets are GH heads x pq queries: pq = 1 unless kQG (b is
  // then the query group of queries b0 .. b_last).
  const int pq = kQG ? p.pq : 1;
  const int GH = kQG ? G / pq : G;
  const int h0 = kvh * p.gqa + sub * GH;
  const int b0 = b * pq;
  const int b_last = kQG ? min(b0 + pq - 1, p.nq - 1) : b;

  const SplitRange rg = kQG ? prefill_range(p, b0, b_last, split) : split_range(p, b, split);
  if (split >= rg.S) return;
  const int t_begin = rg.t_begin, t_end = rg.t_end;
  // this column's causal / window limits (the queries of a group differ)
  const int pos = p.n + b0 + (hn / GH);
  const int col_hi = pos;
  const int col_lo = p.window > 0 ? pos - p.window + 1 : 0;

  // One partial result per wave; with packed columns a wave leaves its hi-
  // and lo-part rows and their corrections as two slots, which the
  // workgroup combine sums (a lane holds 64 values of one column part; a
  // cross-lane sum and a correction per value in every wave would cost
  // ~200 instructions on the workgroup's critical path).
  using Fin = Finalize<G, D, NW, NW * 64, PACK ? 2 : 1, PACK>;
  __shared__ __align__(16) float arena[Fin::kArena];
  // scales staged per wave as [array][group][key pair] fp16x2, or
  // [array][group][key] fp32
  __shared__ __align__(16) uint32_t sc_lds[NW][4][NG][SKP];
  // B operands of the K MFMAs: one compact image per wave (built by the wave
  // itself, see the prologue), and one all-zero image of the same layout
  // ([NW]) that lanes read where their column has no digits.
  __shared__ __align__(16) uint4 qimg[NW + 1][QWORDS];
  // iterations processed, per wave (issue pacing; each wave zeroes its own
  // entry, and a partner's read before that only sets an issue priority)
  __shared__ int s_done[NW];
  if ((threadIdx.x & 63) == 0) s_done[threadIdx.x >> 6] = 0;

  // ---- first loads, issued before the prologue to overlap its latency ------
  const int64_t row0 = (static_cast<int64_t>(cache_batch(p, b)) * p.Hkv + kvh) * p.cap;
  const uint32_t* kq_row0 = p.kq + row0 * RW;
  const uint32_t* vq_row0 = p.vq + row0 * RW;
  // (a select chain over kernel-argument pointers keeps the global address
  // space visible: a lane-indexed pointer table would turn these into FLAT
  // loads, which the waitcnt logic cannot order and drains with vmcnt(0))
  const int arr = lane >> 4, k16 = lane & 15;  // this lane's scale array / key pair
  const void* sc_base = arr == 0 ? p.ks : (arr == 1 ? p.kb : (arr == 2 ? p.vs : p.vb));
  const uint32_t* sc_arr = static_cast<const uint32_t*>(sc_base) + row0 * Gm::SCW;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  // wave wv streams keys with the NWK waves of its V half (wv / NWK)
  const int vhalf = VS == 1 ? 0 : wv / NWK;  // (a constant without a V split)
  LaneOffs lo;
  lo.k = m * (D / 2) + c * Gm::KW * 4;
  lo.v = 4 * c * (D / 2) + (m * Gm::VW + vhalf * Gm::VWH) * 4;
  lo.s = 2 * k16 * Gm::SCW * 4;
  const int base0 = t_begin + (wv - vhalf * NWK) * 32;
  const int nit = base0 < t_end ? (t_end - base0 + kIter - 1) / kIter : 0;
  // First row of the 32-row block read for the iteration at key t0: t0
  // itself while the block lies below t_end; else moved back to end at
  // t_end (rows of the sequence, the keys before t0 masked in process), and
  // to row 0 for sequences shorter than 32 keys, whose rows [t_end, 32) lie
  // past the sequence (process zeroes their scales and biases).  Rows stay
  // in [0, max(t_end, 32)), inside the cache: the planner gives this kernel
  // capacities of at least 32 rows.  Wave-uniform (scalar).
  auto block_row = [&](int t0) { return max(0, min(t0, t_end - 32)); };

  // q is loaded first, then the first block's K/V, which stay in flight
  // while the prologue runs.  Every wave loads all G * D q elements of its
  // column sets (8 per lane and chunk: one or two 16-byte loads, the same
  // two loads for every dtype, so no branch separates them from the K/V
  // loads and the prologue's wait covers q only).
  uint4 qa[NCH], qb[NCH];
  const bool q32 = p.q_dtype == TQ_F32;
#pragma unroll
  for (int s = 0; s < NCH; ++s) {
    // chunk ch: elements 8 ch .. 8 ch + 7 of column set v = 8 ch / D, i.e.
    // query min(b0 + v / GH, b_last), head h0 + v % GH (clamped chunks are
    // dropped below)
    const int ch = min(lane + 64 * s, G * D / 8 - 1);
    const int v = 8 * ch / D;
    const int64_t qrow = static_cast<int64_t>(min(b0 + v / GH, b_last)) * p.Hq + h0 + v % GH;
    const char* qp = static_cast<const char*>(p.q) + (qrow * D + (8 * ch - v * D)) * (q32 ? 4 : 2);
    qa[s] = *reinterpret_cast<const uint4*>(qp);
    qb[s] = *reinterpret_cast<const uint4*>(qp + (q32 ? 16 : 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  // Issued unconditionally (a load under a branch makes the compiler drain
  // every outstanding load at the join): block_row keeps the rows of a wave
  // or split with no keys inside the cache.
  // 4-wave workgroups (one wave per SIMD, short splits) issue only the
  // first block's scales and K rows here and its V rows after the prologue:
  // the K rows every wave's first products need reach the CU's address unit
  // first (sliding layer 7.73 -> 7.43 us; no gain at 8 waves)
  constexpr bool kLateV = NW == 4 && VS == 1;
  IterBuf<D, F32> bufA, bufB;
  if constexpr (kLateV)
    load_part<0, D, G, F32, kStreamNT>(bufA, kq_row0, vq_row0, sc_arr, lo, block_row(base0));
  else
    load_iter<D, G, F32, kStreamNT>(bufA, kq_row0, vq_row0, sc_arr, lo, block_row(base0));
  __builtin_amdgcn_sched_barrier(0);

  // ---- prologue: q as 22-bit fixed point per column set, B image per wave ---
  // Each wave builds the whole image it reads, so no barrier orders the
  // prologue: a wave starts its stream as soon as its own q has arrived.
  // The digits equal those of one image shared by the workgroup (the
  // exponent F is the column set's, from its maximum over all D dims).
  {
    uint4* zi = &qimg[wv][0];
    uint4* zz = &qimg[NW][0];  // every wave writes the same zeros here
#pragma unroll
    for (int i = lane; i < QWORDS; i += 64) {
      zi[i] = uint4{0u, 0u, 0u, 0u};
      zz[i] = uint4{0u, 0u, 0u, 0u};
    }
  }
  int Fs[NCH];
  float qhs[NCH];
#pragma unroll
  for (int s = 0; s < NCH; ++s) {
    const int ch = lane + 64 * s;
    const bool ok = ch < G * D / 8;
    // (one uniform dtype branch per chunk, straight-line conversions inside)
    float f[8];
    if (q32) {
      const uint32_t w[8] = {qa[s].x, qa[s].y, qa[s].z, qa[s].w, qb[s].x, qb[s].y, qb[s].z, qb[s].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = __uint_as_float(w[e]);
    } else if (p.q_dtype == TQ_F16) {
      const uint32_t w[4] = {qa[s].x, qa[s].y, qa[s].z, qa[s].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[2 * e] = half_lo(w[e]);
        f[2 * e + 1] = half_hi(w[e]);
      }
    } else {
      const uint32_t w[4] = {qa[s].x, qa[s].y, qa[s].z, qa[s].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[2 * e] = __uint_as_float(w[e] << 16);
        f[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = ok ? f[e] * p.scale_log2 : 0.0f;
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[e]));
    // the column set's D / 8 chunks are D / 8 consecutive lanes of one slot
    amax = group_max<(D / 8 < 64 ? D / 8 : 64)>(amax);
    int ex = 0;
    if (amax > 0.0f) frexpf(amax, &ex);  // amax < 2^ex
    const int F = 22 - ex;               // |round(q * 2^F)| <= 2^22
    const float sF = ldexpf(1.0f, F);
    // three signed base-256 digits per element: the low byte of X, then of
    // X1 = (X - sext(byte)) / 256, then of X2 = (X1 - sext(byte)) / 256
    uint32_t dg[3][8];
    int xs = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int X = static_cast<int>(__builtin_rintf(f[e] * sF));
      xs += X;
      const int X1 = (X - __builtin_amdgcn_sbfe(X, 0, 8)) >> 8;
      const int X2 = (X1 - __builtin_amdgcn_sbfe(X1, 0, 8)) >> 8;
      dg[0][e] = static_cast<uint32_t>(X);
      dg[1][e] = static_cast<uint32_t>(X1);
      dg[2][e] = static_cast<uint32_t>(X2);
    }
    // sum over the quant group's 64 dims (8 lanes), exact: 64 * 2^22 < 2^31
    xs = group_sum_i<8>(xs);
    Fs[s] = F;
    qhs[s] = static_cast<float>(xs) * ldexpf(1.0f, -F);
    // the low bytes of elements 0, 2, 4, 6 (even) and 1, 3, 5, 7 (odd) form
    // two dwords of the 16 k-slots of this chunk's MFMA, lane group and
    // column (three byte permutes per dword)
    uint32_t ev[3], od[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const uint32_t e02 = __builtin_amdgcn_perm(dg[k][2], dg[k][0], 0x0C0C0400u);
      const uint32_t e46 = __builtin_amdgcn_perm(dg[k][6], dg[k][4], 0x0C0C0400u);
      const uint32_t o13 = __builtin_amdgcn_perm(dg[k][3], dg[k][1], 0x0C0C0400u);
      const uint32_t o57 = __builtin_amdgcn_perm(dg[k][7], dg[k][5], 0x0C0C0400u);
      ev[k] = __builtin_amdgcn_perm(e46, e02, 0x05040100u);
      od[k] = __builtin_amdgcn_perm(o57, o13, 0x05040100u);
    }
    if (ok) {
      const int v = 8 * ch / D, dim0 = 8 * ch - v * D;
      const int nn = v * NG + dim0 / 64;                       // column
      const int cc = dim0 / (D / 4), off = dim0 - cc * (D / 4);  // lane group, k-slot offset
      const int i = off >> 4, half = (off >> 3) & 1;
      char* w0 = reinterpret_cast<char*>(&qimg[wv][(i * QCOL + nn) * QCC + cc % QCC]) + 8 * half;
#pragma unroll
      for (int k = 0; k < 3; ++k)
        *reinterpret_cast<uint2*>(w0 + k * (KM * QCOL * QCC * 16)) = uint2{ev[k], od[k]};
    }
  }
  // this lane's column: its set's exponent and the group's sum of q, from the
  // lane holding the group's first chunk
  float sf = 0.0f, qhat = 0.0f;
  {
    const int chn = col_used ? (hn * D + 64 * gn) / 8 : 0;
#pragma unroll
    for (int s = 0; s < NCH; ++s) {
      const int Fv = __shfl(Fs[s], chn & 63, 64);
      const float qv = __shfl(qhs[s], chn & 63, 64);
      if ((chn >> 6) == s && col_used) {
        sf = ldexpf(1.0f, -Fv);
        qhat = qv;
      }
    }
  }
  // B operand addresses of this lane, per key tile: its wave's image where
  // its (column, lane group) pair carries digits, else the zero image
  const uint4* bq_addr[NTB];
  {
    const bool grp = D == 128 ? (c >> 1) == gn : (D == 256 ? c == gn : c == (gn >> 1));
    const int wofs = n * QCC + (D == 128 ? (c & 1) : 0);
#pragma unroll
    for (int t = 0; t < NTB; ++t) {
      const bool has = col_used && grp && (!PACK || T == t);
      bq_addr[t] = &qimg[has ? wv : NW][wofs];
    }
  }

  if constexpr (kLateV) {
    __builtin_amdgcn_sched_barrier(0);
    load_part<1, D, G, F32, kStreamNT>(bufA, kq_row0, vq_row0, sc_arr, lo, block_row(base0));
    load_part<2, D, G, F32, kStreamNT>(bufA, kq_row0, vq_row0, sc_arr, lo, block_row(base0));
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- main loop ----------------------------------------------------------
  float m_run = -INFINITY, l_run = 0.0f, wsum = 0.0f, bacc = 0.0f;
  v4f cv[VM];
#pragma unroll
  for (int f = 0; f < VM; ++f) cv[f] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // bf16 magic of (128 + nibble), kept in a VGPR so each A-operand word is
  // one v_and_or_b32 (a gfx9 VOP3 instruction takes at most one literal/SGPR)
  uint32_t magic = 0x43004300u;
  asm volatile("" : "+v"(magic));

  // The 4 staged scales of array a, group g, keys 16 * tile + 4c + {0..3}.
  auto scale4 = [&](int a, int g, int tile) -> v4f {
    if constexpr (F32) {
      return *reinterpret_cast<const v4f*>(&sc_lds[wv][a][g][16 * tile + 4 * c]);
    } else {
      const uint2 u = *reinterpret_cast<const uint2*>(&sc_lds[wv][a][g][8 * tile + 2 * c]);
      return v4f{half_lo(u.x), half_hi(u.x), half_lo(u.y), half_hi(u.y)};
    }
  };

  // `issue(part)` puts out part 0, 1, 2 of the next block's loads at three
  // points of the products (before the scale staging, after the K MFMAs,
  // before the V products): a wave's loads go out in three smaller bursts,
  // so the waves of a CU stay closer together than with one burst of all
  // thirteen loads per iteration.
  auto process = [&](const IterBuf<D, F32>& B, int t0, auto&& issue) {
    // B holds the block of rows r0 .. r0 + 31 (r0 <= t0); its keys below t0
    // or from t_end on are masked
    const int r0 = block_row(t0);
    issue(std::integral_constant<int, 0>{});
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t n_keep = static_cast<uint32_t>(t_end - t0);  // > 0 for a processed iteration
    // This lane's scale words (keys r0 + 2 k16, r0 + 2 k16 + 1).  A sequence
    // shorter than one block reads rows [t_end, 32) too (block_row moves the
    // block to row 0): rows past the sequence, possibly never written.  Their
    // keys get zero weight, but 0 * NaN is NaN, so their scales and biases
    // are replaced by zero before any product sees them.
    uint32_t scv[2][Gm::SCW];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int w = 0; w < Gm::SCW; ++w) scv[e][w] = B.sc[e][w];
    if (t_end < 32) {  // uniform, and rare: only then can a block row pass t_end
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const bool in_seq = r0 + 2 * k16 + e < t_end;
#pragma unroll
        for (int w = 0; w < Gm::SCW; ++w) scv[e][w] = in_seq ? scv[e][w] : 0u;
      }
    }
    // scales -> LDS [array][group][key]
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if constexpr (F32) {
        *reinterpret_cast<uint2*>(&sc_lds[wv][arr][g][2 * k16]) = uint2{scv[0][g], scv[1][g]};
      } else {
        const uint32_t a0 = scv[0][g >> 1], a1 = scv[1][g >> 1];
        const uint32_t v = (g & 1) ? ((a0 >> 16) | (a1 & 0xFFFF0000u))
                                   : ((a0 & 0xFFFFu) | (a1 << 16));
        sc_lds[wv][arr][g][k16] = v;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // K . q on the int8 matrix cores.  Score slot 4*u + i of this lane is key
    // r0 + 16*tile(u) + 4c + i of column n: tile(u) = T with packed columns
    // (one score tile), u otherwise (two).
    constexpr int NU = PACK ? 1 : 2;
    float sc[4 * NU];
    auto kq_tile = [&](int tile, v4i (&acc)[3], int img) {
      // B operands live in LDS (16 B per lane per MFMA) to keep the wave
      // within 256 registers; those of half the tile's k-steps are read
      // ahead of their products (the compiler otherwise keeps two reads in
      // flight)
      constexpr int RS = KM >= 2 ? KM / 2 : 1;
#pragma unroll
      for (int i0 = 0; i0 < KM; i0 += RS) {
        uint4 bu[RS][3];
#pragma unroll
        for (int ii = 0; ii < RS; ++ii)
#pragma unroll
          for (int k = 0; k < 3; ++k) bu[ii][k] = bq_addr[img][(k * KM + i0 + ii) * QCOL * QCC];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ii = 0; ii < RS; ++ii) {
          const int i = i0 + ii;
          const uint32_t w0 = B.kw[tile][2 * i], w1 = B.kw[tile][2 * i + 1];
          const v4i a = v4i{static_cast<int>(w0 & 0x0F0F0F0Fu),
                            static_cast<int>((w0 >> 4) & 0x0F0F0F0Fu),
                            static_cast<int>(w1 & 0x0F0F0F0Fu),
                            static_cast<int>((w1 >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
          for (int k = 0; k < 3; ++k) {
            const uint4 u = bu[ii][k];
            const v4i bq = v4i{static_cast<int>(u.x), static_cast<int>(u.y), static_cast<int>(u.z),
                               static_cast<int>(u.w)};
            acc[k] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bq, acc[k], 0, 0, 0);
          }
        }
      }
    };
    // With packed columns (every lane's column used) and no per-column
    // limits, a block whose 32 rows all lie in [t0, t_end) needs no mask.
    constexpr bool kMaskAll = !PACK || kQG;
    const bool full = r0 == t0 && n_keep >= 32;  // uniform
    auto scores = [&](const v4i (&acc)[3], int u, int tile) {
      const v4f ks = scale4(0, gn, tile), kb = scale4(1, gn, tile);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // digits 0 and 1 combine exactly in int32 (|.| < 2^25)
        const int lo01 = acc[0][i] + (acc[1][i] << 8);
        const float dot = static_cast<float>(lo01) + 65536.0f * static_cast<float>(acc[2][i]);
        // (fma with + 0: the fp16 scale converts inside the multiply)
        const float kss = fmaf(ks[i], sf, 0.0f), kbq = fmaf(kb[i], qhat, 0.0f);
        float part = fmaf(dot, kss, kbq);
        part = group_sum<NG>(part);
        if constexpr (kMaskAll) {
          const int t = r0 + 16 * tile + 4 * c + i;
          // t0 <= t < t_end, as one unsigned compare
          bool keep = static_cast<uint32_t>(t - t0) < n_keep && col_used;
          if constexpr (kQG) keep = keep && t <= col_hi && t >= col_lo;
          sc[4 * u + i] = keep ? part : -INFINITY;
        } else {
          sc[4 * u + i] = part;
        }
      }
      if constexpr (!kMaskAll) {
        if (!full) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = r0 + 16 * tile + 4 * c + i;
            if (static_cast<uint32_t>(t - t0) >= n_keep) sc[4 * u + i] = -INFINITY;
          }
        }
      }
    };
    if constexpr (PACK) {
      v4i acc[3];
#pragma unroll
      for (int k = 0; k < 3; ++k) acc[k] = v4i{0, 0, 0, 0};
      kq_tile(0, acc, 0);
      kq_tile(1, acc, 1);
      __builtin_amdgcn_sched_barrier(0);
      issue(std::integral_constant<int, 1>{});
      __builtin_amdgcn_sched_barrier(0);
      scores(acc, 0, T);
    } else {
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        v4i acc[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) acc[k] = v4i{0, 0, 0, 0};
        kq_tile(tile, acc, 0);
        if (tile == 1) {
          __builtin_amdgcn_sched_barrier(0);
          issue(std::integral_constant<int, 1>{});
          __builtin_amdgcn_sched_barrier(0);
        }
        scores(acc, tile, tile);
      }
    }

    // online softmax over the 32 keys (log2 domain)
    float mt = sc[0];
#pragma unroll
    for (int j = 1; j < 4 * NU; ++j) mt = fmaxf(mt, sc[j]);
    if constexpr (PACK) mt = fmaxf(mt, ror8(mt));
    mt = xor16_max(mt);
    mt = xor32_max(mt);
    const float m_new = fmaxf(m_run, mt);
    if (t0 == base0) {
      m_run = m_new;  // first batch: nothing accumulated yet
    } else if (__any(m_new > m_run + kLazyMax)) {
      const float f = (m_new == m_run) ? 1.0f : merge_factor(m_run, m_new);
      l_run *= f;
      wsum *= f;
      bacc *= f;
#pragma unroll
      for (int ff = 0; ff < VM; ++ff) cv[ff] *= f;
      m_run = m_new;
    }
    // weights of this lane's own scores; the denominator and the V bias
    // term count each key once (the lane of its score)
    float pw[4 * NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const v4f vb = scale4(3, gn, PACK ? T : u);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // (a masked score gives 2^-inf = 0 as long as m_run is finite: with
        // packed columns every column scores every key, and a processed
        // iteration holds at least one key, so only the other forms test)
        const float pj = (PACK && !kQG) || sc[4 * u + i] != -INFINITY ? fast_exp2(sc[4 * u + i] - m_run) : 0.0f;
        pw[4 * u + i] = pj;
        l_run += pj;
        bacc = fmaf(pj, vb[i], bacc);
      }
    }
    // the weights of the P.V k-slots: slot j = key 16*(j/4) + 4c + j%4
    float ps[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (PACK) {
        const float other = ror8(pw[i]);  // the other tile's key, same column
        ps[i] = T ? other : pw[i];
        ps[4 + i] = T ? pw[i] : other;
      } else {
        ps[i] = pw[i];
        ps[4 + i] = pw[4 + i];
      }
    }
    const v4f vs0 = scale4(2, gn, 0), vs1 = scale4(2, gn, 1);
    // Weights in bf16 pairs (slots 2k, 2k + 1: one B operand word), hi part
    // and lo = w - hi, each pair converted by one packed conversion; the
    // weight sum of the 128 offset takes a word per v_dot2 with (1, 1).
    uint32_t bh[4], bl[4];
    const v2bf ones = __builtin_bit_cast(v2bf, 0x3F803F80u);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int j = 2 * k;
      // (fma with + 0: the fp16 scale converts inside the multiply)
      const float w0 = fmaf(ps[j], j < 4 ? vs0[j] : vs1[j - 4], 0.0f);
      const float w1 = fmaf(ps[j + 1], j + 1 < 4 ? vs0[j + 1] : vs1[j - 3], 0.0f);
      uint32_t hb = __builtin_bit_cast(uint32_t, v2bf{static_cast<__bf16>(w0), static_cast<__bf16>(w1)});
      asm("" : "+v"(hb));  // h0, h1 from the packed word (no second conversion of w0)
      const float h0 = __uint_as_float(hb << 16), h1 = __uint_as_float(hb & 0xFFFF0000u);
      const uint32_t lb =
          __builtin_bit_cast(uint32_t, v2bf{static_cast<__bf16>(w0 - h0), static_cast<__bf16>(w1 - h1)});
      if constexpr (PACK) {
        // column n + 8T takes part T of the weight
        bh[k] = T ? lb : hb;
        wsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, bh[k]), ones, wsum, false);
      } else {
        bh[k] = hb;
        bl[k] = lb;
        wsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, hb), ones, wsum, false);
        wsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, lb), ones, wsum, false);
      }
    }
    const v8bf bhi = __builtin_bit_cast(v8bf, u32x4{bh[0], bh[1], bh[2], bh[3]});
    const v8bf blo = __builtin_bit_cast(v8bf, u32x4{bl[0], bl[1], bl[2], bl[3]});

    __builtin_amdgcn_sched_barrier(0);
    issue(std::integral_constant<int, 2>{});
    __builtin_amdgcn_sched_barrier(0);
    // P . V on the bf16 matrix cores: A = (128 + nibble) of 16 dims x 32 keys
#pragma unroll
    for (int s = 0; s < VWH; ++s) {
#pragma unroll
      for (int by = 0; by < 4; ++by) {
        const uint32_t sel = static_cast<uint32_t>(by) | (0x0Cu << 8) |
                             (static_cast<uint32_t>(4 + by) << 16) | (0x0Cu << 24);
        uint32_t alo[4], ahi[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t x = __builtin_amdgcn_perm(B.vw[2 * r + 1][s], B.vw[2 * r][s], sel);
          alo[r] = (x & 0x000F000Fu) | magic;
          ahi[r] = ((x >> 4) & 0x000F000Fu) | magic;
        }
        const v4i ilo = v4i{static_cast<int>(alo[0]), static_cast<int>(alo[1]),
                            static_cast<int>(alo[2]), static_cast<int>(alo[3])};
        const v4i ihi = v4i{static_cast<int>(ahi[0]), static_cast<int>(ahi[1]),
                            static_cast<int>(ahi[2]), static_cast<int>(ahi[3])};
        const v8bf a_lo = __builtin_bit_cast(v8bf, ilo);
        const v8bf a_hi = __builtin_bit_cast(v8bf, ihi);
        const int fe = 8 * s + 2 * by, fo = fe + 1;
        cv[fe] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, bhi, cv[fe], 0, 0, 0);
        cv[fo] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, bhi, cv[fo], 0, 0, 0);
        if constexpr (!PACK) {
          cv[fe] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, blo, cv[fe], 0, 0, 0);
          cv[fo] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, blo, cv[fo], 0, 0, 0);
        }
      }
    }
  };

  // the next block's loads (into B, rows from key t0), issued in parts by process
  auto next_of = [&](IterBuf<D, F32>& B, int t0) {
    const int r0 = block_row(t0);
    return [&B, r0, &kq_row0, &vq_row0, &sc_arr, &lo](auto part) {
      load_part<decltype(part)::value, D, G, F32, kStreamNT>(B, kq_row0, vq_row0, sc_arr, lo, r0);
    };
  };
  auto no_loads = [](auto) {};

  auto pace = [&](int done) { pace_waves<NW>(s_done, wv, lane, done); };
  pace(0);
  // Steady state: every load in the body is for an iteration of this wave.
  // The last one or two iterations are peeled, so no load is issued past
  // the stream: the registers of such a load would have to be waited for
  // before their reuse after the loop, a full memory round trip per wave.
  int it = 0;
  for (; it + 2 < nit; it += 2) {
    process(bufA, base0 + it * kIter, next_of(bufB, base0 + (it + 1) * kIter));
    pace(it + 1);
    __builtin_amdgcn_sched_barrier(0);
    process(bufB, base0 + (it + 1) * kIter, next_of(bufA, base0 + (it + 2) * kIter));
    pace(it + 2);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (it + 1 < nit) {
    process(bufA, base0 + it * kIter, next_of(bufB, base0 + (it + 1) * kIter));
    __builtin_amdgcn_sched_barrier(0);
    process(bufB, base0 + (it + 1) * kIter, no_loads);
  } else if (it < nit) {
    process(bufA, base0 + it * kIter, no_loads);
  }

  // ---- per-wave result into the finalisation arena --------------------------
  // The V MFMAs contract over the keys of all four lane groups, so the
  // per-lane sums (softmax denominator, weight sum of the 128 offset, bias
  // term) are totalled over the lane groups of the same column.
  float l_sum = xor16_sum(l_run);
  l_sum = xor32_sum(l_sum);
  wsum = xor16_sum(wsum);
  wsum = xor32_sum(wsum);
  bacc = xor16_sum(bacc);
  bacc = xor32_sum(bacc);
  if constexpr (PACK) {
    // columns n and n + 8 hold tile 0's / tile 1's keys (denominator, bias
    // term): add the two; the hi / lo weight parts' products are added
    // below, each with its own 128 offset removed
    l_sum += ror8(l_sum);
    bacc += ror8(bacc);
    if (T) bacc = 0.0f;  // counted once, in the hi part
  }
  // packed: slot 2 * wave + T holds column n's part T (hi / lo)
  const int slot = PACK ? 2 * wave + T : wave;
  const float corr = bacc - 128.0f * wsum;  // bias term and the 128 offset
  if (col_used) {
    // Accumulator element (s, j) of C row 4c + i is dim 8 * (VW * (4c + i) +
    // s) + j: for one (c, i) the 8 * VW dims are contiguous and lie in one
    // quant group, so a lane writes the rows of its column's group as whole
    // vectors.  A wave's arena slot covers every dim: its own V words' dims
    // get the result, the other V half's dims zero; only V half 0 counts the
    // denominator (both halves scored the same keys).  Packed columns write
    // raw rows, and the correction once per (slot, column).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int dim0 = 8 * VW * (4 * c + i);
      if ((dim0 >> 6) == gn) {
        float row[8 * VW];
#pragma unroll
        for (int sg = 0; sg < VW; ++sg)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int so = sg - vhalf * VWH;  // this wave's word index, if owned
            float v = 0.0f;
#pragma unroll
            for (int s2 = 0; s2 < VWH; ++s2)
              if (s2 == so) v = PACK ? cv[8 * s2 + j][i] : cv[8 * s2 + j][i] + corr;
            row[8 * sg + j] = v;
          }
        v4f* dst = reinterpret_cast<v4f*>(Fin::o(arena, slot, hn) + dim0);
#pragma unroll
        for (int q4 = 0; q4 < 2 * VW; ++q4)
          dst[q4] = v4f{row[4 * q4], row[4 * q4 + 1], row[4 * q4 + 2], row[4 * q4 + 3]};
      }
    }
    if constexpr (PACK) {
      if (c == 0) Fin::corr(arena, slot)[n] = corr;
    }
    if (gn == 0 && c == 0 && T == 0) {
      Fin::m(arena, wave)[hn] = m_run;
      Fin::l(arena, wave)[hn] = vhalf == 0 ? l_sum : 0.0f;
    }
  }
  if constexpr (kQG)
    Fin::run(p, arena, static_cast<int64_t>(b0) * p.Hq + h0, rg.S, split, b * p.Hq + hy, GH,
             p.Hq, (b_last - b0 + 1) * GH);
  else
    Fin::run(p, arena, static_cast<int64_t>(b) * p.Hq + h0, rg.S, split, b * p.Hq + hy);
}

template <int D, int G, bool F32>
int launch_dgs(const SdpaParams& p, dim3 grid, hipStream_t s) {
  constexpr int NW = D == 512 ? 4 : kMfmaWaves;
  if (p.prefill && p.pq > 1)
    sdpa_int4_mfma_kernel<D, G, NW, true, true, F32><<<grid, NW * 64, 0, s>>>(p);
  else if (p.seq_lens)  // batched sequences of their own lengths
    sdpa_int4_mfma_kernel<D, G, NW, false, false, F32><<<grid, NW * 64, 0, s>>>(p);
  else if (NW == 8 && p.chunk <= 4 * 32)
    // splits of at most 128 keys (short contexts, e.g. a 786-key sliding
    // layer): at 8 waves half of them would hold no 32-key block yet issue
    // their clamped first loads; 4 waves each take one block (sliding layer
    // 9.93 -> 9.61 us)
    sdpa_int4_mfma_kernel<D, G, 4, false, true, F32><<<grid, 4 * 64, 0, s>>>(p);
  else
    sdpa_int4_mfma_kernel<D, G, NW, false, true, F32><<<grid, NW * 64, 0, s>>>(p);
  TQ_CHECK_LAUNCH("sdpa_int4_mfma_kernel");
  return TQ_OK;
}

template <int D, int G>
int launch_dg(const SdpaParams& p, int sb_dtype, dim3 grid, hipStream_t s) {
  return sb_dtype == TQ_F32 ? launch_dgs<D, G, true>(p, grid, s) : launch_dgs<D, G, false>(p, grid, s);
}

}  // namespace

bool mfma_serves(int D, int cols, int sb_dtype) {
  if (sb_dtype != TQ_F16 && sb_dtype != TQ_F32) return false;
  if (D == 256) return cols == 1 || cols == 2 || cols == 4;
  if (D == 512) return cols == 1 || cols == 2;
  if (D == 128) return cols == 1 || cols == 2 || cols == 4 || cols == 8;
  return false;
}

int launch_sdpa_mfma(const SdpaParams& p, int D, int G, int sb_dtype, dim3 grid,
                     hipStream_t stream) {
  if (!mfma_serves(D, G, sb_dtype)) return -1;
  if (D == 256) {
    if (G == 1) return launch_dg<256, 1>(p, sb_dtype, grid, stream);
    if (G == 2) return launch_dg<256, 2>(p, sb_dtype, grid, stream);
    if (G == 4) return launch_dg<256, 4>(p, sb_dtype, grid, stream);
  } else if (D == 512) {
    if (G == 1) return launch_dg<512, 1>(p, sb_dtype, grid, stream);
    if (G == 2) return launch_dg<512, 2>(p, sb_dtype, grid, stream);
  } else if (D == 128) {
    if (G == 1) return launch_dg<128, 1>(p, sb_dtype, grid, stream);
    if (G == 2) return launch_dg<128, 2>(p, sb_dtype, grid, stream);
    if (G == 4) return launch_dg<128, 4>(p, sb_dtype, grid, stream);
    if (G == 8) return launch_dg<128, 8>(p, sb_dtype, grid, stream);
  }
  return -1;
}

}  // namespace tq
