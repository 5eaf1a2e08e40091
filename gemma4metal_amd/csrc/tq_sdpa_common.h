// Shared pieces of the two fused int4 decode-attention kernels (the VALU
// kernel in tq_sdpa.hip and the matrix-core kernel in tq_sdpa_mfma.hip):
// launch parameters, the per-sequence key range, q loading, and the
// workgroup finalisation (cross-wave merge, split-K partials, and the
// last-workgroup log-sum-exp merge).
#pragma once

#include <math.h>

#include <algorithm>

// The split-K completion protocol below (Finalize::run: relaxed agent-scope
// partial stores and loads, one relaxed counter atomic, no L2 write-back or
// invalidate) is correct because of how gfx950 executes those instructions:
// write-through stores acknowledged at the point every XCD shares, and
// counter atomics performed at that same point in one order.  That argument
// has not been made for any other target, so device code for one is refused.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "tq_sdpa_common.h: the split-K merge protocol is argued for gfx950 only; build with --offload-arch=gfx950"
#endif

#include "tq_internal.h"

namespace tq {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kMaxSplits = 256;  // splits per (sequence, kv head)
// Split counters at the head of the workspace (ints); batch * num_heads of
// them are in use at once.
constexpr int64_t kMaxCounters = 1 << 16;

struct SdpaParams {
  const void* q;
  int q_dtype;
  const uint32_t* kq;
  const void* ks;
  const void* kb;
  const uint32_t* vq;
  const void* vs;
  const void* vb;
  float* out;
  float* ws_o;    // [B][Hq][max_splits][D]
  float* ws_ml;   // [B][Hq][max_splits][2]
  int* ws_cnt;    // [B][Hq]  (one counter per (sequence, kv head, head subgroup))
  int Hq, Hkv, cap, gqa, n_sub;
  int n;                   // single-sequence length (seq_lens == nullptr)
  const int* seq_lens;     // device [B] or nullptr
  const int* windows;      // device [B] or nullptr
  int window;
  int n_clamp;             // upper bound applied to every sequence length
  float scale_log2;        // scale * log2(e)
  int chunk;
  int max_splits;
  // Output normalisation: 0 -> out = l > 0 ? O / l : 0 (sdpa_int4,
  // lib/turboquant.metal:886); > 0 -> out = O / (l + denom_eps)
  // (sdpa_tq_sequential, lib/turboquant.metal:222).
  float denom_eps;
  // 0: the last workgroup of a split sequence merges the partials; 1: the
  // kernel only writes them and launch_merge_splits merges them afterwards.
  int ext_merge;
  // Prefill: batch element b is the query at position n + b over the one
  // cache of batch 0, attending its first n + b + 1 rows (causal), under
  // `window` (engine/gemma4_multilayer.cpp:349-358).
  int prefill;
  // Prefill on the matrix-core kernel: each workgroup takes pq consecutive
  // queries (grid z = query groups) of its heads, nq queries in all.
  int pq;
  int nq;
  // Ragged launches of at most 64 sequences: the chunk is chosen on the
  // device from the lengths, and workgroups take their (sequence, split)
  // from the longest-first order of ragged_job.  cus: compute units.
  int lpt;
  int cus;
  // ints between the split counters of consecutive (sequence, head) rows
  // (counter_stride of the launch's counter count, set on the host)
  int cnt_stride;
};

// Counter `c` of a launch with n counters in use sits at ws_cnt[c * stride]:
// up to 32 ints (one 128 B line) from its neighbours, as far as the counter
// region allows -- the atomics of every head's last splits arrive together
// at the end of a launch, and on one shared line they serialise.
inline int counter_stride(int64_t n) {
  return static_cast<int>(std::min<int64_t>(32, kMaxCounters / std::max<int64_t>(n, 1)));
}

// Kernel arguments arrive through scalar loads from the kernarg segment, one
// memory round trip per batch of loads.  Left to itself, the compiler places
// each field's load near its first use: behind the split-range arithmetic
// and its early exit, that made three dependent round trips before the
// first K/V load could issue (1.3 us after a wave's start at L = 786).
// Pinning the fields the prologue needs into SGPRs at kernel entry issues
// them as one batch.
__device__ __forceinline__ void pin_args(const SdpaParams& p) {
  asm volatile("" ::"s"(p.q), "s"(p.kq), "s"(p.ks), "s"(p.kb), "s"(p.vq), "s"(p.vs), "s"(p.vb),
               "s"(p.seq_lens), "s"(p.windows), "s"(p.q_dtype), "s"(p.Hq), "s"(p.Hkv), "s"(p.cap),
               "s"(p.gqa), "s"(p.n_sub), "s"(p.n), "s"(p.window), "s"(p.n_clamp),
               "s"(p.scale_log2), "s"(p.chunk), "s"(p.prefill), "s"(p.ws_cnt), "s"(p.cnt_stride));
}

// Batch index of the cache that batch element b reads.
__device__ __forceinline__ int cache_batch(const SdpaParams& p, int b) { return p.prefill ? 0 : b; }

// The keys one workgroup attends: rows [t_begin, t_end) of its sequence's
// cache.  Key ki survives the reference window rule (skip ki when
// W > 0 and n-1-ki >= W, lib/turboquant.metal:779) iff ki >= n - W.
struct SplitRange {
  int S;        // number of splits of this sequence (>= 1)
  int t_begin;  // first row of this split
  int t_end;    // one past the last row
};

__device__ __forceinline__ SplitRange split_range(const SdpaParams& p, int b, int split) {
  int n_b = p.prefill ? p.n + b + 1 : (p.seq_lens ? p.seq_lens[b] : p.n);
  n_b = min(n_b, p.n_clamp);
  const int W = p.windows ? p.windows[b] : p.window;
  const int lo = W > 0 ? max(0, n_b - W) : 0;
  const int L = max(n_b - lo, 0);
  SplitRange r;
  r.S = L > 0 ? (L + p.chunk - 1) / p.chunk : 1;
  r.t_begin = lo + split * p.chunk;
  r.t_end = min(r.t_begin + p.chunk, n_b);
  return r;
}

// Job of a workgroup in a ragged launch with p.lpt set (at most 64
// sequences).
// - The chunk is chosen here, from the actual lengths (the host knows only
//   the longest, and sizes the grid and workspace for p.max_splits chunks
//   of it): of the candidates ceil(Lmax / k) (rounded up to 128 keys),
//   k = 1 .. p.max_splits, the one with the least estimated makespan
//   max(F + c, (F * jobs(c) + keys) / CUs), F = kLptFixedKeys, a
//   workgroup's fixed cost (prologue, split merge) in keys streamed.  One
//   chunk per sequence (no merge) wins when many sequences fill the chip;
//   a few long sequences among short ones get split.
// - The (sequence, kv-head column, split) cells then run in longest-first
//   order, so that the chunks that take longest start first and the launch
//   does not end on a few long chunks dispatched last: all full chunks
//   first (sequence, then split order), then each sequence's last, partial
//   chunk by size, largest first (ties: lower sequence first); the heads
//   of one cell are consecutive.
// Every wave computes the same mapping from one load of the lengths (lane
// i: sequence i), so no barrier is needed.  A job's work and its split
// merge order do not depend on which workgroup runs it.  Returns false for
// a workgroup beyond the last job.
constexpr int kLptFixedKeys = 870;

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) v = max(v, __shfl_xor(v, d, 64));
  return v;
}

__device__ __forceinline__ bool ragged_job(const SdpaParams& p, int& b, int& hy, int& split, int& chunk) {
  const int lane = threadIdx.x & 63;
  const int H = static_cast<int>(gridDim.y);
  const int64_t wg = blockIdx.x + static_cast<int64_t>(gridDim.x) * (blockIdx.y + static_cast<int64_t>(gridDim.y) * blockIdx.z);
  const bool mine = lane < p.nq;
  const int n_b = mine ? min(p.seq_lens[lane], p.n_clamp) : 0;
  const int W = mine ? (p.windows ? p.windows[lane] : p.window) : 0;
  const int lo = W > 0 ? max(0, n_b - W) : 0;
  const int len = max(n_b - lo, 0);
  // ---- chunk: candidates k = 1 .. max_splits, one wave-wide job count each
  const int lmax = wave_max_i(len);
  const float keys = static_cast<float>(wave_sum_dpp(len)) * H;
  const float cus = static_cast<float>(max(p.cus, 1));
  float best = INFINITY;
  chunk = p.chunk;
  for (int k = 1; k <= p.max_splits; ++k) {  // uniform loop
    const int cand = max(128, ((lmax + k - 1) / k + 127) / 128 * 128);
    const int jobs = wave_sum_dpp(mine ? (len > 0 ? (len + cand - 1) / cand : 1) : 0);
    const float est = fmaxf(static_cast<float>(kLptFixedKeys + cand),
                            (static_cast<float>(kLptFixedKeys) * jobs * H + keys) / cus);
    if (est < best) {  // uniform: strictly better, so ties keep the smaller k
      best = est;
      chunk = cand;
    }
  }
  // ---- longest-first order ------------------------------------------------------
  const int full = mine ? len / chunk : 0;
  const int rem = len - full * chunk;
  const bool part = mine && (rem > 0 || len == 0);  // one partial (or empty) chunk
  const int F = wave_sum_dpp(full);  // full chunks in all
  const int64_t r = wg / H;
  hy = static_cast<int>(wg - r * H);
  if (r >= F + static_cast<int>(__builtin_popcountll(__ballot(part)))) return false;  // no job
  if (r < F) {
    // inclusive prefix sum of the full-chunk counts over the lanes
    int pre = full;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(pre, d, 64);
      if (lane >= d) pre += v;
    }
    const uint64_t m = __ballot(pre > r);
    b = __builtin_ffsll(static_cast<long long>(m)) - 1;
    split = static_cast<int>(r) - (__builtin_amdgcn_readlane(pre, b) - __builtin_amdgcn_readlane(full, b));
    return true;
  }
  // rank of this lane's partial chunk among all partial chunks
  int rank = 0;
  for (int j = 0; j < 64; ++j) {
    const int rj = __builtin_amdgcn_readlane(rem, j);
    const bool pj = __builtin_amdgcn_readlane(static_cast<int>(part), j) != 0;
    rank += (pj && (rj > rem || (rj == rem && j < lane))) ? 1 : 0;
  }
  const uint64_t m = __ballot(part && rank == static_cast<int>(r - F));
  b = __builtin_ffsll(static_cast<long long>(m)) - 1;
  split = __builtin_amdgcn_readlane(full, b);
  return true;
}

// Key range of the prefill query group b0 .. b_last (positions n + b0 ..):
// the union of their causal windows, cut into chunks as split_range does.
__device__ __forceinline__ SplitRange prefill_range(const SdpaParams& p, int b0, int b_last,
                                                    int split) {
  const int lo = p.window > 0 ? max(0, p.n + b0 + 1 - p.window) : 0;
  const int hi = p.n + b_last + 1;
  SplitRange r;
  r.S = (hi - lo + p.chunk - 1) / p.chunk;
  r.t_begin = lo + split * p.chunk;
  r.t_end = min(r.t_begin + p.chunk, hi);
  return r;
}

// E contiguous elements of a q row, any of the three input dtypes (one
// uniform branch, then straight-line 16 B loads).
template <int E, bool kF16>
__device__ __forceinline__ void load_q16(const uint16_t* p, float out[E]) {
  const uint4* v4 = reinterpret_cast<const uint4*>(p);
  uint32_t w[E / 2];
#pragma unroll
  for (int i = 0; i < E / 8; ++i) {
    const uint4 v = v4[i];
    w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
  }
#pragma unroll
  for (int k = 0; k < E / 2; ++k) {
    if constexpr (kF16) {
      out[2 * k] = __half2float(__ushort_as_half(static_cast<uint16_t>(w[k] & 0xFFFFu)));
      out[2 * k + 1] = __half2float(__ushort_as_half(static_cast<uint16_t>(w[k] >> 16)));
    } else {
      out[2 * k] = __uint_as_float(w[k] << 16);
      out[2 * k + 1] = __uint_as_float(w[k] & 0xFFFF0000u);
    }
  }
}

template <int E>
__device__ __forceinline__ void load_q_slice(const void* q, int dtype, int64_t off, float out[E]) {
  if (dtype == TQ_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(q) + off);
#pragma unroll
    for (int i = 0; i < E / 4; ++i) {
      const float4 v = p[i];
      out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
    }
  } else if (dtype == TQ_F16) {
    load_q16<E, true>(static_cast<const uint16_t*>(q) + off, out);
  } else {
    load_q16<E, false>(static_cast<const uint16_t*>(q) + off, out);
  }
}

// Agent-scope (all XCDs) coherent store / load of split-K partials.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// VEC (2 or 4) consecutive floats as one agent-scope (sc1) 8- or 16-byte
// buffer access, the cache policy of the relaxed agent-scope atomics above.
constexpr int kBufSc1 = 16;  // buffer instruction cache-policy bits: sc1
template <int VEC>
struct CoherentVec {
  static_assert(VEC == 1 || VEC == 2 || VEC == 4, "VEC");
  typedef float FV __attribute__((ext_vector_type(VEC)));
  typedef uint32_t UV __attribute__((ext_vector_type(VEC)));
  __device__ static __amdgpu_buffer_rsrc_t rsrc(float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7FFFFFFF, 0x00020000);
  }
  __device__ static FV load(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    FV v;
    if constexpr (VEC == 1) {
      v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, kBufSc1));
    } else if constexpr (VEC == 2) {
      v = __builtin_bit_cast(FV, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, kBufSc1));
    } else {
      v = __builtin_bit_cast(FV, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kBufSc1));
    }
    return v;
  }
  __device__ static void store(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, FV v) {
    if constexpr (VEC == 1)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[0]), r, byte_off, 0, kBufSc1);
    else if constexpr (VEC == 2)
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(UV, v), r, byte_off, 0, kBufSc1);
    else
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(UV, v), r, byte_off, 0, kBufSc1);
  }
};

// A split's (m, l) pair as one 8-byte access (p 8-byte aligned).
__device__ __forceinline__ void store_coherent_pair(float* p, float m, float l) {
  const uint64_t v = static_cast<uint64_t>(__float_as_uint(m)) | (static_cast<uint64_t>(__float_as_uint(l)) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_coherent_pair(const float* p) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return float2{__uint_as_float(static_cast<uint32_t>(v)), __uint_as_float(static_cast<uint32_t>(v >> 32))};
}

__device__ __forceinline__ float normalise(float O, float L, float eps) {
  return eps > 0.0f ? O / (L + eps) : (L > 0.0f ? O / L : 0.0f);
}

__device__ __forceinline__ float merge_factor(float m, float M) {
  return m == -INFINITY ? 0.0f : fast_exp2(m - M);
}

// Lazy online-softmax rescale: a kernel's running max m moves (and its
// accumulators are rescaled) only when a new score exceeds m by more than
// this many log2 units, so every weight 2^(s - m) stays <= 2^kLazyMax.
// Every partial (O, l) is still exact relative to its own m, so the merges
// are unchanged; the rescale, a read-multiply-write of every accumulator,
// then runs about once per wave instead of whenever the max grows.
constexpr float kLazyMax = 8.0f;

// Issue pacing of 8-wave workgroups with a static key stream per wave.
// Waves w and w ^ 4 share a SIMD, whose arbiter favours the older wave: left
// alone, waves 0-3 finish their (equal) streams long before waves 4-7 (at
// 256k keys per head: 142 vs 189 us), the CU streaming with half its loads
// in flight in between.  After each iteration a wave publishes its count in
// `done_lds` (one int per wave, zeroed before the workgroup's first barrier)
// and takes the higher issue priority while it is behind its SIMD partner,
// or level with it and the younger of the two.  Only issue order changes,
// so results do not depend on timing.
template <int NW>
__device__ __forceinline__ void pace_waves(int* done_lds, int wv, int lane, int done) {
  if constexpr (NW == 8) {
    if (lane == 0) __hip_atomic_store(&done_lds[wv], done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int other = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(&done_lds[wv ^ (NW / 2)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    if (other > done || (other == done && wv >= NW / 2))
      __builtin_amdgcn_s_setprio(1);
    else
      __builtin_amdgcn_s_setprio(0);
  } else if constexpr (NW == 16) {
    // four waves per SIMD (w, w + 4, w + 8, w + 12): a wave behind the
    // furthest of its partners takes priority 1, or 2 when two or more
    // steps behind
    if (lane == 0) __hip_atomic_store(&done_lds[wv], done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    int mx = done;
#pragma unroll
    for (int j = 1; j < 4; ++j)
      mx = max(mx, __hip_atomic_load(&done_lds[(wv + 4 * j) & 15], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    const int behind = __builtin_amdgcn_readfirstlane(mx) - done;
    if (behind >= 2)
      __builtin_amdgcn_s_setprio(2);
    else if (behind == 1)
      __builtin_amdgcn_s_setprio(1);
    else
      __builtin_amdgcn_s_setprio(0);
  }
}

// LDS arena of the finalisation: [o: NW*SPW*G*D | m: NW*G | l: NW*G |
// corr: NW*SPW*G*(D/64)] (sized to at least 2*G*kMaxSplits floats).  NW =
// partial results per workgroup (one per wave, or per key stream), NT =
// threads.  A wave may leave its partial O as SPW rows per head (slots
// SPW*w .. SPW*w + SPW - 1, summed here) and, with CORR, one additive term
// per slot and (head, quant group) that applies to every dim of the group
// (the matrix-core kernel's hi and lo weight parts and their corrections).
template <int G, int D, int NW = kWaves, int NT = NW * 64, int SPW = 1, bool CORR = false>
struct Finalize {
  static constexpr int kNT = NT;
  static constexpr int NGc = D / 64;
  static constexpr int kUsed = NW * SPW * G * D + 2 * NW * G + (CORR ? NW * SPW * G * NGc : 0);
  static constexpr int kArena = kUsed > 2 * G * kMaxSplits ? kUsed : 2 * G * kMaxSplits;
  __device__ static float* o(float* arena, int slot, int h) { return arena + (slot * G + h) * D; }
  __device__ static float* m(float* arena, int w) { return arena + NW * SPW * G * D + w * G; }
  __device__ static float* l(float* arena, int w) {
    return arena + NW * SPW * G * D + NW * G + w * G;
  }
  // [h * (D / 64) + group] of a slot
  __device__ static float* corr(float* arena, int slot) {
    return arena + NW * SPW * G * D + 2 * NW * G + slot * G * NGc;
  }

  // Called by all threads after every wave stored its unnormalised output
  // O[h][d] (relative to its running max m[h]) and denominator l[h] into the
  // arena (no barrier needed before the call).  Column h is output row
  // head_base + (h / gh) * qstride + h % gh (decode: head_base = b*Hq + first
  // head, rows head_base + h); columns h >= nvalid are dropped.
  //
  // Both merges here (the NW per-wave partials of this workgroup, then the S
  // split partials in the last workgroup) weight partial k by
  // f_k = 2^(m_k - M), M = max m_k.  A wave's 64 outputs share one head (64
  // divides D), so the weights are wave-uniform: lane k computes f_k (one
  // exp2 per lane, not one per output and partial), the denominator is a
  // lane reduction, and each output then takes one FMA per partial with f_k
  // read back as a scalar.
  __device__ static void run(const SdpaParams& p, float* arena, int64_t head_base, int S,
                             int split, int counter, int gh = G, int64_t qstride = 0,
                             int nvalid = G) {
    static_assert(D % 64 == 0, "one head per wave");
    static_assert(NW <= 16, "per-wave partials fit one row of 16 lanes");
    // A thread takes VEC consecutive dims of one head: the arena rows are
    // read as VEC-float LDS vectors and the split partials move as one 4-,
    // 8- or 16-byte agent-scope access per split (fewer memory instructions,
    // which the CU's address unit serialises).  VEC is as large as keeps
    // every wave busy (G * D / threads outputs each; concentrating the
    // combine on fewer waves was slower) and at most 4, and a wave's
    // 64 * VEC dims lie in one head.
    constexpr int VPT = G * D / kNT;  // outputs per thread
    constexpr int VEC = (VPT >= 4 && D >= 256) ? 4 : ((VPT >= 2 && D >= 128) ? 2 : 1);
    using CV = CoherentVec<VEC>;
    using FV = float __attribute__((ext_vector_type(VEC)));
    constexpr int NU = G * D / VEC;             // (head, dim vector) units
    constexpr int NI = (NU + kNT - 1) / kNT;    // units per thread
    auto row = [&](int h) -> int64_t { return head_base + (h / gh) * qstride + h % gh; };
    const int lane = threadIdx.x & 63;
    // split partials: [row][split][D] floats, byte offsets below 2^31
    // (checked on the host)
    const __amdgpu_buffer_rsrc_t wso = CV::rsrc(p.ws_o);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int u = threadIdx.x + i * kNT;
      const int h = u * VEC / D, d = u * VEC - (u * VEC / D) * D;
      if (u >= NU || h >= nvalid) continue;  // wave-uniform
      // lane w < NW: wave w's (m, l) of head h (each row of 16 lanes holds
      // the same copy, so a row reduction is the workgroup's).  With up to
      // four waves, every LDS read of this unit (m, l, corrections, the
      // waves' rows) goes out before the arithmetic: one LDS latency on the
      // path, not two (sliding layer 6.70 -> 6.66 us).  With eight waves the
      // rows are read as they are summed: reading them ahead there measured
      // 28.43 us at 32k against 28.40.
      constexpr bool kPre = NW <= 4;
      const int w = lane & 15;
      // (with the reads hoisted, lanes w >= NW read wave NW - 1's copy and
      // drop it: no branch around the reads)
      const int wc = kPre ? (w < NW ? w : NW - 1) : w;
      float mw = 0.0f, lw = 0.0f, cw = 0.0f;
      if (kPre || w < NW) {
        mw = m(arena, wc)[h];
        lw = l(arena, wc)[h];
        if constexpr (CORR) {
          // the corrections of this wave's group (d / 64 is wave-uniform)
#pragma unroll
          for (int t = 0; t < SPW; ++t) cw += corr(arena, wc * SPW + t)[h * NGc + d / 64];
        }
      }
      FV ov[kPre ? NW : 1][SPW];
      if constexpr (kPre) {
#pragma unroll
        for (int k = 0; k < NW; ++k)
#pragma unroll
          for (int t = 0; t < SPW; ++t) ov[k][t] = *reinterpret_cast<const FV*>(o(arena, k * SPW + t, h) + d);
      }
      mw = w < NW ? mw : -INFINITY;
      lw = w < NW ? lw : 0.0f;
      const float M = row16_max(mw);
      const float fw = merge_factor(mw, M);
      const float Ls = group_sum<16>(lw * fw);
      FV O;
      {
        float c0 = 0.0f;
        if constexpr (CORR) c0 = group_sum<16>((w < NW ? cw : 0.0f) * fw);
#pragma unroll
        for (int e = 0; e < VEC; ++e) O[e] = c0;
      }
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const float fk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fw), k));
#pragma unroll
        for (int t = 0; t < SPW; ++t) {
          const FV v = kPre ? ov[kPre ? k : 0][t] : *reinterpret_cast<const FV*>(o(arena, k * SPW + t, h) + d);
#pragma unroll
          for (int e = 0; e < VEC; ++e) O[e] = fmaf(v[e], fk, O[e]);
        }
      }
      if (S == 1) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) p.out[row(h) * D + d + e] = normalise(O[e], Ls, p.denom_eps);
      } else {
        const int64_t slot = row(h) * p.max_splits + split;
        CV::store(wso, static_cast<uint32_t>((slot * D + d) * 4), O);
        if (d == 0) store_coherent_pair(p.ws_ml + slot * 2, M, Ls);
      }
    }
    if (S == 1 || p.ext_merge) return;

    // The last workgroup of this (sequence, kv head, subgroup) to finish merges
    // the splits.  Partials are written with agent-scope stores (write-through
    // to the coherence point shared by all XCDs) and read with agent-scope
    // loads, so no L2 write-back/invalidate fence is needed -- such a fence
    // costs ~4 us per workgroup here.  vmcnt(0) before the barrier makes every
    // wave's partial stores complete before thread 0 bumps the counter.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    __shared__ int s_last;
    if (threadIdx.x == 0) {
      // counter `counter` < gridDim.z * Hq (checked on the host); its
      // spacing comes with the arguments, so nothing but the atomic lies
      // between the barrier and the counter's value
      int* cnt = p.ws_cnt + static_cast<int64_t>(counter) * p.cnt_stride;
      const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = (old == S - 1);
      // leave the workspace zeroed for the next call -- with an atomic RMW,
      // the same kind of operation as the increments (a plain store, even a
      // write-through one, is not ordered with them)
      if (old == S - 1) __hip_atomic_exchange(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;

    // Merge, KC splits at a time: lane k (mod 16) loads split s0 + k's
    // (m, l), and every thread the KC partial vectors of its units.  All
    // loads of a chunk, for all of a thread's units, go out before the first
    // use: one memory round trip per chunk, one in all for S <= KC.
    constexpr int KC = 16;
    float Mr[NI], Lr[NI];
    FV Or[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      Mr[i] = -INFINITY;
      Lr[i] = 0.0f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) Or[i][e] = 0.0f;
    }
    for (int s0 = 0; s0 < S; s0 += KC) {
      float2 mlv[NI];
      FV ok[NI][KC];
      const int sl = min(s0 + (lane & (KC - 1)), S - 1);
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int u = min(static_cast<int>(threadIdx.x) + i * kNT, NU - 1);
        // (past the last unit: a valid row, loaded and dropped below)
        const int h = min(u * VEC / D, nvalid - 1), d = u * VEC - (u * VEC / D) * D;
        mlv[i] = load_coherent_pair(p.ws_ml + (row(h) * p.max_splits + sl) * 2);
        const int64_t base = row(h) * p.max_splits * D + d;
        // only the chunk's existing splits are loaded (a clamped duplicate
        // load would still take an address-unit slot); full chunks without
        // the per-split branches
        if (s0 + KC <= S) {
#pragma unroll
          for (int k = 0; k < KC; ++k)
            ok[i][k] = CV::load(wso, static_cast<uint32_t>((base + static_cast<int64_t>(s0 + k) * D) * 4));
        } else {
#pragma unroll
          for (int k = 0; k < KC; ++k) {
            if (s0 + k < S)
              ok[i][k] = CV::load(wso, static_cast<uint32_t>((base + static_cast<int64_t>(s0 + k) * D) * 4));
            else
              ok[i][k] = FV{};
          }
        }
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        // lanes past the splits get m = -inf, hence weight 0
        const float mk = s0 + (lane & (KC - 1)) < S ? mlv[i].x : -INFINITY;
        const float Mn = fmaxf(Mr[i], row16_max(mk));
        const float fr = merge_factor(Mr[i], Mn);
        const float fk = merge_factor(mk, Mn);
        Lr[i] = fmaf(Lr[i], fr, group_sum<16>(mlv[i].y * fk));
        FV O = Or[i] * fr;
#pragma unroll
        for (int k = 0; k < KC; ++k) {
          const float f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fk), k));
#pragma unroll
          for (int e = 0; e < VEC; ++e) O[e] = fmaf(ok[i][k][e], f, O[e]);
        }
        Or[i] = O;
        Mr[i] = Mn;
      }
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int u = threadIdx.x + i * kNT;
      const int h = u * VEC / D, d = u * VEC - (u * VEC / D) * D;
      if (u >= NU || h >= nvalid) continue;
#pragma unroll
      for (int e = 0; e < VEC; ++e) p.out[row(h) * D + d + e] = normalise(Or[i][e], Lr[i], p.denom_eps);
    }
  }
};

// ---- host-side split planning (tq_sdpa.hip) ---------------------------------
// Workspace: [split counters | (m, l) partials | O partials].  The counter
// region has a FIXED size at offset 0 so that no call's partials ever overlap
// another call's counters: counters must read zero on entry (the kernels
// return every counter they use to zero), whatever shapes earlier calls had.

struct WsLayout {
  size_t cnt_off, ml_off, o_off, total;
};

int target_wgs();                                   // CUs of the current device
int head_subgroup(int gqa);                         // query heads per workgroup
int plan_chunk(int max_len, int64_t groups, int min_splits);        // keys per workgroup
int max_splits_bound(int max_len, int64_t groups, int min_splits);  // bound of ceil(L / chunk)
int min_splits_for(int batch);                                      // 5 for batched launches
WsLayout ws_layout(int batch, int Hq, int D, int max_splits);

// Kernel-choice switches for tests and measurement.  They are read from the
// environment once per process; tq_reload_options() reads them again.
//   TQ_SDPA_IMPL=valu       the VALU decode kernel for every shape
//   TQ_SDPA_CHUNK=n         keys per split (overrides the planner)
//   TQ_PREFILL_IMPL=splitk  prefill on the split-K decode kernels
//   TQ_PREFILL_WS=0         the one-role prefill tile kernel
//   TQ_HC_IMPL=1            the one-wave D=512 heads-as-columns kernel
struct Options {
  bool sdpa_valu;
  int sdpa_chunk;
  bool prefill_splitk;
  bool prefill_ws;
  bool hc_one;
};
Options options();

// Which kernel a decode / ragged / prefill call launches, and its split plan.
enum class SdpaKernel { valu, mfma, hc, prefill_tiles };
struct SdpaPlan {
  SdpaKernel kernel;
  int G;           // query heads per workgroup (before query grouping)
  int n_sub;       // workgroups per kv head along the head axis (gqa / G)
  int pq;          // consecutive prefill queries per workgroup (1 otherwise)
  int chunk;       // keys per split
  int max_splits;  // grid.x: bound of the splits of any sequence
  WsLayout wl;     // workspace layout
  bool lpt;        // ragged: device-chosen chunk, longest-first order (ragged_job)
};
// mode: 0 single sequence (n = kv_len), 1 ragged batch (max_len bounds the
// lengths), 2 prefill (batch = queries, max_len = n_prior + n_new); cap =
// the cache's rows per (sequence, kv head).
SdpaPlan plan_sdpa(int mode, int batch, int Hq, int Hkv, int D, int max_len, int gqa, int window,
                   int sb_dtype, int cap);
// Smallest cache capacity (rows) the matrix-core kernel serves: it reads
// whole 32-row blocks.
constexpr int kMfmaMinRows = 32;
const char* kernel_name(const SdpaPlan& pl, int D, int sb_dtype);

// (D, query columns) served by the matrix-core kernel, for a scale dtype.
bool mfma_serves(int D, int cols, int sb_dtype);
// Scale dtypes the D = 512 heads-as-columns kernels serve.
bool hc_serves(int sb_dtype);
// Shapes the prefill tile kernels serve.
bool prefill_tiles_serve(int D, int sb_dtype, int gqa);

// Launch of the matrix-core kernel (tq_sdpa_mfma.hip).  Returns TQ_OK,
// a tq_status error, or -1 when (D, G) is not served by that kernel.
int launch_sdpa_mfma(const SdpaParams& p, int D, int G, int sb_dtype, dim3 grid,
                     hipStream_t stream);
// D = 512, 8 query heads per workgroup (heads as matrix-core columns), fp16
// scale/bias: tq_sdpa_hc.hip.
int launch_sdpa_hc(const SdpaParams& p, int sb_dtype, dim3 grid, hipStream_t stream);
// Prefill with K/V tiles shared by 64 (query, head) rows (tq_prefill.hip);
// -1 when the shape is not served (D other than 128 / 256, fp32 scales,
// gqa not dividing 64).
int launch_prefill_tiles(const SdpaParams& p, int D, int sb_dtype, hipStream_t stream);
// Merge of the split partials of a launch with ext_merge = 1 (batch b of
// grid.y): tq_sdpa_hc.hip.
int launch_merge_splits(const SdpaParams& p, int D, int batch, hipStream_t stream);

}  // namespace tq
