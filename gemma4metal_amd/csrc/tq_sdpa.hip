// Fused int4-KV decode attention (sdpa_int4) for gfx950.
//
// Replaces sdpa_int4_vector<D,BN> (lib/turboquant.metal:723-889) and its host
// dispatch FusedInt4SDPA::eval_gpu (lib/turboquant.cpp:367-403).
//
// Work decomposition (flash-decoding):
//   grid = (splits, kv-head x head-subgroup, batch); a workgroup of 4 wave64s
//   owns one kv head, one contiguous chunk of keys and ALL the GQA query heads
//   that read that kv head (G of them), so every packed K/V byte is fetched
//   from HBM exactly once per call (the reference re-reads K/V once per query
//   head, lib/turboquant.metal:744-745).
//   Inside a wave, LPT = D/E consecutive lanes share one key row, each lane
//   owning E contiguous dims (E/2 bytes of nibbles: a 16 B dwordx4 load when
//   E = 32), so one load instruction covers 64*E/2 contiguous bytes of
//   K (or V) rows.  The 4 waves interleave over the chunk's rows.
//   Each lane keeps an online softmax (log2 domain) for each of its G heads;
//   rescaling of the running output happens only when some lane's maximum
//   grows (a wave-uniform branch), which after the first rows is rare.
//   Epilogue: xor-exchange merge across the row groups of a wave, an LDS merge
//   across the 4 waves, then either the final normalised output (one split)
//   or an (O, m, l) partial in the workspace.  The last workgroup of a
//   (sequence, kv head) -- found with one device-scope atomic counter that it
//   resets to zero -- merges the partials with the same log-sum-exp rule, so
//   a call is ONE kernel launch at every context length.
//
// Math: score_h = sum_g s_g * (q_h . n_g) + b_g * sum(q_h over g), i.e. the
// bias term of the dequantized key (s*n + b) is folded into a per-lane
// constant sum(q); V likewise accumulates (p*s_v)*n per element plus a per
// group sum of p*b_v.  q is pre-multiplied by scale*log2(e) so p = exp2(.)
// (the reference pre-scales q by scale, lib/turboquant.metal:762, and uses
// exp; the normalised result is the same).
#include <math.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

#include "tq_sdpa_common.h"

namespace tq {

// ---- split planning and workspace layout (shared with tq_polar.hip) ----------

// Workgroups per launch the split planner aims for: one per CU (the matrix
// kernel runs one 4-wave workgroup per CU at its register budget; more,
// smaller splits only add per-split fixed cost).  Queried once per process
// from the current device.
int target_wgs() {
  static int cached = [] {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    return cus;
  }();
  return cached;
}
namespace {
constexpr int kMinChunk = 128;
constexpr int kChunkGranule = 128;
}  // namespace

namespace {
// The switches of Options, as atomics so that a reload while other threads
// plan calls is well defined (each call sees old or new values).
struct OptionStore {
  std::atomic<int> sdpa_valu{0}, sdpa_chunk{0}, prefill_splitk{0}, prefill_ws{1}, hc_one{0};
};
OptionStore g_opts;
std::once_flag g_opts_once;

void read_options() {
  auto env = [](const char* name) -> const char* { return std::getenv(name); };
  const char* v = env("TQ_SDPA_IMPL");
  g_opts.sdpa_valu.store(v && std::string(v) == "valu", std::memory_order_relaxed);
  v = env("TQ_SDPA_CHUNK");
  g_opts.sdpa_chunk.store(v ? std::atoi(v) : 0, std::memory_order_relaxed);
  v = env("TQ_PREFILL_IMPL");
  g_opts.prefill_splitk.store(v && std::string(v) == "splitk", std::memory_order_relaxed);
  v = env("TQ_PREFILL_WS");
  g_opts.prefill_ws.store(!(v && v[0] == '0'), std::memory_order_relaxed);
  v = env("TQ_HC_IMPL");
  g_opts.hc_one.store(v && v[0] == '1', std::memory_order_relaxed);
}
}  // namespace

Options options() {
  std::call_once(g_opts_once, read_options);
  Options o;
  o.sdpa_valu = g_opts.sdpa_valu.load(std::memory_order_relaxed) != 0;
  o.sdpa_chunk = g_opts.sdpa_chunk.load(std::memory_order_relaxed);
  o.prefill_splitk = g_opts.prefill_splitk.load(std::memory_order_relaxed) != 0;
  o.prefill_ws = g_opts.prefill_ws.load(std::memory_order_relaxed) != 0;
  o.hc_one = g_opts.hc_one.load(std::memory_order_relaxed) != 0;
  return o;
}

int head_subgroup(int gqa) {
  for (int g : {8, 4, 2}) if (gqa % g == 0) return g;
  return 1;
}

// Keys per workgroup: about one workgroup per CU over `groups` (sequence,
// kv head, head subgroup) groups of max_len keys, never fewer than kMinChunk
// rows.  A batched (ragged) launch also splits every sequence of max_len into
// at least min_splits chunks: its sequences differ in length, and a long one
// in a few large chunks is the tail of the whole launch.  (Measured on the
// B=64 ragged workload, ms per step: chunks of max_len/2 0.721, /4 0.664,
// /5 0.630, /6 0.634, /10 0.646.  Each chunk adds a workgroup's prologue and
// finalisation, a few us in which its CU does not stream.)
int plan_chunk(int max_len, int64_t groups, int min_splits) {
  // never more than kMaxSplits chunks per sequence
  const int64_t floor_c = (static_cast<int64_t>(max_len) + kMaxSplits - 1) / kMaxSplits;
  const int forced = options().sdpa_chunk;
  if (forced > 0) return static_cast<int>(std::max<int64_t>(forced, floor_c));
  const int64_t want = (static_cast<int64_t>(max_len) * groups + target_wgs() - 1) / target_wgs();
  int64_t c = (want + kChunkGranule - 1) / kChunkGranule * kChunkGranule;
  if (min_splits > 1) {
    const int64_t per = (static_cast<int64_t>(max_len) + min_splits - 1) / min_splits;
    c = std::min(c, (per + kChunkGranule - 1) / kChunkGranule * kChunkGranule);
  }
  c = std::max<int64_t>({c, int64_t{kMinChunk}, floor_c});
  return static_cast<int>(std::min<int64_t>(c, 1 << 30));
}

// Upper bound of ceil(L / plan_chunk(L, groups, min_splits)) over every
// L <= max_len (plan_chunk is not monotone in L, the bound is): sizes grids
// and workspaces.
int max_splits_bound(int max_len, int64_t groups, int min_splits) {
  if (max_len <= 0) return 1;
  const int forced = options().sdpa_chunk;
  if (forced > 0) return std::min((max_len + forced - 1) / forced, kMaxSplits);  // chunk >= ceil(L/kMaxSplits)
  const int64_t by_len = (static_cast<int64_t>(max_len) + kMinChunk - 1) / kMinChunk;
  const int64_t by_wgs = std::max<int64_t>((target_wgs() + groups - 1) / groups, min_splits);
  return static_cast<int>(std::max<int64_t>(1, std::min({by_len, by_wgs, int64_t{kMaxSplits}})));
}

// Chunks per sequence of max_len a launch of `batch` sequences uses at least.
int min_splits_for(int batch) { return batch > 1 ? 5 : 1; }

// Workspace: [split counters | (m, l) partials | O partials].  The counter
// region has a FIXED size at offset 0 so that no call's partials ever overlap
// another call's counters: counters must read zero on entry (the kernels
// return every counter they use to zero), whatever shapes earlier calls had.
WsLayout ws_layout(int batch, int Hq, int D, int max_splits) {
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  WsLayout w;
  w.cnt_off = 0;
  w.ml_off = sizeof(int) * static_cast<size_t>(kMaxCounters);
  w.o_off = w.ml_off + up(sizeof(float) * 2 * static_cast<size_t>(batch) * Hq * max_splits);
  w.total = w.o_off + up(sizeof(float) * static_cast<size_t>(batch) * Hq * max_splits * D);
  return w;
}

// Kernel choice and split plan of a call (validated arguments).
// - D = 512 with GQA a multiple of 8: the heads-as-columns kernel (8 heads
//   per workgroup, each K/V byte unpacked once), merged by a separate
//   kernel.
// - Otherwise the matrix-core kernel where it serves (D, G); at D = 512 it
//   takes at most 2 query heads per workgroup (2 heads x 8 quant groups
//   fill its 16 columns): the head subgroups of one kv head then read the
//   same K/V, concurrently and on one XCD, so the repeats are served mostly
//   from L2.  (The workspace bound of tq_sdpa_int4_workspace_size, planned
//   with the largest subgroup, covers this: more groups never means more
//   splits.)
// - Prefill of >= 64 queries: the K/V-tile kernels where they serve.
// - The VALU kernel under TQ_SDPA_IMPL=valu.
SdpaPlan plan_sdpa(int mode, int batch, int Hq, int Hkv, int D, int max_len, int gqa, int window,
                   int sb_dtype, int cap) {
  (void)Hq;
  const Options o = options();
  const bool prefill = mode == 2;
  SdpaPlan pl{};
  const bool hc = !o.sdpa_valu && D == 512 && gqa % 8 == 0 && hc_serves(sb_dtype);
  // the matrix-core kernel reads whole 32-row blocks of the cache
  const bool try_mfma = !o.sdpa_valu && cap >= kMfmaMinRows;
  int G = head_subgroup(gqa);
  // the matrix-core kernel takes at most 16 (head, quant group) columns:
  // halve the head subgroup until it serves the shape
  if (try_mfma && !hc)
    while (G > 1 && !mfma_serves(D, G, sb_dtype)) G /= 2;
  pl.G = G;
  pl.n_sub = gqa / G;
  const int64_t groups = static_cast<int64_t>(batch) * Hkv * pl.n_sub;
  // Prefill on the matrix-core kernel: pq consecutive queries share a
  // workgroup (its G * pq column sets fill the 16 MFMA columns), so each K/V
  // byte serves pq queries.  Split planning stays per query, and a group's
  // key range is the union of its windows (at most window + pq - 1 keys).
  int pq = 1;
  if (prefill && try_mfma && !hc && mfma_serves(D, G, sb_dtype)) {
    const int max_cols = D == 128 ? 8 : (D == 256 ? 4 : 2);  // G * pq the kernel serves
    while (G * pq * 2 <= max_cols && pq * 2 <= batch && mfma_serves(D, G * pq * 2, sb_dtype))
      pq *= 2;
  }
  pl.pq = pq;
  int eff_len = max_len;
  if (mode == 0 && window > 0) eff_len = std::min(max_len, window);
  if (prefill && window > 0) eff_len = std::min(max_len, window + pq - 1);
  // (a prefill's queries are many short-to-long sequences: no minimum split)
  const int min_splits = prefill ? 1 : min_splits_for(batch);
  pl.chunk = plan_chunk(eff_len, groups, min_splits);
  pl.max_splits = max_splits_bound(eff_len, groups, min_splits);
  pl.wl = ws_layout(batch, Hq, D, pl.max_splits);
  if (prefill && batch >= 64 && !o.prefill_splitk && prefill_tiles_serve(D, sb_dtype, gqa))
    pl.kernel = SdpaKernel::prefill_tiles;
  else if (hc)
    pl.kernel = SdpaKernel::hc;
  else if (try_mfma && mfma_serves(D, G * pq, sb_dtype))
    pl.kernel = SdpaKernel::mfma;
  else
    pl.kernel = SdpaKernel::valu;
  // Ragged batches of up to 64 sequences on the matrix-core kernel choose
  // their chunk on the device (ragged_job), among 1 .. max_splits chunks of
  // the longest sequence.  Every sequence is at least one job, so with two
  // or more workgroups' worth of (sequence, head) jobs per CU the grid
  // allows at most two chunks per sequence: fewer grid workgroups then go
  // without a job (each still costs its CU a dispatch and a load of the
  // lengths).
  pl.lpt = mode == 1 && batch <= 64 && pl.kernel == SdpaKernel::mfma;
  if (pl.lpt && groups >= 2 * static_cast<int64_t>(target_wgs()) && pl.max_splits > 2) {
    pl.max_splits = 2;
    const int64_t half = (static_cast<int64_t>(eff_len) + 1) / 2;
    pl.chunk = std::max<int>(pl.chunk, static_cast<int>((half + kChunkGranule - 1) / kChunkGranule * kChunkGranule));
    pl.wl = ws_layout(batch, Hq, D, pl.max_splits);
  }
  return pl;
}

const char* kernel_name(const SdpaPlan& pl, int D, int sb_dtype) {
  (void)sb_dtype;
  switch (pl.kernel) {
    case SdpaKernel::prefill_tiles:
      return (D != 512 && options().prefill_ws) ? "prefill_int4_ws_kernel" : "prefill_int4_kernel";
    case SdpaKernel::hc:
      return options().hc_one ? "sdpa_int4_hc_kernel" : "sdpa_int4_hc2_kernel";
    case SdpaKernel::mfma: return "sdpa_int4_mfma_kernel";
    default: return "sdpa_int4_kernel";
  }
}


namespace {

constexpr int kPrefetch = 4;  // row steps in flight per wave

template <int D, int G>
struct Geom {
  static constexpr int E = G <= 2 ? 32 : (G == 4 ? 16 : 8);  // dims per lane
  static constexpr int LPT = D / E;                          // lanes per key row
  static constexpr int TPS = 64 / LPT;                       // rows per wave step
  static constexpr int WPL = E / 8;                          // packed words per lane
  static constexpr int NG = D / 64;                          // quant groups per row
  static_assert(LPT <= 64 && 64 % LPT == 0, "bad geometry");
};

template <int WPL>
__device__ __forceinline__ void load_words(const uint32_t* p, uint32_t w[WPL]) {
  if constexpr (WPL == 4) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    w[0] = u.x; w[1] = u.y; w[2] = u.z; w[3] = u.w;
  } else if constexpr (WPL == 2) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    w[0] = u.x; w[1] = u.y;
  } else {
    w[0] = *p;
  }
}

// One key/value row slice of one lane: packed K and V words plus the
// scale/bias of the lane's quant group.  Pointers are pre-offset to the lane's
// words / group; t is the row index.
template <int D, int WPL, typename SB>
struct RowBuf {
  uint32_t kw[WPL], vw[WPL];
  SB ks, kb, vs, vb;
  __device__ __forceinline__ void load(const uint32_t* kq, const uint32_t* vq, const SB* ksp,
                                       const SB* kbp, const SB* vsp, const SB* vbp, int64_t t) {
    load_words<WPL>(kq + t * (D / 8), kw);
    load_words<WPL>(vq + t * (D / 8), vw);
    ks = ksp[t * (D / 64)];
    kb = kbp[t * (D / 64)];
    vs = vsp[t * (D / 64)];
    vb = vbp[t * (D / 64)];
  }
};

// The 8 nibbles of a word as floats, element order (nibble i at bits 4i).
__device__ __forceinline__ void unpack8(uint32_t w, float n[8]) {
  const uint32_t lo = w & 0x0F0F0F0Fu;         // nibbles 0,2,4,6 in bytes 0..3
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // nibbles 1,3,5,7
  n[0] = static_cast<float>(lo & 0xFF);
  n[1] = static_cast<float>(hi & 0xFF);
  n[2] = static_cast<float>((lo >> 8) & 0xFF);
  n[3] = static_cast<float>((hi >> 8) & 0xFF);
  n[4] = static_cast<float>((lo >> 16) & 0xFF);
  n[5] = static_cast<float>((hi >> 16) & 0xFF);
  n[6] = static_cast<float>(lo >> 24);
  n[7] = static_cast<float>(hi >> 24);
}

template <int D, int G, typename SB>
__global__ __launch_bounds__(kThreads) void sdpa_int4_kernel(SdpaParams p) {
  pin_args(p);
  using Gm = Geom<D, G>;
  constexpr int E = Gm::E, LPT = Gm::LPT, TPS = Gm::TPS, WPL = Gm::WPL, NG = Gm::NG;
  constexpr int RW = D / 8;  // packed words per row

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tok = lane / LPT, j = lane % LPT;
  const int grp = (j * E) >> 6;
  const int b = blockIdx.z, hy = blockIdx.y, split = blockIdx.x;
  const int kvh = hy / p.n_sub, sub = hy - kvh * p.n_sub;
  const int h0 = kvh * p.gqa + sub * G;

  const SplitRange rg = split_range(p, b, split);
  if (split >= rg.S) return;
  const int S = rg.S, t_begin = rg.t_begin, t_end = rg.t_end;

  const int64_t row0 = (static_cast<int64_t>(cache_batch(p, b)) * p.Hkv + kvh) * p.cap;
  const uint32_t* kq = p.kq + row0 * RW + j * WPL;
  const uint32_t* vq = p.vq + row0 * RW + j * WPL;
  const SB* ks = static_cast<const SB*>(p.ks) + row0 * NG + grp;
  const SB* kb = static_cast<const SB*>(p.kb) + row0 * NG + grp;
  const SB* vs = static_cast<const SB*>(p.vs) + row0 * NG + grp;
  const SB* vb = static_cast<const SB*>(p.vb) + row0 * NG + grp;

  // q slice of every head in the group, pre-scaled by scale*log2(e).  The
  // dtype branch is uniform and taken once; each lane reads E contiguous
  // elements with 16 B loads.
  float q[G][E], qsum[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const int64_t qoff = (static_cast<int64_t>(b) * p.Hq + h0 + h) * D + j * E;
    load_q_slice<E>(p.q, p.q_dtype, qoff, q[h]);
    qsum[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      q[h][i] *= p.scale_log2;
      qsum[h] += q[h][i];
    }
  }

  float m[G], l[G], ob[G], o[G][E];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
    ob[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < E; ++i) o[h][i] = 0.0f;
  }

  // Rows are consumed through a ring of kPrefetch register buffers: step u is
  // computed while the loads of the next kPrefetch-1 steps are in flight
  // (vmcnt retires them in order).  Step counts are made provably uniform
  // (readfirstlane) and every load is unconditional with a clamped row index,
  // so the waitcnt pass sees straight-line code and can wait for just the
  // oldest buffer instead of draining the queue.
  constexpr int kStride = kWaves * TPS;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int base0 = t_begin + wv * TPS;
  const int nsteps = base0 < t_end ? (t_end - base0 + kStride - 1) / kStride : 0;
  if (nsteps > 0) {
    const int last = t_end - 1;
    RowBuf<D, WPL, SB> buf[kPrefetch];
#pragma unroll
    for (int u = 0; u < kPrefetch; ++u)
      buf[u].load(kq, vq, ks, kb, vs, vb, min(base0 + u * kStride + tok, last));

    for (int s0 = 0; s0 < nsteps; s0 += kPrefetch) {
#pragma unroll
      for (int u = 0; u < kPrefetch; ++u) {
        const int step = s0 + u;
        if (step < nsteps) {  // uniform
          const bool valid = base0 + step * kStride + tok < t_end;
          const RowBuf<D, WPL, SB>& r = buf[u];
      const float ksc = sb_to_f32<SB>(r.ks), kbi = sb_to_f32<SB>(r.kb);
      const float vsc = sb_to_f32<SB>(r.vs), vbi = sb_to_f32<SB>(r.vb);
      float part[G];
#pragma unroll
      for (int h = 0; h < G; ++h) part[h] = 0.0f;
#pragma unroll
      for (int w = 0; w < WPL; ++w) {
        float n[8];
        unpack8(r.kw[w], n);
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int i = 0; i < 8; ++i) part[h] = fmaf(q[h][w * 8 + i], n[i], part[h]);
      }
#pragma unroll
      for (int h = 0; h < G; ++h) part[h] = ksc * part[h] + kbi * qsum[h];
#pragma unroll
      for (int h = 0; h < G; ++h) part[h] = group_sum<LPT>(part[h]);

      bool need = false;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        part[h] = valid ? part[h] : -INFINITY;
        need |= part[h] > m[h];
      }
      if (__any(need)) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float mn = fmaxf(m[h], part[h]);
          const float f = (mn == m[h]) ? 1.0f : fast_exp2(m[h] - mn);
          l[h] *= f;
          ob[h] *= f;
#pragma unroll
          for (int i = 0; i < E; ++i) o[h][i] *= f;
          m[h] = mn;
        }
      }
      float ps[G];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pp = valid ? fast_exp2(part[h] - m[h]) : 0.0f;
        l[h] += pp;
        ob[h] = fmaf(pp, vbi, ob[h]);
        ps[h] = pp * vsc;
      }
#pragma unroll
      for (int w = 0; w < WPL; ++w) {
        float n[8];
        unpack8(r.vw[w], n);
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int i = 0; i < 8; ++i) o[h][w * 8 + i] = fmaf(ps[h], n[i], o[h][w * 8 + i]);
      }
        }
        buf[u].load(kq, vq, ks, kb, vs, vb, min(base0 + (step + kPrefetch) * kStride + tok, last));
      }
    }
  }

  // ---- epilogue: fold bias sums, merge row groups, merge waves ---------------
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < E; ++i) o[h][i] += ob[h];

#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float mo = shfl_xor_f(m[h], off);
      const float lo2 = shfl_xor_f(l[h], off);
      const float M = fmaxf(m[h], mo);
      const float fs = merge_factor(m[h], M), fo = merge_factor(mo, M);
      l[h] = l[h] * fs + lo2 * fo;
#pragma unroll
      for (int i = 0; i < E; ++i) o[h][i] = o[h][i] * fs + shfl_xor_f(o[h][i], off) * fo;
      m[h] = M;
    }
  }

  using Fin = Finalize<G, D>;
  __shared__ __align__(16) float arena[Fin::kArena];
  if (tok == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int i = 0; i < E; ++i) Fin::o(arena, wave, h)[j * E + i] = o[h][i];
      if (j == 0) {
        Fin::m(arena, wave)[h] = m[h];
        Fin::l(arena, wave)[h] = l[h];
      }
    }
  }
  Fin::run(p, arena, static_cast<int64_t>(b) * p.Hq + h0, S, split, b * p.Hq + hy);
}

// ---- host side ---------------------------------------------------------------

template <int D, int G>
int launch_dg(const SdpaParams& p, int sb_dtype, dim3 grid, hipStream_t s) {
  if (sb_dtype == TQ_F16)
    sdpa_int4_kernel<D, G, __half><<<grid, kThreads, 0, s>>>(p);
  else
    sdpa_int4_kernel<D, G, float><<<grid, kThreads, 0, s>>>(p);
  TQ_CHECK_LAUNCH("sdpa_int4_kernel");
  return TQ_OK;
}

template <int D>
int launch_d(const SdpaParams& p, int G, int sb_dtype, dim3 grid, hipStream_t s) {
  switch (G) {
    case 1: return launch_dg<D, 1>(p, sb_dtype, grid, s);
    case 2: return launch_dg<D, 2>(p, sb_dtype, grid, s);
    case 4: return launch_dg<D, 4>(p, sb_dtype, grid, s);
    default: return launch_dg<D, 8>(p, sb_dtype, grid, s);
  }
}

int sdpa_common(const void* q, int q_dtype, const uint32_t* kq, const void* ks, const void* kb,
                const uint32_t* vq, const void* vs, const void* vb, int sb_dtype, float* out,
                int batch, int Hq, int Hkv, int D, int cap, int n, const int32_t* seq_lens,
                const int32_t* windows, int max_len, int gqa, float scale, int window,
                void* workspace, size_t ws_bytes, void* stream, const char* fn,
                int prefill = 0) {
  TQ_CHECK_ARG(valid_dtype(q_dtype), "%s: bad q_dtype %d", fn, q_dtype);
  TQ_CHECK_ARG(sb_dtype == TQ_F16 || sb_dtype == TQ_F32, "%s: sb_dtype must be f16 or f32", fn);
  if (D != 128 && D != 256 && D != 512) {
    set_error("%s: head_dim must be 128, 256 or 512 (got %d)", fn, D);
    return TQ_ERR_UNSUPPORTED;
  }
  TQ_CHECK_ARG(batch >= 1 && Hkv >= 1 && gqa >= 1, "%s: batch, num_kv_heads, gqa must be >= 1", fn);
  TQ_CHECK_ARG(Hq == Hkv * gqa, "%s: num_heads (%d) != num_kv_heads (%d) * gqa_factor (%d)", fn,
               Hq, Hkv, gqa);
  TQ_CHECK_ARG(window >= 0, "%s: sliding_window must be >= 0", fn);
  TQ_CHECK_ARG(max_len >= 0 && cap >= 1 && max_len <= cap,
               "%s: need 0 <= kv_len <= kv_capacity (got %d, %d)", fn, max_len, cap);
  TQ_CHECK_ARG(q && kq && ks && kb && vq && vs && vb && out, "%s: null tensor pointer", fn);
  TQ_CHECK_ARG(reinterpret_cast<uintptr_t>(kq) % 16 == 0 && reinterpret_cast<uintptr_t>(vq) % 16 == 0,
               "%s: k_quant / v_quant must be 16-byte aligned", fn);
  TQ_CHECK_ARG(reinterpret_cast<uintptr_t>(q) % 16 == 0, "%s: queries must be 16-byte aligned", fn);
  TQ_CHECK_ARG(std::isfinite(scale), "%s: scale must be finite", fn);

  const int mode = prefill ? 2 : (seq_lens ? 1 : 0);
  const SdpaPlan pl = plan_sdpa(mode, batch, Hq, Hkv, D, max_len, gqa, window, sb_dtype, cap);
  const int n_sub = pl.n_sub, pq = pl.pq, max_splits = pl.max_splits;
  const WsLayout wl = pl.wl;
  if (max_splits > 1) {
    if (!workspace || ws_bytes < wl.total) {
      set_error("%s: workspace of %zu bytes needed (got %zu)", fn, wl.total, ws_bytes);
      return TQ_ERR_WORKSPACE;
    }
    TQ_CHECK_ARG(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "%s: workspace must be 16-byte aligned", fn);
    // the split partials are addressed with 32-bit byte offsets
    TQ_CHECK_ARG(wl.total - wl.o_off < (size_t{1} << 31), "%s: split-K partials exceed 2 GiB", fn);
  }
  TQ_CHECK_ARG(Hkv * n_sub <= 65535 && batch <= 65535, "%s: grid too large", fn);
  TQ_CHECK_ARG(static_cast<int64_t>(batch) * Hq <= kMaxCounters || (prefill && max_splits == 1),
               "%s: batch (queries) * num_heads must be <= %lld", fn,
               static_cast<long long>(kMaxCounters));

  SdpaParams p{};
  p.q = q;
  p.q_dtype = q_dtype;
  p.kq = kq; p.ks = ks; p.kb = kb;
  p.vq = vq; p.vs = vs; p.vb = vb;
  p.out = out;
  char* ws = static_cast<char*>(workspace);
  p.ws_cnt = ws ? reinterpret_cast<int*>(ws + wl.cnt_off) : nullptr;
  p.ws_ml = ws ? reinterpret_cast<float*>(ws + wl.ml_off) : nullptr;
  p.ws_o = ws ? reinterpret_cast<float*>(ws + wl.o_off) : nullptr;
  p.Hq = Hq; p.Hkv = Hkv; p.cap = cap; p.gqa = gqa; p.n_sub = n_sub;
  p.n = prefill ? n : max_len;  // prefill: positions before the first query
  p.seq_lens = seq_lens;
  p.windows = windows;
  p.window = window;
  p.n_clamp = max_len;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.chunk = pl.chunk;
  p.max_splits = max_splits;
  p.prefill = prefill;
  p.pq = pq;
  p.nq = batch;
  // ragged batches of up to 64 sequences on the matrix-core kernel: chunk
  // chosen on the device from the lengths, longest-first workgroup order
  // (ragged_job); the grid and workspace stay sized for pl.max_splits
  p.lpt = pl.lpt ? 1 : 0;
  p.cus = target_wgs();

  dim3 grid(max_splits, Hkv * n_sub, (batch + pq - 1) / pq);
  p.cnt_stride = counter_stride(static_cast<int64_t>(grid.z) * Hq);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (pl.kernel) {
    case SdpaKernel::prefill_tiles:
      return launch_prefill_tiles(p, D, sb_dtype, s);
    case SdpaKernel::hc: {
      // 8 heads x 512 dims of partials per split: merged by a separate,
      // parallel kernel rather than one workgroup per kv head
      p.ext_merge = max_splits > 1 ? 1 : 0;
      const int r = launch_sdpa_hc(p, sb_dtype, grid, s);
      if (r != TQ_OK || !p.ext_merge) return r;
      return launch_merge_splits(p, D, batch, s);
    }
    case SdpaKernel::mfma:
      return launch_sdpa_mfma(p, D, pl.G * pq, sb_dtype, grid, s);
    default:
      switch (D) {
        case 128: return launch_d<128>(p, pl.G, sb_dtype, grid, s);
        case 256: return launch_d<256>(p, pl.G, sb_dtype, grid, s);
        default: return launch_d<512>(p, pl.G, sb_dtype, grid, s);
      }
  }
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" size_t tq_sdpa_int4_workspace_size(int batch, int num_heads, int num_kv_heads,
                                              int head_dim, int max_kv_len) {
  if (batch < 1 || num_kv_heads < 1 || num_heads < num_kv_heads || max_kv_len < 0) return 0;
  const int gqa = num_heads / num_kv_heads;
  const int G = head_subgroup(gqa);
  const int64_t groups = static_cast<int64_t>(batch) * num_kv_heads * (gqa / G);
  const int splits = max_splits_bound(max_kv_len, groups, min_splits_for(batch));
  return ws_layout(batch, num_heads, head_dim, splits).total;
}

extern "C" int tq_sdpa_int4_plan(int mode, int batch, int num_heads, int num_kv_heads,
                                 int head_dim, int max_kv_len, tq_dtype sb_dtype,
                                 int sliding_window, int* splits, int* chunk_keys,
                                 char* kernel, size_t kernel_bytes) {
  clear_error();
  const char* fn = "tq_sdpa_int4_plan";
  TQ_CHECK_ARG(mode >= 0 && mode <= 2, "%s: mode must be 0 (decode), 1 (ragged) or 2 (prefill)", fn);
  TQ_CHECK_ARG(sb_dtype == TQ_F16 || sb_dtype == TQ_F32, "%s: sb_dtype must be f16 or f32", fn);
  TQ_CHECK_ARG(head_dim == 128 || head_dim == 256 || head_dim == 512, "%s: bad head_dim %d", fn,
               head_dim);
  TQ_CHECK_ARG(batch >= 1 && num_kv_heads >= 1 && num_heads >= num_kv_heads &&
                   num_heads % num_kv_heads == 0 && max_kv_len >= 0 && sliding_window >= 0,
               "%s: bad shape", fn);
  const SdpaPlan pl = plan_sdpa(mode, batch, num_heads, num_kv_heads, head_dim, max_kv_len,
                                num_heads / num_kv_heads, sliding_window, sb_dtype, max_kv_len);
  if (splits) *splits = pl.max_splits;
  if (chunk_keys) *chunk_keys = pl.chunk;
  if (kernel && kernel_bytes > 0) {
    const char* name = kernel_name(pl, head_dim, sb_dtype);
    std::snprintf(kernel, kernel_bytes, "%s", name);
  }
  return TQ_OK;
}

extern "C" int tq_reload_options(void) {
  clear_error();
  options();  // the first read, if not done yet
  read_options();
  return TQ_OK;
}

// ---- decode with library-owned scratch (no caller workspace) -----------------
//
// tq_sdpa_int4_noalloc runs the same kernels as tq_sdpa_int4 with the split-K
// workspace in a file-scope device array instead of a caller buffer, for
// callers that cannot allocate (HIP graph capture, allocation-free serving
// loops).  Each GPU the library runs on holds its own copy of `scratch` until
// the process ends.  Host code never passes the array's name to a kernel: it
// is a host-side stand-in, not a device address.  The device address comes
// from hipGetSymbolAddress, once per device with that device current, and is
// kept per device.
namespace {
constexpr size_t kScratchBytes = size_t{8} << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Zeroes the split counters at the head of a fresh scratch array (the
// array is zero at module load already; this makes the starting state
// explicit).  A kernel, not hipMemsetAsync, so that a first call made under
// graph capture records an ordinary kernel node.
__global__ void zero_words_kernel(int* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// This device's scratch address (set up on the first call on the device).
int device_scratch(hipStream_t stream, void** out) {
  int dev = 0;
  TQ_CHECK_HIP(hipGetDevice(&dev));
  TQ_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "tq_sdpa_int4_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    TQ_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    TQ_CHECK_ARG(ptr != nullptr, "tq_sdpa_int4_noalloc: no device address for the scratch array");
    const int n = static_cast<int>(kMaxCounters);
    zero_words_kernel<<<(n + 255) / 256, 256, 0, stream>>>(static_cast<int*>(ptr), n);
    TQ_CHECK_LAUNCH("zero_words_kernel");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return TQ_OK;
}
}  // namespace

extern "C" int tq_sdpa_int4_noalloc(const void* q, tq_dtype q_dtype, const uint32_t* k_quant,
                                    const void* k_scales, const void* k_biases,
                                    const uint32_t* v_quant, const void* v_scales,
                                    const void* v_biases, tq_dtype sb_dtype, float* out,
                                    int num_heads, int num_kv_heads, int head_dim, int kv_len,
                                    int kv_capacity, int gqa_factor, float scale,
                                    int sliding_window, void* stream) {
  clear_error();
  const char* fn = "tq_sdpa_int4_noalloc";
  // the scratch bound is checked before any device call
  if ((head_dim == 128 || head_dim == 256 || head_dim == 512) && num_kv_heads >= 1 &&
      gqa_factor >= 1 && num_heads == num_kv_heads * gqa_factor && kv_len >= 0 &&
      sliding_window >= 0 && (sb_dtype == TQ_F16 || sb_dtype == TQ_F32)) {
    const SdpaPlan pl = plan_sdpa(0, 1, num_heads, num_kv_heads, head_dim, kv_len, gqa_factor,
                                  sliding_window, sb_dtype, kv_capacity);
    if (pl.max_splits > 1 && pl.wl.total > kScratchBytes) {
      set_error("%s: this shape needs %zu bytes of split-K scratch, more than the library's "
                "static %zu bytes; call tq_sdpa_int4 with a workspace instead",
                fn, pl.wl.total, kScratchBytes);
      return TQ_ERR_UNSUPPORTED;
    }
  }
  void* ws = nullptr;
  const int st = device_scratch(static_cast<hipStream_t>(stream), &ws);
  if (st != TQ_OK) return st;
  return sdpa_common(q, q_dtype, k_quant, k_scales, k_biases, v_quant, v_scales, v_biases,
                     sb_dtype, out, 1, num_heads, num_kv_heads, head_dim, kv_capacity, kv_len,
                     nullptr, nullptr, kv_len, gqa_factor, scale, sliding_window, ws,
                     kScratchBytes, stream, fn);
}

extern "C" int tq_sdpa_int4(const void* q, tq_dtype q_dtype, const uint32_t* k_quant,
                            const void* k_scales, const void* k_biases, const uint32_t* v_quant,
                            const void* v_scales, const void* v_biases, tq_dtype sb_dtype,
                            float* out, int num_heads, int num_kv_heads, int head_dim, int kv_len,
                            int kv_capacity, int gqa_factor, float scale, int sliding_window,
                            void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return sdpa_common(q, q_dtype, k_quant, k_scales, k_biases, v_quant, v_scales, v_biases,
                     sb_dtype, out, 1, num_heads, num_kv_heads, head_dim, kv_capacity, kv_len,
                     nullptr, nullptr, kv_len, gqa_factor, scale, sliding_window, workspace,
                     workspace_bytes, stream, "tq_sdpa_int4");
}

extern "C" int tq_sdpa_int4_ragged(const void* q, tq_dtype q_dtype, const uint32_t* k_quant,
                                   const void* k_scales, const void* k_biases,
                                   const uint32_t* v_quant, const void* v_scales,
                                   const void* v_biases, tq_dtype sb_dtype, float* out, int batch,
                                   int num_heads, int num_kv_heads, int head_dim, int kv_capacity,
                                   const int32_t* seq_lens, const int32_t* windows, int max_kv_len,
                                   int gqa_factor, float scale, int sliding_window,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  TQ_CHECK_ARG(seq_lens != nullptr, "tq_sdpa_int4_ragged: seq_lens is NULL");
  return sdpa_common(q, q_dtype, k_quant, k_scales, k_biases, v_quant, v_scales, v_biases,
                     sb_dtype, out, batch, num_heads, num_kv_heads, head_dim, kv_capacity,
                     max_kv_len, seq_lens, windows, max_kv_len, gqa_factor, scale,
                     sliding_window, workspace, workspace_bytes, stream, "tq_sdpa_int4_ragged");
}

extern "C" int tq_sdpa_int4_prefill(const void* q, tq_dtype q_dtype, const uint32_t* k_quant,
                                    const void* k_scales, const void* k_biases,
                                    const uint32_t* v_quant, const void* v_scales,
                                    const void* v_biases, tq_dtype sb_dtype, float* out,
                                    int num_heads, int num_kv_heads, int head_dim, int n_prior,
                                    int n_new, int kv_capacity, int gqa_factor, float scale,
                                    int sliding_window, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  clear_error();
  const char* fn = "tq_sdpa_int4_prefill";
  TQ_CHECK_ARG(n_prior >= 0 && n_new >= 0, "%s: n_prior and n_new must be >= 0", fn);
  TQ_CHECK_ARG(static_cast<int64_t>(n_prior) + n_new <= kv_capacity,
               "%s: n_prior + n_new (%d + %d) exceeds kv_capacity %d", fn, n_prior, n_new,
               kv_capacity);
  if (n_new == 0) return TQ_OK;
  TQ_CHECK_ARG(n_new <= 65535, "%s: at most 65535 queries per call", fn);
  return sdpa_common(q, q_dtype, k_quant, k_scales, k_biases, v_quant, v_scales, v_biases,
                     sb_dtype, out, n_new, num_heads, num_kv_heads, head_dim, kv_capacity,
                     n_prior, nullptr, nullptr, n_prior + n_new, gqa_factor, scale,
                     sliding_window, workspace, workspace_bytes, stream, fn, 1);
}
