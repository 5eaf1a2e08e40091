/*
 * C restatement of the reference's int4-KV decode-attention algorithm.
 *
 * TEST INFRASTRUCTURE ONLY: compiled into oracle/libtq_oracle.so and loaded
 * by tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py as
 * the checker / the timed CPU baseline.  The shipped library never links it.
 *
 * Built with -ffp-contract=off so every float32 operation rounds exactly as
 * written (the bit-exact quantize contract needs IEEE division and rint with
 * no fused multiply-add).
 *
 *   tqo_quantize_int4   MLX affine quantize(x, 64, 4), CPU rule (rint, IEEE
 *                       fp32 division); call sites
 *                       engine/gemma4_multilayer.cpp:228-229,
 *                       tests/test_sdpa_int4.cpp:25-26.
 *   tqo_sdpa_int4_f64   dequantize (lib/turboquant.metal:719) + softmax
 *                       attention in double, GQA h/gqa (:745), window rule
 *                       (:779), zero denominator -> 0 (:886).
 *   tqo_sdpa_dequant_f32
 *                       the reference's fallback/oracle composition
 *                       (tests/test_sdpa_int4.cpp:31-42,
 *                       engine/gemma4_multilayer.cpp:307-308,349): materialise
 *                       fp32 K and V, then fp32 softmax attention, OpenMP
 *                       over (head, key-chunk) with a log-sum-exp merge.  This
 *                       is the CPU baseline timed beside the GPU.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define TQO_GS 64

/* mode 0: MLX rule; mode 1: literal min/max rule (scale=(max-min)/15, bias=min) */
void tqo_quantize_int4(const float* x, int64_t rows, int D, int mode,
                       uint32_t* wq, float* scales, float* biases) {
  const float n_bins = 15.0f, eps = 1e-7f;
  const int ng = D / TQO_GS;
  for (int64_t r = 0; r < rows; ++r) {
    for (int g = 0; g < ng; ++g) {
      const float* w = x + r * D + g * TQO_GS;
      float mx = -INFINITY, mn = INFINITY;
      for (int j = 0; j < TQO_GS; ++j) {
        mx = w[j] > mx ? w[j] : mx;
        mn = w[j] < mn ? w[j] : mn;
      }
      float scale, bias;
      float d = (mx - mn) / n_bins;
      scale = d < eps ? eps : d;
      if (mode == 0) {
        int side = fabsf(mn) > fabsf(mx);
        scale = side ? scale : -scale;
        float edge = side ? mn : mx;
        float q0 = rintf(edge / scale);
        bias = 0.0f;
        if (q0 != 0.0f) {
          scale = edge / q0;
          bias = edge;
        }
      } else {
        bias = mn;
      }
      for (int j = 0; j < TQO_GS / 8; ++j) {
        uint32_t word = 0;
        for (int k = 0; k < 8; ++k) {
          float v = rintf((w[j * 8 + k] - bias) / scale);
          v = v < 0.0f ? 0.0f : (v > n_bins ? n_bins : v);
          word |= ((uint32_t)v) << (4 * k);
        }
        wq[r * (D / 8) + g * 8 + j] = word;
      }
      scales[r * ng + g] = scale;
      biases[r * ng + g] = bias;
    }
  }
}

static inline double deq_elem(const uint32_t* wq, const float* s, const float* b, int d) {
  uint32_t n = (wq[d >> 3] >> (4 * (d & 7))) & 0xFu;
  return (double)s[d / TQO_GS] * (double)n + (double)b[d / TQO_GS];
}

/* q: (Hq, D) float; caches (Hkv, cap, .) with scales/biases already widened
 * to float; attends rows [lo, n) of each kv head.  out (Hq, D) double. */
void tqo_sdpa_int4_f64(const float* q, const uint32_t* kq, const float* ks, const float* kb,
                       const uint32_t* vq, const float* vs, const float* vb,
                       int Hq, int Hkv, int D, int cap, int n, int gqa, float scale,
                       int window, double* out) {
  const int lo = window > 0 ? (n - window > 0 ? n - window : 0) : 0;
  const int ng = D / TQO_GS, nw = D / 8;
  double* sc = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
  for (int h = 0; h < Hq; ++h) {
    const int kvh = h / gqa;
    double* o = out + (size_t)h * D;
    for (int d = 0; d < D; ++d) o[d] = 0.0;
    if (kvh >= Hkv || n - lo <= 0) continue;
    double m = -INFINITY;
    for (int t = lo; t < n; ++t) {
      const size_t row = (size_t)kvh * cap + t;
      double acc = 0.0;
      for (int d = 0; d < D; ++d)
        acc += (double)q[(size_t)h * D + d] * deq_elem(kq + row * nw, ks + row * ng, kb + row * ng, d);
      sc[t - lo] = acc * (double)scale;
      if (sc[t - lo] > m) m = sc[t - lo];
    }
    double den = 0.0;
    for (int t = lo; t < n; ++t) {
      const size_t row = (size_t)kvh * cap + t;
      double p = exp(sc[t - lo] - m);
      den += p;
      for (int d = 0; d < D; ++d)
        o[d] += p * deq_elem(vq + row * nw, vs + row * ng, vb + row * ng, d);
    }
    for (int d = 0; d < D; ++d) o[d] = den == 0.0 ? 0.0 : o[d] / den;
  }
  free(sc);
}

/* ---------------------------------------------------------------------------
 * CPU baseline: dequantize to fp32 (materialised, as MLX dequantize does) and
 * run fp32 softmax attention.  kdq/vdq are caller-provided (Hkv, n, D) fp32
 * scratch buffers; chunk partials live in a malloc'd buffer.
 * ------------------------------------------------------------------------- */
void tqo_sdpa_dequant_f32(const float* q, const uint32_t* kq, const float* ks, const float* kb,
                          const uint32_t* vq, const float* vs, const float* vb,
                          int Hq, int Hkv, int D, int cap, int n, int gqa, float scale,
                          int window, float* kdq, float* vdq, float* out, int threads) {
  const int lo = window > 0 ? (n - window > 0 ? n - window : 0) : 0;
  const int L = n - lo;
  const int ng = D / TQO_GS, nw = D / 8;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#endif
  /* 1. dequantize (the materialisation MLX performs) */
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < (int64_t)Hkv * L; ++r) {
    const int kvh = (int)(r / L), t = (int)(r % L) + lo;
    const size_t src = (size_t)kvh * cap + t;
    float* kd = kdq + (size_t)r * D;
    float* vd = vdq + (size_t)r * D;
    for (int d = 0; d < D; ++d) {
      const uint32_t sh = 4 * (d & 7);
      const float kn = (float)((kq[src * nw + (d >> 3)] >> sh) & 0xFu);
      const float vn = (float)((vq[src * nw + (d >> 3)] >> sh) & 0xFu);
      kd[d] = ks[src * ng + d / TQO_GS] * kn + kb[src * ng + d / TQO_GS];
      vd[d] = vs[src * ng + d / TQO_GS] * vn + vb[src * ng + d / TQO_GS];
    }
  }
  /* 2. attention: (head, chunk) tasks, each an online-softmax partial */
  const int CH = 1024;
  const int nchunk = L > 0 ? (L + CH - 1) / CH : 1;
  float* part = (float*)malloc(sizeof(float) * (size_t)Hq * nchunk * (D + 2));
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t task = 0; task < (int64_t)Hq * nchunk; ++task) {
    const int h = (int)(task / nchunk), c = (int)(task % nchunk);
    const int kvh = h / gqa;
    float* pr = part + (size_t)task * (D + 2);
    float m = -INFINITY, l = 0.0f;
    for (int d = 0; d < D; ++d) pr[2 + d] = 0.0f;
    const int t0 = c * CH, t1 = (t0 + CH < L) ? t0 + CH : L;
    const float* qh = q + (size_t)h * D;
    for (int t = t0; t < t1 && kvh < Hkv; ++t) {
      const float* kd = kdq + ((size_t)kvh * L + t) * D;
      const float* vd = vdq + ((size_t)kvh * L + t) * D;
      float s = 0.0f;
      for (int d = 0; d < D; ++d) s += qh[d] * kd[d];
      s *= scale;
      if (s > m) {
        const float f = expf(m - s);
        l *= f;
        for (int d = 0; d < D; ++d) pr[2 + d] *= f;
        m = s;
      }
      const float p = expf(s - m);
      l += p;
      for (int d = 0; d < D; ++d) pr[2 + d] += p * vd[d];
    }
    pr[0] = m;
    pr[1] = l;
  }
  for (int h = 0; h < Hq; ++h) {
    float M = -INFINITY;
    for (int c = 0; c < nchunk; ++c) {
      const float mc = part[((size_t)h * nchunk + c) * (D + 2)];
      M = mc > M ? mc : M;
    }
    float l = 0.0f;
    float* o = out + (size_t)h * D;
    for (int d = 0; d < D; ++d) o[d] = 0.0f;
    for (int c = 0; c < nchunk && M > -INFINITY; ++c) {
      const float* pr = part + ((size_t)h * nchunk + c) * (D + 2);
      if (pr[1] == 0.0f) continue;
      const float f = expf(pr[0] - M);
      l += pr[1] * f;
      for (int d = 0; d < D; ++d) o[d] += pr[2 + d] * f;
    }
    for (int d = 0; d < D; ++d) o[d] = l == 0.0f ? 0.0f : o[d] / l;
  }
  free(part);
}

int tqo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
