// sdpa_int4 through the C++ API of include/turboquant.h, mirroring the
// reference's tests/test_sdpa_int4.cpp: random Q/K/V, quantize(K|V, 64, 4),
// the reference composition dequantize + softmax attention (here in double on
// the host) against the fused kernel.  Exits 0 on pass.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "turboquant.h"

using turboquant::array;
using turboquant::Dtype;

static int run_case(int nh, int nkv, int N, int hd, int window, std::mt19937& gen) {
  const int gqa = nh / nkv;
  const float scale = 1.0f;
  std::normal_distribution<float> nd(0.0f, 1.0f);
  std::vector<float> q(nh * hd), k(static_cast<size_t>(nkv) * N * hd), v(k.size());
  for (auto& x : q) x = nd(gen);
  for (auto& x : k) x = nd(gen);
  for (auto& x : v) x = nd(gen);
  printf("Testing sdpa_int4: nh=%d nkv=%d N=%d hd=%d gqa=%d window=%d\n", nh, nkv, N, hd, gqa, window);

  array Q = array::from_host(q.data(), {nh, hd}, Dtype::float32);
  array K = array::from_host(k.data(), {nkv, N, hd}, Dtype::float32);
  array V = array::from_host(v.data(), {nkv, N, hd}, Dtype::float32);
  auto kq = turboquant::quantize(K, 64, 4);
  auto vq = turboquant::quantize(V, 64, 4);
  array Kd = turboquant::dequantize(kq[0], kq[1], kq[2], 64, 4);
  array Vd = turboquant::dequantize(vq[0], vq[1], vq[2], 64, 4);
  array fused = turboquant::sdpa_int4(Q, kq[0], kq[1], kq[2], vq[0], vq[1], vq[2], gqa, scale, window);

  std::vector<float> kd(k.size()), vd(v.size()), out(nh * hd);
  Kd.to_host(kd.data());
  Vd.to_host(vd.data());
  fused.to_host(out.data());

  // reference: softmax(scale q.k) v over the kept keys, in double
  const int lo = window > 0 ? std::max(0, N - window) : 0;
  double max_err = 0.0, ref_norm = 0.0;
  std::vector<double> ref(nh * hd, 0.0);
  for (int h = 0; h < nh; ++h) {
    const int kv = h / gqa;
    std::vector<double> s(N);
    double m = -INFINITY;
    for (int n = lo; n < N; ++n) {
      double acc = 0.0;
      for (int d = 0; d < hd; ++d)
        acc += static_cast<double>(q[h * hd + d]) * kd[(static_cast<size_t>(kv) * N + n) * hd + d];
      s[n] = scale * acc;
      m = std::max(m, s[n]);
    }
    double l = 0.0;
    for (int n = lo; n < N; ++n) l += std::exp(s[n] - m);
    for (int n = lo; n < N; ++n) {
      const double p = std::exp(s[n] - m) / l;
      for (int d = 0; d < hd; ++d)
        ref[h * hd + d] += p * vd[(static_cast<size_t>(kv) * N + n) * hd + d];
    }
  }
  for (int i = 0; i < nh * hd; ++i) {
    max_err = std::max(max_err, std::fabs(ref[i] - out[i]));
    ref_norm += ref[i] * ref[i];
  }
  ref_norm = std::sqrt(ref_norm);
  printf("Reference norm:  %.4f\nMax error:       %.6e\n", ref_norm, max_err);
  printf("Ref  [0, :4]: %.4f %.4f %.4f %.4f\n", ref[0], ref[1], ref[2], ref[3]);
  printf("Fused[0, :4]: %.4f %.4f %.4f %.4f\n", out[0], out[1], out[2], out[3]);
  const bool pass = max_err < 2e-3;
  printf("%s (max_err=%.6e)\n\n", pass ? "PASS" : "FAIL", max_err);
  return pass ? 0 : 1;
}

// The same call three ways on the same inputs: the library's workspace on
// the null stream, on two streams running concurrently (each stream gets its
// own workspace), and with a caller-owned workspace.  All outputs must be
// bit-identical.
static int run_streams_case(std::mt19937& gen) {
  const int nh = 32, nkv = 16, N = 20000, hd = 256, gqa = nh / nkv;
  std::normal_distribution<float> nd(0.0f, 1.0f);
  std::vector<float> q(nh * hd), k(static_cast<size_t>(nkv) * N * hd), v(k.size());
  for (auto& x : q) x = nd(gen);
  for (auto& x : k) x = nd(gen);
  for (auto& x : v) x = nd(gen);
  printf("Testing sdpa_int4 on concurrent streams and with a caller workspace: N=%d\n", N);
  array Q = array::from_host(q.data(), {nh, hd}, Dtype::float32);
  array K = array::from_host(k.data(), {nkv, N, hd}, Dtype::float32);
  array V = array::from_host(v.data(), {nkv, N, hd}, Dtype::float32);
  auto kq = turboquant::quantize(K, 64, 4);
  auto vq = turboquant::quantize(V, 64, 4);
  array ref = turboquant::sdpa_int4(Q, kq[0], kq[1], kq[2], vq[0], vq[1], vq[2], gqa);
  hipStream_t s1 = nullptr, s2 = nullptr;
  if (hipStreamCreate(&s1) != hipSuccess || hipStreamCreate(&s2) != hipSuccess) return 1;
  array o1 = array::empty({nh, hd}, Dtype::float32), o2 = array::empty({nh, hd}, Dtype::float32);
  array o3 = array::empty({nh, hd}, Dtype::float32);
  for (int rep = 0; rep < 3; ++rep) {
    turboquant::sdpa_int4_into(o1, Q, kq[0], kq[1], kq[2], vq[0], vq[1], vq[2], gqa, 1.0f, 0, -1, s1);
    turboquant::sdpa_int4_into(o2, Q, kq[0], kq[1], kq[2], vq[0], vq[1], vq[2], gqa, 1.0f, 0, -1, s2);
  }
  const size_t wsb = turboquant::sdpa_int4_workspace_size(1, nh, nkv, hd, N);
  void* ws = nullptr;
  if (hipMalloc(&ws, wsb) != hipSuccess || hipMemset(ws, 0, wsb) != hipSuccess) return 1;
  turboquant::sdpa_int4_into(o3, Q, kq[0], kq[1], kq[2], vq[0], vq[1], vq[2], gqa, 1.0f, 0, -1,
                             ws, wsb, s2);
  turboquant::synchronize(s1);
  turboquant::synchronize(s2);
  turboquant::synchronize();
  std::vector<float> a(nh * hd), b(nh * hd), c(nh * hd), d(nh * hd);
  ref.to_host(a.data());
  o1.to_host(b.data());
  o2.to_host(c.data());
  o3.to_host(d.data());
  const size_t bytes = a.size() * sizeof(float);
  const bool pass = std::memcmp(a.data(), b.data(), bytes) == 0 &&
                    std::memcmp(a.data(), c.data(), bytes) == 0 &&
                    std::memcmp(a.data(), d.data(), bytes) == 0;
  (void)hipFree(ws);
  (void)hipStreamDestroy(s1);
  (void)hipStreamDestroy(s2);
  printf("%s (outputs %s)\n\n", pass ? "PASS" : "FAIL", pass ? "bit-identical" : "differ");
  return pass ? 0 : 1;
}

int main() {
  turboquant::set_metallib_path("unused");
  std::mt19937 gen(1234);
  int fails = 0;
  fails += run_case(16, 16, 10, 256, 0, gen);      // the reference test's shape
  fails += run_case(32, 16, 786, 256, 1024, gen);  // sliding layer
  fails += run_case(32, 4, 300, 512, 0, gen);      // global layer
  fails += run_case(2, 1, 33, 128, 0, gen);        // tiny decode (the reference test shape)
  fails += run_case(32, 16, 3000, 256, 1024, gen); // window active
  fails += run_streams_case(gen);
  return fails == 0 ? 0 : 1;
}
