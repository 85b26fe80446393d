// moe_ffn_hip (the moe_ffn_cuda-signature shim) against a double-precision CPU evaluation of the
// MoE FFN: the procedure of the reference's tools/moe_ffn_test.cu (E 8, k 2, d 96, d_ff 160, weights
// N(0, 0.3), inputs 3 x N(0, 0.3), renorm and raw gates, T in {1, 2, 5, 16, 17, 40}, pass when
// max |error| < 1e-4), here run through the HIP path. Built by ember.cpp_amd/Makefile; run by
// tests/test_gpu_compat.py. Prints one line per case and "all ok" on success.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <random>
#include <vector>

#include "ember_moe_compat.hpp"

#define CHECK(x)                                                            \
  do {                                                                      \
    if ((x) != hipSuccess) {                                                \
      std::printf("HIP error %s at line %d\n", #x, __LINE__);               \
      return 2;                                                             \
    }                                                                       \
  } while (0)

int main() {
  const int E = 8, k = 2, d = 96, d_ff = 160;
  std::mt19937 rng(3);
  std::normal_distribution<float> nd(0.f, 0.3f);
  auto fill = [&](std::vector<float>& v) {
    for (auto& x : v) x = nd(rng);
  };
  std::vector<float> R((size_t)E * d), G((size_t)E * d_ff * d), U(G.size()), D((size_t)E * d * d_ff);
  fill(R);
  fill(G);
  fill(U);
  fill(D);
  float *dR, *dG, *dU, *dD;
  CHECK(hipMalloc(&dR, R.size() * 4));
  CHECK(hipMalloc(&dG, G.size() * 4));
  CHECK(hipMalloc(&dU, U.size() * 4));
  CHECK(hipMalloc(&dD, D.size() * 4));
  CHECK(hipMemcpy(dR, R.data(), R.size() * 4, hipMemcpyHostToDevice));
  CHECK(hipMemcpy(dG, G.data(), G.size() * 4, hipMemcpyHostToDevice));
  CHECK(hipMemcpy(dU, U.data(), U.size() * 4, hipMemcpyHostToDevice));
  CHECK(hipMemcpy(dD, D.data(), D.size() * 4, hipMemcpyHostToDevice));
  int fails = 0;
  for (int renorm = 1; renorm >= 0; --renorm) {
    for (int T : {1, 2, 5, 16, 17, 40}) {
      std::vector<float> x((size_t)T * d);
      for (auto& v : x) v = nd(rng) * 3.0f;
      std::vector<double> ref((size_t)T * d, 0.0);
      for (int t = 0; t < T; ++t) {
        const float* xt = x.data() + (size_t)t * d;
        std::vector<double> r(E);
        for (int e = 0; e < E; ++e) {
          double s = 0;
          for (int i = 0; i < d; ++i) s += (double)R[(size_t)e * d + i] * xt[i];
          r[e] = s;
        }
        std::vector<int> sel;
        std::vector<bool> taken(E, false);
        for (int j = 0; j < k; ++j) {
          int best = -1;
          for (int e = 0; e < E; ++e)
            if (!taken[e] && (best < 0 || r[e] > r[best])) best = e;
          taken[best] = true;
          sel.push_back(best);
        }
        double mx = -1e300, z = 0;
        for (int e = 0; e < E; ++e)
          if (!renorm || taken[e]) mx = std::max(mx, r[e]);
        for (int e = 0; e < E; ++e)
          if (!renorm || taken[e]) z += std::exp(r[e] - mx);
        for (int e : sel) {
          const double gate = std::exp(r[e] - mx) / z;
          std::vector<double> hid(d_ff);
          for (int i = 0; i < d_ff; ++i) {
            double gv = 0, uv = 0;
            for (int c = 0; c < d; ++c) {
              gv += (double)G[((size_t)e * d_ff + i) * d + c] * xt[c];
              uv += (double)U[((size_t)e * d_ff + i) * d + c] * xt[c];
            }
            hid[i] = gv / (1.0 + std::exp(-gv)) * uv;
          }
          for (int o = 0; o < d; ++o) {
            double acc = 0;
            for (int i = 0; i < d_ff; ++i) acc += (double)D[((size_t)e * d + o) * d_ff + i] * hid[i];
            ref[(size_t)t * d + o] += gate * acc;
          }
        }
      }
      float *dx, *dout, *dscratch;
      CHECK(hipMalloc(&dx, x.size() * 4));
      CHECK(hipMalloc(&dout, x.size() * 4));
      CHECK(hipMalloc(&dscratch, moe_ffn_scratch_floats(T, d, d_ff, E, k) * 4));
      CHECK(hipMemcpy(dx, x.data(), x.size() * 4, hipMemcpyHostToDevice));
      moe_ffn_hip(dx, T, d, d_ff, E, k, renorm != 0, dR, dG, dU, dD, dscratch, dout, nullptr);
      std::vector<float> out(x.size());
      CHECK(hipMemcpy(out.data(), dout, out.size() * 4, hipMemcpyDeviceToHost));
      double err = 0;
      for (size_t i = 0; i < out.size(); ++i) err = std::max(err, std::fabs(out[i] - ref[i]));
      const bool ok = err < 1e-4;
      fails += !ok;
      std::printf("%s T %2d max |err| %.2e %s\n", renorm ? "renorm" : "raw   ", T, err, ok ? "ok" : "FAIL");
      CHECK(hipFree(dx));
      CHECK(hipFree(dout));
      CHECK(hipFree(dscratch));
    }
  }
  std::printf(fails ? "FAILED %d\n" : "all ok\n", fails);
  return fails != 0;
}
