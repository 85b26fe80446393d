// Checks the engine-facing shim (include/ember_moe_compat.hpp: moe_ffn_hip, moe_ffn_scratch_floats,
// moe_ffn_hip_typed) on layers drawn from this project's counter-based generator
// (ember_fill_normal, libember_moe_host.so), against the CPU oracle (oracle/liboracle.so, loaded with
// dlopen from the path given as argv[1]; test infrastructure only).
//
// Cases: two F32 layer shapes (and a wider-router one with k = 4) at batch sizes
// from one token to past the decode / prefill crossover, renorm and raw gates, held to the F32 bar
// (max |err| <= 1e-4 and rel-L2 <= 1e-5); one Q8_0 layer through moe_ffn_hip_typed at the 2e-3 rel-L2
// bar against the oracle on the dequantized stacks.
//
// HIP-graph capture (the engine captures its decode step, model.cpp:1246, 1321): for the decode batch
// the shim call is captured once on a side stream, and the graph is replayed three times with
// different inputs copied into the captured x buffer and an eager shim call on other buffers between
// replays; every replay must equal the eager call on the same input bit for bit.
//
// Exit status 0 and a last line "all ok" on success; one line per case.
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "ember_moe.h"
#include "ember_moe_compat.hpp"

namespace {

using OracleLayerFn = void (*)(const float*, int, int, int, int, int, int, int, const float*, int, int, float,
                               const float*, const float*, const float*, const float*, int, const float*,
                               const float*, const float*, float*, int);
OracleLayerFn oracle_layer = nullptr;

bool hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  std::printf("HIP error in %s: %s\n", what, hipGetErrorString(e));
  return false;
}

// A device copy of a host vector, freed by the owner.
struct Dev {
  void* p = nullptr;
  size_t n = 0;
  bool put(const void* src, size_t bytes) {
    n = bytes;
    return hip_ok(hipMalloc(&p, bytes), "hipMalloc") && hip_ok(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice), "H2D");
  }
  bool alloc(size_t bytes) {
    n = bytes;
    return hip_ok(hipMalloc(&p, bytes), "hipMalloc");
  }
  ~Dev() {
    if (p) (void)hipFree(p);
  }
  float* f() const { return static_cast<float*>(p); }
};

struct Shape {
  int d, d_ff, E, k;
  uint64_t seed;
};

// Layer tensors on the host in F32; gate/up/down are the values the device stacks decode to.
struct HostLayer {
  Shape s;
  std::vector<float> router, gate, up, down;
};

HostLayer make_layer(const Shape& s) {
  HostLayer h{s, {}, {}, {}, {}};
  h.router.resize((size_t)s.E * s.d);
  h.gate.resize((size_t)s.E * s.d_ff * s.d);
  h.up.resize(h.gate.size());
  h.down.resize((size_t)s.E * s.d * s.d_ff);
  // streams 11..14 of the seed; router scale 1/sqrt(d) keeps the routing non-degenerate
  ember_fill_normal(h.router.data(), (int64_t)h.router.size(), s.seed, 11, 0.0f, 1.0f / std::sqrt((float)s.d));
  ember_fill_normal(h.gate.data(), (int64_t)h.gate.size(), s.seed, 12, 0.0f, 0.05f);
  ember_fill_normal(h.up.data(), (int64_t)h.up.size(), s.seed, 13, 0.0f, 0.05f);
  ember_fill_normal(h.down.data(), (int64_t)h.down.size(), s.seed, 14, 0.0f, 0.05f);
  return h;
}

std::vector<float> make_x(const Shape& s, int T, uint64_t stream) {
  std::vector<float> x((size_t)T * s.d);
  ember_fill_normal(x.data(), (int64_t)x.size(), s.seed, stream, 0.0f, 1.0f);
  return x;
}

std::vector<float> expected(const HostLayer& h, const std::vector<float>& x, int T, bool renorm) {
  std::vector<float> out((size_t)T * h.s.d);
  oracle_layer(x.data(), T, h.s.d, h.s.d_ff, h.s.E, h.s.k, renorm ? 1 : 0, 0, nullptr, 1, 1, 1.0f, h.router.data(),
               h.gate.data(), h.up.data(), h.down.data(), 0, nullptr, nullptr, nullptr, out.data(), 0);
  return out;
}

struct Err {
  double max_abs, rel_l2;
};
Err compare(const std::vector<float>& got, const std::vector<float>& want) {
  double m = 0, num = 0, den = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    const double e = (double)got[i] - (double)want[i];
    m = std::fmax(m, std::fabs(e));
    num += e * e;
    den += (double)want[i] * want[i];
  }
  if (!(m == m)) m = INFINITY;  // a NaN anywhere fails
  return {m, std::sqrt(num / (den > 0 ? den : 1e-300))};
}

bool fetch(const Dev& d, std::vector<float>& host) {
  host.resize(d.n / 4);
  return hip_ok(hipMemcpy(host.data(), d.p, d.n, hipMemcpyDeviceToHost), "D2H");
}

// One F32 layer through moe_ffn_hip at several batch sizes; graph capture on the decode batch.
int run_f32(const Shape& s) {
  const HostLayer h = make_layer(s);
  Dev R, G, U, D;
  if (!R.put(h.router.data(), h.router.size() * 4) || !G.put(h.gate.data(), h.gate.size() * 4) ||
      !U.put(h.up.data(), h.up.size() * 4) || !D.put(h.down.data(), h.down.size() * 4))
    return 1;
  int fails = 0;
  for (bool renorm : {true, false}) {
    for (int T : {1, 3, 8, 33, 130}) {
      const std::vector<float> x = make_x(s, T, 100 + T);
      const std::vector<float> want = expected(h, x, T, renorm);
      Dev dx, dout, dscr;
      if (!dx.put(x.data(), x.size() * 4) || !dout.alloc(x.size() * 4) ||
          !dscr.alloc(moe_ffn_scratch_floats(T, s.d, s.d_ff, s.E, s.k) * 4))
        return 1;
      moe_ffn_hip(dx.f(), T, s.d, s.d_ff, s.E, s.k, renorm, R.f(), G.f(), U.f(), D.f(), dscr.f(), dout.f(), nullptr);
      if (!hip_ok(hipDeviceSynchronize(), "sync")) return 1;
      std::vector<float> got;
      if (!fetch(dout, got)) return 1;
      const Err e = compare(got, want);
      const bool ok = e.max_abs <= 1e-4 && e.rel_l2 <= 1e-5;
      fails += !ok;
      std::printf("f32 d%d E%d k%d %s T=%d: max|err| %.3e rel-L2 %.3e %s\n", s.d, s.E, s.k,
                  renorm ? "renorm" : "raw", T, e.max_abs, e.rel_l2, ok ? "ok" : "FAIL");
    }
  }

  // graph capture of the decode call, replayed on fresh inputs
  const int T = 1;
  Dev gx, gout, gscr, ex, eout, escr;
  const size_t scr = moe_ffn_scratch_floats(T, s.d, s.d_ff, s.E, s.k) * 4;
  if (!gx.alloc((size_t)T * s.d * 4) || !gout.alloc((size_t)T * s.d * 4) || !gscr.alloc(scr) ||
      !ex.alloc((size_t)T * s.d * 4) || !eout.alloc((size_t)T * s.d * 4) || !escr.alloc(scr))
    return 1;
  hipStream_t cs;
  if (!hip_ok(hipStreamCreate(&cs), "stream")) return 1;
  {
    const std::vector<float> x0 = make_x(s, T, 500);
    if (!hip_ok(hipMemcpy(gx.p, x0.data(), gx.n, hipMemcpyHostToDevice), "H2D")) return 1;
  }
  hipGraph_t graph;
  hipGraphExec_t exec;
  if (!hip_ok(hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal), "begin capture")) return 1;
  moe_ffn_hip(gx.f(), T, s.d, s.d_ff, s.E, s.k, true, R.f(), G.f(), U.f(), D.f(), gscr.f(), gout.f(), cs);
  if (!hip_ok(hipStreamEndCapture(cs, &graph), "end capture") ||
      !hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate"))
    return 1;
  for (int rep = 0; rep < 3; ++rep) {
    const std::vector<float> x = make_x(s, T, 600 + rep);
    if (!hip_ok(hipMemcpyAsync(gx.p, x.data(), gx.n, hipMemcpyHostToDevice, cs), "H2D") ||
        !hip_ok(hipStreamSynchronize(cs), "sync"))
      return 1;
    if (!hip_ok(hipGraphLaunch(exec, cs), "graph launch") || !hip_ok(hipStreamSynchronize(cs), "sync")) return 1;
    // eager call on the same input, other buffers, on the null stream between replays
    if (!hip_ok(hipMemcpy(ex.p, x.data(), ex.n, hipMemcpyHostToDevice), "H2D")) return 1;
    moe_ffn_hip(ex.f(), T, s.d, s.d_ff, s.E, s.k, true, R.f(), G.f(), U.f(), D.f(), escr.f(), eout.f(), nullptr);
    if (!hip_ok(hipDeviceSynchronize(), "sync")) return 1;
    std::vector<float> g, e;
    if (!fetch(gout, g) || !fetch(eout, e)) return 1;
    const bool same = std::memcmp(g.data(), e.data(), g.size() * 4) == 0;
    const Err er = compare(g, expected(h, x, T, true));
    const bool ok = same && er.max_abs <= 1e-4 && er.rel_l2 <= 1e-5;
    fails += !ok;
    std::printf("f32 d%d graph replay %d: bits %s eager, max|err| %.3e %s\n", s.d, rep, same ? "==" : "!=",
                er.max_abs, ok ? "ok" : "FAIL");
  }
  (void)hipGraphExecDestroy(exec);
  (void)hipGraphDestroy(graph);
  (void)hipStreamDestroy(cs);
  return fails;
}

// A Q8_0 layer through moe_ffn_hip_typed (stacks kept in their GGUF encoding).
int run_q8(const Shape& s) {
  HostLayer h = make_layer(s);
  auto encode = [](std::vector<float>& v, std::vector<uint8_t>& q, int K) {
    const int64_t rows = (int64_t)v.size() / K;
    q.resize((size_t)(rows * ember_row_bytes(EMBER_TYPE_Q8_0, K)));
    ember_quantize(EMBER_TYPE_Q8_0, v.data(), (int64_t)v.size(), q.data());
    ember_dequantize(EMBER_TYPE_Q8_0, q.data(), (int64_t)v.size(), v.data());  // the values the oracle sees
  };
  std::vector<uint8_t> qg, qu, qd;
  encode(h.gate, qg, s.d);
  encode(h.up, qu, s.d);
  encode(h.down, qd, s.d_ff);
  Dev R, G, U, D;
  if (!R.put(h.router.data(), h.router.size() * 4) || !G.put(qg.data(), qg.size()) || !U.put(qu.data(), qu.size()) ||
      !D.put(qd.data(), qd.size()))
    return 1;
  int fails = 0;
  for (int T : {1, 5, 64}) {
    const std::vector<float> x = make_x(s, T, 300 + T);
    const std::vector<float> want = expected(h, x, T, true);
    Dev dx, dout, dscr;
    if (!dx.put(x.data(), x.size() * 4) || !dout.alloc(x.size() * 4) ||
        !dscr.alloc(moe_ffn_scratch_floats_typed(T, s.d, s.d_ff, s.E, s.k, EMBER_TYPE_Q8_0) * 4))
      return 1;
    moe_ffn_hip_typed(dx.f(), T, s.d, s.d_ff, s.E, s.k, true, R.f(), G.p, U.p, D.p, EMBER_TYPE_Q8_0, dscr.f(),
                      dout.f(), nullptr);
    if (!hip_ok(hipDeviceSynchronize(), "sync")) return 1;
    std::vector<float> got;
    if (!fetch(dout, got)) return 1;
    const Err e = compare(got, want);
    const bool ok = e.rel_l2 <= 2e-3;
    fails += !ok;
    std::printf("q8_0 d%d E%d k%d T=%d: rel-L2 %.3e %s\n", s.d, s.E, s.k, T, e.rel_l2, ok ? "ok" : "FAIL");
  }
  return fails;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::printf("usage: %s <path to oracle/liboracle.so>\n", argv[0]);
    return 2;
  }
  void* so = dlopen(argv[1], RTLD_NOW);
  if (!so || !(oracle_layer = reinterpret_cast<OracleLayerFn>(dlsym(so, "oracle_moe_layer")))) {
    std::printf("cannot load the oracle from %s: %s\n", argv[1], dlerror());
    return 2;
  }
  int fails = 0;
  try {
    fails += run_f32({256, 688, 8, 2, 0});
    fails += run_f32({512, 384, 16, 4, 7});
    fails += run_q8({1024, 512, 8, 2, 3});
  } catch (const std::exception& ex) {
    std::printf("shim threw: %s\n", ex.what());
    return 1;
  }
  std::printf(fails ? "FAILED %d\n" : "all ok\n", fails);
  return fails != 0;
}
