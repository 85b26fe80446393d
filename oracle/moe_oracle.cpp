// ORACLE — TEST INFRASTRUCTURE ONLY.
//
// A CPU restatement of ember.cpp's mixture-of-experts FFN, used solely as the parity checker for the
// HIP implementation. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
// The product path (libember_moe.so) never links, loads or calls anything in this directory.
//
// Every function cites the reference file:line whose arithmetic it restates. The translation unit is
// compiled with -ffp-contract=off, as the reference compiles its arithmetic TUs (CMakeLists.txt:302-317),
// so every float/double multiply and add rounds separately, exactly as in the reference.
//
// Pins (each checked by tests/test_oracle.py):
//   dot_f32_f64          — closed form of cpu_dot.h:12-21, vs oracle/_ref and brute-force double sums
//   fp16/bf16 decode     — exhaustive over all 65536 codes vs oracle/_ref and IEEE half semantics
//   Q8_0 / Q4_K dequant  — vs oracle/_ref (quantization.cpp) and closed-form reconstruction
//   route (top-k, gates) — vs oracle/_ref full-layer goldens, brute force, softmax identities
//   dispatch permutation — closed form: std::stable_sort of (token, slot) by expert (no reference
//                          counterpart exists; the reference never sorts tokens)
//   moe_ffn_f32 / routed — bit-exact vs oracle/_ref goldens (tests/golden), and vs an FP64 brute force
//                          at the reference's own 1e-4 bar (tools/moe_ffn_test.cu:82-84)
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>
#include <omp.h>

namespace {

// cpu_dot.h:12-21 (dot_f32_f64_portable; the AVX2 variant at :31-49 is bit-identical by construction):
// eight FP64 chains over i = 8q + lane, a serial tail, then ((0+1)+(2+3)) + ((4+5)+(6+7)) + tail.
double dot64(const float* a, const float* b, int n) {
  double lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const int n8 = n - n % 8;
  for (int base = 0; base < n8; base += 8)
    for (int l = 0; l < 8; ++l) lane[l] += (double)a[base + l] * (double)b[base + l];
  double rest = 0.0;
  for (int i = n8; i < n; ++i) rest += (double)a[i] * (double)b[i];
  const double left = (lane[0] + lane[1]) + (lane[2] + lane[3]);
  const double right = (lane[4] + lane[5]) + (lane[6] + lane[7]);
  return (left + right) + rest;
}

// quantization.cpp:47-90 (fp16_to_fp32 with is_gguf_scale_field = false): IEEE binary16 → binary32,
// subnormals normalised, Inf/NaN payloads kept in the top mantissa bits.
float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      int shift = 0;
      while (!(m & 0x400)) { m <<= 1; ++shift; }
      m &= 0x3ff;
      bits = sign | ((uint32_t)(127 - 15 + 1 - shift) << 23) | (m << 13);
    }
  } else if (e == 0x1f) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// quantization.cpp:145-155 (get_scale_min_k4): the 6-bit scale and min of 32-element group j of a Q4_K
// super-block, packed into 12 bytes.
void q4k_scale_min(int j, const uint8_t* s, int* sc, int* mn) {
  if (j < 4) {
    *sc = s[j] & 0x3f;
    *mn = s[j + 4] & 0x3f;
  } else {
    *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
    *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_BF16 = 30 };

// weight_management.cpp:802-877 (dequant_span_to_f32) for the element range [first, first + n).
// F16 via fp16_to_fp32 (:803-811); BF16 as bits << 16 (:813-820); Q8_0 by dequantize_q8_0_block
// (quantization.cpp:1092-1097: d * (float)q, d keeping its sign); Q4_K by dequantize_q4_k_m
// (quantization.cpp:171-224: per 64-element chunk, d1 = d*sc1, m1 = dmin*m1, low nibbles then high
// nibbles, y = d1*(float)q - m1). F32 is a copy (the reference's memcpy in bind_tensor).
int dequant_span(int type, const uint8_t* src, size_t first, size_t n, float* out) {
  if (type == T_F32) {
    std::memcpy(out, src + 4 * first, 4 * n);
    return 0;
  }
  if (type == T_F16) {
    for (size_t i = 0; i < n; ++i) {
      uint16_t h;
      std::memcpy(&h, src + 2 * (first + i), 2);
      out[i] = half_to_float(h);
    }
    return 0;
  }
  if (type == T_BF16) {
    for (size_t i = 0; i < n; ++i) {
      uint16_t h;
      std::memcpy(&h, src + 2 * (first + i), 2);
      const uint32_t bits = (uint32_t)h << 16;
      std::memcpy(out + i, &bits, 4);
    }
    return 0;
  }
  if (type == T_Q8_0) {
    if (first % 32 || n % 32) return -1;
    for (size_t b = 0; b < n / 32; ++b) {
      const uint8_t* blk = src + (first / 32 + b) * 34;
      uint16_t dh;
      std::memcpy(&dh, blk, 2);
      const float d = half_to_float(dh);
      for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
    }
    return 0;
  }
  if (type == T_Q4_K) {
    if (first % 256 || n % 256) return -1;
    for (size_t b = 0; b < n / 256; ++b) {
      const uint8_t* blk = src + (first / 256 + b) * 144;
      uint16_t dh, mh;
      std::memcpy(&dh, blk, 2);
      std::memcpy(&mh, blk + 2, 2);
      const float d = half_to_float(dh), dmin = half_to_float(mh);
      const uint8_t* scales = blk + 4;
      const uint8_t* qs = blk + 16;
      float* y = out + b * 256;
      for (int c = 0; c < 4; ++c) {
        int sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, scales, &sc0, &m0);
        q4k_scale_min(2 * c + 1, scales, &sc1, &m1);
        const float dA = d * (float)sc0, mA = dmin * (float)m0;
        const float dB = d * (float)sc1, mB = dmin * (float)m1;
        for (int l = 0; l < 32; ++l) y[64 * c + l] = dA * (float)(qs[32 * c + l] & 0x0f) - mA;
        for (int l = 0; l < 32; ++l) y[64 * c + 32 + l] = dB * (float)(qs[32 * c + l] >> 4) - mB;
      }
    }
    return 0;
  }
  return -2;
}

// std::max(a, b) as the reference calls it: (a < b) ? b : a.
inline float smax(float a, float b) { return (a < b) ? b : a; }

// utils.cpp:706-733 — routing of moe_ffn_f32_cpu given one token's logits r[E]: k passes of argmax over
// the untaken experts with strict > (ties keep the lower index), the picks sorted ascending, then gates
// (float)(exp((double)(r_e - mx)) / z) with mx and the double sum z over the selected experts (renorm)
// or over all E (raw), both in ascending expert order. Writes k (or E if E < k) indices and gates.
int route_softmax(const float* r, int E, int k, bool renorm, int32_t* idx, float* gate) {
  std::vector<int> sel;
  std::vector<char> taken(E, 0);
  for (int j = 0; j < k && j < E; ++j) {
    int best = -1;
    for (int e = 0; e < E; ++e)
      if (!taken[e] && (best < 0 || r[e] > r[best])) best = e;
    taken[best] = 1;
    sel.push_back(best);
  }
  std::sort(sel.begin(), sel.end());
  float mx = -std::numeric_limits<float>::infinity();
  double z = 0.0;
  if (renorm) {
    for (int e : sel) mx = smax(mx, r[e]);
    for (int e : sel) z += std::exp((double)(r[e] - mx));
  } else {
    for (int e = 0; e < E; ++e) mx = smax(mx, r[e]);
    for (int e = 0; e < E; ++e) z += std::exp((double)(r[e] - mx));
  }
  for (size_t j = 0; j < sel.size(); ++j) {
    idx[j] = sel[j];
    gate[j] = (float)(std::exp((double)(r[sel[j]] - mx)) / z);
  }
  return (int)sel.size();
}

// utils.cpp:758-820 — the DeepSeek-V3 router of moe_ffn_routed_f32_cpu: float scores (E-way float softmax
// with expf and an ascending float sum, or sigmoid 1/(1+expf(-r))), selection scores c = s + bias,
// optional group limiting (group score = top-2 sum of c, top groups by strict >), k picks by strict >
// over the candidates, ascending sort, gates s_e (/ the ascending float sum of the picked s under renorm).
// Returns the number of picks (fewer than k only if the candidates run out).
int route_routed(const float* r, int E, int k, bool renorm, bool sigmoid, const float* bias, int groups_n,
                 int groups_top, int32_t* idx, float* gate) {
  if (!sigmoid && !bias && groups_n <= 1) return route_softmax(r, E, k, renorm, idx, gate);
  std::vector<float> s(E), c(E);
  if (sigmoid) {
    for (int e = 0; e < E; ++e) s[e] = 1.0f / (1.0f + std::exp(-r[e]));
  } else {
    float mx = -std::numeric_limits<float>::infinity();
    for (int e = 0; e < E; ++e) mx = smax(mx, r[e]);
    float z = 0.0f;
    for (int e = 0; e < E; ++e) {
      s[e] = std::exp(r[e] - mx);
      z += s[e];
    }
    for (int e = 0; e < E; ++e) s[e] = s[e] / z;
  }
  for (int e = 0; e < E; ++e) c[e] = bias ? s[e] + bias[e] : s[e];
  std::vector<char> cand(E, 1);
  if (groups_n > 1) {
    const int per = E / groups_n;
    std::vector<float> gscore(groups_n);
    const float ninf = -std::numeric_limits<float>::infinity();
    for (int g = 0; g < groups_n; ++g) {
      float top1 = ninf, top2 = ninf;
      for (int e = g * per; e < (g + 1) * per; ++e) {
        if (c[e] > top1) {
          top2 = top1;
          top1 = c[e];
        } else if (c[e] > top2) {
          top2 = c[e];
        }
      }
      gscore[g] = per == 1 ? top1 : top1 + top2;
    }
    std::vector<char> keep(groups_n, 0);
    for (int j = 0; j < groups_top && j < groups_n; ++j) {
      int best = -1;
      for (int g = 0; g < groups_n; ++g)
        if (!keep[g] && (best < 0 || gscore[g] > gscore[best])) best = g;
      keep[best] = 1;
    }
    for (int e = 0; e < E; ++e) cand[e] = keep[e / per];
  }
  std::vector<int> sel;
  std::vector<char> taken(E, 0);
  for (int j = 0; j < k; ++j) {
    int best = -1;
    for (int e = 0; e < E; ++e)
      if (cand[e] && !taken[e] && (best < 0 || c[e] > c[best])) best = e;
    if (best < 0) break;
    taken[best] = 1;
    sel.push_back(best);
  }
  std::sort(sel.begin(), sel.end());
  float z = 0.0f;
  for (int e : sel) z += s[e];
  for (size_t j = 0; j < sel.size(); ++j) {
    idx[j] = sel[j];
    gate[j] = renorm ? s[sel[j]] / z : s[sel[j]];
  }
  return (int)sel.size();
}

// utils.cpp:735-747 — the expert loop for one token: for each selected expert in ascending order,
// h_i = gv * (1/(1+expf(-gv))) * uv with gv, uv the FP64 dots rounded to float, then
// out[o] += w * (float)dot64(down_e[o], h), out starting at zero.
void experts_one_token(const float* x, int d, int d_ff, const int32_t* idx, const float* gate, int n_sel,
                       const float* G, const float* U, const float* D, float* out) {
  std::fill(out, out + d, 0.0f);
  std::vector<float> h(d_ff);
  for (int j = 0; j < n_sel; ++j) {
    const int e = idx[j];
    const float w = gate[j];
    const float* g = G + (size_t)e * d_ff * d;
    const float* u = U + (size_t)e * d_ff * d;
    const float* dn = D + (size_t)e * d * d_ff;
    for (int i = 0; i < d_ff; ++i) {
      const float gv = (float)dot64(g + (size_t)i * d, x, d);
      const float uv = (float)dot64(u + (size_t)i * d, x, d);
      h[i] = gv * (1.0f / (1.0f + std::exp(-gv))) * uv;
    }
    for (int o = 0; o < d; ++o) out[o] += w * (float)dot64(dn + (size_t)o * d_ff, h.data(), d_ff);
  }
}

}  // namespace

extern "C" {

double oracle_dot_f32_f64(const float* a, const float* b, int n) { return dot64(a, b, n); }

float oracle_fp16_to_fp32(uint16_t h) { return half_to_float(h); }

int oracle_dequant(int type, const void* src, size_t first, size_t n, float* out) {
  return dequant_span(type, (const uint8_t*)src, first, n, out);
}

// Router logits r[t][e] = (float)dot64(R[e], x[t]) (utils.cpp:707).
void oracle_router_logits(const float* x, int T, int d, int E, const float* router, float* logits) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t)
    for (int e = 0; e < E; ++e) logits[(size_t)t * E + e] = (float)dot64(router + (size_t)e * d, x + (size_t)t * d, d);
}

// Routing for T tokens given logits. scoring: 0 = moe_ffn_f32_cpu's softmax gates (double exp),
// 1 = moe_ffn_routed_f32_cpu (float softmax, or sigmoid if `sigmoid`, with optional bias / groups).
// Writes idx[T][k], gates[T][k]; returns the minimum pick count over tokens (k unless candidates ran out).
int oracle_route(const float* logits, int T, int E, int k, int renorm, int sigmoid, const float* bias, int groups_n,
                 int groups_top, int32_t* idx, float* gates) {
  int min_picks = k;
  for (int t = 0; t < T; ++t) {
    const int n = route_routed(logits + (size_t)t * E, E, k, renorm != 0, sigmoid != 0, bias, groups_n, groups_top,
                               idx + (size_t)t * k, gates + (size_t)t * k);
    for (int j = n; j < k; ++j) {
      idx[(size_t)t * k + j] = -1;
      gates[(size_t)t * k + j] = 0.0f;
    }
    min_picks = std::min(min_picks, n);
  }
  return min_picks;
}

// The dispatch permutation (no reference counterpart; see header): slots s = t*k + j ordered by
// (expert, s) — a stable sort of the slots by expert id. offsets[E+1] are the per-expert starts,
// perm[p] = the slot at sorted position p. Slots with idx < 0 are left out.
void oracle_dispatch(const int32_t* idx, int T, int k, int E, int32_t* offsets, int32_t* perm) {
  std::vector<int32_t> slots;
  for (int s = 0; s < T * k; ++s)
    if (idx[s] >= 0) slots.push_back(s);
  std::stable_sort(slots.begin(), slots.end(), [&](int32_t a, int32_t b) { return idx[a] < idx[b]; });
  std::fill(offsets, offsets + E + 1, 0);
  for (int32_t s : slots) offsets[idx[s] + 1]++;
  for (int e = 0; e < E; ++e) offsets[e + 1] += offsets[e];
  for (size_t p = 0; p < slots.size(); ++p) perm[p] = slots[p];
}

// The whole routed layer on F32 stacks, token-parallel as cpu_batch_processor.cpp:223-231 and the IR's
// moe_ffn op (graph_ir.cpp:2704-2709): router, routing (as oracle_route), experts (utils.cpp:735-747),
// then — IR deepseek2 graph (graph_ir.cpp:919-928) — f = (f * scale) + 0 when scale != 1 and, with a
// shared expert of width d_ff_sh, f = f + sf, sf = down_sh · ((g * (1/(1+expf(-g)))) * u) with g, u, sf
// the FP64-dot rows of matmul_f32_f32_batch_cpu (utils.cpp:867-909) and silu_cpu (utils.cpp:838-844);
// with Wsg (qwen2moe's ffn_gate_inp_shexp, graph_ir.cpp:694-705) sf is first scaled by sigmoid(Wsg · x).
// nthreads <= 0 leaves OpenMP's default.
void oracle_moe_layer_gated(const float* x, int T, int d, int d_ff, int E, int k, int renorm, int sigmoid,
                            const float* bias, int groups_n, int groups_top, float scale, const float* router,
                            const float* G, const float* U, const float* D, int d_ff_sh, const float* Gs,
                            const float* Us, const float* Ds, const float* Wsg, float* sgate_out, float* out,
                            int nthreads) {
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : omp_get_max_threads())
  for (int t = 0; t < T; ++t) {
    const float* xt = x + (size_t)t * d;
    float* ot = out + (size_t)t * d;
    std::vector<float> r(E);
    for (int e = 0; e < E; ++e) r[e] = (float)dot64(router + (size_t)e * d, xt, d);
    std::vector<int32_t> idx(std::max(k, 1));
    std::vector<float> gate(std::max(k, 1));
    const int n = route_routed(r.data(), E, k, renorm != 0, sigmoid != 0, bias, groups_n, groups_top, idx.data(),
                               gate.data());
    experts_one_token(xt, d, d_ff, idx.data(), gate.data(), n, G, U, D, ot);
    if (scale != 1.0f)
      for (int o = 0; o < d; ++o) ot[o] = ot[o] * scale + 0.0f;
    if (d_ff_sh > 0) {
      std::vector<float> hs(d_ff_sh);
      for (int i = 0; i < d_ff_sh; ++i) {
        const float g = (float)dot64(Gs + (size_t)i * d, xt, d);
        const float u = (float)dot64(Us + (size_t)i * d, xt, d);
        const float sg = g * (1.0f / (1.0f + std::exp(-g)));
        hs[i] = sg * u;
      }
      // qwen2moe (graph_ir.cpp:704-705): sgate = linear(h2, ffn_gate_inp_shexp), a one-row FP64 dot
      // (utils.cpp:867-909); sigmoid 1 / (1 + expf(-s)) (graph_ir_ops.cpp:22); sf * sgate per token
      // (mul_col, graph_ir_ops.cpp:61); then f + sf
      float c = 1.0f;
      if (Wsg) {
        const float s = (float)dot64(Wsg, xt, d);
        if (sgate_out) sgate_out[t] = s;
        c = 1.0f / (1.0f + std::exp(-s));
      }
      for (int o = 0; o < d; ++o) {
        float sf = (float)dot64(Ds + (size_t)o * d_ff_sh, hs.data(), d_ff_sh);
        if (Wsg) sf = sf * c;
        ot[o] = ot[o] + sf;
      }
    }
  }
}

void oracle_moe_layer(const float* x, int T, int d, int d_ff, int E, int k, int renorm, int sigmoid,
                      const float* bias, int groups_n, int groups_top, float scale, const float* router,
                      const float* G, const float* U, const float* D, int d_ff_sh, const float* Gs,
                      const float* Us, const float* Ds, float* out, int nthreads) {
  oracle_moe_layer_gated(x, T, d, d_ff, E, k, renorm, sigmoid, bias, groups_n, groups_top, scale, router, G, U, D,
                         d_ff_sh, Gs, Us, Ds, nullptr, nullptr, out, nthreads);
}

}  // extern "C"
