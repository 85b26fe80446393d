// Device-side routing of one token per wave (top-k, gates, the DeepSeek-style router) and the block
// prefix scan used by the dispatch; shared by the routing kernels and the fused decode kernel.
// Reference: utils.cpp:704-836 (softmax top-k and gates), graph_ir.cpp:2689-2740 (routed scoring).
#pragma once
#include "moe_internal.hpp"

namespace ember_moe {
using namespace ember_math;


__device__ inline float smax(float a, float b) { return (a < b) ? b : a; }  // std::max(a, b)

// a is a strictly better argmax candidate than b: larger value, ties to the lower index; -1 = none.
__device__ inline bool better(float va, int ia, float vb, int ib) {
  if (ia < 0) return false;
  if (ib < 0) return true;
  return va > vb || (va == vb && ia < ib);
}

__device__ inline void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// moe_ffn_f32_cpu's routing (utils.cpp:706-733), serial, for rows holding a NaN.
__device__ inline void route_softmax_serial(const float* r, int E, int k, int renorm, char* taken, int* picks,
                                     int32_t* idx, float* gates) {
  for (int e = 0; e < E; ++e) taken[e] = 0;
  const int kk = min(k, E);
  for (int j = 0; j < kk; ++j) {
    int best = -1;
    for (int e = 0; e < E; ++e)
      if (!taken[e] && (best < 0 || r[e] > r[best])) best = e;
    taken[best] = 1;
    picks[j] = best;
  }
  for (int a = 1; a < kk; ++a)
    for (int b = a; b > 0 && picks[b - 1] > picks[b]; --b) {
      const int tmp = picks[b];
      picks[b] = picks[b - 1];
      picks[b - 1] = tmp;
    }
  float mx = -__builtin_inff();
  double z = 0.0;
  if (renorm) {
    for (int j = 0; j < kk; ++j) mx = smax(mx, r[picks[j]]);
    for (int j = 0; j < kk; ++j) z = z + exp_glibc((double)(r[picks[j]] - mx));
  } else {
    for (int e = 0; e < E; ++e) mx = smax(mx, r[e]);
    for (int e = 0; e < E; ++e) z = z + exp_glibc((double)(r[e] - mx));
  }
  for (int j = 0; j < k; ++j) {
    idx[j] = j < kk ? picks[j] : -1;
    gates[j] = j < kk ? (float)(exp_glibc((double)(r[picks[j]] - mx)) / z) : 0.0f;
  }
}

// moe_ffn_routed_f32_cpu's router (utils.cpp:766-820), serial: float scores, selection bias, groups.
__device__ inline void route_routed_serial(const float* r, int E, int k, int renorm, int sigmoid, const float* bias,
                                    int groups_n, int groups_top, float* s, float* c, char* cand, char* taken,
                                    int* picks, int32_t* idx, float* gates) {
  if (sigmoid) {
    for (int e = 0; e < E; ++e) s[e] = 1.0f / (1.0f + expf_glibc(-r[e]));
  } else {
    float mx = -__builtin_inff();
    for (int e = 0; e < E; ++e) mx = smax(mx, r[e]);
    float z = 0.0f;
    for (int e = 0; e < E; ++e) {
      s[e] = expf_glibc(r[e] - mx);
      z = z + s[e];
    }
    for (int e = 0; e < E; ++e) s[e] = s[e] / z;
  }
  for (int e = 0; e < E; ++e) c[e] = bias ? s[e] + bias[e] : s[e];
  for (int e = 0; e < E; ++e) cand[e] = 1;
  if (groups_n > 1) {
    const int per = E / groups_n;
    float* gscore = c + E;  // the caller reserves 2E floats at c; groups_n <= E
    for (int g = 0; g < groups_n; ++g) {
      float top1 = -__builtin_inff(), top2 = -__builtin_inff();
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
    for (int g = 0; g < groups_n; ++g) taken[g] = 0;
    for (int j = 0; j < groups_top && j < groups_n; ++j) {
      int best = -1;
      for (int g = 0; g < groups_n; ++g)
        if (!taken[g] && (best < 0 || gscore[g] > gscore[best])) best = g;
      taken[best] = 1;
    }
    for (int e = 0; e < E; ++e) cand[e] = taken[e / per];
  }
  for (int e = 0; e < E; ++e) taken[e] = 0;
  int n = 0;
  for (int j = 0; j < k; ++j) {
    int best = -1;
    for (int e = 0; e < E; ++e)
      if (cand[e] && !taken[e] && (best < 0 || c[e] > c[best])) best = e;
    if (best < 0) break;
    taken[best] = 1;
    picks[n++] = best;
  }
  for (int a = 1; a < n; ++a)
    for (int b = a; b > 0 && picks[b - 1] > picks[b]; --b) {
      const int tmp = picks[b];
      picks[b] = picks[b - 1];
      picks[b - 1] = tmp;
    }
  float z = 0.0f;
  for (int j = 0; j < n; ++j) z = z + s[picks[j]];
  for (int j = 0; j < k; ++j) {
    idx[j] = j < n ? picks[j] : -1;
    gates[j] = j < n ? (renorm ? s[picks[j]] / z : s[picks[j]]) : 0.0f;
  }
}

// Per-wave LDS footprint of route_kernel for E experts.
// LDS bytes of one routing wave: the exp tables (copies of kExp2Tab128 and kExp2Tab32, staged with
// the logits so that no exponential waits on a global table load), then the work arrays.
constexpr size_t kRouteTabBytes = (256 + 32) * 8;
__host__ __device__ inline size_t route_wave_lds(int E) {
  const size_t bytes = kRouteTabBytes + (size_t)E * 8 /*ex*/ + (size_t)E * 4 /*s*/ + (size_t)2 * E * 4 /*c + group scores*/ +
                       (size_t)64 * 4 /*picks*/ + (size_t)((2 * E + 3) & ~3) /*cand, taken*/ + (size_t)E * 4 /*row*/;
  return (bytes + 15) & ~(size_t)15;
}

// k passes of a wave-wide argmax over val[e] (LDS, NaN-free), each pass taking the largest untaken
// value with ties to the lower index — the result of the reference's serial strict-> scans. Experts
// with cand[e] == 0 are skipped (cand may be null); a pass that finds nothing ends the search. Lane 0
// writes the picks in pick order; returns their number (uniform across the wave).
__device__ __attribute__((always_inline)) inline int wave_topk_passes(const float* val, const char* cand, int E, int k, int* picks);

// The same selection by ranks, for larger k: expert e is picked iff it is a candidate and fewer than k
// candidates are strictly better (larger value, ties to the lower index) — exactly the experts the k
// argmax passes pick, and already in ascending index order, the order the picks are returned in.
// O(E^2 / 64) compares per lane against k dependent wave reductions.
__device__ inline int wave_topk_rank(const float* val, const char* cand, int E, int k, int* picks) {
  const int lane = threadIdx.x & 63;
  int n = 0;  // picks so far (uniform)
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    bool sel = false;
    if (e < E && (!cand || cand[e])) {
      const float v = val[e];
      int rank = 0;
      for (int o = 0; o < E; ++o)
        if ((!cand || cand[o]) && better(val[o], o, v, e)) ++rank;
      sel = rank < k;
    }
    const uint64_t m = __ballot(sel);
    if (sel) picks[n + __builtin_popcountll(m & ((1ull << lane) - 1))] = e;
    n += __builtin_popcountll(m);
  }
  wave_sync_lds();
  return n;
}

// Order key of a NaN-free float: key(a) > key(b) iff a > b, and both zeros share the key of +0 (they
// compare equal, so they tie).
__device__ inline uint32_t order_key(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f == 0.0f ? 0.0f : f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The same selection as wave_topk_rank with the values in registers (E <= 64 Q, lane holds experts
// lane + 64 q), by a radix select: the k-th largest key t is built bit by bit (the largest t with at
// least k candidate keys >= t, 32 ballot counts), then the picks are the candidates above t and, of
// those equal to t, the lowest-indexed ones up to k. That is the set the k strict-> argmax passes take
// (larger value first, ties to the lower index); returned in ascending index order.
template <int Q>
__device__ __attribute__((always_inline)) inline int wave_topk_regs(const float* val, const char* cand, int E, int k,
                                                                    int* picks) {
  const int lane = threadIdx.x & 63;
  // E and k are wave-uniform: kept in scalar registers, the search below runs on the scalar unit except
  // for one compare per register slot and step
  E = __builtin_amdgcn_readfirstlane(E);
  k = __builtin_amdgcn_readfirstlane(k);
  uint32_t key[Q];
  uint64_t cm[Q];  // candidate masks
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int e = lane + 64 * q;
    const bool c = e < E && (!cand || cand[e]);
    key[q] = c ? order_key(val[e]) : 0u;  // a candidate's key is > 0 (-inf has 0x007fffff), others 0
    cm[q] = __ballot(c);
  }
  // t stays 0 when there are fewer than k candidates: then every candidate is above it. Every trial is
  // >= 1, so the zero keys of non-candidates never count.
  uint32_t t = 0;
  // kept rolled: unrolled, the 32 steps of each register-count variant added ~10 KB of code to every
  // launch that routes inline (the one-token kernels: 58 -> 45 KB), for no measured gain
#pragma unroll 1
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t trial = t | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int q = 0; q < Q; ++q) cnt += __builtin_popcountll(__ballot(key[q] >= trial));
    t = cnt >= k ? trial : t;
  }
  int gt = 0;
#pragma unroll
  for (int q = 0; q < Q; ++q) gt += __builtin_popcountll(__ballot(key[q] > t));
  const int need = k - gt;  // picks among the candidate keys equal to t
  const uint64_t below = (1ull << lane) - 1;
  int n = 0, eq_before = 0;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const uint64_t eqm = __ballot(key[q] == t) & cm[q];
    const bool eq = (eqm >> lane) & 1;
    const bool sel = key[q] > t || (eq && eq_before + __builtin_popcountll(eqm & below) < need);
    const uint64_t m = __ballot(sel);
    if (sel) picks[n + __builtin_popcountll(m & below)] = lane + 64 * q;
    n += __builtin_popcountll(m);
    eq_before += __builtin_popcountll(eqm);
  }
  wave_sync_lds();
  return n;
}

// Largest of a wave's 32-bit values, every lane's (DPP: row_shr 1, 2, 4, 8 within rows of 16 lanes, then
// row_bcast 15 and 31 across rows; lane 63 ends with the maximum).
__device__ __attribute__((always_inline)) inline uint32_t wave_max_u32(uint32_t v) {
  auto step = [](uint32_t x, auto CTRL, auto ROWS) {
    const uint32_t y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, decltype(CTRL)::value,
                                                             decltype(ROWS)::value, 0xf, false);
    return x > y ? x : y;
  };
  using I = std::integral_constant<int, 0xf>;
  v = step(v, std::integral_constant<int, 0x111>{}, I{});
  v = step(v, std::integral_constant<int, 0x112>{}, I{});
  v = step(v, std::integral_constant<int, 0x114>{}, I{});
  v = step(v, std::integral_constant<int, 0x118>{}, I{});
  v = step(v, std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xa>{});
  v = step(v, std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xc>{});
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// The same selection as wave_topk_regs for small k (E <= 64 Q): the reference's k argmax passes
// themselves, each a wave maximum of the candidates' order keys (larger value first) and the lowest index
// holding it (ties to the lower index); picks returned in ascending index order.
template <int Q>
__device__ __attribute__((always_inline)) inline int wave_topk_argmax(const float* val, const char* cand, int E, int k,
                                                                      int* picks) {
  const int lane = threadIdx.x & 63;
  E = __builtin_amdgcn_readfirstlane(E);
  k = __builtin_amdgcn_readfirstlane(k);
  uint32_t key[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int e = lane + 64 * q;
    key[q] = e < E && (!cand || cand[e]) ? order_key(val[e]) : 0u;  // a candidate's key is > 0
  }
  uint64_t sel[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) sel[q] = 0;
  for (int j = 0; j < k; ++j) {
    uint32_t mine = key[0];
#pragma unroll
    for (int q = 1; q < Q; ++q) mine = mine > key[q] ? mine : key[q];
    const uint32_t m = wave_max_u32(mine);
    if (m == 0u) break;  // fewer candidates than k
    bool done = false;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const uint64_t hit = __ballot(key[q] == m);
      if (!done && hit) {
        const int l = __builtin_ctzll(hit);
        sel[q] |= 1ull << l;
        if (lane == l) key[q] = 0u;
        done = true;
      }
    }
  }
  const uint64_t below = (1ull << lane) - 1;
  int n = 0;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if ((sel[q] >> lane) & 1) picks[n + __builtin_popcountll(sel[q] & below)] = lane + 64 * q;
    n += __builtin_popcountll(sel[q]);
  }
  wave_sync_lds();
  return n;
}

__device__ __attribute__((always_inline)) inline int wave_topk(const float* val, const char* cand, int E, int k, int* picks) {
  if (k <= 8 && E <= 64) return wave_topk_argmax<1>(val, cand, E, k, picks);
  if (k <= 8 && E <= 128) return wave_topk_argmax<2>(val, cand, E, k, picks);
  if (E <= 64) return wave_topk_regs<1>(val, cand, E, k, picks);
  if (E <= 128) return wave_topk_regs<2>(val, cand, E, k, picks);
  if (E <= 256) return wave_topk_regs<4>(val, cand, E, k, picks);
  return k >= 4 ? wave_topk_rank(val, cand, E, k, picks) : wave_topk_passes(val, cand, E, k, picks);
}

__device__ __attribute__((always_inline)) inline int wave_topk_passes(const float* val, const char* cand, int E, int k, int* picks) {
  const int lane = threadIdx.x & 63;
  uint32_t mine_taken = 0;  // bit q: expert lane + 64q taken (E <= 2048)
  int n = 0;
  for (int j = 0; j < k; ++j) {
    float bv = 0.0f;
    int bi = -1;
    for (int e = lane, q = 0; e < E; e += 64, ++q)
      if (!((mine_taken >> q) & 1u) && (!cand || cand[e]) && better(val[e], e, bv, bi)) {
        bv = val[e];
        bi = e;
      }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi < 0) break;
    if ((bi & 63) == lane) mine_taken |= 1u << (bi >> 6);
    if (lane == 0) picks[n] = bi;
    ++n;
  }
  wave_sync_lds();
  if (lane == 0)
    for (int a = 1; a < n; ++a)
      for (int b = a; b > 0 && picks[b - 1] > picks[b]; --b) {
        const int tmp = picks[b];
        picks[b] = picks[b - 1];
        picks[b - 1] = tmp;
      }
  wave_sync_lds();
  return n;
}

// moe_ffn_routed_f32_cpu's router (utils.cpp:766-820) across the wave for NaN-free scores: every
// per-expert float operation is the reference's; the float sums that fix rounding (the softmax
// normaliser, the renorm denominator) stay serial in ascending expert order on lane 0; the maximum,
// the group top-2 and the argmax passes are order-independent for NaN-free values. Returns false
// (nothing written) when a NaN appears in the scores, so the caller falls back to the serial scan.
__device__ inline bool route_routed_wave(const float* row, int E, int k, int renorm, int sigmoid, const float* bias,
                                  int groups_n, int groups_top, float* s, float* c, char* cand, int* picks,
                                  int32_t* idx_t, float* gate_t, const uint64_t* tab32) {
  const int lane = threadIdx.x & 63;
  if (sigmoid) {
    for (int e = lane; e < E; e += 64) s[e] = 1.0f / (1.0f + expf_glibc_t(-row[e], tab32));
  } else {
    float mx = -__builtin_inff();
    for (int e = lane; e < E; e += 64) mx = smax(mx, row[e]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = smax(mx, __shfl_xor(mx, off, 64));
    for (int e = lane; e < E; e += 64) s[e] = expf_glibc_t(row[e] - mx, tab32);
    wave_sync_lds();
    float z = 0.0f;
    if (lane == 0)
      for (int e = 0; e < E; ++e) z = z + s[e];
    z = __shfl(z, 0, 64);
    for (int e = lane; e < E; e += 64) s[e] = s[e] / z;
  }
  bool bad = false;
  for (int e = lane; e < E; e += 64) {
    const float v = bias ? s[e] + bias[e] : s[e];
    c[e] = v;
    bad |= (v != v) || (s[e] != s[e]);
  }
  if (__any(bad)) return false;
  wave_sync_lds();
  const char* cmask = nullptr;
  if (groups_n > 1) {
    const int per = E / groups_n;
    float* gsc = c + E;
    for (int g = lane; g < groups_n; g += 64) {
      float top1 = -__builtin_inff(), top2 = -__builtin_inff();
      for (int e = g * per; e < (g + 1) * per; ++e) {
        if (c[e] > top1) {
          top2 = top1;
          top1 = c[e];
        } else if (c[e] > top2) {
          top2 = c[e];
        }
      }
      gsc[g] = per == 1 ? top1 : top1 + top2;
    }
    wave_sync_lds();
    const int ng = wave_topk(gsc, nullptr, groups_n, groups_top, picks);
    for (int e = lane; e < E; e += 64) cand[e] = 0;
    wave_sync_lds();
    for (int j = 0; j < ng; ++j)
      for (int e = picks[j] * per + lane; e < (picks[j] + 1) * per; e += 64) cand[e] = 1;
    wave_sync_lds();
    cmask = cand;
  }
  const int n = wave_topk(c, cmask, E, k, picks);
  float z = 0.0f;
  for (int j = 0; j < n; ++j) z = z + s[picks[j]];
  if (lane < k) {
    if (lane < n) {
      const int e = picks[lane];
      idx_t[lane] = e;
      gate_t[lane] = renorm ? s[e] / z : s[e];
    } else {
      idx_t[lane] = -1;
      gate_t[lane] = 0.0f;
    }
  }
  return true;
}

// Routes one token on one wave (all 64 lanes call it). NaN-free rows run wave-parallel scans whose
// results equal the reference's serial scans; rows with a NaN (in the logits or in the DeepSeek-style
// scores) run the reference's serial algorithm on lane 0. wl: route_wave_lds(E) bytes of LDS owned by
// this wave.
__device__ inline void route_stage_tables(unsigned char* wl) {
  const int lane = threadIdx.x & 63;
  uint64_t* tab128 = reinterpret_cast<uint64_t*>(wl);
#pragma unroll
  for (int i = 0; i < 4; ++i) tab128[lane + 64 * i] = ember_math::kExp2Tab128[lane + 64 * i];
  if (lane < 32) tab128[256 + lane] = ember_math::kExp2Tab32[lane];
}

// tables_ready: the exp tables are already in wl (route_stage_tables ran earlier on this wave).
// ROUTED = false compiles the DeepSeek-style paths out (callers then pass routed = 0): a launch that
// inlines route_token keeps only the code its router needs.
template <bool ROUTED = true>
__device__ __attribute__((always_inline)) inline void route_token(const float* __restrict__ r, int E, int k, int renorm, int routed, int sigmoid,
                            const float* __restrict__ bias, int groups_n, int groups_top, unsigned char* wl,
                            int32_t* __restrict__ idx_t, float* __restrict__ gate_t, bool tables_ready = false) {
  const int lane = threadIdx.x & 63;
  uint64_t* tab128 = reinterpret_cast<uint64_t*>(wl);
  uint64_t* tab32 = tab128 + 256;
  double* ex = reinterpret_cast<double*>(wl + kRouteTabBytes);
  float* s = reinterpret_cast<float*>(wl + kRouteTabBytes + (size_t)E * 8);
  float* cbuf = s + E;
  int* picks = reinterpret_cast<int*>(cbuf + 2 * E);
  char* cand = reinterpret_cast<char*>(picks + 64);
  char* taken = cand + E;
  float* row = reinterpret_cast<float*>(wl + route_wave_lds(E) - (size_t)E * 4);
  bool has_nan = false;
  {
    // the tables and the logits in one round of loads
    uint64_t t[4], t32 = 0;
    if (!tables_ready) {
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = ember_math::kExp2Tab128[lane + 64 * i];
      t32 = ember_math::kExp2Tab32[lane & 31];
    }
    for (int e = lane; e < E; e += 64) {
      const float v = r[e];
      row[e] = v;
      has_nan |= (v != v);
    }
    if (!tables_ready) {
#pragma unroll
      for (int i = 0; i < 4; ++i) tab128[lane + 64 * i] = t[i];
      if (lane < 32) tab32[lane] = t32;
    }
  }
  has_nan = __any(has_nan);
  wave_sync_lds();
  if constexpr (ROUTED) {
    if (routed && !has_nan && groups_n <= 64 &&
        route_routed_wave(row, E, k, renorm, sigmoid, bias, groups_n, groups_top, s, cbuf, cand, picks, idx_t, gate_t,
                          tab32))
      return;
  }
  if (routed || has_nan) {
    wave_sync_lds();
    if (lane == 0) {
      if (ROUTED && routed)
        route_routed_serial(row, E, k, renorm, sigmoid, bias, groups_n, groups_top, s, cbuf, cand, taken, picks, idx_t,
                            gate_t);
      else
        route_softmax_serial(row, E, k, renorm, taken, picks, idx_t, gate_t);
    }
    return;
  }
  const int kk = wave_topk(row, nullptr, E, min(k, E), picks);
  float mx = -__builtin_inff();
  double z = 0.0;
  if (renorm) {
    for (int j = 0; j < kk; ++j) mx = smax(mx, row[picks[j]]);
    // lane j evaluates the j-th exponential (all at once); every lane adds them in pick order
    const double exj = lane < kk ? exp_glibc_t((double)(row[picks[lane]] - mx), tab128) : 0.0;
    for (int j = 0; j < kk; ++j) z = z + __shfl(exj, j, 64);
    if (lane < k) {
      idx_t[lane] = lane < kk ? picks[lane] : -1;
      gate_t[lane] = lane < kk ? (float)(exj / z) : 0.0f;
    }
    return;
  } else {
    // The maximum of a NaN-free row does not depend on the scan order (only the sign of a zero
    // maximum can, and r - (+0) and r - (-0) round to equal exp arguments for every r).
    for (int e = lane; e < E; e += 64) mx = smax(mx, row[e]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = smax(mx, __shfl_xor(mx, off, 64));
    for (int e = lane; e < E; e += 64) ex[e] = exp_glibc_t((double)(row[e] - mx), tab128);
    wave_sync_lds();
    if (lane == 0)
      for (int e = 0; e < E; ++e) z = z + ex[e];  // ascending, as the reference sums
    z = __shfl(z, 0, 64);
  }
  if (lane < k) {
    if (lane < kk) {
      const int e = picks[lane];
      idx_t[lane] = e;
      gate_t[lane] = (float)(ex[e] / z);  // the exponential the sum used
    } else {
      idx_t[lane] = -1;
      gate_t[lane] = 0.0f;
    }
  }
}

// Exclusive prefix sum over the threads of a block (one value per thread, blockDim.x <= 1024);
// tmp: 16 ints of LDS. Every thread of the block must call it.
__device__ inline int block_exclusive_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int t = lane < nw ? tmp[lane] : 0;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const int y = __shfl_up(t, off, 64);
      if (lane >= off) t += y;
    }
    if (lane < nw) tmp[lane] = t;
  }
  __syncthreads();
  const int base = wave ? tmp[wave - 1] : 0;
  *total = tmp[nw - 1];
  __syncthreads();
  return base + x - v;
}

// The GEMM tile table (DispatchScratch::tiles) from the per-expert segment sizes, by the block that
// computed them: thread q holds expert q's count (q < E; other threads 0). Every thread of the block
// calls it (the scan synchronises), after which ds.tiles holds ceil(count / tile_bm) tiles per expert.
__device__ inline void write_tiles(int q, int E, int cnt, const DispatchScratch& ds, int* tmp) {
  if (!ds.tiles) return;  // uniform over the block
  const int nt = q < E ? (cnt + ds.tile_bm - 1) / ds.tile_bm : 0;
  int all = 0;
  const int base = block_exclusive_scan(nt, tmp, &all);
  for (int i = 0; i < nt; ++i) {
    ds.tiles[2 * (base + i)] = q;
    ds.tiles[2 * (base + i) + 1] = i * ds.tile_bm;
  }
  if (q == 0) *ds.n_tiles = all;
}

}  // namespace ember_moe
