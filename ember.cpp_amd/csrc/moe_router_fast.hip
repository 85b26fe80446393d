// Router for batches of tokens with a renormalised softmax router (the reference's moe_ffn_f32_cpu with
// renorm, utils.cpp:704-724): the picks are proven from exact-integer fast logits with a rigorous error
// bound, and the reference's FP64 eight-chain logit (utils.cpp:707, cpu_dot.h:12-21) is computed only for
// the experts the bound cannot rule out. Under renorm the gates read only the picks' logits (the maximum
// and the sum run over the picks, utils.cpp:720-724), so picks and gates equal the reference's bit for bit.
//
// Fast logits. Every row v (a token of x, an expert of the router) is scaled by a power of two s (max |v| /
// s in (63.5, 127]); X = v / s is written as two int8 planes, a1 = rint(X) and a2 = rint(254 (X - a1)), so
// that X = a1 + a2 / 254 + eps with |eps| <= kEps (1/508 and the one f32 rounding of 254 (X - a1)). The
// int8 MFMA sums the four plane products exactly in int32, and
//   fast = s_x s_r (254^2 a1.b1 + 254 (a1.b2 + a2.b1) + a2.b2) / 254^2
// differs from the real dot product sum x_i r_i by at most s_x s_r ((sum |X| + sum |R|) kEps + d kEps^2)
// (expand (A + eps)(B + eta) with A = a1 + a2/254: the dropped terms are X eta + eps B, and |B| <= |R| +
// kEps). Added to that: the f64 chains' own rounding (gamma_{d/8+8} times sum |x_i r_i| <= 127 s_x s_r
// min(sum |X|, sum |R|)), the f32 rounding of the reference's logit, and the f64 rounding of the bound's
// own arithmetic, each overestimated. L = fast - B and U = fast + B (rounded outward to f32) then bracket
// the reference's f32 logit l: L <= l <= U. No property of the MFMA beyond exact integer arithmetic is
// assumed (int32 sums of at most 2 * 127^2 * d < 2^31 for d <= 65536).
//
// Candidates. With theta the k-th largest L of a token, every expert e with U_e < theta has k experts
// whose logits are >= theta > l_e, so it is not a pick whatever the ties; the others (U_e >= theta) are
// the candidates, whose exact logits are computed. The token's logits row then holds the exact logit of
// every candidate and L_e (< theta <= the k-th largest logit) elsewhere, so the routing's top-k over that
// row picks exactly the reference's experts, ties included, and its renormalised gates are the
// reference's. A token or an expert row with a non-finite value takes exact logits for all experts.
#include "moe_conv.hpp"
#include "moe_route_dev.hpp"

namespace ember_moe {
using namespace ember_math;

typedef long i8x16 __attribute__((ext_vector_type(2)));  // 16 int8 MFMA operands per lane
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kFastTok = 8;       // tokens per refine block
constexpr int kFastMaxE = 256;    // experts a refine wave holds (4 per lane)
constexpr int kFastKWaves = 8;    // waves splitting K in a fast-logit block
constexpr int kFastGroups = 2;    // 128-element K groups whose loads a fast-logit wave issues at once

// ---- row quantisation: one wave per row (rows 0..T-1 of x, then the E rows of the router), the row's
// slice held in registers (d <= 64 * 4 * kQuantV; longer rows are read twice); blocks past the rows convert
// activations for the MFMA paths (act_conv_row). f32 arithmetic: X = ldexp(v, -q) is exact unless it is
// subnormal (then |X| < 2^-126 and a1 = a2 = 0 leave eps = X); X - a1 is exact; 254 (X - a1) rounds once,
// so |eps| <= 1/508 + 2^-25 = kEps. stat[row] = (s, sum |X| rounded up), s = -1 for a non-finite row.
constexpr int kQuantV = 16;
constexpr double kEps = 1.0 / 508.0 + 0x1p-25;
__device__ inline float quant4(const float4 v, int q, bool bad, uint32_t& w1, uint32_t& w2) {
  const float vv[4] = {v.x, v.y, v.z, v.w};
  float sa = 0.0f;
  w1 = w2 = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float X = bad ? 0.0f : __builtin_ldexpf(vv[j], -q);
    const float a1 = __builtin_rintf(X);
    const float a2 = __builtin_rintf((X - a1) * 254.0f);
    sa += __builtin_fabsf(X);
    w1 |= (uint32_t)((int)a1 & 0xff) << (8 * j);
    w2 |= (uint32_t)((int)a2 & 0xff) << (8 * j);
  }
  return sa;
}
__device__ inline void max4(const float4 v, float& mx, bool& bad) {
  bad |= !__builtin_isfinite(v.x) || !__builtin_isfinite(v.y) || !__builtin_isfinite(v.z) || !__builtin_isfinite(v.w);
  mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
}

__global__ void __launch_bounds__(256) router_quant_kernel(const float* __restrict__ x, int T,
                                                           const float* __restrict__ R, int E, int d,
                                                           int8_t* __restrict__ p1, int8_t* __restrict__ p2,
                                                           double2* __restrict__ stat, ActConv conv) {
  const int nqb = (T + E + 3) / 4;
  if ((int)blockIdx.x >= nqb) {
    act_conv_row(conv, blockIdx.x - nqb);
    return;
  }
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= T + E) return;
  const float* src = row < T ? x + (size_t)row * d : R + (size_t)(row - T) * d;
  const bool held = d <= 256 * kQuantV;
  float4 v[kQuantV];
  float mx = 0.0f;
  bool bad = false;
  if (held) {
#pragma unroll
    for (int j = 0; j < kQuantV; ++j)
      if (lane * 4 + 256 * j < d) v[j] = *reinterpret_cast<const float4*>(src + lane * 4 + 256 * j);
#pragma unroll
    for (int j = 0; j < kQuantV; ++j)
      if (lane * 4 + 256 * j < d) max4(v[j], mx, bad);
  } else {
    for (int i = lane * 4; i < d; i += 256) max4(*reinterpret_cast<const float4*>(src + i), mx, bad);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  bad = __any(bad);
  // s = 2^q with max / s in (63.5, 127]: max = f 2^ex, f in [0.5, 1); 128 f <= 127 decides q
  int q = 0;
  if (mx > 0.0f && !bad) {
    int ex;
    const float f = __builtin_frexpf(mx, &ex);
    q = f * 128.0f <= 127.0f ? ex - 7 : ex - 6;
  }
  double sa = 0.0;  // each 4-term f32 sum rounds up to 3 times (relative 2^-24 each)
  int8_t* d1 = p1 + (size_t)row * d;
  int8_t* d2 = p2 + (size_t)row * d;
  if (held) {
#pragma unroll
    for (int j = 0; j < kQuantV; ++j) {
      const int i = lane * 4 + 256 * j;
      if (i < d) {
        uint32_t w1, w2;
        sa += (double)quant4(v[j], q, bad, w1, w2);
        *reinterpret_cast<uint32_t*>(d1 + i) = w1;
        *reinterpret_cast<uint32_t*>(d2 + i) = w2;
      }
    }
  } else {
    for (int i = lane * 4; i < d; i += 256) {
      uint32_t w1, w2;
      sa += (double)quant4(*reinterpret_cast<const float4*>(src + i), q, bad, w1, w2);
      *reinterpret_cast<uint32_t*>(d1 + i) = w1;
      *reinterpret_cast<uint32_t*>(d2 + i) = w2;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sa += __shfl_xor(sa, off, 64);
  // rounding of the sums, and the subnormal X whose rounding the sum does not see (2^-149 each)
  if (lane == 0)
    stat[row] = make_double2(bad ? -1.0 : __builtin_ldexp(1.0, q), sa * (1.0 + 0x1p-20) + (double)d * 0x1p-140);
}

// ---- fast logits: block (32 tokens, 32 experts), eight waves each summing an eighth of K with the int8
// MFMA, the eighths added exactly in LDS. lu[t][e] = (L, U).
// the next float toward -inf / +inf of a finite f (a step of the bit pattern; +-0 step to -+ the least
// subnormal)
__device__ inline float f32_step(float f, bool down) {
  if (f == 0.0f) return down ? -0x1p-149f : 0x1p-149f;
  const uint32_t b = __float_as_uint(f);
  return __uint_as_float((f > 0.0f) == down ? b - 1 : b + 1);
}
__device__ inline float f32_down(double v) {
  const float f = (float)v;
  return (double)f > v && __builtin_isfinite(f) ? f32_step(f, true) : f;
}
__device__ inline float f32_up(double v) {
  const float f = (float)v;
  return (double)f < v && __builtin_isfinite(f) ? f32_step(f, false) : f;
}

__global__ void __launch_bounds__(64 * kFastKWaves) router_fast_kernel(const int8_t* __restrict__ p1,
                                                                       const int8_t* __restrict__ p2,
                                                                       const double2* __restrict__ stat, int T,
                                                                       int E, int d, float2* __restrict__ lu) {
  __shared__ int red[3][16][64];  // the waves' sums, added with exact integer LDS atomics
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < 3 * 16 * 64; i += 64 * kFastKWaves) (&red[0][0][0])[i] = 0;
  const int t0 = blockIdx.x * 32, e0 = blockIdx.y * 32;
  const int ta = min(t0 + (lane & 31), T - 1), ea = T + min(e0 + (lane & 31), E - 1);  // rows past the end
  const int h = lane >> 5;                                                             // repeat the last
  const size_t xo = (size_t)ta * d, ro = (size_t)ea * d;
  i32x16 c11 = {}, cx = {}, c22 = {};
  auto mfma4 = [&](const i8x16& a1, const i8x16& a2, const i8x16& b1, const i8x16& b2) {
    c11 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, c11, 0, 0, 0);
    cx = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b2, cx, 0, 0, 0);
    cx = __builtin_amdgcn_mfma_i32_32x32x32_i8(a2, b1, cx, 0, 0, 0);
    c22 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a2, b2, c22, 0, 0, 0);
  };
  // K in groups of 128 elements, one 128-byte line of each row and plane: lane (row, h) loads the line's
  // 64-byte half h and feeds its four 16-byte quarters to four MFMA steps. A and B take the same element
  // at every step, so the sums run over each element once whatever order the MFMA gives K.
  const int ng = d / 128, gq = (ng + kFastKWaves - 1) / kFastKWaves;
  const int g0 = wave * gq, g1 = min(ng, g0 + gq);
  for (int gb = g0; gb < g1; gb += kFastGroups) {
    i8x16 a1[kFastGroups][4], a2[kFastGroups][4], b1[kFastGroups][4], b2[kFastGroups][4];
#pragma unroll
    for (int u = 0; u < kFastGroups; ++u)
      if (gb + u < g1) {
        const size_t o = (size_t)(gb + u) * 128 + 64 * h;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a1[u][j] = *reinterpret_cast<const i8x16*>(p1 + xo + o + 16 * j);
          a2[u][j] = *reinterpret_cast<const i8x16*>(p2 + xo + o + 16 * j);
          b1[u][j] = *reinterpret_cast<const i8x16*>(p1 + ro + o + 16 * j);
          b2[u][j] = *reinterpret_cast<const i8x16*>(p2 + ro + o + 16 * j);
        }
      }
#pragma unroll
    for (int u = 0; u < kFastGroups; ++u)
      if (gb + u < g1)
#pragma unroll
        for (int j = 0; j < 4; ++j) mfma4(a1[u][j], a2[u][j], b1[u][j], b2[u][j]);
  }
  if (wave == kFastKWaves - 1)  // the last d % 128 elements, 32 per step (d % 32 == 0)
    for (int k = ng * 128; k < d; k += 32) {
      const size_t o = (size_t)k + 16 * h;
      mfma4(*reinterpret_cast<const i8x16*>(p1 + xo + o), *reinterpret_cast<const i8x16*>(p2 + xo + o),
            *reinterpret_cast<const i8x16*>(p1 + ro + o), *reinterpret_cast<const i8x16*>(p2 + ro + o));
    }
  __syncthreads();  // red cleared
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    atomicAdd(&red[0][r][lane], c11[r]);
    atomicAdd(&red[1][r][lane], cx[r]);
    atomicAdd(&red[2][r][lane], c22[r]);
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    c11[r] = red[0][r][lane];
    cx[r] = red[1][r][lane];
    c22[r] = red[2][r][lane];
  }
  const int e = e0 + (lane & 31);
  if (e >= E) return;
  const double2 se = stat[T + e];
  const double gam = ((double)(d / 8) + 8.0) * 0x1.2p-53;  // the f64 chains' relative error, overestimated
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int t = t0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if (t >= T) continue;
    const double2 st = stat[t];
    // every term an integer below 2^53: exact
    const double F = 64516.0 * (double)c11[r] + 254.0 * (double)cx[r] + (double)c22[r];
    const double ss = st.x * se.x;  // exact: powers of two
    const double fast = F * ss / 64516.0;
    double B = ss * ((st.y + se.y) * kEps + (double)d * (kEps * kEps));
    B += ss * 127.0 * fmin(st.y, se.y) * gam;
    B = B * (1.0 + 0x1p-40) + __builtin_fabs(fast) * 0x1p-48;
    B += (__builtin_fabs(fast) + B) * 0x1p-23 + 0x1p-148;  // the f32 rounding of the logit
    lu[(size_t)t * E + e] = make_float2(f32_down(fast - B), f32_up(fast + B));
  }
}

// ---- refine + route: block of kFastTok tokens. (A) wave w takes tokens w, w + 4: theta, the candidates
// (appended to the block's pair list), the row's lower bounds as the default logits. (B) two lanes per
// (token, candidate) pair: lane h runs the reference's chains 4h .. 4h + 3 (elements 8q + c, one 16-byte
// load of x and of the router row per q) straight from global memory, the next kSteps loads in flight
// while the current ones are summed; the lanes' ((c0 + c1) + (c2 + c3)) and ((c4 + c5) + (c6 + c7)) are
// added in the reference's order. (C) wave w writes tokens w, w + 4's logits rows and routes them
// (route_token, as the exact router's route launch does).
struct FastRefineArgs {
  const float* x;
  const float* R;
  const float2* lu;
  const double2* stat;
  int T, d, E, k;
  int check;  // every logit exact, and one outside its [L, U] turns its token's picks to -1 / NaN gates
  float* logits;
  int32_t* idx;
  float* gates;
};

constexpr int kSteps = 8;    // chain steps per load batch

__host__ __device__ inline size_t fast_refine_lds(int E) {
  return 4 * route_wave_lds(E) + (size_t)kFastTok * E * 4 /*vals*/ + (size_t)kFastTok * E * 4 /*pairs*/ + 64;
}

__global__ void __launch_bounds__(256) router_refine_kernel(FastRefineArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int E = a.E, d = a.d, k = a.k;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  float* vals = reinterpret_cast<float*>(lds_raw + 4 * route_wave_lds(E));  // [kFastTok][E]
  int* pairs = reinterpret_cast<int*>(vals + kFastTok * E);                  // (token << 16) | expert
  int* np = pairs + kFastTok * E;
  int* viol = np + 1;  // [kFastTok] check mode: a logit outside its bounds
  const int tb = blockIdx.x * kFastTok;
  const int ntok = min(kFastTok, a.T - tb);
  if (tid == 0) *np = 0;
  if (tid < kFastTok) viol[tid] = 0;
  __syncthreads();
  // (A)
  for (int tl = wave; tl < ntok; tl += 4) {
    const int t = tb + tl;
    bool all = a.check || a.stat[t].x < 0.0 || k >= E;
    float Lv[4], Uv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      Lv[j] = -__builtin_inff();
      Uv[j] = -__builtin_inff();
      if (e < E) {
        const float2 v = a.lu[(size_t)t * E + e];
        Lv[j] = v.x;
        Uv[j] = v.y;
        all |= a.stat[a.T + e].x < 0.0;
        vals[tl * E + e] = v.x;
      }
    }
    all = __any(all);
    float theta = -__builtin_inff();
    if (!all) {
      // the k-th largest L, counted with multiplicity: k passes, each removing one occurrence of the maximum
      unsigned tk = 0;  // bit j: this lane's Lv[j] already taken
      for (int p = 0; p < k; ++p) {
        float m = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (!(tk >> j & 1)) m = fmaxf(m, Lv[j]);
        float wm = m;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) wm = fmaxf(wm, __shfl_xor(wm, off, 64));
        theta = wm;
        const unsigned long long holders = __ballot(m == wm);
        if (lane == __builtin_ctzll(holders)) {
          bool done = false;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (!done && !(tk >> j & 1) && Lv[j] == wm) {
              tk |= 1u << j;
              done = true;
            }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      const bool cand = e < E && (all || Uv[j] >= theta);
      const unsigned long long b = __ballot(cand);
      int base = 0;
      if (lane == 0 && b) base = atomicAdd(np, __builtin_popcountll(b));
      base = __shfl(base, 0, 64);
      if (cand) pairs[base + __builtin_popcountll(b & ((1ull << lane) - 1))] = (tl << 16) | e;
    }
  }
  __syncthreads();
  // (B)
  const int P = *np, h = tid & 1;
  for (int p0 = 0; p0 < P; p0 += 128) {  // passes of 128 pairs, two lanes each
    const int pp = p0 + (tid >> 1);
    const bool on = pp < P;
    const int pr = pairs[on ? pp : p0];  // a lane past the end reads the pass's first pair
    const float4* xr = reinterpret_cast<const float4*>(a.x + (size_t)(tb + (pr >> 16)) * d) + h;
    const float4* rr = reinterpret_cast<const float4*>(a.R + (size_t)(pr & 0xffff) * d) + h;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};  // chains 4h .. 4h + 3
    const int nq = d / 8, nb = nq / kSteps;
    float4 xv[kSteps], rv[kSteps];
    if (nb > 0)
#pragma unroll
      for (int j = 0; j < kSteps; ++j) {
        xv[j] = xr[2 * j];
        rv[j] = rr[2 * j];
      }
    for (int bb = 0; bb < nb; ++bb) {
      float4 xn[kSteps], rn[kSteps];
      if (bb + 1 < nb)
#pragma unroll
        for (int j = 0; j < kSteps; ++j) {
          xn[j] = xr[2 * (kSteps * (bb + 1) + j)];
          rn[j] = rr[2 * (kSteps * (bb + 1) + j)];
        }
#pragma unroll
      for (int j = 0; j < kSteps; ++j) {
        acc[0] = __builtin_fma((double)rv[j].x, (double)xv[j].x, acc[0]);
        acc[1] = __builtin_fma((double)rv[j].y, (double)xv[j].y, acc[1]);
        acc[2] = __builtin_fma((double)rv[j].z, (double)xv[j].z, acc[2]);
        acc[3] = __builtin_fma((double)rv[j].w, (double)xv[j].w, acc[3]);
      }
#pragma unroll
      for (int j = 0; j < kSteps; ++j) {
        xv[j] = xn[j];
        rv[j] = rn[j];
      }
    }
    for (int q = kSteps * nb; q < nq; ++q) {
      const float4 xq = xr[2 * q], rq = rr[2 * q];
      acc[0] = __builtin_fma((double)rq.x, (double)xq.x, acc[0]);
      acc[1] = __builtin_fma((double)rq.y, (double)xq.y, acc[1]);
      acc[2] = __builtin_fma((double)rq.z, (double)xq.z, acc[2]);
      acc[3] = __builtin_fma((double)rq.w, (double)xq.w, acc[3]);
    }
    const double half = (acc[0] + acc[1]) + (acc[2] + acc[3]);  // lane h: ((c4h + c4h+1) + (c4h+2 + c4h+3))
    const double other = __shfl_xor(half, 1, 64);
    if (on && h == 0) {
      const int tl = pr >> 16, e = pr & 0xffff;
      const float v = (float)(half + other);
      vals[tl * E + e] = v;
      if (a.check && a.stat[tb + tl].x >= 0.0 && a.stat[a.T + e].x >= 0.0) {
        const float2 b = a.lu[(size_t)(tb + tl) * E + e];
        if (!(b.x <= v && v <= b.y)) viol[tl] = 1;
      }
    }
  }
  __syncthreads();
  // (C)
  unsigned char* wl = lds_raw + wave * route_wave_lds(E);
  for (int tl = wave; tl < ntok; tl += 4) {
    const int t = tb + tl;
    float* lrow = a.logits + (size_t)t * E;
    for (int e = lane; e < E; e += 64) lrow[e] = vals[tl * E + e];  // route_token reads e on this same lane
    route_token<false>(lrow, E, k, 1, 0, 0, nullptr, 1, 1, wl, a.idx + (size_t)t * k, a.gates + (size_t)t * k);
    if (viol[tl] && lane < k) {
      a.idx[(size_t)t * k + lane] = -1;
      a.gates[(size_t)t * k + lane] = __builtin_nanf("");
    }
  }
}

bool router_fast_fits(int T, int d, int E, int k, int renorm, int routed) {
  if (!renorm || routed || E > kFastMaxE || k > 64 || d % 32 || d > 65536) return false;
  // read per call (tests switch it): off unless EMBER_ROUTER_FAST=1 (measured no faster than the exact
  // router: the per-pair exact chains re-read a router row per candidate through L2); EMBER_ROUTER_FAST_T
  // sets the smallest batch that takes it
  const char* v = std::getenv("EMBER_ROUTER_FAST");
  if (!v || atoi(v) == 0) return false;
  const char* tv = std::getenv("EMBER_ROUTER_FAST_T");
  return T >= (tv ? std::max(1, atoi(tv)) : 64);
}

size_t router_fast_work_bytes(int T, int d, int E) {
  const size_t rows = (size_t)T + E;
  return 2 * rows * d + rows * sizeof(double2) + (size_t)T * E * sizeof(float2) + 3 * 256;
}

int launch_router_fast(const float* x, int T, int d, int E, int k, const float* R, float* logits, int32_t* idx,
                       float* gates, void* work, const ActConv* conv, hipStream_t st) {
  if (T <= 0) return EMBER_OK;
  const size_t rows = (size_t)T + E;
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  unsigned char* w = static_cast<unsigned char*>(work);
  int8_t* p1 = reinterpret_cast<int8_t*>(w);
  int8_t* p2 = reinterpret_cast<int8_t*>(w + up(rows * d));
  double2* stat = reinterpret_cast<double2*>(w + 2 * up(rows * d));
  float2* lu = reinterpret_cast<float2*>(w + 2 * up(rows * d) + up(rows * sizeof(double2)));
  const ActConv c = conv ? *conv : ActConv{};
  router_quant_kernel<<<(unsigned)((rows + 3) / 4) + c.rows, 256, 0, st>>>(x, T, R, E, d, p1, p2, stat, c);
  router_fast_kernel<<<dim3((T + 31) / 32, (E + 31) / 32), 64 * kFastKWaves, 0, st>>>(p1, p2, stat, T, E, d, lu);
  const char* cv = std::getenv("EMBER_ROUTER_FAST_CHECK");  // read per call: tests switch it
  const int check = cv ? atoi(cv) : 0;
  FastRefineArgs fa{x, R, lu, stat, T, d, E, k, check, logits, idx, gates};
  const size_t lds = fast_refine_lds(E);
  static const bool lds_ok = hipFuncSetAttribute(reinterpret_cast<const void*>(&router_refine_kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)fast_refine_lds(kFastMaxE)) == hipSuccess;
  if (!lds_ok) return EMBER_ERR_LAUNCH;
  router_refine_kernel<<<(T + kFastTok - 1) / kFastTok, 256, lds, st>>>(fa);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

}  // namespace ember_moe
