// Expert projections of the MoE FFN for decode-sized segments: a bandwidth kernel that streams each
// selected expert's rows once, dequantizes the llama.cpp blocks in registers and reduces across
// lanes with cross-lane shuffles. Also the activation quantizer and the ordered combine.
//
// Reference semantics (utils.cpp:735-747): per selected expert, g = W_gate x, u = W_up x,
// h = g * (1/(1+expf(-g))) * u, y = W_down h, out = sum over experts ascending of gate * y.
// The reference evaluates these as FP64 dots over F32 weights dequantized at load
// (weight_management.cpp:802-877). Here:
//  * F32 / F16 / BF16 weights: FP32 dots over the exactly-decoded weights and FP32 activations
//    (F32 layers stay within 1e-4 max-abs / 1e-5 rel-L2 of the reference);
//  * Q8_0 / Q4_K weights: the activations are quantized to int16 per 32-element block (scale
//    amax/32767, relative error ~2e-5) and each block's integer dot runs exactly in int32 (Q8_0: on
//    v_dot2_i32_i16 with the quants zero-extended to 16 bits, offset by +128 and corrected with the
//    block's activation sum; Q4_K: the nibbles straight into v_dot4 against the activations staged as
//    byte planes), then scaled in FP32. Relative error stays near 1e-5, far inside 2e-3.
//
// Work layout (proj_kernel): a lane owns a 32/64-element "chunk" of a row (fixed byte offset in the
// ggml row); L lanes (a power of two <= 64) cover a row, so a wave covers 64/L rows; a ring of register
// buffers keeps the next loads in flight. The launch is one resident wave of blocks that share the
// expert segments (experts that received tokens, from the dispatch step, read on the device: no host
// synchronisation) in proportion to their rows (seg_view).
//
// One-token calls fuse the router, the routing and the dispatch into the first launch (router blocks
// publish tagged logits; the other blocks prove the pick set from bounded fast logits or wait for the
// exact ones; block 0 writes the exact record and flags a contradiction), then run either the down
// launch with the combine fused in (down1_kernel), or, with a Q8_0 / Q4_K prefill pack, the whole layer
// as one launch over 64-column slices of d_ff (slice_kernel) plus an ordered reduce.
#include <cstdlib>
#include <type_traits>

#include <hip/hip_ext.h>

#include "moe_fmt.hpp"
#include "moe_route_dev.hpp"

namespace ember_moe {
using namespace ember_math;

// Timeline probe for profiling builds (-DEMBER_PROBE): thread 0 of each block stamps the 100 MHz
// real-time counter into probe[(launch slot * grid + block) * 8 + point]. Compiled out otherwise.
#ifdef EMBER_PROBE
__constant__ unsigned long long* g_probe;
#define EMBER_STAMP(slot, pt)                                                                        \
  do {                                                                                              \
    if (g_probe && threadIdx.x == 0)                                                                \
      g_probe[((size_t)(slot) * 4096 + blockIdx.x) * 8 + (pt)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define EMBER_STAMP(slot, pt) \
  do {                        \
  } while (0)
#endif


constexpr int kProjLdsBytes = 80 * 1024;     // staged activation rows per block (two blocks per CU)

// f(integral_constant<int, j>) for j = 0 .. N-1 (compile-time ring positions)
template <int N, class Fn, int... J>
__device__ inline void ring_for_impl(Fn&& f, std::integer_sequence<int, J...>) {
  (f(std::integral_constant<int, J>{}), ...);
}
template <int N, class Fn>
__device__ inline void ring_for(Fn&& f) {
  ring_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

// Which segment block b of G serves, and its share of that segment's rows. Blocks go to segments in
// proportion to their work, rows x (passes over the weights + kTokW / kPassW per extra token of a pass):
// a segment's weight bytes set its streaming time and its tokens its dot-product time (on the
// decode path a segment with four tokens costs well over one with a single token). Every segment gets
// at least one block. Each wave computes the split itself (a prefix sum over the segments with
// shuffles), so blocks need no coordination.
constexpr int kPassW = 2, kTokW = 1;

// The dispatch order a launch schedules from.
struct Dispatch {
  int n_used;
  const int32_t* used;
  const int32_t* offsets;
  const int32_t* perm;
};

struct SegView {
  const uint8_t* W0;
  const uint8_t* W1;
  int rows, K, p0, M;
  const float* in;
  float* out;
  bool by_perm;
  int jb, nb;  // block index within the segment, blocks of the segment
};

__device__ inline float seg_work(int rows, int M, int MT) {
  const int passes = (M + MT - 1) / MT;
  return (float)rows * (float)(kPassW * passes + kTokW * (M - passes));
}

// inclusive prefix sum over the wave's lanes (every wave computes it identically)
__device__ inline float wave_incl_scan(float v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float y = __shfl_up(v, off, 64);
    if (lane >= off) v += y;
  }
  return v;
}
__device__ inline int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ONE_TOKEN: every routed segment holds one token (a one-token launch, at most 64 picks), so each has the
// same work w and the prefix sums are s w (integer-valued floats: the same values the scans give)
// gr_fixed >= 0: the routed blocks are 0 .. gr_fixed - 1 whatever the number of segments (the one-token
// launches fix the split before the routing is known, so that the shared segment's blocks need not wait)
template <bool GATED, int MT, bool ONE_TOKEN = false>
__device__ inline bool seg_view(const ProjArgs& a, const Dispatch& dp, int b, int G, SegView& v, int gr_fixed = -1) {
  const int nseg = a.used ? dp.n_used : 0;
  const int lane = threadIdx.x & 63;
  // routed work: total, then this block's segment from the prefix sums
  float w_routed = 0.0f;
  const float w1 = seg_work(a.rows, 1, MT);
  if constexpr (ONE_TOKEN) {
    w_routed = (float)nseg * w1;
  } else {
    for (int s0 = 0; s0 < nseg; s0 += 64) {
      const int s = s0 + lane;
      float w = 0.0f;
      if (s < nseg) {
        const int e = dp.used[s];
        w = seg_work(a.rows, dp.offsets[e + 1] - dp.offsets[e], MT);
      }
      w_routed += __shfl(wave_incl_scan(w), 63, 64);
    }
  }
  const float w_shared = a.s_w0 ? seg_work(a.s_rows, a.T, MT) : 0.0f;
  if (w_routed + w_shared == 0.0f) return false;
  int Gr = 0;
  if (gr_fixed >= 0)
    Gr = gr_fixed;
  else if (nseg > 0)
    Gr = w_shared ? uniform(max(nseg, min(G - 1, (int)(G * (w_routed / (w_routed + w_shared)))))) : G;
  if (b < Gr) {
    if (nseg == 0) return false;  // (a fixed split whose token has no valid pick)
    // block start of segment s: s + floor((Gr - nseg) * W(<s) / W); the block's segment is the one
    // whose [start, next start) holds b
    const float spare = (float)(Gr - nseg);
    int seg = 0, bs = 0, be = Gr;
    float carry = 0.0f;
    for (int s0 = 0; s0 < nseg; s0 += 64) {
      const int s = s0 + lane;
      float w = 0.0f, incl;
      if constexpr (ONE_TOKEN) {
        w = s < nseg ? w1 : 0.0f;
        incl = (float)min(s + 1, nseg) * w1;
      } else {
        if (s < nseg) {
          const int e = dp.used[s];
          w = seg_work(a.rows, dp.offsets[e + 1] - dp.offsets[e], MT);
        }
        incl = carry + wave_incl_scan(w);
      }
      const float excl = incl - w;
      const int start = s + min(Gr - nseg, (int)(spare * (excl / w_routed)));
      const int next = s + 1 + min(Gr - nseg, (int)(spare * (incl / w_routed)));
      const uint64_t m = __ballot(s < nseg && start <= b && b < next);
      if (m) {
        const int src = __builtin_ctzll(m);
        seg = __shfl(s, src, 64);
        bs = __shfl(start, src, 64);
        be = __shfl(next, src, 64);
      }
      carry = __shfl(incl, 63, 64);
    }
    seg = uniform(seg);
    bs = uniform(bs);
    be = uniform(be);
    v.jb = b - bs;
    v.nb = be - bs;
    const int e = uniform(dp.used[seg]);
    v.p0 = uniform(dp.offsets[e]);
    v.M = uniform(dp.offsets[e + 1]) - v.p0;
    v.W0 = static_cast<const uint8_t*>(a.w0) + (int64_t)e * a.expert_stride;
    v.W1 = GATED ? static_cast<const uint8_t*>(a.w1) + (int64_t)e * a.expert_stride : v.W0;
    v.rows = a.rows;
    v.K = a.K;
    v.in = a.in;
    v.out = a.out;
    v.by_perm = a.in_by_perm;
  } else {
    if (w_shared == 0.0f) return false;
    v.jb = b - Gr;
    v.nb = G - Gr;
    v.p0 = 0;
    v.M = a.T;
    v.W0 = static_cast<const uint8_t*>(a.s_w0);
    v.W1 = GATED ? static_cast<const uint8_t*>(a.s_w1) : v.W0;
    v.rows = a.s_rows;
    v.K = a.s_K;
    v.in = a.s_in;
    v.out = a.s_out;
    v.by_perm = false;
  }
  return true;
}

// One projection. The blocks of a segment share its rows, interleaved over their waves (see below). L
// lanes (a power of two <= 64) cover a row, one chunk per lane per step (looping NC rounds when a row
// has more than L chunks), so a step covers 64 / L rows. Weight loads run through a ring of NB
// register buffers ahead of the dots. MT tokens per pass over the weights; their activation rows are
// staged in LDS (quantized on the way for Q8_0 / Q4_K).
// The body of proj_kernel for one segment view.
// PRESTAGED (one-token launches only): the activation row is already at the start of the dynamic LDS,
// staged at the start of the launch, so the pass skips its staging.
// COHERENT_OUT: the outputs are device-coherent stores (no L2 write-back needed before another XCD
// reads them in the same launch: the one-launch layer's h rows).
template <int FMT, int MT, bool GATED, int NB, int NT, bool COHERENT_OUT = false, bool PRESTAGED = false>
__device__ inline void proj_body(const ProjArgs& a, const Dispatch& dp, const SegView& v) {
  using F = Fmt<FMT>;
  constexpr int G2 = GATED ? 2 : 1;
  extern __shared__ __align__(16) uint8_t act_lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = NT / 64;
  const int K = v.K;
  const int C = (K + F::CE - 1) / F::CE;
  int Lg = 0;
  while ((1 << Lg) < C && Lg < 6) ++Lg;
  const int L = 1 << Lg, RPS = 64 >> Lg;
  const int sub = lane >> Lg, rl = lane & (L - 1);
  const int NC = (C + L - 1) / L;
  // Rows are interleaved over the segment's waves: step st of wave w (w-th of the segment's W waves)
  // covers row group (st / NC) * W + w, so that at any time the segment's waves read adjacent rows
  // (DRAM pages stay open), rather than each wave streaming its own distant range.
  const int wseg = v.jb * nwaves + wave, Wseg = v.nb * nwaves;
  const int gt = (v.rows + RPS - 1) / RPS;
  const int rbase = wseg * RPS, rstride = Wseg * RPS, rend = v.rows;
  const int ngroups = wseg < gt ? (gt - wseg + Wseg - 1) / Wseg : 0;
  const int nsteps = ngroups * NC;
  const int64_t rb = F::row_bytes(K);
  const int row_lds = act_lds_bytes(F::QX, K);

  __shared__ int rows_idx[MT];

  // weights of matrix g (0: gate or the only one, 1: up) for step st; out-of-range (row, chunk) pairs
  // load a valid neighbour, which dot() then ignores
  auto load_step = [&](int st, int g, uint32_t (&buf)[F::NW]) {
    const int r = max(0, min(rbase + (st / NC) * rstride + sub, rend - 1));
    const int c = min(rl + (st % NC) * L, C - 1);
    F::load((g ? v.W1 : v.W0) + (int64_t)r * rb, c, K, buf);
  };

  // Weight loads form one sequence q = 0, 1, ... (gated: gate and up of a step alternate) that runs
  // through a ring of NB register buffers: NB - 1 loads are in flight while one buffer is consumed.
  const int nloads = nsteps * G2;
#pragma unroll 1
  for (int m0 = 0; m0 < v.M; m0 += MT) {
    const int nvalid = min(MT, v.M - m0);
    uint32_t buf[NB][F::NW];
    // the first weights travel while the activations are staged
    // loads past the end of the stream are clamped to valid addresses and their dots masked, so that
    // the ring below is straight-line code (divergent guards make the compiler drain every load)
    auto pre = [&](auto J) {
      constexpr int j = decltype(J)::value;
      load_step(j / G2, j % G2, buf[j]);
    };
    if (nloads > 0) ring_for<NB - 1>(pre);  // wave-uniform: a wave without rows loads nothing
    if constexpr (!PRESTAGED) {
      __syncthreads();  // the previous pass no longer reads the staged rows
      if (threadIdx.x < nvalid) {
        const int p = v.p0 + m0 + threadIdx.x;
        rows_idx[threadIdx.x] = v.by_perm ? dp.perm[p] / a.k : p;
      }
      __syncthreads();
      if constexpr (F::QX)
        stage_rows_quant<F::PLANES>(v.in, K, rows_idx, nvalid, act_lds, row_lds);
      else
        stage_rows_f32<F::NGL>(v.in, K, rows_idx, nvalid, act_lds, row_lds);
      __syncthreads();
    }
    EMBER_STAMP(GATED ? 0 : 1, 5);

    float acc[G2][MT];
#pragma unroll
    for (int g = 0; g < G2; ++g)
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[g][m] = 0.0f;

    auto dot = [&](int q, const uint32_t (&b)[F::NW], float (&ac)[MT]) {
      const int st = q / G2;
      const int r = rbase + (st / NC) * rstride + sub;
      const int c = rl + (st % NC) * L;
      const bool ok = q < nloads && c < C && r < rend;
      float t[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) t[m] = 0.0f;
      F::template dot_tokens<MT>(b, act_lds, row_lds, min(c, C - 1), K, nvalid, t);
#pragma unroll
      for (int m = 0; m < MT; ++m) ac[m] += ok ? t[m] : 0.0f;
    };
    auto finish = [&](int st) {
      if (st >= nsteps || st % NC != NC - 1) return;  // the row is complete: reduce over the lane group, write
      const int r = rbase + (st / NC) * rstride + sub;
#pragma unroll
      for (int g = 0; g < G2; ++g)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          float t = acc[g][m];
#pragma unroll
          for (int off = 32; off >= 1; off >>= 1)
            if (off < L) t += __shfl_xor(t, off, 64);
          acc[g][m] = t;
        }
      if (rl == 0 && r < rend) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
          if (m < nvalid)
          {
            const float o = GATED ? swiglu(acc[0][m], acc[G2 - 1][m]) : acc[0][m];
            float* dst = v.out + (size_t)(v.p0 + m0 + m) * v.rows + r;
            if constexpr (COHERENT_OUT)
              __hip_atomic_store(dst, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
              *dst = o;
          }
      }
#pragma unroll
      for (int g = 0; g < G2; ++g)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[g][m] = 0.0f;
    };
    // One ring position per call, with compile-time buffer indices so the ring stays in registers. The
    // walk advances U = lcm(NB, G2) loads per iteration, so that both the buffer (q % NB) and the
    // matrix (q % G2) of load q are compile-time constants.
    constexpr int U = (NB % G2 == 0) ? NB : NB * G2;
    auto slot = [&](int q0, auto J) {
      constexpr int j = decltype(J)::value;
      const int q = q0 + j;
      load_step((q + NB - 1) / G2, (j + NB - 1) % G2, buf[(j + NB - 1) % NB]);
      dot(q, buf[j % NB], acc[j % G2]);
      if (q == 0) EMBER_STAMP(GATED ? 0 : 1, 6);
      if (j % G2 == G2 - 1) finish(q / G2);
    };
#pragma unroll 1
    for (int q0 = 0; q0 < nloads; q0 += U) ring_for<U>([&](auto J) { slot(q0, J); });
  }
}

// ---- routing fused into a one-token gate/up launch (ProjArgs::route)
// Words of the flag area: [0] the count of blocks that computed a missing logit themselves, [1] the
// count of calls whose exact picks differed from the fast ones; [2 + e] expert e's logit under the
// call's logit tag (Route::logit_tag in the high half, the f32 bits in the low half). A word is read
// with one device-coherent load and carries its own data, so no ordering between a payload and a flag
// is needed. The tags change from call to call (a per-process call counter mixed into two constants),
// so a word left behind by an earlier call never matches.
constexpr int kFusedMaxK = 8;
// The launch's own tag: its AQL dispatch packet's address (distinct for consecutive dispatches on a
// queue, graph replays included, whose packets take new queue slots) mixed with the call's host tag. A
// word written by an earlier launch therefore never carries the current launch's tag, even when no later
// launch of that call cleared it or a captured graph replays the same host tags.
__device__ inline uint32_t launch_tag(uint32_t host) {
  const uint64_t p = (uint64_t)__builtin_amdgcn_dispatch_ptr();
  uint32_t t = ((uint32_t)(p >> 6) ^ ((uint32_t)(p >> 38) * 0x85ebca6bu)) ^ host;
  t *= 0x9e3779b1u;
  return t ^ (t >> 15);
}
__device__ inline uint32_t logit_tag(const ProjArgs::Route& r) { return launch_tag(r.logit_tag) | 1u; }
__device__ inline uint32_t fast_tag(const ProjArgs::Route& r) {
  const uint32_t t = launch_tag(r.fast_tag) & ~1u;
  return t ? t : 2u;
}
// Words [2 + E + e]: expert e's fast logit under the call's fast tag — the same exact products summed as a
// tree (so available ~4 us before the reference's eight chains are added), as binary32 with the low 8
// mantissa bits replaced by a bound: |fast - the reference's double logit| <= 2^(low byte - 160) (255: no
// bound). Word [2 + 2E]: this call's conflict status (block 0 sets it to 0 at the start of the launch and
// to 1 if its exact picks contradict the fast words); the launch that writes the output rows reads it and
// writes NaN rows when it is set, so a wrong pick set can never pass as a valid result.

// The fast word of a logit whose exact products sum to s (tree order) with sum |p| = S, for a dot of
// nq groups of eight. Bound (Higham, recursive sums): a sum of exact terms whose every term passes
// through at most D additions is within D u / (1 - D u) * S of the true sum, u = 2^-53. The tree's D is
// at most 16 products per thread + 7 tail products + 6 wave levels + 16 wave partials = 45; the
// reference's chains add nq terms, then 3 combining levels and the tail (an fma chain of at most 7
// exact products, then one add): D <= nq + 11. 2 (nq + 64) u S covers both with room for the rounding
// of S itself; truncating the binary32 value to 16 significant bits adds at most 2^-14 |s| + 2^-140.
__device__ inline unsigned long long fast_word(double s, double S, int nq, uint32_t tag) {
  const float f = (float)s;
  uint32_t eb = 255;
  const double B = 2.0 * (double)(nq + 64) * 0x1p-53 * S + fabs(s) * 0x1p-14 + 0x1p-140;
  if (__builtin_isfinite(f) && __builtin_isfinite(B)) {
    // B >= 2^-140 is a normal double: its exponent field is floor(log2 B), so 2^ex > B
    const int ex = (int)((__builtin_bit_cast(unsigned long long, B) >> 52) & 0x7ff) - 1023 + 1;
    eb = ex + 160 < 0 ? 0u : ex + 160 > 254 ? 255u : (uint32_t)(ex + 160);
  }
  return ((unsigned long long)tag << 32) | (__builtin_bit_cast(uint32_t, f) & 0xffffff00u) | eb;
}
// LDS of a router block (the products, f64, chain-major) and, after it, every block's routing area
// (logits, picks, gates, one routing wave's work area)
__host__ __device__ inline size_t fused_router_lds(int d) { return (size_t)8 * d + 8 * 8 * 6 + 256; }
__host__ __device__ inline size_t fused_route_lds(int E) { return 2048 + 512 + route_wave_lds(E); }
// the staged activation row of a one-token launch (16-byte multiple)
__host__ __device__ inline size_t fused_x_lds(int type, int d) {
  return ((size_t)act_lds_bytes(type == EMBER_TYPE_Q8_0 || type == EMBER_TYPE_Q4_K, d) + 15) & ~(size_t)15;
}

// Router block e (blocks 0..E-1): the logit of expert e as the reference computes it (cpu_dot.h:
// eight FP64 chains over i = 8q + c, combined ((c0+c1)+(c2+c3))+((c4+c5)+(c6+c7)), plus the tail).
// Every product (exact in f64) is formed from one round of 16-byte loads and stored chain-major, then
// eight lanes add their chain's products in order — the rounding sequence of acc += (double)r * (double)x.
// Returns the logit in thread 0.
template <int NT, bool FAST>
__device__ __attribute__((always_inline)) float router_block_logit(const ProjArgs& a, int e, uint8_t* lds) {
  const ProjArgs::Route& r = a.route;
  const int t = threadIdx.x, d = r.d, n8 = d - d % 8, nq = n8 / 8;
  // chain stride in doubles: even (16-byte pair reads stay aligned) and 2 mod 4 doubles past a multiple
  // of 64 banks' worth, so the eight chains' pair reads fall on distinct banks
  const int ld = (nq + 3) / 4 * 4 + 2;
  double* pd = reinterpret_cast<double*>(lds);
  const float* row = r.router + (size_t)e * d;
  constexpr int NW = NT / 64;
  __shared__ double fpart[2 * NW];
  double fs = 0.0, fa = 0.0;  // this thread's products: sum, sum of magnitudes (the fast word)
  if (d % 4 == 0) {
    constexpr int PER = 4;  // float4s per thread: d <= 16 * NT
    const int n4 = n8 / 4;
    const float4* x4 = reinterpret_cast<const float4*>(r.x);
    const float4* r4 = reinterpret_cast<const float4*>(row);
    float4 xv[PER], rv[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i4 = min(t + j * NT, n4 - 1);
      xv[j] = x4[i4];
      rv[j] = r4[i4];
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i4 = t + j * NT;
      if (i4 < n4) {
        const int c0 = (4 * i4) & 7, q = i4 >> 1;
        const double p0 = (double)rv[j].x * (double)xv[j].x, p1 = (double)rv[j].y * (double)xv[j].y;
        const double p2 = (double)rv[j].z * (double)xv[j].z, p3 = (double)rv[j].w * (double)xv[j].w;
        pd[(c0 + 0) * ld + q] = p0;
        pd[(c0 + 1) * ld + q] = p1;
        pd[(c0 + 2) * ld + q] = p2;
        pd[(c0 + 3) * ld + q] = p3;
        fs = fs + p0 + p1 + p2 + p3;
        fa = fa + fabs(p0) + fabs(p1) + fabs(p2) + fabs(p3);
      }
    }
  } else {
    for (int i = t; i < n8; i += NT) {
      const double p = (double)row[i] * (double)r.x[i];
      pd[(i & 7) * ld + (i >> 3)] = p;
      fs = fs + p;
      fa = fa + fabs(p);
    }
  }
  if constexpr (FAST) {
    if (t == 0)
      for (int i = n8; i < d; ++i) {
        const double p = (double)row[i] * (double)r.x[i];
        fs = fs + p;
        fa = fa + fabs(p);
      }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      fs = fs + __shfl_xor(fs, off, 64);
      fa = fa + __shfl_xor(fa, off, 64);
    }
    if ((t & 63) == 0) {
      fpart[t >> 6] = fs;
      fpart[NW + (t >> 6)] = fa;
    }
  }
  __syncthreads();
  if (FAST && (t == 64 || (NT == 64 && t == 0))) {  // the fast word, published while wave 0 adds the chains
    double s = 0.0, S = 0.0;
    for (int w = 0; w < NW; ++w) {
      s = s + fpart[w];
      S = S + fpart[NW + w];
    }
    // (test hook: a wrong value under a tight bound, the contradiction block 0 must catch)
    if (r.test_corrupt) s = -s;
    __hip_atomic_store(r.flag + 2 + r.E + e, fast_word(s, S, nq, fast_tag(r)), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  double acc = 0.0;
  if (t < 8) {
    // the chain in order, in bursts of 16 products (8 pair reads) held in two alternating buffers: one
    // burst's reads are in flight while the other is added
    const double* p = pd + (size_t)t * ld;
    const int n32 = nq / 32;
    double2 A[8], B[8];
    if (n32 > 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) A[j] = *reinterpret_cast<const double2*>(p + 2 * j);
    }
    for (int i = 0; i < n32; ++i) {
      const double* pb = p + 32 * i;
      // the scheduling barriers keep each burst's reads ahead of the other burst's adds
#pragma unroll
      for (int j = 0; j < 8; ++j) B[j] = *reinterpret_cast<const double2*>(pb + 16 + 2 * j);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc = acc + A[j].x;
        acc = acc + A[j].y;
      }
      __builtin_amdgcn_sched_barrier(0);
      // the next burst, unconditionally (after the last one these reads are unused; they stay inside the
      // block's LDS, which the launch sizes with room past the products)
#pragma unroll
      for (int j = 0; j < 8; ++j) A[j] = *reinterpret_cast<const double2*>(pb + 32 + 2 * j);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc = acc + B[j].x;
        acc = acc + B[j].y;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    int q = 32 * n32;
    for (; q < nq; ++q) acc = acc + p[q];
  }
  double c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) c[j] = __shfl(acc, j, 64);
  float v = 0.0f;
  if (t == 0) {
    double tail = 0.0;
    for (int i = n8; i < d; ++i) tail = __builtin_fma((double)row[i], (double)r.x[i], tail);
    v = (float)((((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]))) + tail);
  }
  __syncthreads();  // the products area is reused by the caller
  return v;
}

// The one-token dispatch from the picks (ascending, distinct, nv valid): used = the picks, perm the
// identity (a stable sort of the slots by expert), offsets[e] = picks below e.
__device__ inline void fused_dispatch(const int* picks, int nv, int E, int32_t* s_off, int32_t* s_used, int32_t* s_n,
                                      int32_t* s_perm) {
  const int t = threadIdx.x;
  if (t < nv) {
    s_used[t] = picks[t];
    s_perm[t] = t;
  }
  for (int e = t; e <= E; e += blockDim.x) {
    int cnt = 0;
    for (int j = 0; j < nv; ++j) cnt += picks[j] < e;
    s_off[e] = cnt;
  }
  if (t == 0) *s_n = nv;
}

// Block 0's record of the routing for the later launches (logits, idx, gates, pos, used, perm, offsets,
// n_used), from the routing area.
template <int NT, bool ROUTED>
__device__ __attribute__((always_inline)) void route_publish(const ProjArgs& a, uint8_t* ra) {
  const ProjArgs::Route& r = a.route;
  const int t = threadIdx.x;
  float* lg = reinterpret_cast<float*>(ra);
  int32_t* pidx = reinterpret_cast<int32_t*>(ra + 2048);
  float* pgate = reinterpret_cast<float*>(ra + 2048 + 256);
  const int E = r.E, k = a.k;
  int nv = 0;
  for (int j = 0; j < k; ++j) nv += pidx[j] >= 0;
  {
    for (int e = t; e < E; e += NT) r.logits[e] = lg[e];
    if (t < k) {
      r.idx[t] = pidx[t];
      r.gates[t] = pgate[t];
      r.pos[t] = t < nv ? t : -1;
    }
    if (t < nv) {
      r.used[t] = pidx[t];
      r.perm[t] = t;
    }
    for (int e = t; e <= E; e += NT) {
      int cnt = 0;
      for (int j = 0; j < nv; ++j) cnt += pidx[j] < e;
      r.offsets[e] = cnt;
    }
    if (t == 0) *r.n_used = nv;
  }
}

// Router logits of a few tokens (the launch before the expert GEMMs of a small batch): block (e, t) computes
// logit [t][e] with router_block_logit (the one-token launch's exact FP64 chains: products formed in
// parallel, each chain added in order), so a batch of T tokens costs one such block per pair.
__global__ void __launch_bounds__(512) router_logits_blocks(const float* __restrict__ x, const float* __restrict__ R,
                                                            float* __restrict__ logits, int T, int d, int E) {
  extern __shared__ __align__(16) uint8_t rb_lds[];
  ProjArgs a{};
  a.route.x = x + (size_t)blockIdx.y * d;
  a.route.router = R;
  a.route.d = d;
  a.route.E = E;
  const float v = router_block_logit<512, false>(a, blockIdx.x, rb_lds);
  if (threadIdx.x == 0) logits[(size_t)blockIdx.y * E + blockIdx.x] = v;
}

bool router_blocks_fit(int T, int d, int E) {
  return d % 4 == 0 && d <= 16 * 512 && (int64_t)T * E <= 1024 && T <= 65535;
}

int launch_router_logits_blocks(const float* x, int T, int d, int E, const float* R, float* logits, hipStream_t st) {
  if (!router_blocks_fit(T, d, E)) return EMBER_ERR_SHAPE;
  const size_t lds = fused_router_lds(d);
  if (lds > kProjLdsBytes) return EMBER_ERR_SHAPE;
  static const bool lds_ok = hipFuncSetAttribute(reinterpret_cast<const void*>(&router_logits_blocks),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)kProjLdsBytes) == hipSuccess;
  if (!lds_ok) return EMBER_ERR_LAUNCH;
  router_logits_blocks<<<dim3(E, T), 512, lds, st>>>(x, R, logits, T, d, E);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

// Every block (router blocks after their own logit): collects every expert's tagged logit (bounded
// wait), runs route_token (exp tables staged at the start of the launch; every block computes the same
// routing, so no second hop through one block is needed) and fills its dispatch arrays; block 0 also
// writes the routing and dispatch for the later launches. A logit that has not arrived when the wait's
// bound runs out (its router block not resident, e.g. while other work holds the CUs) is computed by
// the waiting block itself with the same code the router block runs, so the picks never depend on the
// other blocks being resident; each block that does so adds one to the flag area's word 0 (a
// diagnostic count for the host, never cleared by the library).
// The give-up path's logit: the same arithmetic as router_block_logit (every product exact in f64,
// eight chains in order, the same combination), written for few registers rather than speed (it only
// runs when a router block is not resident), so that it costs the launch no registers.
template <int NT>
__device__ float router_logit_slow(const ProjArgs& a, int e, uint8_t* lds) {
  const ProjArgs::Route& r = a.route;
  const int t = threadIdx.x, d = r.d, n8 = d - d % 8, nq = n8 / 8;
  double* pd = reinterpret_cast<double*>(lds);
  const float* row = r.router + (size_t)e * d;
  __syncthreads();
  for (int i = t; i < n8; i += NT) pd[(i & 7) * nq + (i >> 3)] = (double)row[i] * (double)r.x[i];
  __syncthreads();
  double acc = 0.0;
  if (t < 8)
    for (int q = 0; q < nq; ++q) acc = acc + pd[t * nq + q];
  double c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) c[j] = __shfl(acc, j, 64);
  float v = 0.0f;
  if (t == 0) {
    double tail = 0.0;
    for (int i = n8; i < d; ++i) tail = __builtin_fma((double)row[i], (double)r.x[i], tail);
    v = (float)((((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]))) + tail);
  }
  __syncthreads();
  return v;
}

// The softmax router's pick set from the fast words, when they prove it. The reference picks the top k
// of the binary32 logits r_e = (float)c_e (c_e its double dot), ties to the lower index, ascending. With
// every c_e in [v_e - h_e, v_e + h_e] (the fast words), the top k of the v_e (same tie rule) are the
// picks when the lowest lower bound among them, m1, and the highest upper bound among the others, m2,
// satisfy m1 - m2 > 2^-22 max(|m1|, |m2|) + 2^-140: then every picked c_e and unpicked c_u round to
// binary32 values r_e > r_u (rounding is monotone and moves each by at most half an ulp, an ulp being
// <= 2^-23 |x| for normal x and 2^-149 below), so no tie can reorder them. Returns false (block-uniform)
// when a word is missing after the wait's bound, carries no bound, or the margin is too small; the
// caller then routes from the exact logits. On true the block's one-token dispatch is built.
template <int NT>
__device__ __attribute__((always_inline)) bool fast_route(const ProjArgs& a, uint8_t* ra, int32_t* s_off, int32_t* s_used, int32_t* s_n,
                           int32_t* s_perm) {
  __shared__ float fv[kMaxRouteE];
  __shared__ uint8_t feb[kMaxRouteE];
  __shared__ int s_ok, s_margin;  // every word present and bounded; the margin proves the set
  const ProjArgs::Route& r = a.route;
  int32_t* pidx = reinterpret_cast<int32_t*>(ra + 2048);
  const int t = threadIdx.x, E = r.E, kk = min(a.k, r.E);
  if (t == 0) s_ok = 1;
  __syncthreads();
  // an eighth of the exact words' bound: the exact path follows a give-up (and waits for the same router
  // block), and the fast words normally land a few microseconds into the launch
  const unsigned spin = r.spin_limit >> 3;
  const uint32_t ftag = fast_tag(r);
  for (int e = t; e < E; e += NT) {
    unsigned long long w;
    unsigned n = 0;
    while (((w = __hip_atomic_load(r.flag + 2 + E + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) >> 32) !=
           ftag) {
      if (++n > spin) break;
      __builtin_amdgcn_s_sleep(1);
    }
    const float v = __builtin_bit_cast(float, (uint32_t)w & 0xffffff00u);
    if ((w >> 32) != ftag || (w & 0xff) == 0xff || v != v) s_ok = 0;
    fv[e] = v;
    feb[e] = (uint8_t)(w & 0xff);
  }
  __syncthreads();
  if (!s_ok) return false;
  if (t < 64) {
    const int n = wave_topk(fv, nullptr, E, kk, pidx);
    double lo = __builtin_inf(), hi = -__builtin_inf();
    for (int e = t; e < E; e += 64) {
      bool picked = false;
      for (int j = 0; j < n; ++j) picked |= pidx[j] == e;
      const double h = __builtin_bit_cast(double, (unsigned long long)((int)feb[e] - 160 + 1023) << 52);  // 2^(b-160)
      if (picked)
        lo = fmin(lo, (double)fv[e] - h);
      else
        hi = fmax(hi, (double)fv[e] + h);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      lo = fmin(lo, __shfl_xor(lo, off, 64));
      hi = fmax(hi, __shfl_xor(hi, off, 64));
    }
    const bool ok = n == kk && (kk == E || lo - hi > 0x1p-22 * fmax(fabs(lo), fabs(hi)) + 0x1p-140);
    // (a word of its own: other waves may still be reading s_ok from the check above)
    if (t == 0) s_margin = ok;
  }
  __syncthreads();
  if (!s_margin) return false;
  fused_dispatch(pidx, kk, E, s_off, s_used, s_n, s_perm);
  __syncthreads();
  return true;
}

// The check of the fast pick sets against the exact picks (used[0 .. n)). A set proven from the fast words
// differs from the exact one only if some unpicked expert's lower bound lies above some picked expert's
// upper bound: the exact logits would then break the bounds. Returns (block-uniform) whether such a
// contradiction (never expected) exists. Words not (yet) published are skipped: the blocks that missed
// them routed from the exact logits. Block 0 counts a contradiction in the flag area's word 1 and stores
// the call's conflict word (2 + 2E), which makes the output rows NaN (the launch that writes them reads it
// or runs this check itself).
template <int NT>
__device__ __attribute__((always_inline)) bool fast_conflict(const ProjArgs& a, const int32_t* used, int n) {
  __shared__ int s_bad;
  const ProjArgs::Route& r = a.route;
  const int t = threadIdx.x;
  const uint32_t ftag = fast_tag(r);
  if (t < 64) {
    double lo_out = -__builtin_inf(), hi_in = __builtin_inf();  // bounds of the unpicked / picked
    for (int e = t; e < r.E; e += 64) {
      const unsigned long long w = __hip_atomic_load(r.flag + 2 + r.E + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((w >> 32) != ftag || (w & 0xff) == 0xff) continue;
      const double v = (double)__builtin_bit_cast(float, (uint32_t)w & 0xffffff00u);
      const double h = __builtin_bit_cast(double, (unsigned long long)((int)(w & 0xff) - 160 + 1023) << 52);
      bool picked = false;
      for (int j = 0; j < n; ++j) picked |= used[j] == e;
      if (picked)
        hi_in = fmin(hi_in, v + h);
      else
        lo_out = fmax(lo_out, v - h);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      hi_in = fmin(hi_in, __shfl_xor(hi_in, off, 64));
      lo_out = fmax(lo_out, __shfl_xor(lo_out, off, 64));
    }
    if (t == 0) {
      s_bad = lo_out > hi_in;
      if (blockIdx.x == 0) {
        if (lo_out > hi_in) __hip_atomic_fetch_add(r.flag + 1, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(r.flag + 2 + 2 * r.E, lo_out > hi_in ? 1ull : 0ull, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  __syncthreads();
  return s_bad != 0;
}

template <int NT, bool ROUTED>
__device__ __attribute__((always_inline)) void route_block(const ProjArgs& a, uint8_t* lds, uint8_t* ra, int32_t* s_off, int32_t* s_used,
                            int32_t* s_n, int32_t* s_perm) {
  __shared__ uint8_t missing[kMaxRouteE];
  __shared__ int any_missing;
  const ProjArgs::Route& r = a.route;
  const int t = threadIdx.x;
  float* lg = reinterpret_cast<float*>(ra);
  int32_t* pidx = reinterpret_cast<int32_t*>(ra + 2048);
  float* pgate = reinterpret_cast<float*>(ra + 2048 + 256);
  uint8_t* wl = ra + 2048 + 512;
  const int E = r.E, k = a.k;
  if (t == 0) any_missing = 0;
  __syncthreads();
  const uint32_t ltag = logit_tag(r);
  for (int e = t; e < E; e += NT) {
    unsigned long long w;
    unsigned n = 0;
    while (((w = __hip_atomic_load(r.flag + 2 + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) >> 32) != ltag) {
      if (++n > r.spin_limit) break;
      __builtin_amdgcn_s_sleep(1);
    }
    const bool got = (w >> 32) == ltag;
    missing[e] = got ? 0 : 1;
    if (!got) any_missing = 1;
    lg[e] = __builtin_bit_cast(float, (uint32_t)w);
  }
  __syncthreads();
  EMBER_STAMP(0, 2);
  if (any_missing) {  // block-uniform
    for (int e = 0; e < E; ++e)
      if (missing[e]) {
        const float v = router_logit_slow<NT>(a, e, lds);
        if (t == 0) lg[e] = v;
      }
    if (t == 0) __hip_atomic_fetch_add(r.flag, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
  }
  // The softmax router's picks are the top k of the logits themselves: with finite logits every block
  // but block 0 takes only them (the launch's dispatch needs nothing else); block 0 (and every block
  // when a logit is NaN, or with the DeepSeek router) runs the whole routing, and block 0 writes it for
  // the later launches.
  bool picks_only = false;
  if (!ROUTED && blockIdx.x != 0) {
    __shared__ int s_nan;
    if (t < 64) {
      bool nan = false;
      for (int e = t; e < E; e += 64) nan |= lg[e] != lg[e];
      nan = __any(nan);
      if (!nan) {
        const int kk = wave_topk(lg, nullptr, E, min(k, E), pidx);
        if (t >= kk && t < k) pidx[t] = -1;
      }
      if (t == 0) s_nan = nan;
    }
    __syncthreads();
    picks_only = !s_nan;
  }
  if (!picks_only) {
    if (t < 64)
      route_token<ROUTED>(lg, E, k, r.renorm, r.routed, r.sigmoid, r.bias, r.groups_n, r.groups_top, wl, pidx, pgate,
                          true);
    __syncthreads();
  }
  int nv = 0;  // valid picks: a prefix (route_token puts the -1 entries last)
  for (int j = 0; j < k; ++j) nv += pidx[j] >= 0;
  if (blockIdx.x == 0) route_publish<NT, ROUTED>(a, ra);
  fused_dispatch(pidx, nv, E, s_off, s_used, s_n, s_perm);
  __syncthreads();
}



// The one-token launches' routing prologue (ROUTE 1: softmax router, 2: the DeepSeek-style options):
// the token's activation row staged at the start of the dynamic LDS (xs), router blocks 0..E-1 publish
// their expert's logit (and, softmax, a fast word), then every block obtains the pick set and builds
// the one-token dispatch in s_off / s_used / s_n / s_perm; block 0 routes exactly and writes the record.
// `prod` and `ra` are the router products' and routing area's LDS (after xs).
// Returns whether this block's pick set came from the fast words (then not yet checked against the exact
// routing, which block 0 always runs).
template <int FMT, int NT, int ROUTE>
__device__ inline bool fused_route_prologue(const ProjArgs& a, uint8_t* xs, uint8_t* prod, uint8_t* ra, int32_t* s_off,
                                            int32_t* s_used, int32_t* s_n, int32_t* s_perm, int* zero_row,
                                            bool routing = true) {
  const int b = blockIdx.x;
  EMBER_STAMP(0, 0);
  if (threadIdx.x == 0) *zero_row = 0;
  if (threadIdx.x < 64) route_stage_tables(ra + 2048 + 512);
  if (b < a.route.E && !a.route.no_publish) {  // router block: its expert's logit, published tagged
    const float v = router_block_logit<NT, ROUTE == 1>(a, b, prod);
    EMBER_STAMP(0, 1);
    if (threadIdx.x == 0) {
      __hip_atomic_store(a.route.flag + 2 + b, ((unsigned long long)logit_tag(a.route) << 32) | __builtin_bit_cast(uint32_t, v),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  {  // then the activation row (router blocks after their logit, which is on the routing's critical path)
    using F = Fmt<FMT>;
    if constexpr (F::QX)
      stage_rows_quant<F::PLANES>(a.route.x, a.route.d, zero_row, 1, xs, act_lds_bytes(true, a.route.d));
    else
      stage_rows_f32<F::NGL>(a.route.x, a.route.d, zero_row, 1, xs, act_lds_bytes(false, a.route.d));
  }
  if (!routing) {  // a shared-segment block: its rows do not depend on the picks
    __syncthreads();
    return false;
  }
  // softmax router: the pick set from the fast words when they prove it (block 0 then writes the
  // exact routing record after its rows); otherwise, and for the DeepSeek-style router, from the
  // exact logits
  bool fast = false;
  if constexpr (ROUTE == 1) {
    if (b != 0) fast = fast_route<NT>(a, ra, s_off, s_used, s_n, s_perm);
  }
  if (!fast) route_block<NT, ROUTE == 2>(a, prod, ra, s_off, s_used, s_n, s_perm);
  if constexpr (ROUTE == 1) {
    if (b == 0) {
      // block 0 routes from the exact logits (and writes the record); the pick set the other blocks
      // may have proven from the fast words must be the same: a difference (never expected) is
      // counted in the flag area's word 1 and stored in the call's conflict word
      (void)fast_conflict<NT>(a, s_used, *s_n);
    }
  }
  EMBER_STAMP(0, 3);
  __syncthreads();
  return fast;
}

// ROUTE: 0 none; 1 the fused one-token routing with a softmax router; 2 with the DeepSeek-style options
template <int FMT, int MT, bool GATED, int NB, int NT, int WPE, int ROUTE>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(WPE))) proj_kernel(ProjArgs a) {
  if (a.clear_flag && blockIdx.x == 0)
    for (int i = threadIdx.x; i < a.clear_n; i += NT)
      __hip_atomic_store(a.clear_flag + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if constexpr (ROUTE != 0) {
    extern __shared__ __align__(16) uint8_t act_lds[];
    __shared__ int32_t s_off[kMaxRouteE + 1], s_used[kFusedMaxK], s_perm[kFusedMaxK], s_n;
    __shared__ int zero_row;
    const int b = blockIdx.x;
    // the token's activation row, staged once at the start (it does not depend on the routing) at the
    // start of the dynamic LDS, where the expert rows' dots read it (routed and shared segments); the
    // router products and the routing area follow it
    uint8_t* xs = act_lds;
    uint8_t* prod = act_lds + fused_x_lds(FMT, a.route.d);
    uint8_t* ra = prod + fused_router_lds(a.route.d);
    // softmax router: block 0 (the exact routing and its record) takes no rows; blocks 1 .. G-1 share them
    constexpr int B0 = ROUTE == 1 ? 1 : 0;
    const int G1 = gridDim.x - B0;
    // with a shared expert the routed / shared split of the blocks is fixed from k (the segments of a token
    // whose picks are all valid, the split seg_view would compute), so the shared segment's blocks skip the
    // routing and stream their rows while it runs (a token with fewer valid picks spreads its routed blocks
    // over fewer segments)
    int gr = -1;
    if (a.s_w0 && a.used) {
      const float w1 = seg_work(a.rows, 1, MT), ws = seg_work(a.s_rows, a.T, MT), wr = (float)a.k * w1;
      gr = uniform(max(a.k, min(G1 - 1, (int)(G1 * (wr / (wr + ws))))));
    }
    const bool shared_blk = gr >= 0 && b >= B0 && b - B0 >= gr;
    fused_route_prologue<FMT, NT, ROUTE>(a, xs, prod, ra, s_off, s_used, &s_n, s_perm, &zero_row, !shared_blk);
    Dispatch dp{shared_blk ? 0 : s_n, s_used, s_off, s_perm};
    SegView v;
    const bool act = b >= B0 && seg_view<GATED, MT, true>(a, dp, b - B0, G1, v, gr);
    EMBER_STAMP(0, 4);
    if (act) proj_body<FMT, MT, GATED, NB, NT, false, true>(a, dp, v);
    EMBER_STAMP(0, 7);
  } else {
    Dispatch dp{a.used ? *a.n_used : 0, a.used, a.offsets, a.perm};
    SegView v;
    const bool active = seg_view<GATED, MT>(a, dp, blockIdx.x, gridDim.x, v);
    EMBER_STAMP(GATED ? 0 : 1, 0);
    if (active) proj_body<FMT, MT, GATED, NB, NT>(a, dp, v);
    EMBER_STAMP(GATED ? 0 : 1, 7);
  }
}

template <int FMT, int MT, bool GATED, int NB, int NT, int WPE, int ROUTE = 0>
int launch_proj_cfg(const ProjArgs& a_in, size_t act_lds, hipStream_t st) {
  const void* fn = reinterpret_cast<const void*>(&proj_kernel<FMT, MT, GATED, NB, NT, WPE, ROUTE>);
  const ProjArgs& a = a_in;
  const size_t lds =
      ROUTE ? fused_x_lds(FMT, a.route.d) + fused_router_lds(a.route.d) + fused_route_lds(a.route.E) : act_lds;
  // blocks per CU at this LDS size (the launch is sized to one resident wave of blocks)
  const int cached_bpc = blocks_per_cu(fn, NT, lds, kProjLdsBytes);
  const int cus = device_cus();
  if (cached_bpc <= 0 || cus <= 0) return EMBER_ERR_LAUNCH;
  static const int bpc_override = [] { const char* e = std::getenv("EMBER_PROJ_BPC"); return e ? atoi(e) : 0; }();
  int bpc = bpc_override > 0 ? std::min(bpc_override, cached_bpc) : cached_bpc;
  // a launch of a few MB of routed weights and no shared expert runs best with one block per CU (measured
  // one-token layers, default / one: C1 gate/up 1.4 MB 20.2 -> 18.5 us, C3 down 7 MB 30.9 -> 29.1 us per
  // layer; C3 gate/up 14 MB even, C4 46-93 MB and the Mixtral-shaped GEMV slower)
  const double wbytes = (double)(a.used ? a.max_segments : 0) * (double)a.expert_stride * (GATED ? 2 : 1);
  if (bpc_override <= 0 && !a.s_w0 && wbytes > 0 && wbytes < 10e6) bpc = 1;
  const int segs = (a.used ? std::max(a.max_segments, 1) : 0) + (a.s_w0 ? 1 : 0);
  const int G = std::max(std::max(cus * bpc, segs), ROUTE ? a.route.E : 0);
  if (ROUTE && a.route.E > cus) return EMBER_ERR_SHAPE;  // the router blocks could not all be resident
  if (a.ev_start) {
    hipExtLaunchKernelGGL(proj_kernel<FMT, MT, GATED, NB, NT, WPE, ROUTE>, dim3(G), dim3(NT), lds, st, a.ev_start,
                          a.ev_stop, 0, a);
  } else {
    proj_kernel<FMT, MT, GATED, NB, NT, WPE, ROUTE><<<G, NT, lds, st>>>(a);
  }
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

template <int FMT, int MT, bool GATED>
int launch_proj_mt(const ProjArgs& a, size_t lds, hipStream_t st) {
  // two register buffers, 512-thread blocks, four waves per SIMD (measured best of the ring depths
  // 2-4 and block sizes 256 / 512 on MI355X for the Mixtral / Qwen / DeepSeek layer shapes); the
  // two-token gate/up pass needs more than the 128 registers four waves leave (it spilled), and runs
  // best at three waves per SIMD in 256-thread blocks (C2 T = 2 / 4: -6 % / -4 %)
  if constexpr (GATED && MT >= 2)
    return launch_proj_cfg<FMT, MT, GATED, 2, 256, 3>(a, lds, st);
  else
    return launch_proj_cfg<FMT, MT, GATED, 2, 512, 4>(a, lds, st);
}

template <int FMT, bool GATED>
int launch_proj_fmt(const ProjArgs& a, hipStream_t st) {
  using F = Fmt<FMT>;
  int row_lds = 0;
  if (a.used) row_lds = act_lds_bytes(F::QX, a.K);
  if (a.s_w0) row_lds = std::max(row_lds, act_lds_bytes(F::QX, a.s_K));
  if (row_lds == 0) return EMBER_OK;
  if (row_lds > kProjLdsBytes) return EMBER_ERR_SHAPE;
  // tokens per pass: up to 2 for gate/up (its 4-token variant runs out of registers), up to 4 for down
  // (F32 gate/up: four tokens per pass fit the registers; the quantizing formats' two-token limit stays)
  int MT = a.T <= 1 ? 1 : (a.T <= 2 || (GATED && FMT != EMBER_TYPE_F32) ? 2 : 4);
  while (MT > 1 && MT * row_lds > kProjLdsBytes) MT >>= 1;
  const size_t lds = (size_t)MT * row_lds;
  if (a.route.flag) {  // routing fused into a one-token gate/up launch
    if (!GATED || a.T != 1 || !fused_route_fits(a.type, a.route.d, a.route.E, a.k))
      return EMBER_ERR_SHAPE;
    if constexpr (GATED) {
      if (a.route.routed) return launch_proj_cfg<FMT, 1, GATED, 2, 512, 4, 2>(a, (size_t)row_lds, st);
      return launch_proj_cfg<FMT, 1, GATED, 2, 512, 4, 1>(a, (size_t)row_lds, st);
    }
  }
  if (MT == 1) return launch_proj_mt<FMT, 1, GATED>(a, lds, st);
  if (MT == 2) return launch_proj_mt<FMT, 2, GATED>(a, lds, st);
  return launch_proj_mt<FMT, 4, GATED>(a, lds, st);
}

template <bool GATED>
int launch_proj_gated(const ProjArgs& a, hipStream_t st) {
  switch (a.type) {
    case EMBER_TYPE_F32: return launch_proj_fmt<EMBER_TYPE_F32, GATED>(a, st);
    case EMBER_TYPE_F16: return launch_proj_fmt<EMBER_TYPE_F16, GATED>(a, st);
    case EMBER_TYPE_BF16: return launch_proj_fmt<EMBER_TYPE_BF16, GATED>(a, st);
    case EMBER_TYPE_Q8_0: return launch_proj_fmt<EMBER_TYPE_Q8_0, GATED>(a, st);
    case EMBER_TYPE_Q4_K: return launch_proj_fmt<EMBER_TYPE_Q4_K, GATED>(a, st);
    default: return EMBER_ERR_TYPE;
  }
}

int launch_projection(const ProjArgs& a, hipStream_t st) {
  return a.gated ? launch_proj_gated<true>(a, st) : launch_proj_gated<false>(a, st);
}

// ---- one-token layer over d_ff slices (SliceArgs)
// Pack rows (64 columns of one weight row, the prefill pack's layout) against one staged activation row:
// chunk c of the row staged in LDS (act_lds_bytes layout; every lane of a wave reads the same chunk, an
// LDS broadcast). A lane owns one pack row, so a wave's load of 64 consecutive rows is one contiguous
// run of the tile, and each lane's dot is its row's whole 64-column share (no cross-lane reduction).
template <int FMT>
struct PackRow;
template <>
struct PackRow<EMBER_TYPE_Q8_0> {  // the two Q8_0 blocks as they are: Fmt<Q8_0>'s chunk
  static constexpr int NW = 17, RB = kPackRowB;
  __device__ static void load(const uint8_t* p, uint32_t* raw) { Fmt<EMBER_TYPE_Q8_0>::load(p, 0, 0, raw); }
  __device__ static void dot(const uint32_t* raw, const uint8_t* x, int c, int K, float& acc) {
    Fmt<EMBER_TYPE_Q8_0>::dot_tokens<1>(raw, x, 0, c, K, 1, &acc);
  }
};
template <>
struct PackRow<EMBER_TYPE_Q4_K> {  // {a0, m0, a1, m1} fp16, then 32 nibble bytes; weight = a q + m
  static constexpr int NW = 10, RB = kPackRowQ4B;
  __device__ static void load(const uint8_t* p, uint32_t* raw) {
    const u32x4 q0 = *reinterpret_cast<const u32x4_a4*>(p);
    const u32x4 q1 = *reinterpret_cast<const u32x4_a4*>(p + 16);
    const uint2 q2 = *reinterpret_cast<const uint2*>(p + 32);
    raw[0] = q0.x, raw[1] = q0.y, raw[2] = q0.z, raw[3] = q0.w;
    raw[4] = q1.x, raw[5] = q1.y, raw[6] = q1.z, raw[7] = q1.w;
    raw[8] = q2.x, raw[9] = q2.y;
  }
  // the activations as byte planes (Fmt<Q4_K>::PLANES): dot = 256 dot4(nibbles, high) + dot4(nibbles, low)
  __device__ static void dot(const uint32_t* raw, const uint8_t* x, int c, int K, float& acc) {
    int ha = 0, hb = 0;
    uint32_t la = 0u, lb = 0u;
#pragma unroll
    for (int k2 = 0; k2 < 8; k2 += 2) {
      const uint32_t w0 = raw[2 + k2], w1 = raw[3 + k2];
      const uint32_t a0 = w0 & 0x0f0f0f0fu, a1 = w1 & 0x0f0f0f0fu;                // group 0, 8 elements
      const uint32_t b0 = (w0 >> 4) & 0x0f0f0f0fu, b1 = (w1 >> 4) & 0x0f0f0f0fu;  // group 1
      const u32x4 xa = *reinterpret_cast<const u32x4*>(lds_granule<3>(x, c, k2 >> 1));
      const u32x4 xb = *reinterpret_cast<const u32x4*>(lds_granule<3>(x, c, 4 + (k2 >> 1)));
      la = __builtin_amdgcn_udot4(a0, xa.x, la, false);
      la = __builtin_amdgcn_udot4(a1, xa.y, la, false);
      ha = __builtin_amdgcn_sdot4((int)a0, (int)xa.z, ha, false);
      ha = __builtin_amdgcn_sdot4((int)a1, (int)xa.w, ha, false);
      lb = __builtin_amdgcn_udot4(b0, xb.x, lb, false);
      lb = __builtin_amdgcn_udot4(b1, xb.y, lb, false);
      hb = __builtin_amdgcn_sdot4((int)b0, (int)xb.z, hb, false);
      hb = __builtin_amdgcn_sdot4((int)b1, (int)xb.w, hb, false);
    }
    const int ia = 256 * ha + (int)la, ib = 256 * hb + (int)lb;
    const float a0 = half_bits_to_float(raw[0] & 0xffff), m0 = half_bits_to_float(raw[0] >> 16);
    const float a1 = half_bits_to_float(raw[1] & 0xffff), m1 = half_bits_to_float(raw[1] >> 16);
    const float* sc = reinterpret_cast<const float*>(x + K * 2) + 2 * c;
    const int* sm = reinterpret_cast<const int*>(x + K * 2 + (K / 32) * 4) + 2 * c;
    acc += sc[0] * (a0 * (float)ia + m0 * (float)sm[0]) + sc[1] * (a1 * (float)ib + m1 * (float)sm[1]);
  }
};

// Block 1 + item (softmax router; item = b for the DeepSeek-style router, whose block 0 also takes one),
// item = j * ns + c: pick j (s_used[j], ascending), slice c. Each wave walks one sequence of pack-row
// loads through a ring of NB register buffers: first its share of the gate/up K tiles (k-tile wave +
// i * waves, gate then up, lane = slice row), then its share of the down rows (row group wave + i * waves
// of 64 rows, lane = row, the slice's 64 columns). Between the two, at a block-uniform position of the
// sequence (every wave has the same number of loads; surplus loads are clamped and their dots masked),
// the waves' gate/up sums are added in wave order, SwiGLU'd and quantized as the GEMV quantizes h.
template <int FMT, int NB, int NT, int ROUTE>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) slice_kernel(SliceArgs a) {
  using P = PackRow<FMT>;
  using F = Fmt<FMT>;
  constexpr int NWV = NT / 64;
  extern __shared__ __align__(16) uint8_t act_lds[];
  __shared__ int32_t s_off[kMaxRouteE + 1], s_used[kFusedMaxK], s_perm[kFusedMaxK], s_n;
  __shared__ int zero_row;
  __shared__ float red[2][NWV][64];
  __shared__ __align__(16) float hval[64];
  __shared__ __align__(16) uint8_t hrow[2 * 64 + 2 * 8];  // act_lds_bytes(true, 64)
  const ProjArgs& pa = a.p;
  uint8_t* xs = act_lds;
  uint8_t* prod = act_lds + fused_x_lds(FMT, a.d);
  uint8_t* ra = prod + fused_router_lds(a.d);
  fused_route_prologue<FMT, NT, ROUTE>(pa, xs, prod, ra, s_off, s_used, &s_n, s_perm, &zero_row);
  constexpr int B0 = ROUTE == 1 ? 1 : 0;
  const int ns = a.d_ff / 64;
  const int item = (int)blockIdx.x - B0;
  if (item < 0) return;  // block-uniform
  const int j = item / ns, c = item - j * ns;
  if (j >= s_n) return;  // an invalid pick (k > E): block-uniform
  const int e = s_used[j];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int d = a.d, nkt = d / 64, nrg = d / 64;
  const int64_t RB = P::RB, tile = 256 * RB;
  // gate/up: tile (e, c / 2, kt), rows 64 (c % 2) + lane (gate) and 128 + the same (up)
  const uint8_t* gbase = a.pack_gu + (int64_t)(e * ((a.d_ff + 127) / 128) + (c >> 1)) * nkt * tile +
                         (64 * (c & 1) + lane) * RB;
  // down: tile (e, rg / 4, c), row 64 (rg % 4) + lane
  const int ntd = (d + 255) / 256;
  const uint8_t* dbase = a.pack_dn + ((int64_t)e * ntd * ns + c) * tile + lane * RB;
  const int ngu = (nkt + NWV - 1) / NWV, ndn = (nrg + NWV - 1) / NWV;
  const int Q1 = 2 * ngu, Q = Q1 + ndn;
  auto addr = [&](int q) __attribute__((always_inline)) -> const uint8_t* {
    if (q < Q1) {
      const int kt = min(wave + (q >> 1) * NWV, nkt - 1);
      return gbase + (int64_t)kt * tile + (q & 1) * 128 * RB;
    }
    const int rg = min(wave + (q - Q1) * NWV, nrg - 1);
    return dbase + (int64_t)(rg >> 2) * ns * tile + (rg & 3) * 64 * RB;
  };
  float ag = 0.0f, au = 0.0f;
  float* part = a.part + (int64_t)item * d;
  uint32_t buf[NB][P::NW];
  auto use = [&](int q, const uint32_t (&b)[P::NW]) __attribute__((always_inline)) {
    if (q < Q1) {
      const int kt = wave + (q >> 1) * NWV;
      if (kt < nkt) {
        float t = 0.0f;
        P::dot(b, xs, kt, d, t);
        if (q & 1)
          au += t;
        else
          ag += t;
      }
      return;
    }
    if (q == Q1) {  // block-uniform: every wave reaches load Q1 at the same ring position
      red[0][wave][lane] = ag;
      red[1][wave][lane] = au;
      __syncthreads();
      if (wave == 0) {
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; ++w) {
          g = g + red[0][w][lane];
          u = u + red[1][w][lane];
        }
        hval[lane] = swiglu(g, u);
      }
      __syncthreads();
      if (threadIdx.x < 2) {  // the GEMV's activation quantization, one 32-element block per thread
        uint32_t packed[16];
        float sc;
        int sm;
        quant_block32(hval + 32 * threadIdx.x, packed, &sc, &sm);
        store_block_quant<F::PLANES>(packed, sc, sm, threadIdx.x, 64, hrow);
      }
      __syncthreads();
      EMBER_STAMP(0, 5);
    }
    if (q >= Q) return;
    const int rg = wave + (q - Q1) * NWV;
    if (rg < nrg) {
      float t = 0.0f;
      P::dot(b, hrow, 0, 64, t);
      part[rg * 64 + lane] = t;
    }
  };
  ring_for<NB - 1>([&](auto J) { P::load(addr(decltype(J)::value), buf[decltype(J)::value]); });
  EMBER_STAMP(0, 4);
#pragma unroll 1
  for (int q0 = 0; q0 < Q; q0 += NB) {
    ring_for<NB>([&](auto J) {
      constexpr int jj = decltype(J)::value;
      const int q = q0 + jj;
      P::load(addr(min(q + NB - 1, Q - 1)), buf[(jj + NB - 1) % NB]);
      use(q, buf[jj]);
    });
  }
  EMBER_STAMP(0, 7);
}

// 32 outputs per block, the slices summed in 8 groups (group g: slices g, g + 8, ...) added in group order.
// A thread issues its group's loads (up to 32 slices at a time) before adding them in slice order.
__global__ void __launch_bounds__(256) slice_reduce_kernel(const float* __restrict__ part, int ns, int d, int k,
                                                           const int32_t* __restrict__ idx,
                                                           const float* __restrict__ gates, float scale,
                                                           const unsigned long long* conflict,
                                                           unsigned long long* clear_flag, int clear_n,
                                                           float* __restrict__ out) {
  __shared__ float red[8][32];
  const int t = threadIdx.x, o = blockIdx.x * 32 + (t & 31), g = t >> 5;
  if (clear_flag && blockIdx.x == 0)
    for (int i = t; i < clear_n; i += 256)
      __hip_atomic_store(clear_flag + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float acc = 0.0f;
  for (int j = 0; j < k; ++j) {
    if (idx[j] < 0) break;  // the valid picks are a prefix (block-uniform)
    const float* p = part + (int64_t)j * ns * d + o;
    float s = 0.0f;
    for (int c0 = g; c0 < ns; c0 += 8 * 32) {
      float v[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int c = c0 + 8 * i;
        v[i] = c < ns ? p[(int64_t)c * d] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 32; ++i)
        if (c0 + 8 * i < ns) s += v[i];
    }
    red[g][t & 31] = s;
    __syncthreads();
    if (g == 0) {
      float y = red[0][t];
#pragma unroll
      for (int i = 1; i < 8; ++i) y = y + red[i][t];
      acc = acc + gates[j] * y;  // combine_kernel's order: acc = acc + gate * y, picks ascending
    }
    __syncthreads();
  }
  if (g == 0) {
    if (scale != 1.0f) acc = acc * scale + 0.0f;
    out[o] = conflict && *conflict ? __builtin_nanf("") : acc;
  }
}

template <int FMT, int ROUTE>
int launch_slices_cfg(const SliceArgs& a, hipStream_t st) {
  // three register buffers per wave, 512-thread blocks (two per CU): measured on MI355X against two buffers
  // (even), four (spills; C2 97 vs 84 us) and 1024-thread blocks (90 vs 84 us)
  constexpr int NB = 3, NT = 512;
  const void* fn = reinterpret_cast<const void*>(&slice_kernel<FMT, NB, NT, ROUTE>);
  const size_t lds = fused_x_lds(FMT, a.d) + fused_router_lds(a.d) + fused_route_lds(a.p.route.E);
  if (blocks_per_cu(fn, NT, lds, kProjLdsBytes) <= 0) return EMBER_ERR_LAUNCH;
  // every router block (0 .. E-1) must exist, whatever the number of slices
  const int G = std::max((ROUTE == 1 ? 1 : 0) + a.p.k * (a.d_ff / 64), a.p.route.E);
  if (a.p.ev_start)
    hipExtLaunchKernelGGL(slice_kernel<FMT, NB, NT, ROUTE>, dim3(G), dim3(NT), lds, st, a.p.ev_start, a.p.ev_stop, 0,
                          a);
  else
    slice_kernel<FMT, NB, NT, ROUTE><<<G, NT, lds, st>>>(a);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

// The slices pay off once they give every CU at least one block (Mixtral-shaped C2 / C5: 448 slices, 85 vs
// 89 us and 55 vs 64 us against the GEMV path); with fewer (Qwen-shaped top-8 of 768-wide experts: 96
// slices) the GEMV path is faster (30.1 vs 31.7 us).
// (any_size: whenever the kernel can run, whatever the fill)
bool slices_fit(int type, int d, int d_ff, int E, int k, bool any_size) {
  return (type == EMBER_TYPE_Q8_0 || type == EMBER_TYPE_Q4_K) && d % 64 == 0 && d_ff % 64 == 0 &&
         fused_route_fits(type, d, E, k) && (any_size || (int64_t)k * (d_ff / 64) >= device_cus()) &&
         (int64_t)k * (d_ff / 64) < (1 << 30);
}

int launch_slices(const SliceArgs& a, hipStream_t st) {
  if (!a.p.route.flag || !a.pack_gu || !a.pack_dn || !a.part ||
      !slices_fit(a.p.type, a.d, a.d_ff, a.p.route.E, a.p.k, true))
    return EMBER_ERR_SHAPE;
  const bool routed = a.p.route.routed != 0;
  switch (a.p.type) {
    case EMBER_TYPE_Q8_0:
      return routed ? launch_slices_cfg<EMBER_TYPE_Q8_0, 2>(a, st) : launch_slices_cfg<EMBER_TYPE_Q8_0, 1>(a, st);
    case EMBER_TYPE_Q4_K:
      return routed ? launch_slices_cfg<EMBER_TYPE_Q4_K, 2>(a, st) : launch_slices_cfg<EMBER_TYPE_Q4_K, 1>(a, st);
    default: return EMBER_ERR_TYPE;
  }
}

int launch_slice_reduce(const float* part, int ns, int d, int k, const int32_t* idx, const float* gates, float scale,
                        const unsigned long long* conflict, unsigned long long* clear_flag, int clear_n, float* out,
                        hipStream_t st) {
  if (d % 32) return EMBER_ERR_SHAPE;
  slice_reduce_kernel<<<d / 32, 256, 0, st>>>(part, ns, d, k, idx, gates, scale, conflict, clear_flag, clear_n, out);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

// 1 / (1 + expf(-s)) in binary32 with glibc's expf (graph_ir_ops.cpp:22 evaluates it on the host)
__device__ inline float shared_gate_sigmoid(float s) { return 1.0f / (1.0f + expf_glibc(-s)); }

// ---- one-token down projection with the combine fused in
// At T = 1 the token's picks all produce the same output rows: out[o] = sum over picks j ascending of
// gate_j * (W_down[e_j][o] . h_j), then * scale, then + the shared expert's row (times its gate). Block
// b owns a set of output rows ("slots") for every pick, so each row's sum is formed where its dots are,
// and neither a y buffer nor a combine launch is needed. Each dot is computed exactly as proj_body
// computes it (same lane partition of the row, same chunk order, same shuffle reduction, same
// activation quantization) and the sum in combine_kernel's order, so the output bits equal those of
// the down launch followed by the combine launch.
//
// Row ownership: with RPS rows per wave step (the routed row length's lane partition), block b of G owns
// the row groups b, b + G, ... (adjacent blocks read adjacent rows at any time), slot i*RPS + sub of its
// row list holding row sub of its i-th group. Its waves share the (group, pick) pairs, so the picks of a
// row are read side by side, into one LDS row of dots per pick that is then summed in pick order. The
// shared expert's rows (another row length, so another lane partition) are the same rows, walked through
// the slot list.

// Walks the shared expert's down matrix (rows of K elements, rb bytes apart) over the block's slots: the
// dot of slot s's row (rowlist[s]; holes load row 0 and store nothing) with the shared expert's activation
// row `act` is added to obuf[s] (obuf = obuf + dot * (*sgc), or + dot). Its row length sets its own lane
// partition (L lanes per row, RPS rows per wave step), the slot groups of RPS taken by the waves in turn.
template <int FMT, int NB, int NT>
__device__ __attribute__((always_inline)) inline void down1_walk_shared(const uint8_t* w0, int64_t rb, int K,
                                                                        const uint8_t* act, int row_lds,
                                                                        const int* rowlist, int nslots, float* obuf,
                                                                        const float* sgc) {
  using F = Fmt<FMT>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = NT / 64;
  const int C = (K + F::CE - 1) / F::CE;
  int Lg = 0;
  while ((1 << Lg) < C && Lg < 6) ++Lg;
  const int L = 1 << Lg, RPS = 64 >> Lg;
  const int sub = lane >> Lg, rl = lane & (L - 1);
  const int NC = (C + L - 1) / L;
  const int ngt = (nslots + RPS - 1) / RPS;
  const int ngroups = wave < ngt ? (ngt - wave + nwaves - 1) / nwaves : 0;
  const int nloads = ngroups * NC;  // load q: slot group q / NC of this wave, chunk step q % NC
  auto slot_of = [&](int st) { return ((st / NC) * nwaves + wave) * RPS + sub; };
  auto load_q = [&](int q, uint32_t (&buf)[F::NW]) {
    const int st = min(q, nloads - 1);
    const int c = min(rl + (st % NC) * L, C - 1);
    F::load(w0 + (int64_t)max(rowlist[min(slot_of(st), nslots - 1)], 0) * rb, c, K, buf);
  };
  if (nloads == 0) return;
  uint32_t buf[NB][F::NW];
  ring_for<NB - 1>([&](auto J) { load_q(decltype(J)::value, buf[decltype(J)::value]); });
  float acc = 0.0f;
#pragma unroll 1
  for (int q0 = 0; q0 < nloads; q0 += NB) {
    ring_for<NB>([&](auto J) {
      constexpr int jj = decltype(J)::value;
      const int q = q0 + jj;
      load_q(q + NB - 1, buf[(jj + NB - 1) % NB]);
      const int sl = slot_of(q);
      const int c = rl + (q % NC) * L;
      const bool ok = q < nloads && c < C && sl < nslots;
      float tk[1] = {0.0f};
      F::template dot_tokens<1>(buf[jj % NB], act, row_lds, min(c, C - 1), K, 1, tk);
      acc += ok ? tk[0] : 0.0f;
      if (q < nloads && q % NC == NC - 1) {  // the row is complete
        float v = acc;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1)
          if (off < L) v += __shfl_xor(v, off, 64);
        if (rl == 0 && sl < nslots && rowlist[sl] >= 0) {
          float& o = obuf[sl];
          o = o + (sgc ? v * *sgc : v);  // the shared expert's row (qwen2moe: times its gate)
        }
        acc = 0.0f;
      }
    });
  }
}

// The routed picks' dots of the block's row groups (block b owns groups b, b + G, b + 2G, ... of RPS rows):
// the (group, pick) units are spread over the block's waves, pick fastest, so the picks of one row run
// side by side instead of one after another; unit (i, j)'s dot of row sub of group i goes to
// pbuf[j][i * RPS + sub]. Each dot is formed as proj_body forms it (same lane partition, chunk order and
// shuffle reduction); the caller adds them in pick order. before_loop() runs on every thread of the block
// after the first weight loads are issued and before the first dot: the activation staging goes there, so
// that the weights travel while it runs.
template <int FMT, int NB, int NT, class Before>
__device__ __attribute__((always_inline)) inline void down1_walk_picks(const uint8_t* w0, const int* exps,
                                                                       int64_t estride, int npicks, int64_t rb, int K,
                                                                       const uint8_t* act, int row_lds, int rows_total,
                                                                       int nslots, float (*pbuf)[kDown1Slots],
                                                                       Before&& before_loop) {
  using F = Fmt<FMT>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = NT / 64;
  const int C = (K + F::CE - 1) / F::CE;
  int Lg = 0;
  while ((1 << Lg) < C && Lg < 6) ++Lg;
  const int L = 1 << Lg, RPS = 64 >> Lg;
  const int sub = lane >> Lg, rl = lane & (L - 1);
  const int NC = (C + L - 1) / L;
  const int gt = (rows_total + RPS - 1) / RPS, G = gridDim.x, b = blockIdx.x;
  const int ngb = b < gt ? (gt - b + G - 1) / G : 0;
  const int nunits = npicks > 0 ? ngb * npicks : 0;
  const int nu_w = wave < nunits ? (nunits - wave + nwaves - 1) / nwaves : 0;
  const int nloads = nu_w * NC;  // load q: this wave's unit q / NC, chunk step q % NC
  auto unit_of = [&](int q) { return min(wave + (q / NC) * nwaves, nunits - 1); };
  auto load_q = [&](int q, uint32_t (&buf)[F::NW]) {
    const int u = unit_of(q), i = u / npicks, j = u - i * npicks;
    const int e = __builtin_amdgcn_readfirstlane(exps[j]);  // LDS, a wave-uniform index
    const int row = min((b + i * G) * RPS + sub, rows_total - 1);
    const int c = min(rl + (q % NC) * L, C - 1);
    F::load(w0 + (int64_t)e * estride + (int64_t)row * rb, c, K, buf);
  };
  uint32_t buf[NB][F::NW];
  if (nloads > 0) ring_for<NB - 1>([&](auto J) { load_q(decltype(J)::value, buf[decltype(J)::value]); });
  before_loop();
  if (nloads == 0) return;
  float acc = 0.0f;
#pragma unroll 1
  for (int q0 = 0; q0 < nloads; q0 += NB) {
    ring_for<NB>([&](auto J) {
      constexpr int jj = decltype(J)::value;
      const int q = q0 + jj;
      load_q(q + NB - 1, buf[(jj + NB - 1) % NB]);
      const int u = unit_of(q), i = u / npicks, j = u - i * npicks;
      const int c = rl + (q % NC) * L;
      const bool ok = q < nloads && c < C;
      float tk[1] = {0.0f};
      F::template dot_tokens<1>(buf[jj % NB], act + (size_t)j * row_lds, row_lds, min(c, C - 1), K, 1, tk);
      acc += ok ? tk[0] : 0.0f;
      if (q < nloads && q % NC == NC - 1) {  // the row is complete for pick j
        float v = acc;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1)
          if (off < L) v += __shfl_xor(v, off, 64);
        const int sl = i * RPS + sub;
        if (rl == 0 && sl < nslots) pbuf[j][sl] = v;
        acc = 0.0f;
      }
    });
  }
}

template <int FMT, int NB, int NT, int WPE>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(WPE))) down1_kernel(Down1Args a) {
  using F = Fmt<FMT>;
  extern __shared__ __align__(16) uint8_t act_lds[];
  __shared__ float obuf[kDown1Slots];
  __shared__ float pbuf[kDown1MaxPicks][kDown1Slots];  // the routed picks' dots per slot
  __shared__ int rowlist[kDown1Slots];
  __shared__ float gate_s[kDown1MaxPicks], sgc_s;
  __shared__ int pos_s[kDown1MaxPicks], exp_s[kDown1MaxPicks], np_s, zero_row;
  if (a.clear_flag && blockIdx.x == 0)
    for (int i = threadIdx.x; i < a.clear_n; i += NT)
      __hip_atomic_store(a.clear_flag + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int t = threadIdx.x;
  EMBER_STAMP(1, 0);
  // the picks' h rows, quantizing formats with one 32-element block per thread: one token's valid picks
  // sit at dispatch positions 0 .. np-1, so rows 0 .. k-1 are loaded into registers at once, before the
  // picks are read and before the first down rows are requested (loads complete in order, so they do not
  // wait for the weight loads); quantized into LDS once those are in flight
  const int nbh = a.K / 32;
  const bool h_early = F::QX && a.K % 32 == 0 && a.k * nbh <= NT;
  float hv[32];
  if (h_early && t < a.k * nbh) {
    const int m = t / nbh, b = t - m * nbh;
    load_block32(a.h + (size_t)m * a.K + (size_t)b * 32, hv);
  }
  if (t < 64) {  // the valid picks in ascending order (the combine's order): one round of loads, compacted
    int p = -1, e = 0;
    float g = 0.0f;
    if (t < a.k) {
      p = a.pos[t];
      e = a.idx[t];
      g = a.gates[t];
    }
    const unsigned long long m = __ballot(p >= 0);
    if (p >= 0) {
      const int j = __popcll(m & ((1ull << t) - 1));
      pos_s[j] = p;
      exp_s[j] = e;
      gate_s[j] = g;
    }
    if (t == 0) {
      np_s = __popcll(m);
      sgc_s = a.sg_logit ? shared_gate_sigmoid(*a.sg_logit) : 1.0f;
      zero_row = 0;
    }
  }
  // the block's rows: its row groups b, b + G, ... of RPS rows (the routed row length's lane partition),
  // slot i * RPS + sub holding row sub of its i-th group
  {
    const int C = (a.K + F::CE - 1) / F::CE;
    int Lg = 0;
    while ((1 << Lg) < C && Lg < 6) ++Lg;
    const int RPS = 64 >> Lg;
    for (int sl = t; sl < a.nslots; sl += NT) {
      const int i = sl / RPS, sub = sl - i * RPS;
      const int r = (blockIdx.x + i * (int)gridDim.x) * RPS + sub;
      rowlist[sl] = r < a.d ? r : -1;
      obuf[sl] = 0.0f;
    }
  }
  __syncthreads();
  const int np = np_s;
  const int row_lds = act_lds_bytes(F::QX, a.K);
  const int srow_lds = a.s_w ? act_lds_bytes(F::QX, a.s_K) : 0;
  // the first down rows are requested before every pick's h row (then the shared expert's) is staged
  auto stage = [&] {
    if (np > 0) {
      if constexpr (F::QX) {
        if (h_early) {
          if (t < np * nbh) {
            const int m = t / nbh, b = t - m * nbh;
            uint32_t packed[16];
            float sc;
            int sm;
            quant_block32_v(hv, packed, &sc, &sm);
            store_block_quant<F::PLANES>(packed, sc, sm, b, a.K, act_lds + m * row_lds);
          }
        } else {
          stage_rows_quant<F::PLANES>(a.h, a.K, pos_s, np, act_lds, row_lds);
        }
      } else {
        stage_rows_f32<F::NGL>(a.h, a.K, pos_s, np, act_lds, row_lds);
      }
    }
    if (a.s_w) {
      if constexpr (F::QX)
        stage_rows_quant<F::PLANES>(a.s_h, a.s_K, &zero_row, 1, act_lds + (size_t)np * row_lds, srow_lds);
      else
        stage_rows_f32<F::NGL>(a.s_h, a.s_K, &zero_row, 1, act_lds + (size_t)np * row_lds, srow_lds);
    }
    __syncthreads();
    EMBER_STAMP(1, 5);
  };
  down1_walk_picks<FMT, NB, NT>(static_cast<const uint8_t*>(a.w), exp_s, a.expert_stride, np, F::row_bytes(a.K), a.K,
                                act_lds, row_lds, a.d, a.nslots, pbuf, stage);
  __syncthreads();
  // combine_kernel's sum on this block's rows: acc = acc + gate * y, picks ascending
  for (int sl = t; sl < a.nslots; sl += NT)
    if (rowlist[sl] >= 0) {
      float o = 0.0f;
      for (int j = 0; j < np; ++j) o = o + gate_s[j] * pbuf[j][sl];
      obuf[sl] = o;
    }
  __syncthreads();
  // the rest of combine_kernel's sequence on this block's rows: (acc * scale) + 0, then the shared row
  if (a.scale != 1.0f)
    for (int sl = t; sl < a.nslots; sl += NT) obuf[sl] = obuf[sl] * a.scale + 0.0f;
  if (a.s_w) {
    __syncthreads();
    down1_walk_shared<FMT, NB, NT>(static_cast<const uint8_t*>(a.s_w), F::row_bytes(a.s_K), a.s_K,
                                   act_lds + (size_t)np * row_lds, srow_lds, rowlist, a.nslots, obuf,
                                   a.sg_logit ? &sgc_s : nullptr);
  }
  __syncthreads();
  // a pick-set conflict of the fused routing (never expected): NaN rows instead of plausible numbers
  const bool bad = a.conflict && __hip_atomic_load(a.conflict, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
  for (int sl = t; sl < a.nslots; sl += NT)
    if (rowlist[sl] >= 0) a.out[rowlist[sl]] = bad ? __builtin_nanf("") : obuf[sl];
  EMBER_STAMP(1, 7);
}

template <int FMT, int NT>
int launch_down1_cfg(const Down1Args& a_in, hipStream_t st) {
  using F = Fmt<FMT>;
  constexpr int NB = 2, WPE = 4;
  const void* fn = reinterpret_cast<const void*>(&down1_kernel<FMT, NB, NT, WPE>);
  const int row_lds = act_lds_bytes(F::QX, a_in.K);
  const size_t lds = (size_t)a_in.k * row_lds + (a_in.s_w ? act_lds_bytes(F::QX, a_in.s_K) : 0);
  if (a_in.k > kDown1MaxPicks || lds > (size_t)kProjLdsBytes) return EMBER_ERR_SHAPE;
  const int bpc = blocks_per_cu(fn, NT, lds, kProjLdsBytes), cus = device_cus();
  if (bpc <= 0 || cus <= 0) return EMBER_ERR_LAUNCH;
  const int G = cus * bpc;
  const int C = (a_in.K + F::CE - 1) / F::CE;
  int Lg = 0;
  while ((1 << Lg) < C && Lg < 6) ++Lg;
  const int RPS = 64 >> Lg;
  const int gt = (a_in.d + RPS - 1) / RPS;
  Down1Args a = a_in;
  a.nslots = (gt + G - 1) / G * RPS;  // the block's row groups, in slots
  if (a.nslots > kDown1Slots) return EMBER_ERR_SHAPE;
  if (a.ev_start)
    hipExtLaunchKernelGGL(down1_kernel<FMT, NB, NT, WPE>, dim3(G), dim3(NT), lds, st, a.ev_start, a.ev_stop, 0, a);
  else
    down1_kernel<FMT, NB, NT, WPE><<<G, NT, lds, st>>>(a);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

template <int FMT>
int launch_down1_fmt(const Down1Args& a, hipStream_t st) {
  // 1024-thread blocks, or 512 for a few MB of down weights (measured, 1024 / 512: C1-shaped 1.4 MB 17.9 /
  // 16.8 us per layer; Mixtral-shaped Q8_0 125 MB 86.8 / 89.7, Q4_K 68.1 / 71.7); EMBER_DOWN1_NT overrides
  static const int nt_env = [] { const char* v = std::getenv("EMBER_DOWN1_NT"); return v ? atoi(v) : 0; }();
  const double bytes = (double)a.k * (double)a.expert_stride;
  const int nt = nt_env ? nt_env : (bytes < 10e6 ? 512 : 1024);
  return nt == 1024 ? launch_down1_cfg<FMT, 1024>(a, st) : launch_down1_cfg<FMT, 512>(a, st);
}

bool down1_fits(int type, int d, int K, int k, int s_K) {
  if (k > kDown1MaxPicks) return false;
  const bool qx = type_quantizes_activations(type);
  const size_t lds = (size_t)k * act_lds_bytes(qx, K) + (s_K > 0 ? act_lds_bytes(qx, s_K) : 0);
  if (lds > (size_t)kProjLdsBytes) return false;
  const int CE = type == EMBER_TYPE_F32 ? 16 : type == EMBER_TYPE_F16 || type == EMBER_TYPE_BF16 ? 32 : 64;
  const int C = (K + CE - 1) / CE;
  int Lg = 0;
  while ((1 << Lg) < C && Lg < 6) ++Lg;
  const int RPS = 64 >> Lg;
  // at least one block per CU: the slot bound for the smallest grid
  const int cus = device_cus();
  if (cus <= 0) return false;
  const int gt = (d + RPS - 1) / RPS;
  return (gt + cus - 1) / cus * RPS <= kDown1Slots;
}

int launch_down1(const Down1Args& a, hipStream_t st) {
  switch (a.type) {
    case EMBER_TYPE_F32: return launch_down1_fmt<EMBER_TYPE_F32>(a, st);
    case EMBER_TYPE_F16: return launch_down1_fmt<EMBER_TYPE_F16>(a, st);
    case EMBER_TYPE_BF16: return launch_down1_fmt<EMBER_TYPE_BF16>(a, st);
    case EMBER_TYPE_Q8_0: return launch_down1_fmt<EMBER_TYPE_Q8_0>(a, st);
    case EMBER_TYPE_Q4_K: return launch_down1_fmt<EMBER_TYPE_Q4_K>(a, st);
    default: return EMBER_ERR_TYPE;
  }
}

int proj_max_row_bytes() { return kProjLdsBytes; }

#ifdef EMBER_PROBE
}  // namespace ember_moe
extern "C" int ember_moe_probe_set(void* buf) {
  unsigned long long* p = static_cast<unsigned long long*>(buf);
  return hipMemcpyToSymbol(HIP_SYMBOL(ember_moe::g_probe), &p, sizeof(p)) == hipSuccess ? 0 : -1;
}
namespace ember_moe {
#endif

// The fused routing's limits: E <= kMaxRouteE (its per-expert LDS arrays), k <= 8 and the LDS of the
// staged row, the router products and the routing area. (A block that waits for a router
// block's word longer than its bound computes that logit itself, so no block depends on another being
// resident.)
bool fused_route_fits(int type, int d, int E, int k) {
  return E <= kMaxRouteE && k <= kFusedMaxK && d >= 8 && d <= 16 * 512 &&
         fused_x_lds(type, d) + fused_router_lds(d) + fused_route_lds(E) <= (size_t)kProjLdsBytes;
}

bool type_quantizes_activations(int type) { return type == EMBER_TYPE_Q8_0 || type == EMBER_TYPE_Q4_K; }

// out[t][o] = sum over j ascending (= experts ascending) of gate[t][j] * y[pos[t*k+j]][o], starting
// from 0 (utils.cpp:736, 744-747); then (x * scale) + 0 (the IR's affine, graph_ir.cpp:923, 2727)
// and + the shared expert's row (graph_ir.cpp:926-928), which qwen2moe first scales by its token's gate
// sigmoid(s) = 1 / (1 + expf(-s)) of the gate logit s (graph_ir.cpp:704-705; graph_ir_ops.cpp:22, 61).
// A y row given as nparts K-split partial sums is their sum in ascending part order, and so is a shared
// row given as s_parts. One thread per output element.
__device__ inline float y_at(const float* __restrict__ y, int nparts, int64_t part_stride, size_t i) {
  float v = y[i];
  for (int s = 1; s < nparts; ++s) v = v + y[s * part_stride + i];
  return v;
}
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ y, int nparts, int64_t part_stride,
                                                      const float* __restrict__ gates, const int32_t* __restrict__ pos,
                                                      const float* __restrict__ y_shared, int s_parts, int64_t s_stride,
                                                      const float* __restrict__ sg_logit, float scale, int k, int d,
                                                      float* __restrict__ out, const unsigned long long* conflict) {
  const int t = blockIdx.y;
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= d) return;
  const float c = sg_logit ? shared_gate_sigmoid(sg_logit[t]) : 1.0f;
  float acc = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int p = pos[(size_t)t * k + j];
    const float g = gates[(size_t)t * k + j];
    if (p >= 0) acc = acc + g * y_at(y, nparts, part_stride, (size_t)p * d + o);
  }
  if (scale != 1.0f) acc = acc * scale + 0.0f;
  if (y_shared) {
    const float v = y_at(y_shared, s_parts, s_stride, (size_t)t * d + o);
    acc = acc + (sg_logit ? v * c : v);
  }
  out[(size_t)t * d + o] = conflict && *conflict ? __builtin_nanf("") : acc;
}

// The same with four consecutive outputs per thread (d % 4 == 0): 16-byte loads of y rows.
__global__ void __launch_bounds__(256) combine4_kernel(const float* __restrict__ y, int nparts, int64_t part_stride,
                                                       const float* __restrict__ gates, const int32_t* __restrict__ pos,
                                                       const float* __restrict__ y_shared, int s_parts, int64_t s_stride,
                                                       const float* __restrict__ sg_logit, float scale, int k, int d,
                                                       float* __restrict__ out, const unsigned long long* conflict) {
  const int t = blockIdx.y;
  const int o = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (o >= d) return;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int p = pos[(size_t)t * k + j];
    const float g = gates[(size_t)t * k + j];
    if (p >= 0) {
      float4 v = *reinterpret_cast<const float4*>(y + (size_t)p * d + o);
      for (int s = 1; s < nparts; ++s) {
        const float4 w = *reinterpret_cast<const float4*>(y + s * part_stride + (size_t)p * d + o);
        v.x = v.x + w.x;
        v.y = v.y + w.y;
        v.z = v.z + w.z;
        v.w = v.w + w.w;
      }
      a0 = a0 + g * v.x;
      a1 = a1 + g * v.y;
      a2 = a2 + g * v.z;
      a3 = a3 + g * v.w;
    }
  }
  if (scale != 1.0f) {
    a0 = a0 * scale + 0.0f;
    a1 = a1 * scale + 0.0f;
    a2 = a2 * scale + 0.0f;
    a3 = a3 * scale + 0.0f;
  }
  if (y_shared) {
    float4 v = *reinterpret_cast<const float4*>(y_shared + (size_t)t * d + o);
    if (s_parts > 1) {  // every part's load issued before the ordered sum
      float4 w[kMaxDenseKSplit - 1];
#pragma unroll
      for (int s = 1; s < kMaxDenseKSplit; ++s)
        w[s - 1] = s < s_parts ? *reinterpret_cast<const float4*>(y_shared + s * s_stride + (size_t)t * d + o)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int s = 1; s < kMaxDenseKSplit; ++s) {
        if (s < s_parts) {
          v.x = v.x + w[s - 1].x;
          v.y = v.y + w[s - 1].y;
          v.z = v.z + w[s - 1].z;
          v.w = v.w + w[s - 1].w;
        }
      }
    }
    if (sg_logit) {
      const float c = shared_gate_sigmoid(sg_logit[t]);
      v.x = v.x * c;
      v.y = v.y * c;
      v.z = v.z * c;
      v.w = v.w * c;
    }
    a0 = a0 + v.x;
    a1 = a1 + v.y;
    a2 = a2 + v.z;
    a3 = a3 + v.w;
  }
  if (conflict && *conflict) a0 = a1 = a2 = a3 = __builtin_nanf("");  // a pick-set conflict (see Route)
  *reinterpret_cast<float4*>(out + (size_t)t * d + o) = make_float4(a0, a1, a2, a3);
}

int launch_combine(const float* y, int nparts, int64_t part_stride, const float* gates, const int32_t* pos,
                   const float* y_shared, int s_parts, int64_t s_stride, const float* sg, float scale, int T, int k,
                   int d, float* out, hipStream_t st, const unsigned long long* conflict) {
  if (T <= 0) return EMBER_OK;
  if (d % 4 == 0) {
    dim3 grid((d / 4 + 255) / 256, T);
    combine4_kernel<<<grid, 256, 0, st>>>(y, nparts, part_stride, gates, pos, y_shared, s_parts, s_stride, sg, scale,
                                          k, d, out, conflict);
    return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
  }
  dim3 grid((d + 255) / 256, T);
  combine_kernel<<<grid, 256, 0, st>>>(y, nparts, part_stride, gates, pos, y_shared, s_parts, s_stride, sg, scale, k,
                                       d, out, conflict);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

}  // namespace ember_moe
