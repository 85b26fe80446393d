// Router logits, routing (top-k + gates) and the stable counting-sort dispatch for the MoE FFN.
//
// Bit-exactness contract (reference: utils.cpp:704-836, cpu_dot.h:12-21):
//  * logits are the FP64 fixed-order dot of the reference: eight FP64 chains over i = 8q + c,
//    ((c0+c1)+(c2+c3)) + ((c4+c5)+(c6+c7)) + tail, rounded to f32. Products of two f32 are exact
//    in f64, so one FMA per element rounds exactly as the reference's add of the product; the
//    chains are kept strictly sequential.
//  * top-k: k passes of argmax with strict > (ties to the lower index), picks sorted ascending.
//  * gates: (float)(exp((double)(r - mx)) / z), z the ascending double sum, exp = glibc's algorithm
//    (moe_math.hpp); the DeepSeek-style router runs the reference's float algorithm, as wave-parallel
//    scans whose results equal its serial ones (a row with a NaN runs it serially on one lane).
// (Small batches take their logits from router_logits_blocks in moe_experts.hip: the one-token
// launch's per-expert blocks, one per (expert, token).)
// The dispatch permutation has no reference counterpart: slots s = t*k + j are stably sorted by
// expert id (offsets[E+1], perm[p] = s, pos[s] = p), built without atomics on global memory.
#include "moe_conv.hpp"
#include "moe_route_dev.hpp"

namespace ember_moe {
using namespace ember_math;

constexpr int kRouterLdsFloats = 36864;  // 144 KiB of LDS for the row-staged router

// ---------------------------------------------------------------------------------------------
// Router logits, small T: one thread per (token, expert, chain); the 8 chains of a pair are 8
// consecutive lanes of one wave and are combined there in the reference's order.
__global__ void __launch_bounds__(256) router_logits_direct(const float* __restrict__ x, const float* __restrict__ R,
                                                            float* __restrict__ logits, int T, int d, int E) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int c = (int)(gid & 7);
  const int64_t pair = gid >> 3;
  const bool valid = pair < (int64_t)T * E;
  const int t = valid ? (int)(pair / E) : 0;
  const int e = valid ? (int)(pair % E) : 0;
  const float* xr = x + (size_t)t * d;
  const float* rr = R + (size_t)e * d;
  const int n8 = d - d % 8;
  double acc = 0.0;
  if (valid)
    for (int i = c; i < n8; i += 8) acc = __builtin_fma((double)rr[i], (double)xr[i], acc);
  const int lane = threadIdx.x & 63;
  const int base = lane & ~7;
  double a[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = __shfl(acc, base + j, 64);
  if (valid && c == 0) {
    double tail = 0.0;
    for (int i = n8; i < d; ++i) tail = __builtin_fma((double)rr[i], (double)xr[i], tail);
    const double v = (((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]))) + tail;
    logits[pair] = (float)v;
  }
}

// Router logits, small T: block (expert group, token) stages x[t] and EG router rows in LDS with
// coalesced 16-byte loads, then 8*EG threads run the eight FP64 chains of each expert from LDS (rows
// padded by 8 floats so the chains of different experts fall in different banks).
__host__ __device__ inline int router_lds_rows(int d) { return max(1, min(32, kRouterLdsFloats / (d + 8) - 1)); }

__global__ void __launch_bounds__(256) router_logits_lds(const float* __restrict__ x, const float* __restrict__ R,
                                                         float* __restrict__ logits, int T, int d, int E, int EG) {
  extern __shared__ __align__(16) float rl_lds[];
  const int t = blockIdx.y, e0 = blockIdx.x * EG;
  const int ne = min(EG, E - e0);
  const int ld = d + 8;
  float* xs = rl_lds;
  float* rs = rl_lds + ld;
  const bool vec = (d % 4) == 0;
  if (vec) {
    copy16_to_lds(xs, x + (size_t)t * d, d / 4);
    for (int j = 0; j < ne; ++j) copy16_to_lds(rs + j * ld, R + (size_t)(e0 + j) * d, d / 4);
  } else {
    for (int i = threadIdx.x; i < d; i += blockDim.x) xs[i] = x[(size_t)t * d + i];
    for (int j = 0; j < ne; ++j)
      for (int i = threadIdx.x; i < d; i += blockDim.x) rs[j * ld + i] = R[(size_t)(e0 + j) * d + i];
  }
  __syncthreads();
  const int c = threadIdx.x & 7, j = threadIdx.x >> 3;
  const int n8 = d - d % 8;
  double acc = 0.0;
  if (j < ne) {
    const float* rr = rs + j * ld;
#pragma unroll 8
    for (int i = c; i < n8; i += 8) acc = __builtin_fma((double)rr[i], (double)xs[i], acc);
  }
  const int lane = threadIdx.x & 63;
  double a[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) a[q] = __shfl(acc, (lane & ~7) + q, 64);
  if (j < ne && c == 0) {
    const float* rr = rs + j * ld;
    double tail = 0.0;
    for (int i = n8; i < d; ++i) tail = __builtin_fma((double)rr[i], (double)xs[i], tail);
    const double v = (((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]))) + tail;
    logits[(size_t)t * E + e0 + j] = (float)v;
  }
}

// Router logits, many tokens: a block of TT tokens x TE experts (TT * TE = 256 threads, one per
// pair) walks K in tiles of 512 staged in LDS; each thread keeps the pair's eight FP64 chains as
// independent accumulators (8-way ILP), element 8q + c going to chain c in increasing q, exactly the
// reference's order.
template <int TT, int TE, int PT, int PE, int RP_KT>
__global__ void __launch_bounds__(256) router_logits_pt(const float* __restrict__ x, const float* __restrict__ R,
                                                        float* __restrict__ logits, int T, int d, int E) {
  static_assert((TT / PT) * (TE / PE) == 256, "one thread per PT x PE block of pairs");
  extern __shared__ __align__(16) float rp_lds[];
  constexpr int LD = RP_KT + 4;
  constexpr int ROWS = TT + TE;
  constexpr int Q4 = RP_KT / 4;                    // float4 granules per row of a full tile
  constexpr int PER = (ROWS * Q4 + 255) / 256;     // granules per thread per tile
  const int t0 = blockIdx.x * TT, e0 = blockIdx.y * TE;
  const int tq = threadIdx.x / (TE / PE), eq = threadIdx.x % (TE / PE);
  const int n8 = d - d % 8;
  const int ntiles = (n8 + RP_KT - 1) / RP_KT;
  float4 pre[PER];
  // all of a tile's loads are issued before any is used; the next tile's are in flight while this
  // tile's chains run
  auto fetch = [&](int kt) {
    const int k0 = kt * RP_KT, kn = min(RP_KT, n8 - k0);
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = threadIdx.x + u * 256;
      const int row = i / Q4, col = i % Q4;
      pre[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row < ROWS && 4 * col < kn) {
        if (row < TT) {
          if (t0 + row < T) pre[u] = *reinterpret_cast<const float4*>(x + (size_t)(t0 + row) * d + k0 + 4 * col);
        } else if (e0 + row - TT < E) {
          pre[u] = *reinterpret_cast<const float4*>(R + (size_t)(e0 + row - TT) * d + k0 + 4 * col);
        }
      }
    }
  };
  double a[PT][PE][8];
#pragma unroll
  for (int i = 0; i < PT; ++i)
#pragma unroll
    for (int j = 0; j < PE; ++j)
#pragma unroll
      for (int c = 0; c < 8; ++c) a[i][j][c] = 0.0;
  if (ntiles > 0) fetch(0);
  for (int kt = 0; kt < ntiles; ++kt) {
    const int kn = min(RP_KT, n8 - kt * RP_KT);
    float* buf = rp_lds + (kt & 1) * ROWS * LD;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = threadIdx.x + u * 256;
      if (i < ROWS * Q4) *reinterpret_cast<float4*>(buf + (i / Q4) * LD + 4 * (i % Q4)) = pre[u];
    }
    __syncthreads();  // two buffers alternate, so one barrier per tile suffices
    if (kt + 1 < ntiles) fetch(kt + 1);
    for (int k8 = 0; k8 < kn; k8 += 8) {
      float xv[PT][8], rv[PE][8];
#pragma unroll
      for (int i = 0; i < PT; ++i) {
        const float* xr = buf + (tq * PT + i) * LD + k8;
        const float4 u0 = *reinterpret_cast<const float4*>(xr), u1 = *reinterpret_cast<const float4*>(xr + 4);
        xv[i][0] = u0.x; xv[i][1] = u0.y; xv[i][2] = u0.z; xv[i][3] = u0.w;
        xv[i][4] = u1.x; xv[i][5] = u1.y; xv[i][6] = u1.z; xv[i][7] = u1.w;
      }
#pragma unroll
      for (int j = 0; j < PE; ++j) {
        const float* rr = buf + (TT + eq * PE + j) * LD + k8;
        const float4 u0 = *reinterpret_cast<const float4*>(rr), u1 = *reinterpret_cast<const float4*>(rr + 4);
        rv[j][0] = u0.x; rv[j][1] = u0.y; rv[j][2] = u0.z; rv[j][3] = u0.w;
        rv[j][4] = u1.x; rv[j][5] = u1.y; rv[j][6] = u1.z; rv[j][7] = u1.w;
      }
#pragma unroll
      for (int i = 0; i < PT; ++i)
#pragma unroll
        for (int j = 0; j < PE; ++j)
#pragma unroll
          for (int c = 0; c < 8; ++c) a[i][j][c] = __builtin_fma((double)rv[j][c], (double)xv[i][c], a[i][j][c]);
    }
  }
#pragma unroll
  for (int i = 0; i < PT; ++i)
#pragma unroll
    for (int j = 0; j < PE; ++j) {
      const int t = t0 + tq * PT + i, e = e0 + eq * PE + j;
      if (t >= T || e >= E) continue;
      double tail = 0.0;
      for (int q = n8; q < d; ++q) tail = __builtin_fma((double)R[(size_t)e * d + q], (double)x[(size_t)t * d + q], tail);
      const double* c8 = a[i][j];
      const double v = (((c8[0] + c8[1]) + (c8[2] + c8[3])) + ((c8[4] + c8[5]) + (c8[6] + c8[7]))) + tail;
      logits[(size_t)t * E + e] = (float)v;
    }
}

// Router logits, large T: a 32-token x 16-expert tile per 256-thread block. Thread (chain c, group g)
// keeps 4 tokens x 4 experts of chain c; x and R stream through LDS in 64-element K tiles, and each
// chain visits its elements in increasing index order, so the sums are the reference's exactly.
constexpr int RL_TT = 32, RL_TE = 16, RL_KT = 64;
__global__ void __launch_bounds__(256) router_logits_tiled(const float* __restrict__ x, const float* __restrict__ R,
                                                           float* __restrict__ logits, int T, int d, int E) {
  __shared__ float xs[RL_TT][RL_KT + 1];
  __shared__ float rs[RL_TE][RL_KT + 1];
  __shared__ double part[RL_TT * RL_TE][9];
  const int tid = threadIdx.x;
  const int c = tid & 7, g = tid >> 3;
  const int tq = g & 7, eq = g >> 3;  // 8 token quads x 4 expert quads
  const int t0 = blockIdx.x * RL_TT, e0 = blockIdx.y * RL_TE;
  const int n8 = d - d % 8;
  double acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
  for (int k0 = 0; k0 < n8; k0 += RL_KT) {
    const int kn = min(RL_KT, n8 - k0);
    for (int i = tid; i < RL_TT * RL_KT; i += 256) {
      const int tt = i / RL_KT, kk = i % RL_KT;
      const int t = t0 + tt;
      xs[tt][kk] = (t < T && kk < kn) ? x[(size_t)t * d + k0 + kk] : 0.0f;
    }
    for (int i = tid; i < RL_TE * RL_KT; i += 256) {
      const int ee = i / RL_KT, kk = i % RL_KT;
      const int e = e0 + ee;
      rs[ee][kk] = (e < E && kk < kn) ? R[(size_t)e * d + k0 + kk] : 0.0f;
    }
    __syncthreads();
    for (int kk = c; kk < kn; kk += 8) {
      double xv[4], rv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[i] = (double)xs[tq * 4 + i][kk];
#pragma unroll
      for (int j = 0; j < 4; ++j) rv[j] = (double)rs[eq * 4 + j][kk];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fma(rv[j], xv[i], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) part[(tq * 4 + i) * RL_TE + eq * 4 + j][c] = acc[i][j];
  __syncthreads();
  for (int p = tid; p < RL_TT * RL_TE; p += 256) {
    const int t = t0 + p / RL_TE, e = e0 + p % RL_TE;
    if (t >= T || e >= E) continue;
    const double* a = part[p];
    double tail = 0.0;
    for (int i = n8; i < d; ++i) tail = __builtin_fma((double)R[(size_t)e * d + i], (double)x[(size_t)t * d + i], tail);
    const double v = (((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]))) + tail;
    logits[(size_t)t * E + e] = (float)v;
  }
}

__global__ void __launch_bounds__(256) route_kernel(const float* __restrict__ logits, int T, int E, int k, int renorm,
                                                    int routed, int sigmoid, const float* __restrict__ bias,
                                                    int groups_n, int groups_top, int32_t* __restrict__ idx,
                                                    float* __restrict__ gates, ActConv conv) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int nroute = (T + 3) / 4;  // blocks past these convert activations (act_conv_row)
  if ((int)blockIdx.x >= nroute) {
    act_conv_row(conv, blockIdx.x - nroute);
    return;
  }
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  route_token(logits + (size_t)t * E, E, k, renorm, routed, sigmoid, bias, groups_n, groups_top,
              lds_raw + (size_t)wave * route_wave_lds(E), idx + (size_t)t * k, gates + (size_t)t * k);
}

// ---------------------------------------------------------------------------------------------
// Dispatch: stable counting sort of the T*k slots by expert. Slots are cut into 1024-slot chunks, one
// block each. (1) each slot's rank among equal experts earlier in its chunk (within a wave by
// shuffles, across the chunk's waves by a per-expert prefix in LDS) and per-chunk per-expert counts;
// (2) one block scans the counts into per-expert offsets, the list of experts with tokens, and each
// chunk's base position per expert; (3) each slot lands at base[chunk][e] + rank.
constexpr int kChunk = 1024;

__global__ void __launch_bounds__(kChunk) dispatch_count(const int32_t* __restrict__ idx, int nslots, int E,
                                                         int32_t* __restrict__ rank, int32_t* __restrict__ chunk_cnt) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  int* wcnt = reinterpret_cast<int*>(lds_raw);  // [16][E]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x;
  const int s = c * kChunk + threadIdx.x;
  for (int i = threadIdx.x; i < 16 * E; i += kChunk) wcnt[i] = 0;
  const int e = s < nslots ? idx[s] : -1;
  int rk = 0, later = 0;
  for (int j = 0; j < 64; ++j) {
    const int oe = __shfl(e, j, 64);
    if (oe == e) {
      if (j < lane) ++rk;
      if (j > lane) ++later;
    }
  }
  __syncthreads();
  if (e >= 0 && later == 0) wcnt[wave * E + e] = rk + 1;
  __syncthreads();
  for (int q = threadIdx.x; q < E; q += kChunk) {
    int run = 0;
    for (int w = 0; w < 16; ++w) {
      const int t = wcnt[w * E + q];
      wcnt[w * E + q] = run;
      run += t;
    }
    chunk_cnt[(size_t)c * E + q] = run;
  }
  __syncthreads();
  if (s < nslots) rank[s] = e >= 0 ? wcnt[wave * E + e] + rk : 0;
}

// One block of 1024 threads (E <= 1024): offsets[E+1], used[] / n_used, and chunk_cnt overwritten with
// each chunk's base position per expert.
// The counts are staged in LDS with coalesced loads (one memory latency, not one per chunk) when they fit
// (cnt_lds), and the bases written back the same way.
__global__ void __launch_bounds__(1024) dispatch_scan(int32_t* __restrict__ chunk_cnt, int nchunks, int E,
                                                      DispatchScratch ds, int cnt_lds) {
  extern __shared__ __align__(16) int cc[];  // [nchunks][E] when cnt_lds
  int32_t* __restrict__ offsets = ds.offsets;
  int32_t* __restrict__ used = ds.used;
  int32_t* __restrict__ n_used = ds.n_used;
  __shared__ int tmp[16];
  const int e = threadIdx.x, n = nchunks * E;
  int* cnt = cnt_lds ? cc : chunk_cnt;
  if (cnt_lds) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) cc[i] = chunk_cnt[i];
    __syncthreads();
  }
  int tot = 0;
  if (e < E)
    for (int c = 0; c < nchunks; ++c) tot += cnt[(size_t)c * E + e];
  int all = 0, nu = 0;
  const int off = block_exclusive_scan(e < E ? tot : 0, tmp, &all);
  const int upos = block_exclusive_scan(e < E && tot > 0 ? 1 : 0, tmp, &nu);
  if (e < E) {
    offsets[e] = off;
    if (tot > 0) used[upos] = e;
    int run = off;
    for (int c = 0; c < nchunks; ++c) {
      const int v = cnt[(size_t)c * E + e];
      cnt[(size_t)c * E + e] = run;
      run += v;
    }
  }
  if (e == 0) {
    offsets[E] = all;
    *n_used = nu;
  }
  write_tiles(e, E, tot, ds, tmp);
  if (cnt_lds) {
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) chunk_cnt[i] = cc[i];
  }
}

__global__ void __launch_bounds__(256) dispatch_scatter(const int32_t* __restrict__ idx, int nslots, int E,
                                                        const int32_t* __restrict__ rank,
                                                        const int32_t* __restrict__ chunk_base,
                                                        int32_t* __restrict__ perm, int32_t* __restrict__ pos) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= nslots) return;
  const int e = idx[s];
  if (e < 0) {
    pos[s] = -1;
    return;
  }
  const int p = chunk_base[(size_t)(s / kChunk) * E + e] + rank[s];
  perm[p] = s;
  pos[s] = p;
}

// Dispatch of up to kOneBlockChunks chunks (E <= kOneBlockE) in one block: the same three steps as
// dispatch_count / dispatch_scan / dispatch_scatter, with the ranks and experts of the block's slots
// kept in registers and the per-chunk counts in LDS, so the whole sort is one launch. The block walks
// the chunks one after another: one chunk saves ~2 us of launches, four cost ~11 us more than the
// three-kernel sort, so only single-chunk dispatches take it.
constexpr int kOneBlockChunks = 1, kOneBlockE = 256;
__global__ void __launch_bounds__(kChunk) dispatch_one_block(const int32_t* __restrict__ idx, int nslots, int E,
                                                             DispatchScratch ds) {
  int32_t* __restrict__ offsets = ds.offsets;
  int32_t* __restrict__ used = ds.used;
  int32_t* __restrict__ n_used = ds.n_used;
  int32_t* __restrict__ perm = ds.perm;
  int32_t* __restrict__ pos = ds.pos;
  __shared__ int wcnt[16 * kOneBlockE];
  __shared__ int ccnt[kOneBlockChunks * kOneBlockE];
  __shared__ int tmp[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunks = (nslots + kChunk - 1) / kChunk;
  int ex[kOneBlockChunks], rk[kOneBlockChunks];
#pragma unroll
  for (int c = 0; c < kOneBlockChunks; ++c) {
    ex[c] = -1;
    rk[c] = 0;
    if (c >= nchunks) continue;  // uniform over the block
    const int s = c * kChunk + threadIdx.x;
    for (int i = threadIdx.x; i < 16 * E; i += kChunk) wcnt[i] = 0;
    const int e = s < nslots ? idx[s] : -1;
    int r = 0, later = 0;
    for (int j = 0; j < 64; ++j) {
      const int oe = __shfl(e, j, 64);
      if (oe == e) {
        if (j < lane) ++r;
        if (j > lane) ++later;
      }
    }
    __syncthreads();
    if (e >= 0 && later == 0) wcnt[wave * E + e] = r + 1;
    __syncthreads();
    for (int q = threadIdx.x; q < E; q += kChunk) {
      int run = 0;
      for (int w = 0; w < 16; ++w) {
        const int t = wcnt[w * E + q];
        wcnt[w * E + q] = run;
        run += t;
      }
      ccnt[c * E + q] = run;
    }
    __syncthreads();
    ex[c] = e;
    rk[c] = e >= 0 ? wcnt[wave * E + e] + r : 0;
    __syncthreads();  // wcnt is cleared for the next chunk
  }
  const int e = threadIdx.x;
  int tot = 0;
  if (e < E)
    for (int c = 0; c < nchunks; ++c) tot += ccnt[c * E + e];
  int all = 0, nu = 0;
  const int off = block_exclusive_scan(e < E ? tot : 0, tmp, &all);
  const int upos = block_exclusive_scan(e < E && tot > 0 ? 1 : 0, tmp, &nu);
  if (e < E) {
    offsets[e] = off;
    if (tot > 0) used[upos] = e;
    int run = off;
    for (int c = 0; c < nchunks; ++c) {
      const int n = ccnt[c * E + e];
      ccnt[c * E + e] = run;
      run += n;
    }
  }
  if (e == 0) {
    offsets[E] = all;
    *n_used = nu;
  }
  write_tiles(e, E, tot, ds, tmp);
  __syncthreads();
#pragma unroll
  for (int c = 0; c < kOneBlockChunks; ++c) {
    const int s = c * kChunk + threadIdx.x;
    if (c >= nchunks || s >= nslots) continue;
    if (ex[c] < 0) {
      pos[s] = -1;
      continue;
    }
    const int p = ccnt[c * E + ex[c]] + rk[c];
    perm[p] = s;
    pos[s] = p;
  }
}

// Decode-sized batches (T <= 8 tokens, T*k <= 512 slots, E <= 256): routing and the whole dispatch in
// one block of 512 threads. Wave w routes token w; then each slot takes its rank among equal experts
// at lower slots (a scan of the idx list in LDS), the per-expert offsets come from LDS counts.
constexpr int kSmallT = 8, kSmallSlots = 512, kSmallE = 256;

__global__ void __launch_bounds__(512) route_dispatch_small(const float* __restrict__ logits, int T, int E, int k,
                                                            int renorm, int routed, int sigmoid,
                                                            const float* __restrict__ bias, int groups_n,
                                                            int groups_top, int32_t* __restrict__ idx,
                                                            float* __restrict__ gates, DispatchScratch ds,
                                                            ActConv conv) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  if (blockIdx.x > 0) {  // blocks past the first convert activations (act_conv_row)
    act_conv_row(conv, blockIdx.x - 1);
    return;
  }
  const int wave = threadIdx.x >> 6;
  const size_t wl = route_wave_lds(E);
  int* sidx = reinterpret_cast<int*>(lds_raw + kSmallT * wl);
  float* sgate = reinterpret_cast<float*>(sidx + kSmallSlots);
  int* cnt = reinterpret_cast<int*>(sgate + kSmallSlots);
  if (wave < T)  // picks and gates stay in LDS; the block copies them out below
    route_token(logits + (size_t)wave * E, E, k, renorm, routed, sigmoid, bias, groups_n, groups_top,
                lds_raw + wave * wl, sidx + (size_t)wave * k, sgate + (size_t)wave * k);
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  const int n = T * k;
  const int sl = threadIdx.x;
  int e = -1;
  if (sl < n) {
    e = sidx[sl];
    idx[sl] = e;
    gates[sl] = sgate[sl];
    if (e >= 0) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  {
    // E <= 512 = blockDim: one expert per thread
    const int q = threadIdx.x;
    const int c = q < E ? cnt[q] : 0;
    int all = 0, nu = 0;
    const int off = block_exclusive_scan(c, cnt + E, &all);
    const int upos = block_exclusive_scan(c > 0 ? 1 : 0, cnt + E, &nu);
    if (q < E) {
      ds.offsets[q] = off;
      if (c > 0) ds.used[upos] = q;
    }
    __syncthreads();
    write_tiles(q, E, c, ds, cnt + E);
    if (q < E) cnt[q] = off;
    if (q == 0) {
      ds.offsets[E] = all;
      *ds.n_used = nu;
    }
  }
  __syncthreads();
  if (sl < n) {
    if (e < 0) {
      ds.pos[sl] = -1;
    } else {
      int rk = 0;
      for (int q = 0; q < sl; ++q) rk += (sidx[q] == e);
      const int p = cnt[e] + rk;
      ds.perm[p] = sl;
      ds.pos[sl] = p;
    }
  }
}

// Router logits, many tokens x many experts: lane (chain c = lane & 7, pair group g = tid >> 3) runs
// chain c of PT x PE (token, expert) pairs, tokens tq + GT*i and experts eq + GE*j of the block's
// tile; the 32 pair groups of a 256-thread block form a GT x GE grid, so a block covers GT*PT tokens x
// GE*PE experts and a launch has ceil(T / (GT*PT)) x
// ceil(E / (GE*PE)) blocks (one lane per chain instead of one per pair keeps several hundred blocks
// in flight at T ~ 100). x and R rows stream through LDS in KT-element K tiles (two buffers, the next
// tile's loads in flight while this tile's chains run; every tile waits for one memory latency, so
// the tiles are long); each chain visits its elements 8q + c in
// increasing q and the eight chains of a pair sit in eight consecutive lanes, combined by shuffles
// in the reference's order. The eight pair groups of a wave read eight consecutive R rows per step,
// padded to start 8 banks apart. Each thread converts PT + PE staged floats to double per PT * PE
// FMAs, so the large-T variant takes 4 x 4 pairs.
template <int GT, int GE, int PT, int PE, int KT>
__global__ void __launch_bounds__(256) router_logits_chains(const float* __restrict__ x, const float* __restrict__ R,
                                                            float* __restrict__ logits, int T, int d, int E) {
  static_assert(GT * GE == 32, "32 pair groups of 8 chains");
  constexpr int TT = GT * PT, TE = GE * PE, ROWS = TT + TE;
  constexpr int LD = KT + 8;
  constexpr int Q4 = KT / 4;
  constexpr int PER = (ROWS * Q4 + 255) / 256;
  __shared__ __align__(16) float buf2[2][ROWS * LD];
  const int c = threadIdx.x & 7, g = threadIdx.x >> 3;
  const int tq = g / GE, eq = g % GE;
  const int t0 = blockIdx.x * TT, e0 = blockIdx.y * TE;
  const int n8 = d - d % 8;
  const int ntiles = (n8 + KT - 1) / KT;
  float4 pre[PER];
  auto fetch = [&](int kt) {
    const int k0 = kt * KT, kn = min(KT, n8 - k0);
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = threadIdx.x + u * 256;
      const int row = i / Q4, col = i % Q4;
      pre[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row < ROWS && 4 * col < kn) {
        if (row < TT) {
          if (t0 + row < T) pre[u] = *reinterpret_cast<const float4*>(x + (size_t)(t0 + row) * d + k0 + 4 * col);
        } else if (e0 + row - TT < E) {
          pre[u] = *reinterpret_cast<const float4*>(R + (size_t)(e0 + row - TT) * d + k0 + 4 * col);
        }
      }
    }
  };
  double a[PT][PE];
#pragma unroll
  for (int i = 0; i < PT; ++i)
#pragma unroll
    for (int j = 0; j < PE; ++j) a[i][j] = 0.0;
  if (ntiles > 0) fetch(0);
  for (int kt = 0; kt < ntiles; ++kt) {
    const int kn = min(KT, n8 - kt * KT);
    float* buf = buf2[kt & 1];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = threadIdx.x + u * 256;
      if (i < ROWS * Q4) *reinterpret_cast<float4*>(buf + (i / Q4) * LD + 4 * (i % Q4)) = pre[u];
    }
    __syncthreads();  // two buffers alternate, so one barrier per tile suffices
    if (kt + 1 < ntiles) fetch(kt + 1);
    const float* xb = buf + tq * LD + c;
    const float* rb = buf + (TT + eq) * LD + c;
    if (kn == KT) {
      // bursts of NB steps in two register slots: the next burst's LDS reads are issued before this
      // burst's FMAs (the scheduling barriers keep the compiler from interleaving them into one
      // read-wait-FMA sequence per step, which waits for one LDS latency every step or two)
      constexpr int NB = 32 / (PT + PE), NBURST = KT / 8 / NB;
      static_assert(KT / 8 % NB == 0, "whole bursts per tile");
      float xs[2][PT][NB], rs[2][PE][NB];
      auto load = [&](int slot, int b) {
#pragma unroll
        for (int q = 0; q < NB; ++q) {
#pragma unroll
          for (int i = 0; i < PT; ++i) xs[slot][i][q] = xb[i * GT * LD + 8 * (b * NB + q)];
#pragma unroll
          for (int j = 0; j < PE; ++j) rs[slot][j][q] = rb[j * GE * LD + 8 * (b * NB + q)];
        }
      };
      load(0, 0);
#pragma unroll
      for (int b = 0; b < NBURST; ++b) {
        if (b + 1 < NBURST) load((b + 1) & 1, b + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < NB; ++q)
#pragma unroll
          for (int i = 0; i < PT; ++i)
#pragma unroll
            for (int j = 0; j < PE; ++j)
              a[i][j] = __builtin_fma((double)rs[b & 1][j][q], (double)xs[b & 1][i][q], a[i][j]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      for (int k8 = 0; k8 < kn; k8 += 8)
#pragma unroll
        for (int i = 0; i < PT; ++i)
#pragma unroll
          for (int j = 0; j < PE; ++j)
            a[i][j] = __builtin_fma((double)rb[j * GE * LD + k8], (double)xb[i * GT * LD + k8], a[i][j]);
    }
  }
  const int base = (threadIdx.x & 63) & ~7;
#pragma unroll
  for (int i = 0; i < PT; ++i)
#pragma unroll
    for (int j = 0; j < PE; ++j) {
      double ch[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) ch[q] = __shfl(a[i][j], base + q, 64);
      const int t = t0 + tq + GT * i, e = e0 + eq + GE * j;
      if (c != 0 || t >= T || e >= E) continue;
      double tail = 0.0;
      for (int q = n8; q < d; ++q) tail = __builtin_fma((double)R[(size_t)e * d + q], (double)x[(size_t)t * d + q], tail);
      const double v = (((ch[0] + ch[1]) + (ch[2] + ch[3])) + ((ch[4] + ch[5]) + (ch[6] + ch[7]))) + tail;
      logits[(size_t)t * E + e] = (float)v;
    }
}

// ---------------------------------------------------------------------------------------------
// Host-side launchers.

int launch_router_logits(const float* x, int T, int d, int E, const float* R, float* logits, hipStream_t st) {
  if (T <= 0) return EMBER_OK;
  // rows per block: as many as fit, but no more than keeps >= 256 blocks in flight
  const int EG = max(1, min(router_lds_rows(d), (int)(((int64_t)T * E + 255) / 256)));
  const int64_t lds_blocks = (int64_t)T * ((E + EG - 1) / EG);
  if (d % 4 == 0 && ((E >= 16 && T >= 4) || (E >= 8 && T >= 64))) {
    // one lane per chain; the largest tile that still gives >= 256 blocks: 16 x 32 pairs (E >= 32), 8 x 16
    // (E >= 16), else 4 x 8 (with 8 to 15 experts the staged-row kernels below stay ahead up to a few
    // dozen tokens). Measured router times, 4 x 8 / 8 x 16 / 16 x 32: C3-shaped (E = 128, d = 2048) T = 128
    // 14.4 / 17.6 / 34.0 us, T = 256 21.1 / 18.9, T = 512 34.8 / 25.7 / 34.4, T = 1024 - / 40.6 / 36.5;
    // C4-shaped (E = 64) T = 256 13.5 / 16.9, T = 512 20.4 / 18.0, T = 1024 32.4 / 24.7
    const int64_t b16 = (int64_t)((T + 15) / 16) * ((E + 31) / 32), b8 = (int64_t)((T + 7) / 8) * ((E + 15) / 16);
    if (E >= 32 && b16 >= 256) {
      router_logits_chains<4, 8, 4, 4, 128><<<dim3((T + 15) / 16, (E + 31) / 32), 256, 0, st>>>(x, R, logits, T, d, E);
    } else if (E >= 16 && b8 >= 256) {
      router_logits_chains<4, 8, 2, 2, 256><<<dim3((T + 7) / 8, (E + 15) / 16), 256, 0, st>>>(x, R, logits, T, d, E);
    } else {
      router_logits_chains<4, 8, 1, 1, 512><<<dim3((T + 3) / 4, (E + 7) / 8), 256, 0, st>>>(x, R, logits, T, d, E);
    }
  } else if (router_blocks_fit(T, d, E)) {
    // a few pairs: one block each, its products formed in parallel (the one-token launch's router blocks)
    return launch_router_logits_blocks(x, T, d, E, R, logits, st);
  } else if (2 * (d + 8) <= kRouterLdsFloats && (lds_blocks <= 1024 || d % 4)) {
    // few blocks: each stages whole rows once and runs its chains from LDS (one memory latency)
    static const bool lds_ok =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&router_logits_lds), hipFuncAttributeMaxDynamicSharedMemorySize,
                            kRouterLdsFloats * (int)sizeof(float)) == hipSuccess;
    if (!lds_ok) return EMBER_ERR_LAUNCH;
    dim3 grid((E + EG - 1) / EG, T);
    router_logits_lds<<<grid, 256, (size_t)(EG + 1) * (d + 8) * sizeof(float), st>>>(x, R, logits, T, d, E, EG);
  } else if (d % 4 == 0) {
    const size_t lds_small = (size_t)2 * (32 + 8) * (256 + 4) * sizeof(float);
    const size_t lds_big = (size_t)2 * (32 + 32) * (128 + 4) * sizeof(float);
    static const bool lds_ok =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&router_logits_pt<32, 8, 1, 1, 256>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_small) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(&router_logits_pt<32, 32, 2, 2, 128>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_big) == hipSuccess;
    if (!lds_ok) return EMBER_ERR_LAUNCH;
    if (E <= 8) {
      dim3 grid((T + 31) / 32, (E + 7) / 8);
      router_logits_pt<32, 8, 1, 1, 256><<<grid, 256, lds_small, st>>>(x, R, logits, T, d, E);
    } else {
      dim3 grid((T + 31) / 32, (E + 31) / 32);
      router_logits_pt<32, 32, 2, 2, 128><<<grid, 256, lds_big, st>>>(x, R, logits, T, d, E);
    }
  } else if (T >= 32 && E >= 8) {
    dim3 grid((T + RL_TT - 1) / RL_TT, (E + RL_TE - 1) / RL_TE);
    router_logits_tiled<<<grid, 256, 0, st>>>(x, R, logits, T, d, E);
  } else {
    const int64_t threads = (int64_t)T * E * 8;
    router_logits_direct<<<(unsigned)((threads + 255) / 256), 256, 0, st>>>(x, R, logits, T, d, E);
  }
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

int launch_route(const float* logits, int T, int E, int k, int renorm, int routed, int sigmoid, const float* bias,
                 int groups_n, int groups_top, int32_t* idx, float* gates, const ActConv* conv, hipStream_t st) {
  if (T <= 0) return EMBER_OK;
  const size_t lds = 4 * route_wave_lds(E);
  const ActConv c = conv ? *conv : ActConv{};
  route_kernel<<<(T + 3) / 4 + c.rows, 256, lds, st>>>(logits, T, E, k, renorm, routed, sigmoid, bias, groups_n,
                                                       groups_top, idx, gates, c);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

bool route_dispatch_fused(int T, int E, int k) { return T <= kSmallT && T * k <= kSmallSlots && E <= kSmallE; }

int launch_route_dispatch(const float* logits, int T, int E, int k, int renorm, int routed, int sigmoid,
                          const float* bias, int groups_n, int groups_top, int32_t* idx, float* gates,
                          const DispatchScratch& ds, const ActConv* conv, hipStream_t st) {
  if (T <= 0) return EMBER_OK;
  if (!route_dispatch_fused(T, E, k)) {
    int s = launch_route(logits, T, E, k, renorm, routed, sigmoid, bias, groups_n, groups_top, idx, gates, conv, st);
    return s ? s : launch_dispatch(idx, T, k, E, ds, st);
  }
  const size_t lds = kSmallT * route_wave_lds(E) + (size_t)(2 * kSmallSlots + E + 16) * sizeof(int);
  static const bool lds_ok = [] {
    const size_t most = kSmallT * route_wave_lds(kSmallE) + (size_t)(2 * kSmallSlots + kSmallE + 16) * sizeof(int);
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&route_dispatch_small),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)most) == hipSuccess;
  }();
  if (!lds_ok) return EMBER_ERR_LAUNCH;
  const ActConv c = conv ? *conv : ActConv{};
  route_dispatch_small<<<1 + c.rows, 512, lds, st>>>(logits, T, E, k, renorm, routed, sigmoid, bias, groups_n,
                                                     groups_top, idx, gates, ds, c);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

int launch_dispatch(const int32_t* idx, int T, int k, int E, const DispatchScratch& ds, hipStream_t st) {
  const int nslots = T * k;
  const int nchunks = (nslots + kChunk - 1) / kChunk;
  if (nslots <= 0) return EMBER_OK;
  if (nchunks <= kOneBlockChunks && E <= kOneBlockE) {
    dispatch_one_block<<<1, kChunk, 0, st>>>(idx, nslots, E, ds);
    return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
  }
  dispatch_count<<<nchunks, kChunk, 16 * (size_t)E * sizeof(int), st>>>(idx, nslots, E, ds.rank, ds.chunk_cnt);
  const size_t cnt_bytes = (size_t)nchunks * E * sizeof(int);
  const int cnt_lds = cnt_bytes <= 48 * 1024;
  dispatch_scan<<<1, 1024, cnt_lds ? cnt_bytes : 0, st>>>(ds.chunk_cnt, nchunks, E, ds, cnt_lds);
  dispatch_scatter<<<(nslots + 255) / 256, 256, 0, st>>>(idx, nslots, E, ds.rank, ds.chunk_cnt, ds.perm, ds.pos);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

}  // namespace ember_moe
