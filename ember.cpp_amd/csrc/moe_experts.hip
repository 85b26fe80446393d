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
//    amax/32767, relative error ~2e-5) and each block's integer dot runs on v_dot2_i32_i16 with
//    the weights' quants zero-extended to 16 bits (Q8_0 offset by +128, corrected with the block's
//    activation sum), then scaled in FP32. Relative error stays near 1e-5, far inside 2e-3.
//
// Work layout: a lane owns a 32/64-element "chunk" of a row (fixed byte offset in the ggml row);
// L lanes (a power of two <= 64) cover a row (looping when a row has more than L chunks), so a wave
// covers 64/L rows. Each lane group walks row groups of RR rows (x2 for the gate/up pair) across
// the whole segment (grid-stride), with the next step's weights loaded before the current step is
// computed. grid.y enumerates expert segments (experts that received tokens, from the dispatch
// step), so no host synchronisation is needed.
#include "moe_fmt.hpp"

namespace ember_moe {
using namespace ember_math;


// One projection pass. Thread layout: lane group of L lanes per row slot; RR rows per step; MT tokens
// per pass over the weights. Steps (row group, chunk round) are double-buffered.
template <int FMT, int RR, int MT, bool GATED>
__global__ void __launch_bounds__(256) proj_kernel(ProjArgs a, int L_log2) {
  using F = Fmt<FMT>;
  constexpr int G = GATED ? 2 : 1;
  const int L = 1 << L_log2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane >> L_log2, rl = lane & (L - 1);
  const int slots_per_block = 4 * (64 >> L_log2);
  const int slot = blockIdx.x * slots_per_block + wave * (64 >> L_log2) + sub;
  const int nslots = gridDim.x * slots_per_block;
  int e = 0, p0 = 0, M = a.T;
  if (a.used) {
    if ((int)blockIdx.y >= *a.n_used) return;
    e = a.used[blockIdx.y];
    p0 = a.offsets[e];
    M = a.offsets[e + 1] - p0;
  }
  const int K = a.K;
  const int64_t rb = F::row_bytes(K);
  const int C = (K + F::CE - 1) / F::CE;
  const int NC = (C + L - 1) / L;  // chunk rounds per row (uniform across the lane group)
  const uint8_t* W0 = static_cast<const uint8_t*>(a.w0) + (int64_t)e * a.expert_stride;
  const uint8_t* W1 = GATED ? static_cast<const uint8_t*>(a.w1) + (int64_t)e * a.expert_stride : W0;
  const int ngroups = (a.rows + RR - 1) / RR;
  // number of steps this slot walks: row groups slot, slot + nslots, ... times NC chunk rounds
  const int my_groups = slot < ngroups ? (ngroups - 1 - slot) / nslots + 1 : 0;
  const int nsteps = my_groups * NC;

  extern __shared__ __align__(16) uint8_t act_lds[];
  const int row_lds = act_lds_bytes(F::QX, K);
  __shared__ int rows[MT];
  for (int m0 = 0; m0 < M; m0 += MT) {
    __syncthreads();  // the previous token group's rows are no longer read
    if (threadIdx.x < MT && m0 + (int)threadIdx.x < M) {
      const int p = p0 + m0 + threadIdx.x;
      rows[threadIdx.x] = a.in_by_perm ? a.perm[p] / a.k : p;
    }
    __syncthreads();
    stage_rows<F::NGL>(F::QX, StageSrc{a.in, a.act.q, a.act.scale, a.act.sum, a.K}, rows, min(MT, M - m0), act_lds, row_lds);
    __syncthreads();
    float acc[G][RR][MT];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < RR; ++i)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[g][i][m] = 0.0f;
    const int nvalid = min(MT, M - m0);
    // weights of step st -> buf (zeros outside the row range / past the last chunk)
    auto load_step = [&](int st, uint32_t (&buf)[G][RR][F::NW]) {
      const int grp = slot + (st / NC) * nslots;
      const int c = rl + (st % NC) * L;
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < RR; ++i) {
          const int r = grp * RR + i;
          if (c < C && r < a.rows) {
            F::load((g ? W1 : W0) + (int64_t)r * rb, c, K, buf[g][i]);
          } else {
#pragma unroll
            for (int w = 0; w < F::NW; ++w) buf[g][i][w] = 0u;
          }
        }
    };
    for (int st = 0; st < nsteps; ++st) {
      const int grp = slot + (st / NC) * nslots;
      const int c = rl + (st % NC) * L;
      uint32_t raw[G][RR][F::NW];
      load_step(st, raw);
      if (c < C) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int i = 0; i < RR; ++i) F::template dot_tokens<MT>(raw[g][i], act_lds, row_lds, c, K, nvalid, acc[g][i]);
      }
      if (st % NC == NC - 1) {  // row group complete: reduce over the lane group and write
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int i = 0; i < RR; ++i)
#pragma unroll
            for (int m = 0; m < MT; ++m) {
              float v = acc[g][i][m];
              for (int off = L >> 1; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
              acc[g][i][m] = v;
            }
        if (rl == 0) {
#pragma unroll
          for (int i = 0; i < RR; ++i) {
            const int r = grp * RR + i;
            if (r >= a.rows) continue;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
              if (m >= nvalid) continue;
              const size_t o = (size_t)(p0 + m0 + m) * a.rows + r;
              a.out[o] = GATED ? swiglu(acc[0][i][m], acc[G - 1][i][m]) : acc[0][i][m];
            }
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int i = 0; i < RR; ++i)
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[g][i][m] = 0.0f;
      }
    }
  }
}

constexpr int kProjLdsBytes = 64 * 1024;  // activation rows staged per block

template <int FMT, int RR, bool GATED>
int launch_proj_fmt(const ProjArgs& a, int MT, hipStream_t st) {
  using F = Fmt<FMT>;
  const int C = (a.K + F::CE - 1) / F::CE;
  int L_log2 = 0;
  while ((1 << L_log2) < C && L_log2 < 6) ++L_log2;
  const int slots_per_block = 4 * (64 >> L_log2);
  const int ngroups = (a.rows + RR - 1) / RR;
  // enough blocks to fill the chip (~8 per CU over all segments), each slot walking a few groups
  const int segs = std::max(a.max_segments, 1);
  static const int kTarget = [] { const char* v = std::getenv("EMBER_PROJ_BLOCKS"); return v ? atoi(v) : 2048; }();
  int blocks = (kTarget + segs - 1) / segs;
  blocks = std::min(blocks, (ngroups + slots_per_block - 1) / slots_per_block);
  blocks = std::max(blocks, 1);
  dim3 grid(blocks, a.max_segments);
  if (grid.y == 0) return EMBER_OK;
  const int row_lds = act_lds_bytes(F::QX, a.K);
  while (MT > 1 && MT * row_lds > kProjLdsBytes) MT >>= 1;
  if (row_lds > kProjLdsBytes) return EMBER_ERR_SHAPE;
  const size_t lds = (size_t)MT * row_lds;
  if (MT == 1)
    proj_kernel<FMT, RR, 1, GATED><<<grid, 256, lds, st>>>(a, L_log2);
  else if (MT == 2)
    proj_kernel<FMT, RR, 2, GATED><<<grid, 256, lds, st>>>(a, L_log2);
  else
    proj_kernel<FMT, RR, 4, GATED><<<grid, 256, lds, st>>>(a, L_log2);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

template <bool GATED>
int launch_proj_gated(const ProjArgs& a, int MT, hipStream_t st) {
  switch (a.type) {
    case EMBER_TYPE_F32: return launch_proj_fmt<EMBER_TYPE_F32, 1, GATED>(a, MT, st);
    case EMBER_TYPE_F16: return launch_proj_fmt<EMBER_TYPE_F16, 1, GATED>(a, MT, st);
    case EMBER_TYPE_BF16: return launch_proj_fmt<EMBER_TYPE_BF16, 1, GATED>(a, MT, st);
    case EMBER_TYPE_Q8_0: return launch_proj_fmt<EMBER_TYPE_Q8_0, GATED ? 1 : 2, GATED>(a, MT, st);
    case EMBER_TYPE_Q4_K: return launch_proj_fmt<EMBER_TYPE_Q4_K, GATED ? 1 : 2, GATED>(a, MT, st);
    default: return EMBER_ERR_TYPE;
  }
}

bool type_quantizes_activations(int type) { return type == EMBER_TYPE_Q8_0 || type == EMBER_TYPE_Q4_K; }

int launch_projection(const ProjArgs& a, hipStream_t st) {
  const int MT = a.T <= 1 ? 1 : (a.T <= 2 ? 2 : 4);
  return a.gated ? launch_proj_gated<true>(a, MT, st) : launch_proj_gated<false>(a, MT, st);
}

// Per-32-block int16 quantization of activation rows: q = rint(x / s), s = amax / 32767 (s = 0 for
// an all-zero block), plus the block's sum of q. One thread per block of 32.
__global__ void __launch_bounds__(256) quantize_act_kernel(const float* __restrict__ in, int rows, int K,
                                                           int16_t* __restrict__ q, float* __restrict__ scale,
                                                           int* __restrict__ sum) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int nb = K / 32;
  if (b >= (int64_t)rows * nb) return;
  const float4* p = reinterpret_cast<const float4*>(in + b * 32);
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 t = p[i];
    v[4 * i] = t.x;
    v[4 * i + 1] = t.y;
    v[4 * i + 2] = t.z;
    v[4 * i + 3] = t.w;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const float s = amax / 32767.0f;
  const float inv = amax > 0.0f ? 32767.0f / amax : 0.0f;
  int tot = 0;
  uint32_t packed[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int a0 = (int)__builtin_rintf(v[2 * i] * inv), a1 = (int)__builtin_rintf(v[2 * i + 1] * inv);
    const int c0 = max(-32767, min(32767, a0)), c1 = max(-32767, min(32767, a1));
    tot += c0 + c1;
    packed[i] = (uint32_t)(uint16_t)c0 | ((uint32_t)(uint16_t)c1 << 16);
  }
  u32x4* dst = reinterpret_cast<u32x4*>(q + b * 32);
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[i] = u32x4{packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]};
  scale[b] = s;
  sum[b] = tot;
}

int launch_quantize_act(const float* in, int rows, int K, const ActQ& a, hipStream_t st) {
  const int64_t n = (int64_t)rows * (K / 32);
  if (n <= 0) return EMBER_OK;
  quantize_act_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(in, rows, K, a.q, a.scale, a.sum);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

// out[t][o] = sum over j ascending (= experts ascending) of gate[t][j] * y[pos[t*k+j]][o], starting
// from 0 (utils.cpp:736, 744-747); then (x * scale) + 0 (the IR's affine, graph_ir.cpp:923, 2727)
// and + the shared expert's row (graph_ir.cpp:926-928). One thread per output element.
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ y, const float* __restrict__ gates,
                                                      const int32_t* __restrict__ pos,
                                                      const float* __restrict__ y_shared, float scale, int k, int d,
                                                      float* __restrict__ out) {
  const int t = blockIdx.y;
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= d) return;
  float acc = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int p = pos[(size_t)t * k + j];
    const float g = gates[(size_t)t * k + j];
    if (p >= 0) acc = acc + g * y[(size_t)p * d + o];
  }
  if (scale != 1.0f) acc = acc * scale + 0.0f;
  if (y_shared) acc = acc + y_shared[(size_t)t * d + o];
  out[(size_t)t * d + o] = acc;
}

// The same with four consecutive outputs per thread (d % 4 == 0): 16-byte loads of y rows.
__global__ void __launch_bounds__(256) combine4_kernel(const float* __restrict__ y, const float* __restrict__ gates,
                                                       const int32_t* __restrict__ pos,
                                                       const float* __restrict__ y_shared, float scale, int k, int d,
                                                       float* __restrict__ out) {
  const int t = blockIdx.y;
  const int o = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (o >= d) return;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int p = pos[(size_t)t * k + j];
    const float g = gates[(size_t)t * k + j];
    if (p >= 0) {
      const float4 v = *reinterpret_cast<const float4*>(y + (size_t)p * d + o);
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
    const float4 v = *reinterpret_cast<const float4*>(y_shared + (size_t)t * d + o);
    a0 = a0 + v.x;
    a1 = a1 + v.y;
    a2 = a2 + v.z;
    a3 = a3 + v.w;
  }
  *reinterpret_cast<float4*>(out + (size_t)t * d + o) = make_float4(a0, a1, a2, a3);
}

int launch_combine(const float* y, const float* gates, const int32_t* pos, const float* y_shared, float scale, int T,
                   int k, int d, float* out, hipStream_t st) {
  if (T <= 0) return EMBER_OK;
  if (d % 4 == 0) {
    dim3 grid((d / 4 + 255) / 256, T);
    combine4_kernel<<<grid, 256, 0, st>>>(y, gates, pos, y_shared, scale, k, d, out);
    return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
  }
  dim3 grid((d + 255) / 256, T);
  combine_kernel<<<grid, 256, 0, st>>>(y, gates, pos, y_shared, scale, k, d, out);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

}  // namespace ember_moe
