// Expert projections of the MoE FFN for decode-sized segments: a bandwidth kernel that streams each
// selected expert's rows once, dequantizes the llama.cpp blocks in registers and reduces across
// lanes with cross-lane shuffles. Also the ordered combine.
//
// Reference semantics (utils.cpp:735-747): per selected expert, g = W_gate x, u = W_up x,
// h = g * (1/(1+expf(-g))) * u, y = W_down h, out = sum over experts ascending of gate * y.
// The reference evaluates these as FP64 dots over F32 weights dequantized at load
// (weight_management.cpp:802-877); here each dot accumulates in FP32 over the dequantized values,
// which keeps F32 layers within 1e-4 max-abs and quantized layers within 2e-3 rel-L2.
//
// Work layout: a lane owns one 32- or 64-element "chunk" of a row (chunk c of row r sits at a fixed
// byte offset in the ggml row). L lanes (a power of two <= 64, L >= chunks per row when possible)
// cover a row, so one wave covers 64/L rows at once; each thread keeps RR rows (x2 for gate/up)
// in flight. A block is 4 waves; grid.x tiles the rows, grid.y the expert segments (experts that
// received tokens, from the dispatch step), so no host synchronisation is needed.
#include "moe_internal.hpp"

namespace ember_moe {
using namespace ember_math;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));

template <int FMT>
struct Fmt;

// F32: chunk = 32 floats = 128 B.
template <>
struct Fmt<EMBER_TYPE_F32> {
  static constexpr int CE = 32, NW = 32;
  __host__ __device__ static int64_t row_bytes(int K) { return 4 * (int64_t)K; }
  __device__ static void load(const uint8_t* row, int c, int K, uint32_t* raw) {
    const u32x4* p = reinterpret_cast<const u32x4*>(row + (size_t)c * 128);
    const int n = K - c * CE;  // valid elements in this chunk (multiple of 4)
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      u32x4 q = (4 * v < n) ? p[v] : u32x4{0, 0, 0, 0};
      raw[4 * v] = q.x;
      raw[4 * v + 1] = q.y;
      raw[4 * v + 2] = q.z;
      raw[4 * v + 3] = q.w;
    }
  }
  __device__ static float dot(const uint32_t* raw, const float* x, int) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
      a0 = __builtin_fmaf(as_f32(raw[i]), x[i], a0);
      a1 = __builtin_fmaf(as_f32(raw[i + 1]), x[i + 1], a1);
    }
    return a0 + a1;
  }
};

// BF16 / F16: chunk = 64 halves = 128 B.
template <int FMT>
struct FmtHalf {
  static constexpr int CE = 64, NW = 32;
  __host__ __device__ static int64_t row_bytes(int K) { return 2 * (int64_t)K; }
  __device__ static void load(const uint8_t* row, int c, int K, uint32_t* raw) {
    const u32x4* p = reinterpret_cast<const u32x4*>(row + (size_t)c * 128);
    const int n = K - c * CE;  // multiple of 8
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      u32x4 q = (8 * v < n) ? p[v] : u32x4{0, 0, 0, 0};
      raw[4 * v] = q.x;
      raw[4 * v + 1] = q.y;
      raw[4 * v + 2] = q.z;
      raw[4 * v + 3] = q.w;
    }
  }
  __device__ static float lo(uint32_t w) {
    if (FMT == EMBER_TYPE_BF16) return as_f32(w << 16);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffff));
  }
  __device__ static float hi(uint32_t w) {
    if (FMT == EMBER_TYPE_BF16) return as_f32(w & 0xffff0000u);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  __device__ static float dot(const uint32_t* raw, const float* x, int) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      a0 = __builtin_fmaf(lo(raw[i]), x[2 * i], a0);
      a1 = __builtin_fmaf(hi(raw[i]), x[2 * i + 1], a1);
    }
    return a0 + a1;
  }
};
template <>
struct Fmt<EMBER_TYPE_BF16> : FmtHalf<EMBER_TYPE_BF16> {};
template <>
struct Fmt<EMBER_TYPE_F16> : FmtHalf<EMBER_TYPE_F16> {};

__device__ inline int sbyte(const uint32_t* raw, int b) { return (int)(int8_t)((raw[b >> 2] >> (8 * (b & 3))) & 0xff); }
__device__ inline int ubyte(const uint32_t* raw, int b) { return (int)((raw[b >> 2] >> (8 * (b & 3))) & 0xff); }

// Q8_0: chunk = two 34-byte blocks = 68 B = 17 dwords (4-byte aligned when K % 64 == 0).
template <>
struct Fmt<EMBER_TYPE_Q8_0> {
  static constexpr int CE = 64, NW = 17;
  __host__ __device__ static int64_t row_bytes(int K) { return (int64_t)K / 32 * 34; }
  __device__ static void load(const uint8_t* row, int c, int, uint32_t* raw) {
    const uint8_t* p = row + (size_t)c * 68;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 q = *reinterpret_cast<const u32x4_a4*>(p + 16 * v);
      raw[4 * v] = q.x;
      raw[4 * v + 1] = q.y;
      raw[4 * v + 2] = q.z;
      raw[4 * v + 3] = q.w;
    }
    raw[16] = *reinterpret_cast<const uint32_t*>(p + 64);
  }
  __device__ static float dot(const uint32_t* raw, const float* x, int) {
    const float dA = half_bits_to_float(raw[0] & 0xffff);
    const float dB = half_bits_to_float(raw[8] >> 16);
    float sA = 0.0f, sB = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      sA = __builtin_fmaf((float)sbyte(raw, 2 + j), x[j], sA);
      sB = __builtin_fmaf((float)sbyte(raw, 36 + j), x[32 + j], sB);
    }
    return dA * sA + dB * sB;
  }
};

// Q4_K: chunk = one 64-element quarter of a 256-element super-block: the 16-byte header
// {d, dmin, scales[12]} plus the quarter's 32 bytes of nibbles (low: group 2q, high: group 2q+1).
template <>
struct Fmt<EMBER_TYPE_Q4_K> {
  static constexpr int CE = 64, NW = 12;
  __host__ __device__ static int64_t row_bytes(int K) { return (int64_t)K / 256 * 144; }
  __device__ static void load(const uint8_t* row, int c, int, uint32_t* raw) {
    const uint8_t* sb = row + (size_t)(c >> 2) * 144;
    const u32x4 h = *reinterpret_cast<const u32x4*>(sb);
    const u32x4 q0 = *reinterpret_cast<const u32x4*>(sb + 16 + 32 * (c & 3));
    const u32x4 q1 = *reinterpret_cast<const u32x4*>(sb + 32 + 32 * (c & 3));
    raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
    raw[4] = q0.x; raw[5] = q0.y; raw[6] = q0.z; raw[7] = q0.w;
    raw[8] = q1.x; raw[9] = q1.y; raw[10] = q1.z; raw[11] = q1.w;
  }
  // get_scale_min_k4 (quantization.cpp:145-155) on the 12 scale bytes (header bytes 4..15).
  __device__ static void scale_min(const uint32_t* raw, int j, int* sc, int* mn) {
    if (j < 4) {
      *sc = ubyte(raw, 4 + j) & 63;
      *mn = ubyte(raw, 8 + j) & 63;
    } else {
      *sc = (ubyte(raw, 8 + j) & 0xf) | ((ubyte(raw, j) >> 6) << 4);
      *mn = (ubyte(raw, 8 + j) >> 4) | ((ubyte(raw, 4 + j) >> 6) << 4);
    }
  }
  __device__ static float dot(const uint32_t* raw, const float* x, int c) {
    const float d = half_bits_to_float(raw[0] & 0xffff), dmin = half_bits_to_float(raw[0] >> 16);
    const int q = c & 3;
    int scA, mA, scB, mB;
    scale_min(raw, 2 * q, &scA, &mA);
    scale_min(raw, 2 * q + 1, &scB, &mB);
    float sA = 0.0f, sB = 0.0f, xA = 0.0f, xB = 0.0f;
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      const uint32_t byte = (raw[4 + (l >> 2)] >> (8 * (l & 3))) & 0xff;
      sA = __builtin_fmaf((float)(byte & 0xf), x[l], sA);
      sB = __builtin_fmaf((float)(byte >> 4), x[32 + l], sB);
      xA += x[l];
      xB += x[32 + l];
    }
    return (d * (float)scA) * sA - (dmin * (float)mA) * xA + (d * (float)scB) * sB - (dmin * (float)mB) * xB;
  }
};

template <int FMT>
__device__ inline void load_x(const float* row, int c, int K, float* xv) {
  constexpr int CE = Fmt<FMT>::CE;
  const float4* p = reinterpret_cast<const float4*>(row + (size_t)c * CE);
  const int n = K - c * CE;
#pragma unroll
  for (int v = 0; v < CE / 4; ++v) {
    const float4 q = (4 * v < n) ? p[v] : make_float4(0.f, 0.f, 0.f, 0.f);
    xv[4 * v] = q.x;
    xv[4 * v + 1] = q.y;
    xv[4 * v + 2] = q.z;
    xv[4 * v + 3] = q.w;
  }
}

__device__ inline float swiglu(float g, float u) { return g * (1.0f / (1.0f + expf_glibc(-g))) * u; }

template <int FMT, int RR, int MT, bool GATED>
__global__ void __launch_bounds__(256) proj_kernel(ProjArgs a, int L_log2) {
  using F = Fmt<FMT>;
  constexpr int G = GATED ? 2 : 1;
  const int L = 1 << L_log2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane >> L_log2, rl = lane & (L - 1);
  const int rows_per_wave = 64 >> L_log2;
  const int RPW = 4 * rows_per_wave;
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
  const uint8_t* W[2];
  W[0] = static_cast<const uint8_t*>(a.w0) + (int64_t)e * a.expert_stride;
  W[1] = GATED ? static_cast<const uint8_t*>(a.w1) + (int64_t)e * a.expert_stride : W[0];
  int row[RR];
#pragma unroll
  for (int i = 0; i < RR; ++i) row[i] = blockIdx.x * (RPW * RR) + wave * rows_per_wave + sub + RPW * i;

  for (int m0 = 0; m0 < M; m0 += MT) {
    float acc[G][RR][MT];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < RR; ++i)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[g][i][m] = 0.0f;
    int in_row[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int p = p0 + m0 + m;
      in_row[m] = (m0 + m < M) ? (a.in_by_perm ? a.perm[p] / a.k : p) : 0;
    }
    for (int c = rl; c < C; c += L) {
      uint32_t raw[G][RR][F::NW];
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < RR; ++i) {
          if (row[i] < a.rows) {
            F::load(W[g] + (int64_t)row[i] * rb, c, K, raw[g][i]);
          } else {
#pragma unroll
            for (int w = 0; w < F::NW; ++w) raw[g][i][w] = 0u;
          }
        }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m0 + m < M) {
          float xv[F::CE];
          load_x<FMT>(a.in + (size_t)in_row[m] * K, c, K, xv);
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < RR; ++i) acc[g][i][m] += F::dot(raw[g][i], xv, c);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < RR; ++i)
#pragma unroll
        for (int m = 0; m < MT; ++m)
          for (int off = L >> 1; off >= 1; off >>= 1) acc[g][i][m] += __shfl_xor(acc[g][i][m], off, 64);
    if (rl == 0) {
#pragma unroll
      for (int i = 0; i < RR; ++i) {
        if (row[i] >= a.rows) continue;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (m0 + m >= M) continue;
          const size_t o = (size_t)(p0 + m0 + m) * a.rows + row[i];
          a.out[o] = GATED ? swiglu(acc[0][i][m], acc[G - 1][i][m]) : acc[0][i][m];
        }
      }
    }
  }
}

template <int FMT, int RR, bool GATED>
int launch_proj_fmt(const ProjArgs& a, int MT, hipStream_t st) {
  using F = Fmt<FMT>;
  const int C = (a.K + F::CE - 1) / F::CE;
  int L_log2 = 0;
  while ((1 << L_log2) < C && L_log2 < 6) ++L_log2;
  const int RPW = 4 * (64 >> L_log2);
  dim3 grid((a.rows + RPW * RR - 1) / (RPW * RR), a.max_segments);
  if (grid.y == 0) return EMBER_OK;
  if (MT == 1)
    proj_kernel<FMT, RR, 1, GATED><<<grid, 256, 0, st>>>(a, L_log2);
  else if (MT == 2)
    proj_kernel<FMT, RR, 2, GATED><<<grid, 256, 0, st>>>(a, L_log2);
  else
    proj_kernel<FMT, RR, 4, GATED><<<grid, 256, 0, st>>>(a, L_log2);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

template <bool GATED>
int launch_proj_gated(const ProjArgs& a, int MT, hipStream_t st) {
  constexpr int RR = GATED ? 2 : 4;
  switch (a.type) {
    case EMBER_TYPE_F32: return launch_proj_fmt<EMBER_TYPE_F32, GATED ? 1 : 2, GATED>(a, MT, st);
    case EMBER_TYPE_F16: return launch_proj_fmt<EMBER_TYPE_F16, RR, GATED>(a, MT, st);
    case EMBER_TYPE_BF16: return launch_proj_fmt<EMBER_TYPE_BF16, RR, GATED>(a, MT, st);
    case EMBER_TYPE_Q8_0: return launch_proj_fmt<EMBER_TYPE_Q8_0, RR, GATED>(a, MT, st);
    case EMBER_TYPE_Q4_K: return launch_proj_fmt<EMBER_TYPE_Q4_K, RR, GATED>(a, MT, st);
    default: return EMBER_ERR_TYPE;
  }
}

int launch_projection(const ProjArgs& a, hipStream_t st) {
  const int MT = a.T <= 1 ? 1 : (a.T <= 2 ? 2 : 4);
  return a.gated ? launch_proj_gated<true>(a, MT, st) : launch_proj_gated<false>(a, MT, st);
}

// out[t][o] = sum over j ascending (= experts ascending) of gate[t][j] * y[pos[t*k+j]][o], starting
// from 0 (utils.cpp:736, 744-747); then (x * scale) + 0 (the IR's affine, graph_ir.cpp:923, 2727)
// and + the shared expert's row (graph_ir.cpp:926-928).
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ y, const float* __restrict__ gates,
                                                      const int32_t* __restrict__ pos,
                                                      const float* __restrict__ y_shared, float scale, int k, int d,
                                                      float* __restrict__ out) {
  const int t = blockIdx.x;
  for (int o = threadIdx.x; o < d; o += blockDim.x) {
    float acc = 0.0f;
    for (int j = 0; j < k; ++j) {
      const int p = pos[(size_t)t * k + j];
      if (p >= 0) acc = acc + gates[(size_t)t * k + j] * y[(size_t)p * d + o];
    }
    if (scale != 1.0f) acc = acc * scale + 0.0f;
    if (y_shared) acc = acc + y_shared[(size_t)t * d + o];
    out[(size_t)t * d + o] = acc;
  }
}

int launch_combine(const float* y, const float* gates, const int32_t* pos, const float* y_shared, float scale, int T,
                   int k, int d, float* out, hipStream_t st) {
  if (T <= 0) return EMBER_OK;
  combine_kernel<<<T, 256, 0, st>>>(y, gates, pos, y_shared, scale, k, d, out);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

}  // namespace ember_moe
