// Weight-format codecs of the decode kernels: llama.cpp row layouts (F32, F16, BF16, Q8_0, Q4_K)
// split into per-lane 64-element chunks, their dots against activations staged in LDS (f32, or
// int16 per 32-element block for the quantizing formats), and the block-cooperative staging.
// Reference row layouts: ggml-common (block_q8_0, block_q4_K), quantization.cpp:145-155.
#pragma once
#include "moe_internal.hpp"

namespace ember_moe {
using namespace ember_math;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));
typedef short short2_t __attribute__((ext_vector_type(2)));

// Staged activation rows are split into per-lane chunks of 2^NGL 16-byte granules (NGL = 3: 128 B,
// NGL = 4: 256 B). Lane c reads granule i of chunk c while its neighbours read granule i of theirs,
// which at a 128/256-byte stride would fall into the same LDS banks; each chunk's granules are
// therefore stored rotated by a per-chunk amount so that 16 consecutive chunks' granule i occupy all
// 16 bank slots of a 256-byte window.
template <int NGL>
__device__ inline int swz_granule(int c, int i) {
  constexpr int NG = 1 << NGL;
  const int rot = (c >> (4 - NGL)) & (NG - 1);
  return (c << NGL) + ((i + rot) & (NG - 1));
}
template <int NGL>
__device__ inline const uint8_t* lds_granule(const uint8_t* row, int c, int i) {
  return row + 16 * swz_granule<NGL>(c, i);
}
__device__ inline int sdot2(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, a), __builtin_bit_cast(short2_t, b), c, false);
}
// bytes 0,1 (sel 0) or 2,3 (sel 1) of w, zero-extended to two 16-bit lanes
__device__ inline uint32_t u16pair(uint32_t w, int hi) {
  return __builtin_amdgcn_perm(0u, w, hi ? 0x0c030c02u : 0x0c010c00u);
}

__device__ inline void load16(const uint8_t* p, uint32_t* raw) {
  const u32x4 q = *reinterpret_cast<const u32x4*>(p);
  raw[0] = q.x;
  raw[1] = q.y;
  raw[2] = q.z;
  raw[3] = q.w;
}

// Activation operands of one chunk for one token.
struct XF {                 // float activations (F32 / F16 / BF16 weights)
  float v[32];
};

template <int FMT>
struct Fmt;

// F32: chunk = 16 floats = 64 B.
template <>
struct Fmt<EMBER_TYPE_F32> {
  static constexpr int CE = 16, NW = 16, NGL = 2;  // activation chunk: 16 floats = 4 granules
  static constexpr bool QX = false, PLANES = false;
  __host__ __device__ static int64_t row_bytes(int K) { return 4 * (int64_t)K; }
  __device__ static void load(const uint8_t* row, int c, int K, uint32_t* raw) {
    const int n = K - c * CE;  // valid elements (multiple of 4)
#pragma unroll
    for (int v = 0; v < 4; ++v) {  // branch-free: a granule past the row's end reloads granule 0, then zeroes
      const bool ok = 4 * v < n;
      const u32x4 q = *reinterpret_cast<const u32x4*>(row + (size_t)c * 64 + 16 * (ok ? v : 0));
      raw[4 * v] = ok ? q.x : 0u;
      raw[4 * v + 1] = ok ? q.y : 0u;
      raw[4 * v + 2] = ok ? q.z : 0u;
      raw[4 * v + 3] = ok ? q.w : 0u;
    }
  }
  template <int MT>
  __device__ static void dot_tokens(const uint32_t* raw, const uint8_t* lds, int row_lds, int c, int K, int nvalid,
                                    float* out);
  __device__ static float dot(const uint32_t* raw, const XF& x, int) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      a0 = __builtin_fmaf(as_f32(raw[i]), x.v[i], a0);
      a1 = __builtin_fmaf(as_f32(raw[i + 1]), x.v[i + 1], a1);
    }
    return a0 + a1;
  }
};

// BF16 / F16: chunk = 32 halves = 64 B.
template <int FMT>
struct FmtHalf {
  static constexpr int CE = 32, NW = 16, NGL = 3;  // activation chunk: 32 floats = 8 granules
  static constexpr bool QX = false, PLANES = false;
  __host__ __device__ static int64_t row_bytes(int K) { return 2 * (int64_t)K; }
  __device__ static void load(const uint8_t* row, int c, int K, uint32_t* raw) {
    const int n = K - c * CE;  // multiple of 8
#pragma unroll
    for (int v = 0; v < 4; ++v) {  // branch-free: a granule past the row's end reloads granule 0, then zeroes
      const bool ok = 8 * v < n;
      const u32x4 q = *reinterpret_cast<const u32x4*>(row + (size_t)c * 64 + 16 * (ok ? v : 0));
      raw[4 * v] = ok ? q.x : 0u;
      raw[4 * v + 1] = ok ? q.y : 0u;
      raw[4 * v + 2] = ok ? q.z : 0u;
      raw[4 * v + 3] = ok ? q.w : 0u;
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
  template <int MT>
  __device__ static void dot_tokens(const uint32_t* raw, const uint8_t* lds, int row_lds, int c, int K, int nvalid,
                                    float* out);
  __device__ static float dot(const uint32_t* raw, const XF& x, int) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      a0 = __builtin_fmaf(lo(raw[i]), x.v[2 * i], a0);
      a1 = __builtin_fmaf(hi(raw[i]), x.v[2 * i + 1], a1);
    }
    return a0 + a1;
  }
};
template <>
struct Fmt<EMBER_TYPE_BF16> : FmtHalf<EMBER_TYPE_BF16> {};
template <>
struct Fmt<EMBER_TYPE_F16> : FmtHalf<EMBER_TYPE_F16> {};

// Q8_0: chunk = two 34-byte blocks = 68 B = 17 dwords (4-byte aligned when K % 64 == 0).
// Dword 0 = {d_A, q0, q1}; 1..7 = q2..q29; 8 = {q30, q31, d_B}; 9..16 = block B's q0..q31.
template <>
struct Fmt<EMBER_TYPE_Q8_0> {
  static constexpr int CE = 64, NW = 17, NGL = 3;  // activation chunk: 64 int16 = 8 granules
  static constexpr bool QX = true, PLANES = false;
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
  // MT tokens' dots of one chunk; the activation rows are staged in LDS (act_lds_bytes layout).
  // Each weight pair is converted once (q + 128, zero-extended to 16 bits) and used for every token.
  template <int MT>
  __device__ static void dot_tokens(const uint32_t* raw, const uint8_t* lds, int row_lds, int c, int K, int nvalid,
                                    float* out) {
    const float dA = half_bits_to_float(raw[0] & 0xffff);
    const float dB = half_bits_to_float(raw[8] >> 16);
    int ia[MT], ib[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) ia[m] = ib[m] = 0;
#pragma unroll
    for (int j4 = 0; j4 < 16; j4 += 4) {
      uint32_t ua[4], ub[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ua[j] = u16pair(raw[(1 + j4 + j) >> 1] ^ 0x80808080u, (1 + j4 + j) & 1);
        ub[j] = u16pair(raw[9 + ((j4 + j) >> 1)] ^ 0x80808080u, (j4 + j) & 1);
      }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m < nvalid) {
          const uint8_t* xr = lds + m * row_lds;
          const u32x4 xa = *reinterpret_cast<const u32x4*>(lds_granule<3>(xr, c, j4 >> 2));
          const u32x4 xb = *reinterpret_cast<const u32x4*>(lds_granule<3>(xr, c, 4 + (j4 >> 2)));
          ia[m] = sdot2(ua[0], xa.x, ia[m]);
          ia[m] = sdot2(ua[1], xa.y, ia[m]);
          ia[m] = sdot2(ua[2], xa.z, ia[m]);
          ia[m] = sdot2(ua[3], xa.w, ia[m]);
          ib[m] = sdot2(ub[0], xb.x, ib[m]);
          ib[m] = sdot2(ub[1], xb.y, ib[m]);
          ib[m] = sdot2(ub[2], xb.z, ib[m]);
          ib[m] = sdot2(ub[3], xb.w, ib[m]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < nvalid) {
        const uint8_t* xr = lds + m * row_lds;
        const float* sc = reinterpret_cast<const float*>(xr + K * 2) + 2 * c;
        const int* sm = reinterpret_cast<const int*>(xr + K * 2 + (K / 32) * 4) + 2 * c;
        out[m] += dA * (sc[0] * (float)(ia[m] - 128 * sm[0])) + dB * (sc[1] * (float)(ib[m] - 128 * sm[1]));
      }
    }
  }
};

// Q4_K: chunk = one 64-element quarter of a 256-element super-block: the 16-byte header
// {d, dmin, scales[12]} plus the quarter's 32 bytes of nibbles (low: group 2q, high: group 2q+1).
template <>
struct Fmt<EMBER_TYPE_Q4_K> {
  // PLANES: the int16 activations are staged as byte planes (granule: 8 low bytes x & 0xff, then 8 high
  // bytes x >> 8), so the nibbles enter v_dot4 as they are: dot(w, x) = 256 dot4(w, x_hi) + dot4(w, x_lo),
  // exact in int32, instead of being widened to 16-bit pairs for v_dot2
  static constexpr int CE = 64, NW = 12, NGL = 3;
  static constexpr bool QX = true, PLANES = true;
  __host__ __device__ static int64_t row_bytes(int K) { return (int64_t)K / 256 * 144; }
  __device__ static void load(const uint8_t* row, int c, int, uint32_t* raw) {
    const uint8_t* sb = row + (size_t)(c >> 2) * 144;
    load16(sb, raw);
    load16(sb + 16 + 32 * (c & 3), raw + 4);
    load16(sb + 32 + 32 * (c & 3), raw + 8);
  }
  __device__ static int ubyte(const uint32_t* raw, int b) { return (int)((raw[b >> 2] >> (8 * (b & 3))) & 0xff); }
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
  template <int MT>
  __device__ static void dot_tokens(const uint32_t* raw, const uint8_t* lds, int row_lds, int c, int K, int nvalid,
                                    float* out) {
    const float d = half_bits_to_float(raw[0] & 0xffff), dmin = half_bits_to_float(raw[0] >> 16);
    const int q = c & 3;
    int scA, mA, scB, mB;
    scale_min(raw, 2 * q, &scA, &mA);
    scale_min(raw, 2 * q + 1, &scB, &mB);
    int ha[MT], hb[MT];
    uint32_t la[MT], lb[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) ha[m] = hb[m] = 0, la[m] = lb[m] = 0u;
#pragma unroll
    for (int k2 = 0; k2 < 8; k2 += 2) {
      const uint32_t w0 = raw[4 + k2], w1 = raw[5 + k2];
      const uint32_t a0 = w0 & 0x0f0f0f0fu, a1 = w1 & 0x0f0f0f0fu;                // group 2q, 8 elements
      const uint32_t b0 = (w0 >> 4) & 0x0f0f0f0fu, b1 = (w1 >> 4) & 0x0f0f0f0fu;  // group 2q + 1
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m < nvalid) {
          const uint8_t* xr = lds + m * row_lds;
          const u32x4 xa = *reinterpret_cast<const u32x4*>(lds_granule<3>(xr, c, k2 >> 1));
          const u32x4 xb = *reinterpret_cast<const u32x4*>(lds_granule<3>(xr, c, 4 + (k2 >> 1)));
          la[m] = __builtin_amdgcn_udot4(a0, xa.x, la[m], false);
          la[m] = __builtin_amdgcn_udot4(a1, xa.y, la[m], false);
          ha[m] = __builtin_amdgcn_sdot4((int)a0, (int)xa.z, ha[m], false);
          ha[m] = __builtin_amdgcn_sdot4((int)a1, (int)xa.w, ha[m], false);
          lb[m] = __builtin_amdgcn_udot4(b0, xb.x, lb[m], false);
          lb[m] = __builtin_amdgcn_udot4(b1, xb.y, lb[m], false);
          hb[m] = __builtin_amdgcn_sdot4((int)b0, (int)xb.z, hb[m], false);
          hb[m] = __builtin_amdgcn_sdot4((int)b1, (int)xb.w, hb[m], false);
        }
      }
    }
    int ia[MT], ib[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      ia[m] = 256 * ha[m] + (int)la[m];
      ib[m] = 256 * hb[m] + (int)lb[m];
    }
    const float dA = d * (float)scA, mAf = dmin * (float)mA, dB = d * (float)scB, mBf = dmin * (float)mB;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < nvalid) {
        const uint8_t* xr = lds + m * row_lds;
        const float* sc = reinterpret_cast<const float*>(xr + K * 2) + 2 * c;
        const int* sm = reinterpret_cast<const int*>(xr + K * 2 + (K / 32) * 4) + 2 * c;
        out[m] += sc[0] * (dA * (float)ia[m] - mAf * (float)sm[0]) + sc[1] * (dB * (float)ib[m] - mBf * (float)sm[1]);
      }
    }
  }
};

// Bytes of one token's activation row as staged in LDS: f32 values (padded to whole 64-element
// chunks, so that a partial last chunk's rotated granules stay inside the row), or int16 values
// followed by the per-32-block scales and sums.
__host__ __device__ inline int act_lds_bytes(bool qx, int K) { return qx ? K * 2 + (K / 32) * 8 : (K + 63) / 64 * 256; }

// Block-cooperative copy of the activation rows rows[0..nrows) into consecutive LDS slots of
// row_lds bytes (16-byte granules; values rotated per chunk, then the per-block scales and sums).
// All rows' loads are issued in one batch per thread before any store, so staging costs about one
// memory latency instead of one per row and section.
struct StageSrc {
  const float* in;      // f32 rows [*][K] (float formats)
  const int16_t* q;     // int16 rows [*][K] + per-32-block scales / sums (quantizing formats)
  const float* scale;
  const int* sum;
  int K;
};

template <int NGL>
__device__ inline void stage_rows(bool qx, const StageSrc& a, const int* rows, int nrows, uint8_t* lds, int row_lds) {
  typedef uint32_t v4 __attribute__((ext_vector_type(4)));
  const int K = a.K;
  const int nq = qx ? K / 8 : K / 4;  // granules of values per row
  const int nb = K / 32;
  const bool sg = qx && nb % 4 == 0;  // scales and sums start on 16-byte boundaries
  const int per = nq + (sg ? nb / 2 : 0);
  const int n = nrows * per;
  const int stride = blockDim.x;
  for (int base = threadIdx.x; base < n; base += 8 * stride) {
    v4 t[8];
    int dst[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {  // branch-free address math: every load is issued before any store
      const int gi = min(base + u * stride, n - 1);
      const int m = gi / per, r = gi - m * per;
      const size_t row = (size_t)rows[m];
      const bool val = r < nq, isc = !val && r < nq + nb / 4;
      const int rs = val ? r : isc ? r - nq : r - nq - nb / 4;
      const uint8_t* base_p = val ? (qx ? reinterpret_cast<const uint8_t*>(a.q + row * K)
                                        : reinterpret_cast<const uint8_t*>(a.in + row * K))
                                  : isc ? reinterpret_cast<const uint8_t*>(a.scale + row * nb)
                                        : reinterpret_cast<const uint8_t*>(a.sum + row * nb);
      t[u] = *reinterpret_cast<const v4*>(base_p + 16 * rs);
      dst[u] = m * row_lds + (val ? 16 * swz_granule<NGL>(r >> NGL, r & ((1 << NGL) - 1))
                                  : K * 2 + (isc ? 0 : nb * 4) + 16 * rs);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (base + u * stride < n) *reinterpret_cast<v4*>(lds + dst[u]) = t[u];
  }
  if (qx && !sg) {
    for (int i = threadIdx.x; i < nrows * nb; i += stride) {
      const int m = i / nb, b = i - m * nb;
      const size_t row = (size_t)rows[m];
      reinterpret_cast<float*>(lds + m * row_lds + K * 2)[b] = a.scale[row * nb + b];
      reinterpret_cast<int*>(lds + m * row_lds + K * 2 + nb * 4)[b] = a.sum[row * nb + b];
    }
  }
}

// Per-32-element-block int16 quantization of one block of activations, the values quantize_act_kernel
// writes: s = amax / 32767, q = rint(x * (32767 / amax)) clamped to +-32767 (q = 0, s = 0 for an
// all-zero block), plus the block's sum of q.
__device__ inline void load_block32(const float* src, float* v) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 t = reinterpret_cast<const float4*>(src)[i];
    v[4 * i] = t.x;
    v[4 * i + 1] = t.y;
    v[4 * i + 2] = t.z;
    v[4 * i + 3] = t.w;
  }
}
// 32 values (in registers) -> int16 pairs, scale, sum
__device__ inline void quant_block32_v(const float* v, uint32_t* packed, float* scale, int* sum) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const float inv = amax > 0.0f ? 32767.0f / amax : 0.0f;
  int tot = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int a0 = (int)__builtin_rintf(v[2 * i] * inv), a1 = (int)__builtin_rintf(v[2 * i + 1] * inv);
    const int c0 = max(-32767, min(32767, a0)), c1 = max(-32767, min(32767, a1));
    tot += c0 + c1;
    packed[i] = (uint32_t)(uint16_t)c0 | ((uint32_t)(uint16_t)c1 << 16);
  }
  *scale = amax / 32767.0f;
  *sum = tot;
}
__device__ inline void quant_block32(const float* src, uint32_t* packed, float* scale, int* sum) {
  float v[32];
  load_block32(src, v);
  quant_block32_v(v, packed, scale, sum);
}

// Stages f32 activation rows rows[0..nrows) of [*][K] into LDS already quantized (act_lds_bytes
// layout for the quantizing formats: int16 values in rotated 64-element chunks, then the per-block
// scales, then the per-block sums). One thread per 32-element block.
// One block's store into the staged row (act_lds_bytes layout), from its quantized values.
template <bool PLANES = false>
__device__ inline void store_block_quant(const uint32_t* packed, float sc, int sm, int b, int K, uint8_t* row) {
  const int nb = K / 32;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    u32x4 gr{packed[4 * g], packed[4 * g + 1], packed[4 * g + 2], packed[4 * g + 3]};
    if constexpr (PLANES) {
      gr = u32x4{__builtin_amdgcn_perm(gr.y, gr.x, 0x06040200u), __builtin_amdgcn_perm(gr.w, gr.z, 0x06040200u),
                 __builtin_amdgcn_perm(gr.y, gr.x, 0x07050301u), __builtin_amdgcn_perm(gr.w, gr.z, 0x07050301u)};
    }
    *reinterpret_cast<u32x4*>(row + 16 * swz_granule<3>(b >> 1, (b & 1) * 4 + g)) = gr;
  }
  reinterpret_cast<float*>(row + K * 2)[b] = sc;
  reinterpret_cast<int*>(row + K * 2 + nb * 4)[b] = sm;
}

template <bool PLANES = false>
__device__ inline void stage_rows_quant(const float* in, int K, const int* rows, int nrows, uint8_t* lds, int row_lds) {
  const int nb = K / 32;
  const int n = nrows * nb;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int m = i / nb, b = i - m * nb;
    uint32_t packed[16];
    float sc;
    int sm;
    quant_block32(in + (size_t)rows[m] * K + (size_t)b * 32, packed, &sc, &sm);
    uint8_t* row = lds + m * row_lds;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x4 gr{packed[4 * g], packed[4 * g + 1], packed[4 * g + 2], packed[4 * g + 3]};
      if constexpr (PLANES) {
        // eight int16 (pairs in .x .. .w) -> eight low bytes, then eight high bytes
        gr = u32x4{__builtin_amdgcn_perm(gr.y, gr.x, 0x06040200u), __builtin_amdgcn_perm(gr.w, gr.z, 0x06040200u),
                   __builtin_amdgcn_perm(gr.y, gr.x, 0x07050301u), __builtin_amdgcn_perm(gr.w, gr.z, 0x07050301u)};
      }
      *reinterpret_cast<u32x4*>(row + 16 * swz_granule<3>(b >> 1, (b & 1) * 4 + g)) = gr;
    }
    reinterpret_cast<float*>(row + K * 2)[b] = sc;
    reinterpret_cast<int*>(row + K * 2 + nb * 4)[b] = sm;
  }
}

// Stages f32 activation rows rows[0..nrows) of [*][K] into LDS in rotated chunks of 2^NGL granules
// (float formats). Four granules per thread are loaded before any is stored.
template <int NGL>
__device__ inline void stage_rows_f32(const float* in, int K, const int* rows, int nrows, uint8_t* lds, int row_lds) {
  const int nq = K / 4, n = nrows * nq;
  const int stride = blockDim.x;
  for (int base = threadIdx.x; base < n; base += 4 * stride) {
    u32x4 t[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(base + u * stride, n - 1);
      const int m = i / nq, r = i - m * nq;
      t[u] = *reinterpret_cast<const u32x4*>(in + (size_t)rows[m] * K + 4 * r);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = base + u * stride;
      if (i < n) {
        const int m = i / nq, r = i - m * nq;
        *reinterpret_cast<u32x4*>(lds + m * row_lds + 16 * swz_granule<NGL>(r >> NGL, r & ((1 << NGL) - 1))) = t[u];
      }
    }
  }
}

// Activation operands of chunk c (element offset c*CE) from a staged row.
template <int FMT>
__device__ inline void lds_xf(const uint8_t* row, int c, int K, XF& x) {
  constexpr int CE = Fmt<FMT>::CE;
  constexpr int NGL = Fmt<FMT>::NGL;
  const int n = K - c * CE;
#pragma unroll
  for (int v = 0; v < CE / 4; ++v) {
    // rows are padded to whole 64-element chunks, so the read stays in the row; the tail reads zero
    const bool ok = 4 * v < n;
    const float4 q = *reinterpret_cast<const float4*>(lds_granule<NGL>(row, c, v));
    x.v[4 * v] = ok ? q.x : 0.0f;
    x.v[4 * v + 1] = ok ? q.y : 0.0f;
    x.v[4 * v + 2] = ok ? q.z : 0.0f;
    x.v[4 * v + 3] = ok ? q.w : 0.0f;
  }
}
// dot_tokens for the float formats: decode the chunk once per token from the staged f32 rows.
template <int FMT, int MT>
__device__ inline void dot_tokens_f(const uint32_t* raw, const uint8_t* lds, int row_lds, int c, int K, int nvalid,
                                    float* out);
template <int MT>
__device__ void Fmt<EMBER_TYPE_F32>::dot_tokens(const uint32_t* raw, const uint8_t* lds, int row_lds, int c, int K,
                                                int nvalid, float* out) {
  dot_tokens_f<EMBER_TYPE_F32, MT>(raw, lds, row_lds, c, K, nvalid, out);
}
template <int FMT>
template <int MT>
__device__ void FmtHalf<FMT>::dot_tokens(const uint32_t* raw, const uint8_t* lds, int row_lds, int c, int K,
                                         int nvalid, float* out) {
  dot_tokens_f<FMT, MT>(raw, lds, row_lds, c, K, nvalid, out);
}
template <int FMT, int MT>
__device__ inline void dot_tokens_f(const uint32_t* raw, const uint8_t* lds, int row_lds, int c, int K, int nvalid,
                                    float* out) {
  constexpr int CE = Fmt<FMT>::CE;
  constexpr int NGL = Fmt<FMT>::NGL;
  const int n = K - c * CE;
  float a0[MT], a1[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) a0[m] = a1[m] = 0.0f;
#pragma unroll
  for (int v = 0; v < CE / 4; ++v) {
    float w[4];
    if constexpr (FMT == EMBER_TYPE_F32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = as_f32(raw[4 * v + i]);
    } else {
      w[0] = Fmt<FMT>::lo(raw[2 * v]);
      w[1] = Fmt<FMT>::hi(raw[2 * v]);
      w[2] = Fmt<FMT>::lo(raw[2 * v + 1]);
      w[3] = Fmt<FMT>::hi(raw[2 * v + 1]);
    }
    // rows are padded to whole 64-element chunks, so the read stays in the row; the tail reads zero
    const bool ok = 4 * v < n;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < nvalid) {
        const float4 q = *reinterpret_cast<const float4*>(lds_granule<NGL>(lds + m * row_lds, c, v));
        a0[m] = __builtin_fmaf(w[0], ok ? q.x : 0.0f, a0[m]);
        a1[m] = __builtin_fmaf(w[1], ok ? q.y : 0.0f, a1[m]);
        a0[m] = __builtin_fmaf(w[2], ok ? q.z : 0.0f, a0[m]);
        a1[m] = __builtin_fmaf(w[3], ok ? q.w : 0.0f, a1[m]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m)
    if (m < nvalid) out[m] += a0[m] + a1[m];
}

__device__ inline float swiglu(float g, float u) { return g * (1.0f / (1.0f + expf_glibc(-g))) * u; }

}  // namespace ember_moe
