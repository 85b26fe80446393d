// Host-side data utilities for the MoE layer: a counter-based seeded normal generator, fp16/bf16
// encoders and llama.cpp-layout block quantizers (Q8_0, Q4_K). These produce the synthetic expert
// stacks that the benchmark and the tests feed to the HIP path; the reference consumes the same
// byte layouts (quantization.h:58-63 block_q4_K, :137-140 block_q8_0).
#include "ember_moe_host.h"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace {

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

// Element i of stream (seed, stream): Box-Muller on two hashed 53-bit uniforms of the pair i/2;
// even i take the cosine branch, odd i the sine branch. Pure function of (seed, stream, i), so any
// slice can be generated independently and in parallel.
inline double normal_at(uint64_t key, int64_t i) {
  const uint64_t p = (uint64_t)(i >> 1);
  const uint64_t a = mix64(key + (2 * p + 1) * 0x9E3779B97F4A7C15ULL);
  const uint64_t b = mix64(key + (2 * p + 2) * 0x9E3779B97F4A7C15ULL);
  const double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;  // (0, 1]
  const double u2 = (double)(b >> 11) * 0x1.0p-53;        // [0, 1)
  const double r = std::sqrt(-2.0 * std::log(u1));
  const double ang = 6.283185307179586 * u2;
  return (i & 1) ? r * std::sin(ang) : r * std::cos(ang);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
  return mix64(seed ^ mix64(stream * 0xD1B54A32D192ED03ULL + 0x632BE59BD9B4E019ULL));
}

// IEEE binary32 -> binary16, round to nearest even, overflow to Inf, NaN kept quiet.
uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return sign | (ax > 0x7f800000u ? 0x7e00 : 0x7c00);
  if (ax >= 0x477ff000u) return sign | 0x7c00;  // rounds to >= 65520 -> Inf
  if (ax < 0x38800000u) {                       // result subnormal or zero
    if (ax < 0x33000000u) return sign;          // < 2^-25 rounds to 0
    const uint32_t e = ax >> 23;
    const uint32_t m = (ax & 0x7fffff) | 0x800000;
    const int shift = 126 - (int)e;             // value = m * 2^(e-150); target unit 2^-24
    const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    return sign | (uint16_t)(q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0));
  }
  const uint32_t e = (ax >> 23) - 112;
  uint32_t m = ax & 0x7fffff;
  uint32_t h = (e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) ++h;
  return sign | (uint16_t)h;
}

uint16_t f32_to_bf16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40);
  x += 0x7fffu + ((x >> 16) & 1);
  return (uint16_t)(x >> 16);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      int s = 0;
      while (!(m & 0x400)) { m <<= 1; ++s; }
      bits = sign | ((uint32_t)(113 - s) << 23) | ((m & 0x3ff) << 13);
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

// One Q8_0 block (ggml's published scheme): d = amax / 127 stored as fp16, q = round(x / d).
void quant_q8_0_block(const float* x, uint8_t* out) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const uint16_t dh = f32_to_f16(d);
  std::memcpy(out, &dh, 2);
  for (int i = 0; i < 32; ++i) {
    const float v = std::round(x[i] * id);
    out[2 + i] = (uint8_t)(int8_t)std::max(-127.0f, std::min(127.0f, v));
  }
}

// One Q4_K super-block in ggml's layout: {fp16 d, fp16 dmin, 12 bytes of packed 6-bit (scale, min)
// pairs for the 8 groups of 32, 128 bytes of nibbles}; group g's element l is y = d*sc_g*q - dmin*m_g.
// Scales come from each group's range (min clamped to <= 0), then every element is re-quantized
// against the reconstructed 6-bit scale and min, which keeps the error within one step per element.
void quant_q4_k_block(const float* x, uint8_t* out) {
  float gscale[8], gmin[8];
  for (int g = 0; g < 8; ++g) {
    float lo = x[32 * g], hi = x[32 * g];
    for (int l = 1; l < 32; ++l) {
      lo = std::min(lo, x[32 * g + l]);
      hi = std::max(hi, x[32 * g + l]);
    }
    lo = std::min(lo, 0.0f);
    gscale[g] = (hi - lo) / 15.0f;
    gmin[g] = -lo;
  }
  float smax = 0.0f, mmax = 0.0f;
  for (int g = 0; g < 8; ++g) {
    smax = std::max(smax, gscale[g]);
    mmax = std::max(mmax, gmin[g]);
  }
  const uint16_t dh = f32_to_f16(smax / 63.0f), mh = f32_to_f16(mmax / 63.0f);
  const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
  uint8_t sc[8], mn[8];
  for (int g = 0; g < 8; ++g) {
    // Round the scale up so the group's range still fits in 15 steps.
    int s = d > 0.0f ? (int)std::ceil(gscale[g] / d) : 0;
    int m = dmin > 0.0f ? (int)std::lround(gmin[g] / dmin) : 0;
    sc[g] = (uint8_t)std::min(63, std::max(0, s));
    mn[g] = (uint8_t)std::min(63, std::max(0, m));
  }
  std::memcpy(out, &dh, 2);
  std::memcpy(out + 2, &mh, 2);
  uint8_t* s = out + 4;
  for (int j = 0; j < 4; ++j) {
    s[j] = (uint8_t)((sc[j] & 0x3f) | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = (uint8_t)((mn[j] & 0x3f) | ((mn[j + 4] >> 4) << 6));
    s[j + 8] = (uint8_t)((sc[j + 4] & 0x0f) | ((mn[j + 4] & 0x0f) << 4));
  }
  uint8_t q[256];
  for (int g = 0; g < 8; ++g) {
    const float ds = d * (float)sc[g], ms = dmin * (float)mn[g];
    for (int l = 0; l < 32; ++l) {
      int v = ds > 0.0f ? (int)std::lround((x[32 * g + l] + ms) / ds) : 0;
      q[32 * g + l] = (uint8_t)std::min(15, std::max(0, v));
    }
  }
  uint8_t* qs = out + 16;
  for (int c = 0; c < 4; ++c)
    for (int l = 0; l < 32; ++l) qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

}  // namespace

extern "C" {

void ember_fill_normal(float* out, int64_t n, uint64_t seed, uint64_t stream, float mean, float stddev) {
  const uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = (float)(mean + stddev * normal_at(key, i));
}

int64_t ember_row_bytes(int type, int64_t n) {
  switch (type) {
    case EMBER_TYPE_F32: return 4 * n;
    case EMBER_TYPE_F16:
    case EMBER_TYPE_BF16: return 2 * n;
    case EMBER_TYPE_Q8_0: return n % 32 ? -1 : n / 32 * 34;
    case EMBER_TYPE_Q4_K: return n % 256 ? -1 : n / 256 * 144;
    default: return -1;
  }
}

int ember_quantize(int type, const float* x, int64_t n, void* out) {
  uint8_t* o = static_cast<uint8_t*>(out);
  switch (type) {
    case EMBER_TYPE_F32:
      std::memcpy(o, x, 4 * (size_t)n);
      return 0;
    case EMBER_TYPE_F16:
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < n; ++i) {
        const uint16_t h = f32_to_f16(x[i]);
        std::memcpy(o + 2 * i, &h, 2);
      }
      return 0;
    case EMBER_TYPE_BF16:
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < n; ++i) {
        const uint16_t h = f32_to_bf16(x[i]);
        std::memcpy(o + 2 * i, &h, 2);
      }
      return 0;
    case EMBER_TYPE_Q8_0:
      if (n % 32) return EMBER_ERR_SHAPE;
#pragma omp parallel for schedule(static)
      for (int64_t b = 0; b < n / 32; ++b) quant_q8_0_block(x + 32 * b, o + 34 * b);
      return 0;
    case EMBER_TYPE_Q4_K:
      if (n % 256) return EMBER_ERR_SHAPE;
#pragma omp parallel for schedule(static)
      for (int64_t b = 0; b < n / 256; ++b) quant_q4_k_block(x + 256 * b, o + 144 * b);
      return 0;
    default:
      return EMBER_ERR_TYPE;
  }
}

int ember_dequantize(int type, const void* src, int64_t n, float* out) {
  const uint8_t* s = static_cast<const uint8_t*>(src);
  switch (type) {
    case EMBER_TYPE_F32:
      std::memcpy(out, s, 4 * (size_t)n);
      return 0;
    case EMBER_TYPE_F16:
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < n; ++i) {
        uint16_t h;
        std::memcpy(&h, s + 2 * i, 2);
        out[i] = f16_to_f32(h);
      }
      return 0;
    case EMBER_TYPE_BF16:
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < n; ++i) {
        uint16_t h;
        std::memcpy(&h, s + 2 * i, 2);
        const uint32_t bits = (uint32_t)h << 16;
        std::memcpy(out + i, &bits, 4);
      }
      return 0;
    case EMBER_TYPE_Q8_0:
      if (n % 32) return EMBER_ERR_SHAPE;
#pragma omp parallel for schedule(static)
      for (int64_t b = 0; b < n / 32; ++b) {
        uint16_t dh;
        std::memcpy(&dh, s + 34 * b, 2);
        const float d = f16_to_f32(dh);
        for (int i = 0; i < 32; ++i) out[32 * b + i] = d * (float)(int8_t)s[34 * b + 2 + i];
      }
      return 0;
    case EMBER_TYPE_Q4_K:
      if (n % 256) return EMBER_ERR_SHAPE;
#pragma omp parallel for schedule(static)
      for (int64_t b = 0; b < n / 256; ++b) {
        const uint8_t* blk = s + 144 * b;
        uint16_t dh, mh;
        std::memcpy(&dh, blk, 2);
        std::memcpy(&mh, blk + 2, 2);
        const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
        for (int g = 0; g < 8; ++g) {
          int sc, mn;
          if (g < 4) {
            sc = blk[4 + g] & 63;
            mn = blk[8 + g] & 63;
          } else {
            sc = (blk[8 + g] & 0xf) | ((blk[g] >> 6) << 4);
            mn = (blk[8 + g] >> 4) | ((blk[4 + g] >> 6) << 4);
          }
          const float ds = d * (float)sc, ms = dmin * (float)mn;
          for (int l = 0; l < 32; ++l) {
            const uint8_t byte = blk[16 + 32 * (g / 2) + l];
            const int q = (g & 1) ? (byte >> 4) : (byte & 0xf);
            out[256 * b + 32 * g + l] = ds * (float)q - ms;
          }
        }
      }
      return 0;
    default:
      return EMBER_ERR_TYPE;
  }
}

uint16_t ember_f32_to_f16(float f) { return f32_to_f16(f); }
float ember_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t ember_f32_to_bf16(float f) { return f32_to_bf16(f); }

}  // extern "C"
