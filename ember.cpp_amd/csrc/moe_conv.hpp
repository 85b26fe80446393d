// Activation conversion for the MFMA expert GEMMs (device side): fp16 rows scaled by a power of two and
// split bf16 planes. Run by the dedicated kernels of moe_gemm.hip and by extra blocks of the routing
// launch (the conversion depends on x only, so it needs no launch of its own).
#pragma once
#include "moe_internal.hpp"

namespace ember_moe {

__device__ inline uint16_t bf16_rne(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN stays NaN
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ inline float bf16_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// Row r of c.x by the whole block (any block size up to 1024): c.y16 gets the row times 2^-e, e the frexp
// exponent of its largest magnitude (0 for an all-zero or non-finite row), in c.yexp[r]; c.yb gets
// bf16 hi = RNE(x) and lo = RNE(x - hi) (exact in f32) planes, the lo plane c.plane elements on.
__device__ inline void act_conv_row(const ActConv& c, int r) {
  const float* xr = c.x + (size_t)r * c.K;
  const int nt = blockDim.x;
  if (c.y16) {
    __shared__ float red[16];
    float m = 0.0f;
    for (int i = threadIdx.x; i < c.K; i += nt) m = fmaxf(m, fabsf(xr[i]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = 0.0f;
    for (int w = 0; w < (nt + 63) / 64; ++w) m = fmaxf(m, red[w]);
    int e = 0;
    if (m > 0.0f && m <= 3.4028235e38f) (void)__builtin_frexpf(m, &e);
    if (threadIdx.x == 0) c.yexp[r] = e;
    _Float16* yr = c.y16 + (size_t)r * c.K;
    for (int i = threadIdx.x; i < c.K; i += nt) yr[i] = (_Float16)__builtin_ldexpf(xr[i], -e);
  }
  if (c.yb) {
    uint16_t* yr = c.yb + (size_t)r * c.K;
    for (int i = threadIdx.x; i < c.K; i += nt) {
      const float v = xr[i];
      const uint16_t hi = bf16_rne(v);
      yr[i] = hi;
      yr[c.plane + i] = bf16_rne(v - bf16_f32(hi));
    }
  }
}

}  // namespace ember_moe
