// Grouped expert GEMM of the MoE FFN for prefill-sized batches, on CDNA4 MFMA.
//
// For every expert segment (the tokens routed to one expert, contiguous in the dispatch order) and
// every output tile: gate/up:  h[p][n] = silu(x_p . Wg[n]) * (x_p . Wu[n])   (x rows gathered via perm)
//                    down:     y[p][n] = h_p . Wd[n]
// with W rows in their ggml encoding. The reference computes the same products as FP64 dots over
// weights dequantized to F32 at load (utils.cpp:735-747, weight_management.cpp:802-877).
//
// Numerics: weights are decoded to fp16 while they are staged into LDS (Q8_0: d*q with one rounding;
// Q4_K: (d*sc)*q - dmin*m by one fused multiply-add of the fp16-rounded factors; BF16: RNE to fp16),
// activations are fp16, products accumulate in fp32 on v_mfma_f32_32x32x16_f16. The relative error
// of a layer is ~4e-4 (rel-L2), inside the 2e-3 bar for quantized stacks. F32 stacks never take this
// path (their bar is 1e-5).
//
// Kernels: gemm_dma_q8_kernel (Q8_0 rows or the prefill pack's Q8_0 / Q4_K tiles; 256-token tiles,
// weights and activations loaded straight into LDS), gemm_dma64_q8_kernel (the same formats, 64-token
// tiles), gemm_kernel and gemm_skinny_kernel (register-staged 256- / 64-token tiles for the other
// formats). Tiles are (expert, first token) pairs from a table the dispatch step writes (dense rows:
// consecutive token ranges); grids are sized for the most tiles a call can have, blocks take their work
// items XCD-balanced from the device-side tile count, and blocks without one exit at once. The down
// projection can split K over blocks (partial sums added in order by the combine); the 256-token gate/up
// launch splits only the tiles of its partial last round (the tail split), which a fixup launch finishes.
#include <cstdlib>
#include <type_traits>

#include "moe_conv.hpp"

namespace ember_moe {
using namespace ember_math;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));

constexpr int GBM = 256, GBK = 64, LDK = GBK + 8;  // LDS rows padded by 16 bytes

__device__ inline half2_t h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ inline uint32_t u32(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// (1024 + byte) as fp16 for bytes 0,1 (hi = 0) or 2,3 (hi = 1) of w: exact integers 1024..1279.
__device__ inline half2_t magic_pair(uint32_t w, int hi) {
  return h2(__builtin_amdgcn_perm(0x64646464u, w, hi ? 0x04030402u : 0x04010400u));
}

// Row-chunk decoders: the 64 elements [64*kt, +64) of a weight row into 32 dwords of fp16 pairs.
template <int FMT>
struct Deq;

// Q8_0: two 34-byte blocks, 68 bytes from a 4-byte boundary (rows are whole 64-element chunks).
// Dword 0 = {d_A, q0, q1}; 1..7 = q2..q29; 8 = {q30, q31, d_B}; 9..16 = block B's q0..q31.
template <>
struct Deq<EMBER_TYPE_Q8_0> {
  static constexpr int NW = 17;
  __device__ static void load(const uint8_t* row, int c, uint32_t* raw) {
    const uint8_t* p = row + (size_t)c * 68;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 q = *reinterpret_cast<const u32x4_a4*>(p + 16 * v);
      raw[4 * v] = q.x; raw[4 * v + 1] = q.y; raw[4 * v + 2] = q.z; raw[4 * v + 3] = q.w;
    }
    raw[16] = *reinterpret_cast<const uint32_t*>(p + 64);
  }
  // half row: block 2*kt + h, 34 bytes; odd blocks start 2 bytes past a dword boundary, so nine dwords
  // are loaded from the boundary below (they never leave the row) and funnel-shifted
  static constexpr int NWH = 9;
  __device__ static void load_half(const uint8_t* row, int kt, int h, uint32_t* raw) {
    const int blk = 2 * kt + h;
    const uint32_t* p = reinterpret_cast<const uint32_t*>(row + (size_t)(blk * 34 & ~3));
    const u32x4 q0 = *reinterpret_cast<const u32x4_a4*>(p), q1 = *reinterpret_cast<const u32x4_a4*>(p + 4);
    raw[0] = q0.x; raw[1] = q0.y; raw[2] = q0.z; raw[3] = q0.w;
    raw[4] = q1.x; raw[5] = q1.y; raw[6] = q1.z; raw[7] = q1.w;
    raw[8] = p[8];
  }
  __device__ static void decode_half(const uint32_t* raw, int, int h, uint32_t* out) {
    const uint32_t sh = h ? 16u : 0u;
    uint32_t w[9];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = __builtin_amdgcn_alignbit(raw[i + 1], raw[i], sh);
    w[8] = raw[8] >> sh;
    const half2_t dd = h2((w[0] & 0xffffu) * 0x10001u);
    const half2_t off = h2(0xe480e480u);
#pragma unroll
    for (int j = 0; j < 16; ++j) out[j] = u32((magic_pair(w[(1 + j) >> 1] ^ 0x80808080u, (1 + j) & 1) + off) * dd);
  }
  __device__ static void decode(const uint32_t* raw, int, uint32_t* out) {
    const half2_t dA = h2((raw[0] & 0xffffu) * 0x10001u), dB = h2((raw[8] >> 16) * 0x10001u);
    const half2_t off = h2(0xe480e480u);  // -1152 = -(1024 + 128) in each half
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const half2_t qa = magic_pair(raw[(1 + j) >> 1] ^ 0x80808080u, (1 + j) & 1) + off;
      const half2_t qb = magic_pair(raw[9 + (j >> 1)] ^ 0x80808080u, j & 1) + off;
      out[j] = u32(qa * dA);
      out[16 + j] = u32(qb * dB);
    }
  }
};

// Q4_K: quarter kt%4 of super-block kt/4: the 16-byte header and the quarter's 32 nibble bytes
// (low nibbles: group 2q, high nibbles: group 2q+1).
template <>
struct Deq<EMBER_TYPE_Q4_K> {
  static constexpr int NW = 12;
  __device__ static void load(const uint8_t* row, int c, uint32_t* raw) {
    const uint8_t* sb = row + (size_t)(c >> 2) * 144;
    const u32x4 hd = *reinterpret_cast<const u32x4*>(sb);
    const u32x4 q0 = *reinterpret_cast<const u32x4*>(sb + 16 + 32 * (c & 3));
    const u32x4 q1 = *reinterpret_cast<const u32x4*>(sb + 32 + 32 * (c & 3));
    raw[0] = hd.x; raw[1] = hd.y; raw[2] = hd.z; raw[3] = hd.w;
    raw[4] = q0.x; raw[5] = q0.y; raw[6] = q0.z; raw[7] = q0.w;
    raw[8] = q1.x; raw[9] = q1.y; raw[10] = q1.z; raw[11] = q1.w;
  }
  __device__ static int ubyte(const uint32_t* raw, int b) { return (int)((raw[b >> 2] >> (8 * (b & 3))) & 0xff); }
  __device__ static void scale_min(const uint32_t* raw, int j, int* sc, int* mn) {  // quantization.cpp:145-155
    if (j < 4) {
      *sc = ubyte(raw, 4 + j) & 63;
      *mn = ubyte(raw, 8 + j) & 63;
    } else {
      *sc = (ubyte(raw, 8 + j) & 0xf) | ((ubyte(raw, j) >> 6) << 4);
      *mn = (ubyte(raw, 8 + j) >> 4) | ((ubyte(raw, 4 + j) >> 6) << 4);
    }
  }
  // half row: group 2*(kt%4) + h of super-block kt/4 (low nibbles for h = 0, high for h = 1)
  static constexpr int NWH = 12;
  __device__ static void load_half(const uint8_t* row, int kt, int, uint32_t* raw) { load(row, kt, raw); }
  __device__ static void decode_half(const uint32_t* raw, int kt, int h, uint32_t* out) {
    const float d = half_bits_to_float(raw[0] & 0xffff), dmin = half_bits_to_float(raw[0] >> 16);
    int sc, mn;
    scale_min(raw, 2 * (kt & 3) + h, &sc, &mn);
    const _Float16 fd = (_Float16)(d * (float)sc), fm = (_Float16)(-(dmin * (float)mn));
    const half2_t dd = {fd, fd}, mm = {fm, fm};
    const half2_t off = h2(0xe400e400u);
    const uint32_t sh = h ? 4u : 0u;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t nib = (raw[4 + k] >> sh) & 0x0f0f0f0fu;
      out[2 * k] = u32(__builtin_elementwise_fma(magic_pair(nib, 0) + off, dd, mm));
      out[2 * k + 1] = u32(__builtin_elementwise_fma(magic_pair(nib, 1) + off, dd, mm));
    }
  }
  __device__ static void decode(const uint32_t* raw, int c, uint32_t* out) {
    const float d = half_bits_to_float(raw[0] & 0xffff), dmin = half_bits_to_float(raw[0] >> 16);
    int scA, mA, scB, mB;
    scale_min(raw, 2 * (c & 3), &scA, &mA);
    scale_min(raw, 2 * (c & 3) + 1, &scB, &mB);
    const _Float16 fdA = (_Float16)(d * (float)scA), fmA = (_Float16)(-(dmin * (float)mA));
    const _Float16 fdB = (_Float16)(d * (float)scB), fmB = (_Float16)(-(dmin * (float)mB));
    const half2_t dA = {fdA, fdA}, mA2 = {fmA, fmA}, dB = {fdB, fdB}, mB2 = {fmB, fmB};
    const half2_t off = h2(0xe400e400u);  // -1024
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t w = raw[4 + k];
      const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
      out[2 * k] = u32(__builtin_elementwise_fma(magic_pair(lo, 0) + off, dA, mA2));
      out[2 * k + 1] = u32(__builtin_elementwise_fma(magic_pair(lo, 1) + off, dA, mA2));
      out[16 + 2 * k] = u32(__builtin_elementwise_fma(magic_pair(hi, 0) + off, dB, mB2));
      out[16 + 2 * k + 1] = u32(__builtin_elementwise_fma(magic_pair(hi, 1) + off, dB, mB2));
    }
  }
};

template <int FMT>
struct DeqHalf {
  static constexpr int NW = 32, NWH = 16;
  __device__ static void load_half(const uint8_t* row, int kt, int h, uint32_t* raw) {
    const u32x4* p = reinterpret_cast<const u32x4*>(row + (size_t)kt * 128 + 64 * h);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 q = p[v];
      raw[4 * v] = q.x; raw[4 * v + 1] = q.y; raw[4 * v + 2] = q.z; raw[4 * v + 3] = q.w;
    }
  }
  __device__ static void decode_half(const uint32_t* raw, int, int, uint32_t* out) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (FMT == EMBER_TYPE_F16) {
        out[i] = raw[i];
      } else {
        const half2_t v = {(_Float16)as_f32(raw[i] << 16), (_Float16)as_f32(raw[i] & 0xffff0000u)};
        out[i] = u32(v);
      }
    }
  }
  __device__ static void load(const uint8_t* row, int c, uint32_t* raw) {
    const u32x4* p = reinterpret_cast<const u32x4*>(row + (size_t)c * 128);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const u32x4 q = p[v];
      raw[4 * v] = q.x; raw[4 * v + 1] = q.y; raw[4 * v + 2] = q.z; raw[4 * v + 3] = q.w;
    }
  }
  __device__ static void decode(const uint32_t* raw, int, uint32_t* out) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if (FMT == EMBER_TYPE_F16) {
        out[i] = raw[i];
      } else {
        const half2_t v = {(_Float16)as_f32(raw[i] << 16), (_Float16)as_f32(raw[i] & 0xffff0000u)};
        out[i] = u32(v);
      }
    }
  }
};
template <>
struct Deq<EMBER_TYPE_F16> : DeqHalf<EMBER_TYPE_F16> {};
template <>
struct Deq<EMBER_TYPE_BF16> : DeqHalf<EMBER_TYPE_BF16> {};

// The GEMM path carries ~4e-4 relative error from fp16 operands, so SwiGLU uses the hardware exp here.
__device__ inline float swiglu_g(float g, float u) { return g * __frcp_rn(1.0f + __expf(-g)) * u; }

// ---- epilogue stores shared by the MFMA kernels (GemmArgs::a_exp / h_exp / split_bf16)
// the range exponent of the A row behind output row p (0: unscaled)
__device__ inline int row_exp(const GemmArgs& g, int p) {
  return g.a_exp ? g.a_exp[g.perm ? g.perm[p] / g.k : p] : 0;
}
// h[p][n] = SwiGLU of the unscaled gate and up dots, stored in the A format of the down projection; the
// fp16 form is h times 2^-(2 e + eh), eh the expert's weight-range exponent (GemmArgs::w_hexp)
__device__ inline void store_h(const GemmArgs& g, size_t o, int p, int e, float ga, float ua, bool first_col,
                               int eh = 0) {
  const float hv = swiglu_g(__builtin_ldexpf(ga, e), __builtin_ldexpf(ua, e));
  if (g.split_bf16) {
    uint16_t* hb = reinterpret_cast<uint16_t*>(g.out_h);
    const uint16_t hi = bf16_rne(hv);
    hb[o] = hi;
    hb[g.h_plane + o] = bf16_rne(hv - bf16_f32(hi));
  } else {
    g.out_h[o] = (_Float16)__builtin_ldexpf(hv, -2 * e - eh);
    if (first_col && g.h_exp) g.h_exp[p] = 2 * e + eh;
  }
}
__device__ inline float unscale_y(float acc, int e) { return __builtin_ldexpf(acc, e); }
// BF16 weights on the fp16 path: the row's exponent (GemmArgs::w_exp0 / w_exp1; 0 without a table)
__device__ inline int w_exp_of(const int16_t* t, int e, int N, int n) { return t ? (int)t[(int64_t)e * N + n] : 0; }
// 16 dwords of bf16 pairs -> fp16 pairs, each value times sc (a power of two, so the only rounding is
// the fp16 one)
__device__ inline void bf16_to_f16_scaled(const uint32_t* raw, float sc, uint32_t* out) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const half2_t v = {(_Float16)(as_f32(raw[i] << 16) * sc), (_Float16)(as_f32(raw[i] & 0xffff0000u) * sc)};
    out[i] = u32(v);
  }
}
// the tile's row exponents, looked up once into LDS (rows of the tile: positions p0 .. p0 + rows)
__device__ inline void load_row_exps(const GemmArgs& g, int p0, int rows, int* s_rexp) {
  for (int r = threadIdx.x; r < rows; r += blockDim.x) s_rexp[r] = row_exp(g, p0 + r);
}

// m-tiles of a launch: the device-side tile count, or the dense rows' tiles of bm tokens
__device__ inline int launch_mtiles(const GemmArgs& g, int bm) {
  return g.tiles ? *g.n_tiles : (g.T + bm - 1) / bm;
}

// XCD-balanced work item of block b for the 256-token-tile kernels: the W = M x NT x KS work items (m-tile
// major, then n-tile, then K part) are cut into 8 equal runs, one per XCD (the hardware hands block b to
// XCD b % 8), and XCD x's j-th block takes item x ceil(W / 8) + j. Every XCD gets the same share whatever
// the (data-dependent) m-tile count, and the blocks an XCD holds at once mostly share one m-tile of
// activations in its L2. False: no item (the grid is sized for the largest M).
__device__ inline bool xcd_item(int M, int NT, int KS, int& mt, int& rem) {
  const int W = M * NT * KS, C = (W + 7) / 8;
  const int j = blockIdx.x / 8, w = (blockIdx.x % 8) * C + j;
  if (j >= C || w >= W) return false;
  mt = w / (NT * KS);
  rem = w % (NT * KS);
  return true;
}

// The gated DMA kernels' work item of block b: the W = M x NT items, or with a tail split
// (GemmArgs::tail_parts) the first R x slots items (R whole rounds) XCD-balanced as xcd_item takes them, then
// for blocks R slots + i part i % S of tail item R slots + i / S, S = min(tail_parts, slots / tail) (S = 1: no
// split; slots is a multiple of 8). Returns false for a block without an item; part / parts: this block's
// K part.
constexpr int kMaxTailParts = 8;
// The tail split of a gated launch of W = M x NT items: S parts per tail item (1: no split), capped at the
// K tiles so that every part holds at least one; `full` = the items of the whole rounds (W without a split).
__device__ inline int tail_split(const GemmArgs& g, int W, int& full) {
  full = W;
  if (g.tail_parts <= 1 || g.slots <= 0) return 1;
  const int R = W / g.slots, tail = W - R * g.slots;
  if (tail == 0) return 1;
  const int S = min(min(min(g.tail_parts, kMaxTailParts), g.slots / tail), g.K / GBK);
  if (S <= 1) return 1;
  full = R * g.slots;
  return S;
}
__device__ inline bool gated_item(const GemmArgs& g, int NT, int& mt, int& nt, int& part, int& parts) {
  const int W = launch_mtiles(g, GBM) * NT;
  int full;
  const int S = tail_split(g, W, full);
  // the whole rounds' items take blocks 0 .. 8 C - 1 (xcd_item's mapping, C = ceil(full / 8)), the tail
  // parts the blocks after them
  const int b = blockIdx.x, C = (full + 7) / 8;
  part = 0;
  parts = 1;
  if (b < 8 * C) {
    const int j = b / 8, w = (b % 8) * C + j;
    if (w >= full) return false;
    mt = w / NT;
    nt = w % NT;
    return true;
  }
  const int i = b - 8 * C, w = full + i / S;
  if (S == 1 || w >= W) return false;
  mt = w / NT;
  nt = w % NT;
  part = i % S;
  parts = S;
  return true;
}

// Blocks take their tiles XCD-balanced (xcd_item).
//
// 512 threads = 8 waves in a 4 (M) x 2 (N) arrangement (two waves per SIMD, so one wave's waits and
// decode overlap the other's MFMAs), each wave a 64 x 128 tile of accumulators; every thread loads
// half of one activation row and decodes half of one weight row per K tile. Per K tile: issue the
// global loads of tile k+1, run the MFMAs of tile k from one LDS stage, store / decode tile k+1 into
// the other stage, barrier.
constexpr int kGemmThreads = 512;
constexpr int kStageHalves = (GBM + 256) * LDK;
constexpr size_t kGemmLds = 2 * kStageHalves * sizeof(_Float16);

template <int FMT, bool GATED>
__global__ void __launch_bounds__(kGemmThreads) gemm_kernel(GemmArgs g, int NT) {
  using D = Deq<FMT>;
  constexpr int BN = GATED ? 128 : 256;  // output columns per block
  constexpr int WN = GATED ? 2 : 4;      // 32-column subtiles per wave (per matrix)
  constexpr int WM = 2;                  // 32-row subtiles per wave
  constexpr int G = GATED ? 2 : 1;
  extern __shared__ __align__(16) _Float16 smem[];

  // ---- the tile
  int mt, nt;
  if (!xcd_item(launch_mtiles(g, GBM), NT, 1, mt, nt)) return;
  int e = 0, p0 = 0, rows = 0;
  if (g.tiles) {
    e = g.tiles[2 * mt];
    const int m0 = g.tiles[2 * mt + 1];
    p0 = g.offsets[e] + m0;
    rows = min(GBM, g.offsets[e + 1] - p0);
  } else {
    p0 = mt * GBM;
    if (p0 >= g.T) return;
    rows = min(GBM, g.T - p0);
  }
  const int n0 = nt * BN;
  const int K = g.K, N = g.N;
  const int nk = K / GBK;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = tid >> 1, lh = tid & 1;  // this thread's row (of A and of W) and half of the K tile

  const _Float16* a_src = nullptr;
  if (lr < rows) {
    const int p = p0 + lr;
    a_src = g.A + (size_t)(g.perm ? g.perm[p] / g.k : p) * K + 32 * lh;
  }
  const uint8_t* b_row = nullptr;
  float b_sc = 1.0f;  // BF16: 2^-(the row's exponent)
  {
    const int b_g = GATED ? (lr >> 7) : 0;
    const int b_n = n0 + (GATED ? (lr & 127) : lr);
    if (b_n < N) {
      b_row = static_cast<const uint8_t*>(b_g ? g.W1 : g.W0) + (int64_t)e * g.expert_stride + (int64_t)b_n * g.row_bytes;
      if (FMT == EMBER_TYPE_BF16) b_sc = __builtin_ldexpf(1.0f, -w_exp_of(b_g ? g.w_exp1 : g.w_exp0, e, N, b_n));
    }
  }

  u32x4 a_reg[4];
  uint32_t b_raw[D::NWH];
  auto fetch = [&](int kt) {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      a_reg[v] = a_src ? *reinterpret_cast<const u32x4*>(a_src + (size_t)kt * GBK + 8 * v) : u32x4{0, 0, 0, 0};
    if (b_row) {
      D::load_half(b_row, kt, lh, b_raw);
    } else {
#pragma unroll
      for (int w = 0; w < D::NWH; ++w) b_raw[w] = 0u;
    }
  };
  auto stage_in = [&](int kt, int stage) {
    _Float16* As = smem + stage * kStageHalves;
    _Float16* Bs = As + GBM * LDK;
#pragma unroll
    for (int v = 0; v < 4; ++v) *reinterpret_cast<u32x4*>(&As[lr * LDK + 32 * lh + 8 * v]) = a_reg[v];
    uint32_t dq[16];
    if (b_row) {
      if constexpr (FMT == EMBER_TYPE_BF16)
        bf16_to_f16_scaled(b_raw, b_sc, dq);
      else
        D::decode_half(b_raw, kt, lh, dq);
    } else {
#pragma unroll
      for (int w = 0; w < 16; ++w) dq[w] = 0u;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v)
      *reinterpret_cast<u32x4*>(&Bs[lr * LDK + 32 * lh + 8 * v]) = u32x4{dq[4 * v], dq[4 * v + 1], dq[4 * v + 2], dq[4 * v + 3]};
  };

  floatx16 acc[G][WM][WN];
#pragma unroll
  for (int q = 0; q < G; ++q)
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int jn = 0; jn < WN; ++jn)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[q][i][jn][r] = 0.0f;

  auto mfma_stage = [&](int stage) {
    const _Float16* As = smem + stage * kStageHalves;
    const _Float16* Bs = As + GBM * LDK;
#pragma unroll
    for (int ks = 0; ks < GBK / 16; ++ks) {
      const int kk = ks * 16 + 8 * (lane >> 5);
      half8 af[WM];
#pragma unroll
      for (int i = 0; i < WM; ++i) af[i] = *reinterpret_cast<const half8*>(&As[(wm * 64 + 32 * i + (lane & 31)) * LDK + kk]);
#pragma unroll
      for (int q = 0; q < G; ++q)
#pragma unroll
        for (int jn = 0; jn < WN; ++jn) {
          const int brow = (GATED ? q * 128 : 0) + wn * (WN * 32) + 32 * jn + (lane & 31);
          const half8 bf = *reinterpret_cast<const half8*>(&Bs[brow * LDK + kk]);
#pragma unroll
          for (int i = 0; i < WM; ++i)
            acc[q][i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf, acc[q][i][jn], 0, 0, 0);
        }
    }
  };

  __shared__ int s_rexp[GBM];
  load_row_exps(g, p0, rows, s_rexp);
  fetch(0);
  stage_in(0, 0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) fetch(kt + 1);  // in flight during the MFMAs below
    mfma_stage(kt & 1);
    if (kt + 1 < nk) stage_in(kt + 1, (kt + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds column (lane & 31) of each 32x32 subtile, rows 8*ii + 4*(lane>>5) + jj
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int jn = 0; jn < WN; ++jn) {
      const int n = n0 + wn * (WN * 32) + 32 * jn + (lane & 31);
      if (n >= N) continue;
      const int we0 = FMT == EMBER_TYPE_BF16 ? w_exp_of(g.w_exp0, e, N, n) : 0;
      const int we1 = FMT == EMBER_TYPE_BF16 && GATED ? w_exp_of(g.w_exp1, e, N, n) : 0;
      const int weh = FMT == EMBER_TYPE_BF16 && GATED && g.w_hexp ? (int)g.w_hexp[e] : 0;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int m = wm * 64 + 32 * i + 8 * ii + 4 * (lane >> 5) + jj;
          if (m >= rows) continue;
          const size_t o = (size_t)(p0 + m) * N + n;
          const int ex = s_rexp[m];
          if constexpr (GATED) {
            store_h(g, o, p0 + m, ex, __builtin_ldexpf(acc[0][i][jn][4 * ii + jj], we0),
                    __builtin_ldexpf(acc[1][i][jn][4 * ii + jj], we1), n == n0, weh);
          } else {
            g.out_y[o] = unscale_y(__builtin_ldexpf(acc[0][i][jn][4 * ii + jj], we0), ex);
          }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Q8_0 grouped GEMM with direct global->LDS tile loads. Tiles of 256 tokens x 256 weight rows x 64 K
// run through a ring of three LDS stages that global_load_lds fills without passing through
// registers, so two tiles are in flight while one is multiplied (launches of at most 64 tokens: 64-row
// activation stages and five stages, four tiles in flight). Every wave loads a share of both
// operands: the activation tile as 16-byte granules XOR-swizzled by row pair (the 16 rows that one
// 16-lane pass of ds_read_b128 reads fall on distinct bank groups of the 64-bank LDS), the weight
// tile in its Q8_0 bytes: the 68 bytes of a row's K tile as five 16-byte granules, the fifth
// overlapping (bytes 52..67), so a row occupies 80 bytes of LDS. 512 threads = 8 waves (two per
// SIMD) in a 2 (M) x 4 (N) arrangement; a wave owns 128 tokens x 64 weight rows (gated: 32 gate +
// 32 up columns, so SwiGLU pairs meet in one wave) and decodes its own B fragments from the Q8_0
// bytes straight into MFMA operands (fp16 d * q, one rounding, as the decoders above).
typedef __attribute__((address_space(3))) void lds_void_t;
constexpr int kDmaThreads = 512, kDmaStages = 3;
constexpr int kDmaRowB = 80;                     // LDS bytes of one weight row's K tile
constexpr int kDmaA = GBM * GBK * 2;             // activation bytes per stage (32 KiB)
constexpr int kDmaB = 256 * kDmaRowB;            // weight bytes per stage (20 KiB)
constexpr int kDmaStage = kDmaA + kDmaB;
constexpr size_t kDmaLds = (size_t)kDmaStages * kDmaStage;
// launches of at most 64 tokens (every segment, hence every tile, holds at most 64 rows: a token picks an
// expert once): 64 activation rows per stage (8 KiB) and five stages, four tiles in flight
constexpr int kDmaStagesShort = 5, kShortRows = 64;
constexpr int kDmaAShort = kShortRows * GBK * 2;
constexpr size_t kDmaLdsShort = (size_t)kDmaStagesShort * (kDmaAShort + kDmaB);

__device__ inline void lds_dma16(const void* g, uint8_t* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_t*)lds, 16, 0, 0);
}
// s_waitcnt vmcnt(n) alone (expcnt and lgkmcnt left at their no-wait maxima)
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Weight tile formats of the DMA kernels (template parameter WF):
//   kWfQ8Rows  Q8_0 row slices read from the ggml rows (80 LDS bytes per row, as above);
//   kWfQ8Pack  prefill-pack Q8_0 tiles: 17 KiB contiguous, loaded as 17 whole-kilobyte DMA instructions
//              into 68-byte LDS rows (17 dwords: the 32 rows a B fragment read touches fall on distinct
//              banks);
//   kWfQ4Pack  prefill-pack Q4_K tiles: 10 KiB, 40-byte rows {a0, m0, a1, m1, 32 nibble bytes} (10 dwords,
//              again 32 distinct banks).
enum { kWfQ8Rows = 0, kWfQ8Pack = 1, kWfQ4Pack = 2 };
template <int WF>
struct DmaW {
  static constexpr int kRowB = WF == kWfQ8Rows ? kDmaRowB : WF == kWfQ8Pack ? kPackRowB : kPackRowQ4B;
  static constexpr int kInst = (WF == kWfQ8Rows ? kDmaB : 256 * kRowB) / 1024;  // 1 KiB instructions per tile
  static constexpr int64_t kStride = WF == kWfQ8Rows ? 68 : 256 * kRowB;         // global bytes per K tile
};

// The B fragment of K step KS (compile time) from one weight row's K tile in LDS: the lane's 8 elements
// of K granule 2 KS + h, as fp16 MFMA operands.
// Q8_0: K granule gk = 2 ks + h of the 64 = Q8_0 block b = ks / 2, bytes X + 8 h .. + 8 of the row's 68
// with X = 34 b + 2 + 16 (ks % 2); for b = 1 those are dword aligned and, in row slices past byte 52,
// read from the overlapping fifth granule (LDS byte = global byte + 12); for b = 0 they sit two bytes
// past a dword and are funnel-shifted out of three dwords. Value d * q, one rounding.
// Q4_K pack: group b = ks / 2 (its nibble half of the 32 bytes), elements 16 (ks % 2) + 8 h .. + 8 =
// nibble bytes of the same offsets; value a * q + m by one fp16 fused multiply-add (the factors as
// Deq<Q4_K> forms them, so the products are those of the register-staged kernels).
template <int WF, int KS>
__device__ inline half8 b_frag(const uint8_t* row, int h) {
  constexpr int b = KS >> 1;
  if constexpr (WF == kWfQ4Pack) {
    const uint32_t hdr = *reinterpret_cast<const uint32_t*>(row + 4 * b);
    const half2_t a = h2((hdr & 0xffffu) * 0x10001u), m = h2((hdr >> 16) * 0x10001u);
    const uint32_t* qw = reinterpret_cast<const uint32_t*>(row + 8 + 16 * (KS & 1) + 8 * h);
    const uint32_t n0 = (qw[0] >> (4 * b)) & 0x0f0f0f0fu, n1 = (qw[1] >> (4 * b)) & 0x0f0f0f0fu;
    const half2_t off = h2(0xe400e400u);  // -1024 in each half
    const uint32_t o0 = u32(__builtin_elementwise_fma(magic_pair(n0, 0) + off, a, m));
    const uint32_t o1 = u32(__builtin_elementwise_fma(magic_pair(n0, 1) + off, a, m));
    const uint32_t o2 = u32(__builtin_elementwise_fma(magic_pair(n1, 0) + off, a, m));
    const uint32_t o3 = u32(__builtin_elementwise_fma(magic_pair(n1, 1) + off, a, m));
    return __builtin_bit_cast(half8, u32x4{o0, o1, o2, o3});
  } else {
    constexpr int X = 34 * b + 2 + 16 * (KS & 1);
    const uint32_t dbits = b ? (*reinterpret_cast<const uint32_t*>(row + 32) >> 16)
                             : (*reinterpret_cast<const uint32_t*>(row) & 0xffffu);
    const half2_t d = h2(dbits * 0x10001u);
    uint32_t w0, w1;
    if constexpr (b == 0) {
      const uint32_t* qw = reinterpret_cast<const uint32_t*>(row + (X & ~3) + 8 * h);
      w0 = __builtin_amdgcn_alignbit(qw[1], qw[0], 16);
      w1 = __builtin_amdgcn_alignbit(qw[2], qw[1], 16);
    } else {
      const int byte = X + 8 * h;
      const uint32_t* qw =
          reinterpret_cast<const uint32_t*>(row + (WF == kWfQ8Pack || byte + 8 <= 64 ? byte : byte + 12));
      w0 = qw[0];
      w1 = qw[1];
    }
    const half2_t off = h2(0xe480e480u);  // -1152 = -(1024 + 128) in each half
    const uint32_t q0 = w0 ^ 0x80808080u, q1 = w1 ^ 0x80808080u;
    const uint32_t o0 = u32((magic_pair(q0, 0) + off) * d), o1 = u32((magic_pair(q0, 1) + off) * d);
    const uint32_t o2 = u32((magic_pair(q1, 0) + off) * d), o3 = u32((magic_pair(q1, 1) + off) * d);
    return __builtin_bit_cast(half8, u32x4{o0, o1, o2, o3});
  }
}

// TAIL (gated only): the launch carries a tail split (gated_item); the other instantiation is the plain
// XCD-balanced mapping. SHORT: the launch has at most 64 tokens (kDmaStagesShort).
template <bool GATED, int WF, bool TAIL = false, bool SHORT = false>
__global__ void __launch_bounds__(kDmaThreads) gemm_dma_q8_kernel(GemmArgs g, int NT) {
  constexpr int BN = GATED ? 128 : 256;
  constexpr int kRowB = DmaW<WF>::kRowB;       // LDS bytes per weight row
  constexpr int kLastB = DmaW<WF>::kInst - 1;  // last weight DMA instruction
  constexpr int kDmaInstB = (DmaW<WF>::kInst + 7) / 8;  // weight DMA instructions per wave (the last shared)
  constexpr int NS = SHORT ? kDmaStagesShort : kDmaStages;  // LDS stages
  constexpr int kAB = SHORT ? kDmaAShort : kDmaA;           // activation bytes per stage
  constexpr int kStage = kAB + kDmaB;
  constexpr int kInstA = kAB / 1024 / 8;                    // activation DMA instructions per wave (1 or 4)
  constexpr int kInstMax = kInstA > kDmaInstB ? kInstA : kDmaInstB;
  constexpr int kDmaInst = kInstA + kDmaInstB;
  extern __shared__ __align__(16) uint8_t dsm[];

  // block -> (m-tile, n-tile, K split part), XCD-balanced
  int KS, mt, nt, ks;
  if constexpr (GATED && TAIL) {
    if (!gated_item(g, NT, mt, nt, ks, KS)) return;
  } else {
    KS = GATED ? 1 : g.ksplit;
    int rem;
    if (!xcd_item(launch_mtiles(g, GBM), NT, KS, mt, rem)) return;
    nt = rem / KS;
    ks = rem % KS;
  }
  int e = 0, p0 = 0, rows = 0;
  if (g.tiles) {
    e = g.tiles[2 * mt];
    const int m0 = g.tiles[2 * mt + 1];
    p0 = g.offsets[e] + m0;
    rows = min(GBM, g.offsets[e + 1] - p0);
  } else {
    p0 = mt * GBM;
    if (p0 >= g.T) return;
    rows = min(GBM, g.T - p0);
  }
  const int n0 = nt * BN;
  const int K = g.K, N = g.N;
  // this part's K tiles [kt0, kt0 + nk)
  const int nk_all = K / GBK;
  const int kt0 = ks * nk_all / KS, nk = (ks + 1) * nk_all / KS - kt0;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // wave w runs on SIMD w % 4, so each SIMD holds one wave of each M half: a tile whose rows end
  // inside the first half leaves no SIMD with double work
  const int wm = wave >> 2, wn = wave & 3;
  // 32-row subtiles of this wave's M half that hold tokens (0..4; SHORT: 0..2); the others are skipped
  const int msub = min(SHORT ? kShortRows / 32 : 4, max(0, (rows - 128 * wm + 31) >> 5));

  // DMA sources, the same code in every wave (no branches in the K loop): DMA instruction j of a
  // tile fills 16-byte granules 64 j + lane. Activations: instructions 4 w + i (i < 4; SHORT: w, rows
  // 8 w .. 8 w + 7); granule gi is row gi / 8, slot gi % 8 holding K granule slot ^ ((row / 2) % 8); rows
  // past the tile repeat its last row.
  // Weights: instructions min(3 w + i, 19) (i < 3; waves 6 and 7 repeat instruction 19, which rewrites
  // identical bytes); granule gb is row gb / 5, part gb % 5 = bytes 16 part (parts 0-3) or 52.
  const uint8_t* srcA[kInstA];
  const uint8_t* srcB[kDmaInstB];
#pragma unroll
  for (int i = 0; i < kInstA; ++i) {
    const int gi = 64 * (kInstA * wave + i) + lane;
    const int r = gi >> 3, kg = (gi & 7) ^ ((r >> 1) & 7);
    const int p = p0 + min(r, rows - 1);
    srcA[i] = reinterpret_cast<const uint8_t*>(g.A + (size_t)(g.perm ? g.perm[p] / g.k : p) * K + 8 * kg);
  }
#pragma unroll
  for (int i = 0; i < kDmaInstB; ++i) {
    const int gb = 64 * min(kDmaInstB * wave + i, kLastB) + lane;
    if constexpr (WF != kWfQ8Rows) {
      srcB[i] = g.Wp + ((int64_t)e * NT + nt) * nk_all * DmaW<WF>::kStride + 16 * gb;
    } else {
      const int r = gb / 5, part = gb - 5 * r;
      const int q = GATED ? (r >> 7) : 0;
      const int n = min(n0 + (GATED ? (r & 127) : r), N - 1);
      srcB[i] = static_cast<const uint8_t*>(q ? g.W1 : g.W0) + (int64_t)e * g.expert_stride + (int64_t)n * g.row_bytes +
                (part < 4 ? 16 * part : 52);
    }
  }
  // DMA of tile kt (clamped: tiles past the end reload the last, never multiplied), part j of 4 so
  // that the issue is spread over the K steps of a tile: activation instruction j, weight instruction j
  // NOA (compile time): this wave loads no activation rows (its rows lie past the tile's tokens), so its
  // per-tile DMA count, and the waits that count it, are the weights' alone
  auto issue = [&](int kt, int j, auto NOAc) {
    const int kc = kt0 + min(kt, nk - 1);
    uint8_t* st = dsm + (kt % NS) * kStage;
    if constexpr (!decltype(NOAc)::value) {
      if (j < kInstA)
        lds_dma16(srcA[j < kInstA ? j : 0] + (size_t)kc * GBK * 2, st + 1024 * (kInstA * wave + j));
    }
    if (j < kDmaInstB)
      lds_dma16(srcB[j < kDmaInstB ? j : 0] + (size_t)kc * DmaW<WF>::kStride,
                st + kAB + 1024 * min(kDmaInstB * wave + j, kLastB));
  };
  auto issue_all = [&](int kt, auto NOAc) {
#pragma unroll
    for (int j = 0; j < kInstMax; ++j) issue(kt, j, NOAc);
  };

  floatx16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jn = 0; jn < 2; ++jn)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][jn][r] = 0.0f;

  // B tile row of this lane in subtile jn
  auto brow_of = [&](int jn) {
    if constexpr (GATED) return jn * 128 + wn * 32 + (lane & 31);
    return wn * 64 + 32 * jn + (lane & 31);
  };
  const int h = lane >> 5;

  // Fragments of K step ks (compile time) of the tile in stage `st`, for the first MS (compile time)
  // 32-row subtiles
  struct Frags {
    half8 a[4], b[2];
  };
  auto load_frags = [&](const uint8_t* st, auto KS, auto MSc, Frags& f) {
    constexpr int ks = decltype(KS)::value;
    constexpr int MS = decltype(MSc)::value;
    const int gk = 2 * ks + h;
#pragma unroll
    for (int i = 0; i < MS; ++i) {
      const int r = wm * 128 + 32 * i + (lane & 31);
      f.a[i] = *reinterpret_cast<const half8*>(st + 16 * (8 * r + (gk ^ ((r >> 1) & 7))));
    }
    const uint8_t* Bs = st + kAB;
#pragma unroll
    for (int jn = 0; jn < 2; ++jn) f.b[jn] = b_frag<WF, ks>(Bs + kRowB * brow_of(jn), h);
  };
  auto mfmas = [&](const Frags& f, auto MSc) {
#pragma unroll
    for (int i = 0; i < decltype(MSc)::value; ++i)
#pragma unroll
      for (int jn = 0; jn < 2; ++jn)
        acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], f.b[jn], acc[i][jn], 0, 0, 0);
  };
  // A bare barrier: __syncthreads()'s release fence would wait for the DMA in flight as well. The
  // empty asm statements keep the compiler from moving LDS accesses across it.
  auto barrier = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // The K loop, rotated so that no tile starts cold: iteration kt runs the MFMAs of K steps 0-2 of
  // tile kt with the DMA of tile kt + 2 spread between them, then waits for tile kt + 1 (this wave's
  // DMA, then every wave's at the barrier, which also marks the reads of tile kt complete, so stage
  // kt % 3 may be refilled next iteration), and reads and decodes K step 0 of tile kt + 1 while the
  // MFMAs of K step 3 of tile kt run. (The last iteration reads tile nk, a clamped reload, unused.)
  // A wave whose M half holds no tokens (MS = 0) only loads and keeps the barriers.
  // (NS stages: tiles kt + 1 .. kt + NS - 2 are in flight while tile kt is multiplied; the iteration
  // issues tile kt + NS - 1 and then waits for tile kt + 1, leaving NS - 2 tiles' DMA outstanding)
  auto k_loop = [&](auto MSc, auto NOAc) {
    constexpr int kInst = decltype(NOAc)::value ? kDmaInstB : kDmaInst;  // this wave's DMA per tile
    using K0 = std::integral_constant<int, 0>;
    using K1 = std::integral_constant<int, 1>;
    using K2 = std::integral_constant<int, 2>;
    using K3 = std::integral_constant<int, 3>;
#pragma unroll
    for (int t = 0; t < NS - 1; ++t) issue_all(t, NOAc);
    wait_vmcnt<(NS - 2) * kInst>();
    barrier();
    Frags f0, f1;
    if constexpr (decltype(MSc)::value > 0) load_frags(dsm, K0{}, MSc, f0);
    for (int kt = 0; kt < nk; ++kt) {
      if constexpr (decltype(MSc)::value == 0) {
        issue_all(kt + NS - 1, NOAc);
        wait_vmcnt<(NS - 2) * kInst>();
        barrier();
      } else {
        const uint8_t* st = dsm + (kt % NS) * kStage;
        load_frags(st, K1{}, MSc, f1);
        issue(kt + NS - 1, 0, NOAc);
        mfmas(f0, MSc);
        load_frags(st, K2{}, MSc, f0);
        issue(kt + NS - 1, 1, NOAc);
        mfmas(f1, MSc);
        load_frags(st, K3{}, MSc, f1);
        issue(kt + NS - 1, 2, NOAc);
        mfmas(f0, MSc);
        issue(kt + NS - 1, 3, NOAc);
        wait_vmcnt<(NS - 2) * kInst>();
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of tile kt are complete
        barrier();
        load_frags(dsm + ((kt + 1) % NS) * kStage, K0{}, MSc, f0);
        mfmas(f1, MSc);
      }
    }
  };
  __shared__ int s_rexp[GBM];
  load_row_exps(g, p0, rows, s_rexp);
  // waves whose activation rows (32 w .. 32 w + 31; SHORT: 8 w .. 8 w + 7) lie past the tile's tokens load
  // none: a short tile's DMA is then its weights and only the activation rows it holds (wave-uniform)
  using A1 = std::integral_constant<bool, false>;
  using A0 = std::integral_constant<bool, true>;
  // (SHORT: msub <= 2, so the 3- and 4-subtile loops are not built)
  using M4 = std::integral_constant<int, SHORT ? 2 : 4>;
  using M3 = std::integral_constant<int, SHORT ? 2 : 3>;
  if (8 * kInstA * wave >= rows) {
    switch (msub) {
      case 4: k_loop(M4{}, A0{}); break;
      case 3: k_loop(M3{}, A0{}); break;
      case 2: k_loop(std::integral_constant<int, 2>{}, A0{}); break;
      case 1: k_loop(std::integral_constant<int, 1>{}, A0{}); break;
      default: k_loop(std::integral_constant<int, 0>{}, A0{}); break;
    }
  } else {
    switch (msub) {
      case 4: k_loop(M4{}, A1{}); break;
      case 3: k_loop(M3{}, A1{}); break;
      case 2: k_loop(std::integral_constant<int, 2>{}, A1{}); break;
      case 1: k_loop(std::integral_constant<int, 1>{}, A1{}); break;
      default: k_loop(std::integral_constant<int, 0>{}, A1{}); break;
    }
  }
  wait_vmcnt<0>();  // no DMA may still target LDS when the block exits
  __syncthreads();  // the row exponents are visible

  // ---- epilogue: lane holds column (lane & 31) of each 32x32 subtile, rows 8*ii + 4*(lane>>5) + jj
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jn = 0; jn < (GATED ? 1 : 2); ++jn) {
      const int n = n0 + (GATED ? wn * 32 : wn * 64 + 32 * jn) + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int m = wm * 128 + 32 * i + 8 * ii + 4 * (lane >> 5) + jj;
          if (m >= rows) continue;
          const size_t o = (size_t)(p0 + m) * N + n;
          const int ex = s_rexp[m];
          if constexpr (GATED) {
            if (TAIL && KS > 1) {  // a tail item's K part: raw partial dots, gemm_tail_fixup_kernel finishes the tile
              float* part = g.part_h + ((size_t)ks * g.part_rows + p0 + m) * 2 * N + n;
              part[0] = acc[i][0][4 * ii + jj];
              part[N] = acc[i][1][4 * ii + jj];
            } else {
              store_h(g, o, p0 + m, ex, acc[i][0][4 * ii + jj], acc[i][1][4 * ii + jj], n == n0);
            }
          } else {
            g.out_y[ks * g.part_stride + o] = unscale_y(acc[i][jn][4 * ii + jj], ex);
          }
        }
    }
}

// The same with 64-token tiles, for segments of a few to a few dozen tokens (decode batches, short
// prefills), where the layer is bound by streaming the weights: 256 threads = 4 waves side by side
// in N (each 64 tokens x 64 weight rows, gated: 32 gate + 32 up columns), a five-stage LDS ring (four
// tiles in flight), every wave loading 2 activation and 5 weight granules per tile.
constexpr int kD64Threads = 256, kD64Stages = 5, kD64BM = 64;
constexpr int kD64A = kD64BM * GBK * 2;            // 8 KiB
constexpr int kD64Stage = kD64A + kDmaB;          // + 20 KiB of Q8_0 rows
constexpr size_t kD64Lds = (size_t)kD64Stages * kD64Stage;
constexpr int kD64InstA = kD64A / 16 / 64 / 4;     // 2 per wave

// WF: the weight tile format, as in gemm_dma_q8_kernel.
template <bool GATED, int WF>
__global__ void __launch_bounds__(kD64Threads) gemm_dma64_q8_kernel(GemmArgs g, int NT) {
  constexpr int BN = GATED ? 128 : 256;
  constexpr int kRowB = DmaW<WF>::kRowB;
  constexpr int kLastB = DmaW<WF>::kInst - 1;
  constexpr int kD64InstB = (DmaW<WF>::kInst + 3) / 4;  // weight DMA instructions per wave (5, 5, 3)
  extern __shared__ __align__(16) uint8_t dsm[];

  // block -> (m-tile, n-tile, K split part); part ks covers K tiles [kt0, kt0 + nk)
  // (items m-tile fastest, numbered densely: no block of the grid's tail is left waiting behind
  // empty slots)
  const int M = launch_mtiles(g, kD64BM);
  if ((int)blockIdx.x >= M * NT * (g.ksplit < 1 ? 1 : g.ksplit)) return;
  const int mt = blockIdx.x % M, rest = blockIdx.x / M;
  const int nt = rest % NT, ks = rest / NT;
  int e = 0, p0 = 0, rows = 0;
  if (g.tiles) {
    e = g.tiles[2 * mt];
    const int m0 = g.tiles[2 * mt + 1];
    p0 = g.offsets[e] + m0;
    rows = min(kD64BM, g.offsets[e + 1] - p0);
  } else {
    p0 = mt * kD64BM;
    if (p0 >= g.T) return;
    rows = min(kD64BM, g.T - p0);
  }
  const int n0 = nt * BN;
  const int K = g.K, N = g.N;
  const int nk_all = K / GBK;
  const int kt0 = ks * nk_all / g.ksplit, nk = (ks + 1) * nk_all / g.ksplit - kt0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave;

  const uint8_t* srcA[kD64InstA];
  const uint8_t* srcB[kD64InstB];
#pragma unroll
  for (int i = 0; i < kD64InstA; ++i) {
    const int gi = 64 * (kD64InstA * wave + i) + lane;
    const int r = gi >> 3, kg = (gi & 7) ^ ((r >> 1) & 7);
    const int p = p0 + min(r, rows - 1);
    srcA[i] = reinterpret_cast<const uint8_t*>(g.A + (size_t)(g.perm ? g.perm[p] / g.k : p) * K + 8 * kg);
  }
#pragma unroll
  for (int i = 0; i < kD64InstB; ++i) {
    const int gb = 64 * min(kD64InstB * wave + i, kLastB) + lane;
    if constexpr (WF != kWfQ8Rows) {
      srcB[i] = g.Wp + ((int64_t)e * NT + nt) * nk_all * DmaW<WF>::kStride + 16 * gb;
    } else {
      const int r = gb / 5, part = gb - 5 * r;
      const int q = GATED ? (r >> 7) : 0;
      const int n = min(n0 + (GATED ? (r & 127) : r), N - 1);
      srcB[i] = static_cast<const uint8_t*>(q ? g.W1 : g.W0) + (int64_t)e * g.expert_stride + (int64_t)n * g.row_bytes +
                (part < 4 ? 16 * part : 52);
    }
  }
  // DMA of tile kt (clamped past the end), part j of 4: A granule j / 2 on even parts, weight
  // granules spread over the four parts
  // NOA (compile time): this wave's activation rows (16 w .. 16 w + 15) lie past the tile's tokens, so it
  // loads none and its per-tile DMA count is the weights' alone
  auto issue = [&](int kt, int j, auto NOAc) {  // kt: tile index within this block's K range
    const int kc = kt0 + min(kt, nk - 1);
    uint8_t* st = dsm + (kt % kD64Stages) * kD64Stage;
    if (!decltype(NOAc)::value && (j & 1) == 0) {
      const int i = j >> 1;
      lds_dma16(srcA[i] + (size_t)kc * GBK * 2, st + 1024 * (kD64InstA * wave + i));
    }
#pragma unroll
    for (int i = 0; i < kD64InstB; ++i)
      if ((i * 4) / kD64InstB == j)
        lds_dma16(srcB[i] + (size_t)kc * DmaW<WF>::kStride, st + kD64A + 1024 * min(kD64InstB * wave + i, kLastB));
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int jn = 0; jn < 2; ++jn)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][jn][r] = 0.0f;

  auto brow_of = [&](int jn) {
    if constexpr (GATED) return jn * 128 + wn * 32 + (lane & 31);
    return wn * 64 + 32 * jn + (lane & 31);
  };
  const int h = lane >> 5;
  struct Frags {
    half8 a[2], b[2];
  };
  auto load_frags = [&](const uint8_t* st, auto KS, Frags& f) {
    constexpr int ks = decltype(KS)::value;
    const int gk = 2 * ks + h;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = 32 * i + (lane & 31);
      f.a[i] = *reinterpret_cast<const half8*>(st + 16 * (8 * r + (gk ^ ((r >> 1) & 7))));
    }
    const uint8_t* Bs = st + kD64A;
#pragma unroll
    for (int jn = 0; jn < 2; ++jn) f.b[jn] = b_frag<WF, ks>(Bs + kRowB * brow_of(jn), h);
  };
  auto mfmas = [&](const Frags& f) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int jn = 0; jn < 2; ++jn)
        acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], f.b[jn], acc[i][jn], 0, 0, 0);
  };
  auto compute = [&](int kt, auto NOAc) {
    const uint8_t* st = dsm + (kt % kD64Stages) * kD64Stage;
    Frags f0, f1;
    load_frags(st, std::integral_constant<int, 0>{}, f0);
    issue(kt + kD64Stages - 1, 0, NOAc);
    load_frags(st, std::integral_constant<int, 1>{}, f1);
    mfmas(f0);
    issue(kt + kD64Stages - 1, 1, NOAc);
    load_frags(st, std::integral_constant<int, 2>{}, f0);
    mfmas(f1);
    issue(kt + kD64Stages - 1, 2, NOAc);
    load_frags(st, std::integral_constant<int, 3>{}, f1);
    mfmas(f0);
    issue(kt + kD64Stages - 1, 3, NOAc);
    mfmas(f1);
  };

  __shared__ int s_rexp[kD64BM];
  load_row_exps(g, p0, rows, s_rexp);
  auto k_loop = [&](auto NOAc) {
    constexpr int kPerTile = (decltype(NOAc)::value ? 0 : kD64InstA) + kD64InstB;
    static_assert(kD64Stages == 5, "the wait below keeps three tiles in flight beyond the current one");
#pragma unroll
    for (int t = 0; t < kD64Stages - 1; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) issue(t, j, NOAc);
    for (int kt = 0; kt < nk; ++kt) {
      wait_vmcnt<3 * kPerTile>();  // this wave's part of tile kt has landed
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();  // ... every wave's; stage (kt + 4) % 5 is free again
      asm volatile("" ::: "memory");
      compute(kt, NOAc);
    }
  };
  if (16 * wave >= rows)
    k_loop(std::integral_constant<bool, true>{});
  else
    k_loop(std::integral_constant<bool, false>{});
  wait_vmcnt<0>();
  __syncthreads();  // the row exponents are visible

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int jn = 0; jn < (GATED ? 1 : 2); ++jn) {
      const int n = n0 + (GATED ? wn * 32 : wn * 64 + 32 * jn) + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int m = 32 * i + 8 * ii + 4 * (lane >> 5) + jj;
          if (m >= rows) continue;
          const size_t o = (size_t)(p0 + m) * N + n;
          const int ex = s_rexp[m];
          if constexpr (GATED) {
            store_h(g, o, p0 + m, ex, acc[i][0][4 * ii + jj], acc[i][1][4 * ii + jj], n == n0);
          } else {
            g.out_y[ks * g.part_stride + o] = unscale_y(acc[i][jn][4 * ii + jj], ex);
          }
        }
    }
}

// Skinny grouped GEMM for segments of a few dozen tokens (decode batches of 8+ tokens, short prefills):
// 64-token tiles, 256 threads. Each wave owns 32 output columns (gate/up: 32 gate + 32 up rows; down:
// 64 rows) and decodes its own weight rows straight into MFMA B operands: lane (n = lane % 32,
// h = lane / 32) decodes the 32 elements [32h, 32h + 32) of its row's K tile (one Q8_0 block, one
// Q4_K group), which are exactly its four 8-element fragments of the tile's four K steps (the A
// operand uses the same K order). Weights never touch LDS; activations are staged in LDS, two stages.
constexpr int SBM = 64;

// SPLIT (BF16 weights): A holds bf16 hi and lo planes and each product is two bf16 MFMAs, hi * w + lo * w,
// with the weights' bf16 bits as they are (GemmArgs::split_bf16).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int FMT, bool GATED, bool SPLIT = false>
__global__ void __launch_bounds__(256) gemm_skinny_kernel(GemmArgs g, int NT) {
  using D = Deq<FMT>;
  static_assert(!SPLIT || FMT == EMBER_TYPE_BF16, "the split path is for bf16 weights");
  constexpr int G = GATED ? 2 : 1;
  constexpr int WN = GATED ? 1 : 2;     // 32-row subtiles per matrix per wave
  constexpr int BN = GATED ? 128 : 256; // output columns per block
  constexpr int NP = SPLIT ? 2 : 1;     // A planes
  __shared__ __align__(16) _Float16 As[2][NP][SBM][LDK];

  // block -> (m-tile, n-tile, K split part); part ks covers K tiles [kt0, kt0 + nk)
  // (items m-tile fastest, numbered densely: no block of the grid's tail is left waiting behind
  // empty slots)
  const int M = launch_mtiles(g, SBM);
  if ((int)blockIdx.x >= M * NT * (g.ksplit < 1 ? 1 : g.ksplit)) return;
  const int mt = blockIdx.x % M, rest = blockIdx.x / M;
  const int nt = rest % NT, ks = rest / NT;
  const int KS = g.ksplit < 1 ? 1 : g.ksplit;
  int e = 0, p0 = 0, rows = 0;
  if (g.tiles) {
    e = g.tiles[2 * mt];
    const int m0 = g.tiles[2 * mt + 1];
    p0 = g.offsets[e] + m0;
    rows = min(SBM, g.offsets[e + 1] - p0);
  } else {
    p0 = mt * SBM;
    if (p0 >= g.T) return;
    rows = min(SBM, g.T - p0);
  }
  const int K = g.K, N = g.N, nk_all = K / GBK;
  const int kt0 = ks * nk_all / KS, nk = (ks + 1) * nk_all / KS - kt0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, nl = lane & 31;
  const int n0 = nt * BN;
  const int ncol0 = n0 + wave * (GATED ? 32 : 64);  // first output column of this wave

  // A loads: thread -> token row tid / 4, 16-element quarter (tid & 3) of the K tile
  const int a_r = tid >> 2, a_q = tid & 3;
  const _Float16* a_src = nullptr;
  if (a_r < rows) {
    const int p = p0 + a_r;
    a_src = g.A + (size_t)(g.perm ? g.perm[p] / g.k : p) * K + 16 * a_q;
  }
  // B rows of this lane: per matrix q and subtile j, row ncol0 + 32 j + nl
  const uint8_t* b_row[G][WN];
#pragma unroll
  for (int q = 0; q < G; ++q)
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n = ncol0 + 32 * j + nl;
      b_row[q][j] = n < N ? static_cast<const uint8_t*>(q ? g.W1 : g.W0) + (int64_t)e * g.expert_stride +
                                (int64_t)n * g.row_bytes
                          : nullptr;
    }

  // BF16 on the fp16 path: 2^-(row exponent) per B row
  float b_sc[G][WN];
#pragma unroll
  for (int q = 0; q < G; ++q)
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n = ncol0 + 32 * j + nl;
      b_sc[q][j] = FMT == EMBER_TYPE_BF16 && !SPLIT && n < N ? __builtin_ldexpf(1.0f, -w_exp_of(q ? g.w_exp1 : g.w_exp0, e, N, n))
                                                            : 1.0f;
    }
  u32x4 a_reg[NP][2];
  uint32_t b_raw[G][WN][D::NWH];
  auto fetch = [&](int kl) {  // K tile kt0 + kl
    const int kt = kt0 + kl;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl)
#pragma unroll
      for (int v = 0; v < 2; ++v)
        a_reg[pl][v] = a_src ? *reinterpret_cast<const u32x4*>(a_src + pl * g.a_plane + (size_t)kt * GBK + 8 * v)
                             : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < G; ++q)
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        if (b_row[q][j]) {
          D::load_half(b_row[q][j], kt, h, b_raw[q][j]);
        } else {
#pragma unroll
          for (int w = 0; w < D::NWH; ++w) b_raw[q][j][w] = 0u;
        }
      }
  };
  auto stage_a = [&](int st) {
#pragma unroll
    for (int pl = 0; pl < NP; ++pl)
#pragma unroll
      for (int v = 0; v < 2; ++v) *reinterpret_cast<u32x4*>(&As[st][pl][a_r][16 * a_q + 8 * v]) = a_reg[pl][v];
  };

  floatx16 acc[G][2][WN];
#pragma unroll
  for (int q = 0; q < G; ++q)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[q][i][j][r] = 0.0f;

  __shared__ int s_rexp[SBM];
  load_row_exps(g, p0, rows, s_rexp);
  fetch(0);
  stage_a(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int st = kt & 1;
    // decode this tile's weights (registers loaded in the previous iteration) before the loads of
    // the next tile overwrite them (the split path multiplies the bf16 bits as they are)
    uint32_t bq[G][WN][16];
#pragma unroll
    for (int q = 0; q < G; ++q)
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        if constexpr (SPLIT) {
#pragma unroll
          for (int w = 0; w < 16; ++w) bq[q][j][w] = b_raw[q][j][w];
        } else if constexpr (FMT == EMBER_TYPE_BF16) {
          bf16_to_f16_scaled(b_raw[q][j], b_sc[q][j], bq[q][j]);
        } else {
          D::decode_half(b_raw[q][j], kt0 + kt, h, bq[q][j]);
        }
      }
    if (kt + 1 < nk) fetch(kt + 1);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4 af[NP][2];
#pragma unroll
      for (int pl = 0; pl < NP; ++pl)
#pragma unroll
        for (int i = 0; i < 2; ++i) af[pl][i] = *reinterpret_cast<const u32x4*>(&As[st][pl][32 * i + nl][32 * h + 8 * s]);
#pragma unroll
      for (int q = 0; q < G; ++q)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          const u32x4 bw{bq[q][j][4 * s], bq[q][j][4 * s + 1], bq[q][j][4 * s + 2], bq[q][j][4 * s + 3]};
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            if constexpr (SPLIT) {
              acc[q][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[0][i]),
                                                                      __builtin_bit_cast(bf16x8, bw), acc[q][i][j], 0, 0, 0);
              acc[q][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[1][i]),
                                                                      __builtin_bit_cast(bf16x8, bw), acc[q][i][j], 0, 0, 0);
            } else {
              acc[q][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, af[0][i]),
                                                                     __builtin_bit_cast(half8, bw), acc[q][i][j], 0, 0, 0);
            }
          }
        }
    }
    if (kt + 1 < nk) stage_a(st ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n = ncol0 + 32 * j + nl;
      if (n >= N) continue;
      const int we0 = FMT == EMBER_TYPE_BF16 && !SPLIT ? w_exp_of(g.w_exp0, e, N, n) : 0;
      const int we1 = FMT == EMBER_TYPE_BF16 && !SPLIT && GATED ? w_exp_of(g.w_exp1, e, N, n) : 0;
      const int weh = FMT == EMBER_TYPE_BF16 && !SPLIT && GATED && g.w_hexp ? (int)g.w_hexp[e] : 0;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int m = 32 * i + 8 * ii + 4 * h + jj;
          if (m >= rows) continue;
          const size_t o = (size_t)(p0 + m) * N + n;
          const int ex = s_rexp[m];
          if constexpr (GATED) {
            if (KS > 1) {  // raw partial dots; swiglu_parts_kernel finishes the rows
              float* part = g.part_h + ((size_t)ks * g.part_rows + p0 + m) * 2 * N + n;
              part[0] = acc[0][i][j][4 * ii + jj];
              part[N] = acc[1][i][j][4 * ii + jj];
            } else {
              store_h(g, o, p0 + m, ex, __builtin_ldexpf(acc[0][i][j][4 * ii + jj], we0),
                      __builtin_ldexpf(acc[1][i][j][4 * ii + jj], we1), n == n0, weh);
            }
          } else {
            g.out_y[ks * g.part_stride + o] = unscale_y(__builtin_ldexpf(acc[0][i][j][4 * ii + jj], we0), ex);
          }
        }
    }
}

// The gated projection split over K (dense rows, GemmArgs::part_h): h[p][n] from the KS partial gate and
// up dots summed in ascending part order, then the skinny epilogue's scaling and SwiGLU. One thread per
// (row, column).
__global__ void __launch_bounds__(256) swiglu_parts_kernel(GemmArgs g, int rows, int KS) {
  const int N = g.N;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)rows * N) return;
  const int p = (int)(i / N), n = (int)(i % N);
  const float* part = g.part_h + (size_t)p * 2 * N + n;
  const size_t stride = (size_t)g.part_rows * 2 * N;
  // every part's loads issued before the ordered sum
  float pg[kMaxDenseKSplit], pu[kMaxDenseKSplit];
#pragma unroll
  for (int s = 0; s < kMaxDenseKSplit; ++s) {
    pg[s] = s < KS ? part[s * stride] : 0.0f;
    pu[s] = s < KS ? part[s * stride + N] : 0.0f;
  }
  float ga = pg[0], ua = pu[0];
#pragma unroll
  for (int s = 1; s < kMaxDenseKSplit; ++s) {
    if (s < KS) {
      ga = ga + pg[s];
      ua = ua + pu[s];
    }
  }
  const int we0 = w_exp_of(g.w_exp0, 0, N, n), we1 = w_exp_of(g.w_exp1, 0, N, n);
  const int weh = g.w_hexp ? (int)g.w_hexp[0] : 0;
  store_h(g, (size_t)p * N + n, p, row_exp(g, p), __builtin_ldexpf(ga, we0), __builtin_ldexpf(ua, we1), n == 0, weh);
}

// The tail items of a split gated launch (gated_item): block i finishes tail item i — for each of its rows
// and 128 columns the parts' raw gate and up dots summed in ascending part order, then the epilogue of the
// DMA kernel (store_h with the row's exponent). Blocks without a tail item (no split this call) exit.
__global__ void __launch_bounds__(256) gemm_tail_fixup_kernel(GemmArgs g, int NT) {
  constexpr int BN = 128;
  const int W = launch_mtiles(g, GBM) * NT;
  int full;
  const int S = tail_split(g, W, full);
  if (S <= 1 || (int)blockIdx.x >= W - full) return;
  const int w = full + blockIdx.x, mt = w / NT, nt = w % NT;
  const int e = g.tiles[2 * mt], m0 = g.tiles[2 * mt + 1];
  const int p0 = g.offsets[e] + m0, rows = min(GBM, g.offsets[e + 1] - p0);
  const int N = g.N, n0 = nt * BN;
  const size_t stride = (size_t)g.part_rows * 2 * N;
  for (int i = threadIdx.x; i < rows * BN; i += 256) {
    const int m = i / BN, c = i % BN, n = n0 + c;
    if (n >= N) continue;
    const float* part = g.part_h + (size_t)(p0 + m) * 2 * N + n;
    // every part's loads issued before the ordered sum
    float pg[kMaxTailParts], pu[kMaxTailParts];
#pragma unroll
    for (int s = 0; s < kMaxTailParts; ++s) {
      pg[s] = s < S ? part[s * stride] : 0.0f;
      pu[s] = s < S ? part[s * stride + N] : 0.0f;
    }
    float ga = pg[0], ua = pu[0];
#pragma unroll
    for (int s = 1; s < kMaxTailParts; ++s) {
      if (s < S) {
        ga = ga + pg[s];
        ua = ua + pu[s];
      }
    }
    store_h(g, (size_t)(p0 + m) * N + n, p0 + m, row_exp(g, p0 + m), ga, ua, c == 0);
  }
}

// EMBER_GEMM_DMA=0 routes Q8_0 to the register-staged kernels (a debugging switch); they have no K split
static bool dma_enabled() {
  static const bool on = [] { const char* v = std::getenv("EMBER_GEMM_DMA"); return !(v && atoi(v) == 0); }();
  return on;
}

// The DMA tile kernels take Q8_0 stacks (row slices or the prefill pack) and packed Q4_K stacks.
bool dma_path(int type, bool packed) {
  return dma_enabled() && (type == EMBER_TYPE_Q8_0 || (type == EMBER_TYPE_Q4_K && packed));
}

bool gemm_supported(int type, int K) {
  return (type == EMBER_TYPE_Q8_0 || type == EMBER_TYPE_Q4_K || type == EMBER_TYPE_BF16 || type == EMBER_TYPE_F16) &&
         K % GBK == 0;
}

int gemm_max_tiles(int T, int k, int E) { return (T * k + GBM - 1) / GBM + std::min(E, T * k); }

// One 256-token-tile DMA block per CU (its LDS ring takes more than half a CU's LDS).
int gemm_slots() { return device_cus() / 8 * 8; }

// Up to 8 parts and K / 64 (a K tile per part), while the partials (parts x rows x 2N floats) stay within
// 16 MiB (the scratch of a small batch stays well inside the no-allocation entry point's buffer).
// EMBER_TAIL_PARTS (read per call) caps the parts; 1 turns the split off.
int gemm_tail_parts(int type, bool packed, int rows, int N, int K) {
  const char* e = std::getenv("EMBER_TAIL_PARTS");
  const int cap = std::min(e ? atoi(e) : kMaxTailParts, kMaxTailParts);
  if (!dma_path(type, packed) || rows <= 0 || N <= 0) return 0;
  // by default only for K of at least 64 tiles (measured, split / whole: Mixtral-shaped K = 4096, C2 T =
  // 16 294 / 305 us, Q4_K 265 / 277; Qwen-shaped K = 2048, C3 T = 16 127 / 122.5, T = 32 163 / 159)
  if (!e && K / GBK < 64) return 0;
  const int64_t per = (int64_t)rows * 2 * N * 4;
  const int p = (int)std::min<int64_t>(std::min(cap, K / GBK), ((int64_t)16 << 20) / per);
  return p >= 2 ? p : 0;
}

// One DMA tile launch: the weight format's instantiation (Q4_K pack, Q8_0 pack, Q8_0 rows), its LDS.
template <bool GATED, bool TAIL, bool SHORT>
int launch_dma(int type, const GemmArgs& gk, int NT, unsigned nb, hipStream_t st) {
  constexpr size_t lds = SHORT ? kDmaLdsShort : kDmaLds;
  static const bool ok =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_dma_q8_kernel<GATED, kWfQ8Rows, TAIL, SHORT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_dma_q8_kernel<GATED, kWfQ8Pack, TAIL, SHORT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_dma_q8_kernel<GATED, kWfQ4Pack, TAIL, SHORT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess;
  if (!ok) return EMBER_ERR_LAUNCH;
  if (type == EMBER_TYPE_Q4_K)
    gemm_dma_q8_kernel<GATED, kWfQ4Pack, TAIL, SHORT><<<nb, kDmaThreads, lds, st>>>(gk, NT);
  else if (gk.Wp)
    gemm_dma_q8_kernel<GATED, kWfQ8Pack, TAIL, SHORT><<<nb, kDmaThreads, lds, st>>>(gk, NT);
  else
    gemm_dma_q8_kernel<GATED, kWfQ8Rows, TAIL, SHORT><<<nb, kDmaThreads, lds, st>>>(gk, NT);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

template <int FMT, bool GATED>
int launch_gemm_fmt(const GemmArgs& g, int max_mtiles, hipStream_t st) {
  constexpr int BN = GATED ? 128 : 256;
  static const bool lds_ok =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<FMT, GATED>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLds) == hipSuccess;
  if (!lds_ok) return EMBER_ERR_LAUNCH;
  const int NT = (g.N + BN - 1) / BN;
  const int mgroups = (max_mtiles + 7) / 8;
  const unsigned blocks = (unsigned)(8 * mgroups * NT);
  if (max_mtiles == 0 || NT == 0) return EMBER_OK;
  if (dma_path(FMT, g.Wp != nullptr)) {
    GemmArgs gk = g;
    if (GATED || gk.ksplit < 1) gk.ksplit = 1;
    const bool tail = GATED && gk.tail_parts > 1 && gk.slots > 0 && gk.part_h && gk.tiles;
    if (!tail) gk.tail_parts = 1;
    unsigned nb = blocks * (unsigned)gk.ksplit;
    // with a tail split: every whole round plus one round of tail parts, whatever the device-side tile count
    if (tail) nb = std::max(nb, (unsigned)((max_mtiles * NT / gk.slots + 1) * gk.slots));
    // at most 64 tokens: no tile holds more than 64 rows (EMBER_GEMM_SHORT=0, read per call: the
    // three-stage kernel anyway, whose outputs the short one matches bit for bit)
    const char* sv = std::getenv("EMBER_GEMM_SHORT");
    const bool shrt = g.T <= kShortRows && !(sv && atoi(sv) == 0);
    int s = EMBER_OK;
    if constexpr (GATED) {
      if (tail)
        s = shrt ? launch_dma<true, true, true>(FMT, gk, NT, nb, st) : launch_dma<true, true, false>(FMT, gk, NT, nb, st);
      else
        s = shrt ? launch_dma<true, false, true>(FMT, gk, NT, nb, st) : launch_dma<true, false, false>(FMT, gk, NT, nb, st);
    } else {
      s = shrt ? launch_dma<false, false, true>(FMT, gk, NT, nb, st) : launch_dma<false, false, false>(FMT, gk, NT, nb, st);
    }
    if (s) return s;
    if (tail) {
      gemm_tail_fixup_kernel<<<(unsigned)(gk.slots / 2), 256, 0, st>>>(gk, NT);
      if (hipGetLastError() != hipSuccess) return EMBER_ERR_LAUNCH;
    }
    return EMBER_OK;
  }
  if (g.split_bf16) return EMBER_ERR_TYPE;  // the split path runs in the 64-token-tile kernel only
  gemm_kernel<FMT, GATED><<<blocks, kGemmThreads, kGemmLds, st>>>(g, NT);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

template <bool GATED>
int launch_gemm_t(const GemmArgs& g, int max_mtiles, hipStream_t st) {
  switch (g.type) {
    case EMBER_TYPE_Q8_0: return launch_gemm_fmt<EMBER_TYPE_Q8_0, GATED>(g, max_mtiles, st);
    case EMBER_TYPE_Q4_K: return launch_gemm_fmt<EMBER_TYPE_Q4_K, GATED>(g, max_mtiles, st);
    case EMBER_TYPE_BF16: return launch_gemm_fmt<EMBER_TYPE_BF16, GATED>(g, max_mtiles, st);
    case EMBER_TYPE_F16: return launch_gemm_fmt<EMBER_TYPE_F16, GATED>(g, max_mtiles, st);
    default: return EMBER_ERR_TYPE;
  }
}

int launch_gemm(const GemmArgs& g, bool gated, int max_mtiles, hipStream_t st) {
  return gated ? launch_gemm_t<true>(g, max_mtiles, st) : launch_gemm_t<false>(g, max_mtiles, st);
}

template <int FMT, bool GATED>
int launch_skinny_fmt(GemmArgs g, int max_mtiles, hipStream_t st) {
  constexpr int BN = GATED ? 128 : 256;
  const int NT = (g.N + BN - 1) / BN;
  if (max_mtiles == 0 || NT == 0) return EMBER_OK;
  if (dma_path(FMT, g.Wp != nullptr)) {
    static const bool ok =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_dma64_q8_kernel<GATED, kWfQ8Rows>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kD64Lds) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_dma64_q8_kernel<GATED, kWfQ8Pack>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kD64Lds) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_dma64_q8_kernel<GATED, kWfQ4Pack>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kD64Lds) == hipSuccess;
    if (!ok) return EMBER_ERR_LAUNCH;
    if (GATED || g.ksplit < 1) g.ksplit = 1;
    const unsigned blocks = (unsigned)(max_mtiles * NT * g.ksplit);
    if (FMT == EMBER_TYPE_Q4_K)
      gemm_dma64_q8_kernel<GATED, kWfQ4Pack><<<blocks, kD64Threads, kD64Lds, st>>>(g, NT);
    else if (g.Wp)
      gemm_dma64_q8_kernel<GATED, kWfQ8Pack><<<blocks, kD64Threads, kD64Lds, st>>>(g, NT);
    else
      gemm_dma64_q8_kernel<GATED, kWfQ8Rows><<<blocks, kD64Threads, kD64Lds, st>>>(g, NT);
    return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
  }
  // K split: plain projections into out_y parts; gated ones (dense rows only) into part_h, then finished
  if (g.ksplit < 1 || (GATED && (g.tiles || !g.part_h))) g.ksplit = 1;
  const unsigned blocks = (unsigned)(max_mtiles * NT * g.ksplit);
  bool launched = false;
  if constexpr (FMT == EMBER_TYPE_BF16) {
    if (g.split_bf16) {
      gemm_skinny_kernel<FMT, GATED, true><<<blocks, 256, 0, st>>>(g, NT);
      launched = true;
    }
  }
  if (!launched) gemm_skinny_kernel<FMT, GATED><<<blocks, 256, 0, st>>>(g, NT);
  if (hipGetLastError() != hipSuccess) return EMBER_ERR_LAUNCH;
  if (GATED && g.ksplit > 1) {
    const int64_t n = (int64_t)g.T * g.N;
    swiglu_parts_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(g, g.T, g.ksplit);
    if (hipGetLastError() != hipSuccess) return EMBER_ERR_LAUNCH;
  }
  return EMBER_OK;
}

template <bool GATED>
int launch_skinny_t(const GemmArgs& g, int max_mtiles, hipStream_t st) {
  switch (g.type) {
    case EMBER_TYPE_Q8_0: return launch_skinny_fmt<EMBER_TYPE_Q8_0, GATED>(g, max_mtiles, st);
    case EMBER_TYPE_Q4_K: return launch_skinny_fmt<EMBER_TYPE_Q4_K, GATED>(g, max_mtiles, st);
    case EMBER_TYPE_BF16: return launch_skinny_fmt<EMBER_TYPE_BF16, GATED>(g, max_mtiles, st);
    case EMBER_TYPE_F16: return launch_skinny_fmt<EMBER_TYPE_F16, GATED>(g, max_mtiles, st);
    default: return EMBER_ERR_TYPE;
  }
}

int launch_gemm_skinny(const GemmArgs& g, bool gated, int max_mtiles, hipStream_t st) {
  return gated ? launch_skinny_t<true>(g, max_mtiles, st) : launch_skinny_t<false>(g, max_mtiles, st);
}

int gemm_dense_ksplit(bool gated, int T, int N, int K, int64_t weight_bytes) {
  const int mt = (T + SBM - 1) / SBM, nt = (N + (gated ? 127 : 255)) / (gated ? 128 : 256), nk = K / GBK;
  const int64_t part_row = (int64_t)T * N * 4 * (gated ? 2 : 1);  // bytes of one part
  int ks = 1;
  while (2 * ks <= kMaxDenseKSplit && (int64_t)mt * nt * ks < 512 && nk / (2 * ks) >= 2 &&
         2 * ks * part_row <= weight_bytes)
    ks *= 2;
  return ks;
}

int gemm_skinny_max_tiles(int T, int k, int E) { return (T * k + SBM - 1) / SBM + std::min(E, T * k); }

// Expected row tiles (of `bm` rows) of T tokens' k picks over E experts under uniform routing: an expert's
// rows n ~ Binomial(T k, 1 / E) make E[ceil(n / bm)] = sum over j >= 0 of P(n > bm j) tiles (normal
// approximation for j >= 1).
static double expected_row_tiles(int T, int k, int E, int bm) {
  const double m = (double)T * k / E, sd = std::sqrt(m * (1.0 - 1.0 / E));
  double per_e = 1.0 - std::pow(1.0 - 1.0 / E, (double)T * k);  // P(n > 0)
  for (int j = 1; j <= 4096 && bm * j < m + 8 * sd + bm; ++j)
    per_e += sd > 0 ? 0.5 * std::erfc((bm * j + 0.5 - m) / (sd * std::sqrt(2.0))) : (m > bm * j ? 1.0 : 0.0);
  return E * per_e;
}

int gemm_ksplit(int type, bool packed, int T, int k, int E, int N, int K) {
  if (!dma_path(type, packed)) return 1;  // the split lives in the DMA kernels
  // tuning override, clamped so that every part holds at least one K tile
  if (const char* v = std::getenv("EMBER_KSPLIT")) return std::max(1, std::min(std::min(kMaxKSplit, K / GBK), atoi(v)));
  // The launch runs tiles * ks blocks in rounds of `slots`; a part of a round costs a whole round, so ks
  // minimises ceil(tiles * ks / slots) / ks (ties to fewer parts: each part is another y row the combine
  // reads), among the splits that keep >= 32 K tiles per part and are reached while the blocks are fewer
  // than four rounds. tiles: the expected 256-token tiles of uniform routing (an expert's rows n ~
  // Binomial(T k, 1 / E) make E[ceil(n / 256)] tiles; normal approximation) times the n-tiles.
  // Mixtral-shaped down projection (K = 14336), ks 1 / 2 / 4, one box: T = 768 814 / 748 / 769 us,
  // T = 1024 1020 / 1047 / 1017 (about half the experts take a second, short tile), T = 8 - / 278 / 282.
  const double tiles = expected_row_tiles(T, k, E, GBM) * ((N + 255) / 256);
  const double slots = std::max(1, gemm_slots());
  auto rounds = [&](int ks) { return std::ceil(tiles * ks / slots - 1e-6); };  // (a whole count stays whole)
  int best = 1;
  double best_cost = rounds(1);
  for (int ks = 2; ks <= kMaxKSplit && K / GBK >= 32 * ks && tiles * ks / 2 < 4 * slots; ks *= 2) {
    const double cost = rounds(ks) / ks;
    if (cost < best_cost - 1e-9) best = ks, best_cost = cost;
  }
  return best;
}

int gemm_skinny_ksplit(int type, bool packed, int T, int k, int E, int N, int K) {
  (void)type;
  (void)packed;
  // tuning override, clamped so that every part holds at least one K tile
  if (const char* v = std::getenv("EMBER_KSPLIT")) return std::max(1, std::min(std::min(kMaxKSplit, K / GBK), atoi(v)));
  // up to 1024 blocks of the expected 64-token tiles (uniform routing; the worst-case tile count the grid
  // is sized for stopped the split early at small T), with at least 5 K tiles per part. C4-shaped down
  // projection (K = 1408: 22 K tiles), split 1 / 2 / 4: T = 16 151 / 132 / 127 us, T = 64 165 / 146 /
  // 142, T = 128 166 / 150 / 149, T = 256 189 / 186 / 199 (it was the worst-case count: 2 at all four).
  const double blocks = expected_row_tiles(T, k, E, 64) * ((N + 255) / 256);
  int ks = 1;
  while (ks < kMaxKSplit && blocks * ks <= 1023 && K / GBK >= 5 * ks * 2) ks *= 2;  // (a whole 1024 stays)
  return ks;
}

// The activation conversion on its own (act_conv_row): one block per row.
__global__ void __launch_bounds__(256) act_conv_kernel(ActConv c) { act_conv_row(c, blockIdx.x); }

int launch_act_conv(const ActConv& c, hipStream_t st) {
  if (c.rows <= 0 || (!c.y16 && !c.yb)) return EMBER_OK;
  act_conv_kernel<<<(unsigned)c.rows, 256, 0, st>>>(c);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

// Tile table for the grouped GEMMs: (expert, first token) of every bm-token tile of every expert
// segment with tokens, ascending by expert. One thread; E entries of offsets.

int gemm_tile_rows(bool skinny) { return skinny ? SBM : GBM; }


// ---- BF16 row exponents (the prefill pack of a BF16 layer): one wave per row
__global__ void __launch_bounds__(256) bf16_row_exp_kernel(const uint8_t* __restrict__ W, int64_t rows, int K,
                                                           int64_t row_bytes, int16_t* __restrict__ out) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const uint16_t* row = reinterpret_cast<const uint16_t*>(W + r * row_bytes);
  float m = 0.0f;
  for (int i = lane; i < K; i += 64) {
    const float v = fabsf(bf16_f32(row[i]));
    if (v <= 3.4e38f) m = fmaxf(m, v);  // finite values only (NaN fails the test)
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) {
    int ex = 0;
    if (m > 0.0f) (void)__builtin_frexpf(m, &ex);
    out[r] = (int16_t)max(-120, min(120, ex));
  }
}

// per expert: max over its rows n of gate_exp[n] + up_exp[n] (one block per expert)
__global__ void __launch_bounds__(256) bf16_pair_max_kernel(const int16_t* __restrict__ ge, const int16_t* __restrict__ ue,
                                                            int N, int16_t* __restrict__ out) {
  __shared__ int red[4];
  const int e = blockIdx.x;
  int m = -32768;
  for (int n = threadIdx.x; n < N; n += 256) m = max(m, (int)ge[(int64_t)e * N + n] + (int)ue[(int64_t)e * N + n]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) out[e] = (int16_t)max(max(red[0], red[1]), max(red[2], red[3]));
}

int launch_bf16_pair_max(const int16_t* ge, const int16_t* ue, int E, int N, int16_t* out, hipStream_t st) {
  if (E <= 0 || N <= 0) return EMBER_OK;
  bf16_pair_max_kernel<<<dim3((unsigned)E), 256, 0, st>>>(ge, ue, N, out);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

int launch_bf16_row_exps(const void* W, int64_t rows, int K, int64_t row_bytes, int16_t* out, hipStream_t st) {
  if (rows <= 0) return EMBER_OK;
  bf16_row_exp_kernel<<<dim3((unsigned)((rows + 3) / 4)), 256, 0, st>>>(static_cast<const uint8_t*>(W), rows, K,
                                                                         row_bytes, out);
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

// ---- prefill pack: one thread per (tile, row), one pack row each (a one-time copy at weight load)
template <int FMT>
__global__ void __launch_bounds__(256) prefill_pack_kernel(const uint8_t* __restrict__ W0, const uint8_t* __restrict__ W1,
                                                           int64_t expert_stride, int64_t row_bytes, int N, int NT,
                                                           int nk, int64_t total_rows, uint8_t* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total_rows) return;
  const int r = (int)(i % 256);
  int64_t t = i / 256;
  const int kc = (int)(t % nk);
  t /= nk;
  const int nt = (int)(t % NT), e = (int)(t / NT);
  const bool gated = W1 != nullptr;
  const int q = gated ? (r >> 7) : 0;
  const int n = min(nt * (gated ? 128 : 256) + (gated ? (r & 127) : r), N - 1);
  const uint8_t* row = (q ? W1 : W0) + (int64_t)e * expert_stride + (int64_t)n * row_bytes;
  if constexpr (FMT == EMBER_TYPE_Q4_K) {
    // K tile kc = quarter kc % 4 of super-block kc / 4: its groups 2 (kc % 4) and + 1
    uint32_t raw[12];
    Deq<EMBER_TYPE_Q4_K>::load(row, kc, raw);
    const float dd = half_bits_to_float(raw[0] & 0xffff), dmin = half_bits_to_float(raw[0] >> 16);
    uint32_t* d = reinterpret_cast<uint32_t*>(dst + i * kPackRowQ4B);
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      int sc, mn;
      Deq<EMBER_TYPE_Q4_K>::scale_min(raw, 2 * (kc & 3) + gi, &sc, &mn);
      const half2_t am = {(_Float16)(dd * (float)sc), (_Float16)(-(dmin * (float)mn))};
      d[gi] = u32(am);
    }
#pragma unroll
    for (int w = 0; w < 8; ++w) d[2 + w] = raw[4 + w];
  } else {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(row + (int64_t)kc * kPackRowB);
    uint32_t* d = reinterpret_cast<uint32_t*>(dst + i * kPackRowB);
#pragma unroll
    for (int w = 0; w < kPackRowB / 4; ++w) d[w] = src[w];
  }
}

int launch_prefill_pack(int type, const void* W0, const void* W1, int64_t expert_stride, int64_t row_bytes, int E,
                        int N, int K, uint8_t* dst, hipStream_t st) {
  const int NT = W1 ? (N + 127) / 128 : (N + 255) / 256, nk = K / 64;
  const int64_t total = (int64_t)E * NT * nk * 256;
  if (total == 0) return EMBER_OK;
  const int64_t blocks = (total + 255) / 256;
  const uint8_t* w0 = static_cast<const uint8_t*>(W0);
  const uint8_t* w1 = static_cast<const uint8_t*>(W1);
  if (type == EMBER_TYPE_Q4_K)
    prefill_pack_kernel<EMBER_TYPE_Q4_K><<<dim3((unsigned)blocks), 256, 0, st>>>(w0, w1, expert_stride, row_bytes, N, NT,
                                                                                nk, total, dst);
  else if (type == EMBER_TYPE_Q8_0)
    prefill_pack_kernel<EMBER_TYPE_Q8_0><<<dim3((unsigned)blocks), 256, 0, st>>>(w0, w1, expert_stride, row_bytes, N, NT,
                                                                                nk, total, dst);
  else
    return EMBER_ERR_TYPE;
  return hipGetLastError() == hipSuccess ? EMBER_OK : EMBER_ERR_LAUNCH;
}

}  // namespace ember_moe
