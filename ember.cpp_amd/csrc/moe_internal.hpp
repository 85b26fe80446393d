// Internal declarations shared by the MoE FFN translation units (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include "ember_moe.h"
#include "moe_math.hpp"

namespace ember_moe {

// Block-cooperative copy of n 16-byte granules from global memory to LDS. Loads are issued in
// batches of 8 per thread before any store, so a thread waits for one memory latency per batch
// instead of one per granule.
__device__ inline void copy16_to_lds(void* dst, const void* src, int n) {
  typedef uint32_t v4 __attribute__((ext_vector_type(4)));
  v4* d = static_cast<v4*>(dst);
  const v4* g = static_cast<const v4*>(src);
  const int stride = blockDim.x;
  for (int base = threadIdx.x; base < n; base += 8 * stride) {
    v4 t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (base + u * stride < n) t[u] = g[base + u * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (base + u * stride < n) d[base + u * stride] = t[u];
  }
}

// Device buffers of the dispatch step, carved from the caller's scratch.
// Activation conversion for the MFMA paths (act_conv_row): x [rows][K] f32 into fp16 rows scaled by 2^-e
// (y16, e in yexp; null: not needed) and / or split bf16 planes (yb, lo plane `plane` elements on; null:
// not needed).
struct ActConv {
  const float* x;
  int rows, K;
  _Float16* y16;
  int32_t* yexp;
  uint16_t* yb;
  int64_t plane;
};

struct DispatchScratch {
  int32_t* rank;       // [T*k] rank of each slot among equal experts in its 64-slot chunk
  int32_t* chunk_cnt;  // [ceil(T*k/64)][E] counts, then per-chunk base positions
  int32_t* offsets;    // [E+1]
  int32_t* used;       // [E] experts with at least one slot, ascending
  int32_t* n_used;     // [1]
  int32_t* perm;       // [T*k] sorted position -> slot t*k+j
  int32_t* pos;        // [T*k] slot -> sorted position (-1: no pick)
  // optional (null: none): the MFMA GEMMs' tile table, written by the dispatch's last step: tiles of
  // tile_bm rows over each expert's segment, experts ascending, as (expert, first row) pairs
  int32_t* tiles = nullptr;
  int32_t* n_tiles = nullptr;
  int tile_bm = 0;
};

int launch_router_logits(const float* x, int T, int d, int E, const float* R, float* logits, hipStream_t st);
// Router logits of a small batch, one block per (expert, token) pair (router_block_logit's exact chains):
// for T E <= 1024, d % 4 == 0, d <= 8192.
bool router_blocks_fit(int T, int d, int E);
int launch_router_logits_blocks(const float* x, int T, int d, int E, const float* R, float* logits, hipStream_t st);
// Proven-picks router for renormalised softmax routers (moe_router_fast.hip): router logits exact for
// every expert the int8 fast logits' bound cannot rule out (the picks among them), a proven lower bound
// elsewhere, then the routing (idx, gates) as launch_route gives it. work: router_fast_work_bytes.
bool router_fast_fits(int T, int d, int E, int k, int renorm, int routed);
size_t router_fast_work_bytes(int T, int d, int E);
int launch_router_fast(const float* x, int T, int d, int E, int k, const float* R, float* logits, int32_t* idx,
                       float* gates, void* work, const ActConv* conv, hipStream_t st);
// conv (nullable): activation conversion run by extra blocks of the same launch
int launch_route(const float* logits, int T, int E, int k, int renorm, int routed, int sigmoid, const float* bias,
                 int groups_n, int groups_top, int32_t* idx, float* gates, const ActConv* conv, hipStream_t st);
int launch_dispatch(const int32_t* idx, int T, int k, int E, const DispatchScratch& ds, hipStream_t st);
// Routing + dispatch; one fused kernel for decode-sized batches, else launch_route + launch_dispatch.
int launch_route_dispatch(const float* logits, int T, int E, int k, int renorm, int routed, int sigmoid,
                          const float* bias, int groups_n, int groups_top, int32_t* idx, float* gates,
                          const DispatchScratch& ds, const ActConv* conv, hipStream_t st);

bool type_quantizes_activations(int type);
// Compute units of the current device (0 on error); cached per device.
int device_cus();
// Blocks per CU of kernel fn with `threads` threads and `lds` dynamic LDS bytes on the current device
// (its dynamic-LDS limit raised to max_lds first); 0 on error. Cached per (kernel, device, LDS), thread-safe.
int blocks_per_cu(const void* fn, int threads, size_t lds, size_t max_lds);
int proj_max_row_bytes();  // LDS bytes one staged activation row of the decode kernel may take

// One projection launch over expert segments: out[p][row] for rows [0, rows) of a [rows][K] matrix
// per segment. Routed segments are the experts used[0..*n_used) with the dispatch-order positions
// offsets[e]..offsets[e+1); an optional shared-expert segment (s_w0 non-null, same weight type) covers
// tokens 0..T-1 and is scheduled in the same launch. Activations are f32; the quantizing formats
// quantize them to int16 per 32-element block while staging them into LDS.
struct ProjArgs {
  int type;               // ggml type of every matrix of the launch
  bool gated;             // gate/up pair + SwiGLU vs a plain projection
  // routed segments (used non-null)
  const void* w0;         // gate (or the only) stack base
  const void* w1;         // up stack base (gated) or null
  int rows, K;            // matrix shape per expert
  int64_t expert_stride;  // bytes between consecutive experts' matrices
  const float* in;        // x [T][K] (gathered through perm) or h [npos][K]
  float* out;             // h [npos][rows] or y [npos][rows], dispatch order
  const int32_t* offsets;
  const int32_t* used;
  const int32_t* n_used;
  const int32_t* perm;
  int k;                  // slots per token; the input row of position p is perm[p] / k when in_by_perm
  bool in_by_perm;
  int max_segments;       // upper bound on *n_used
  // shared expert segment (s_w0 non-null): tokens 0..T-1, input rows t, output rows t
  const void* s_w0;
  const void* s_w1;
  int s_rows, s_K;
  const float* s_in;
  float* s_out;
  int T;
  // host side only: when set, the launch records these events in its dispatch packet (kernel timing)
  hipEvent_t ev_start, ev_stop;
  // Routing fused into a one-token gate/up launch (route.flag non-null): blocks 0..E-1 each compute
  // one expert's router logit and publish it in a tagged word of the flag area (words 2..E+1); every
  // block collects them (a logit still missing after spin_limit polls it computes itself), computes the
  // same picks and gates and builds the one-token dispatch; block 0 also writes the routing and
  // dispatch (idx, gates, pos, offsets, used, n_used, perm) for the later launches. With the softmax
  // router each router block also publishes a bounded fast logit (words E+2 .. 2E+1), from which the
  // other blocks prove the pick set before the exact logits are summed. A later launch of the same call
  // (clear_flag) zeroes both sets of words, and the tags change per call, so stale words never carry
  // this call's tag (a word of uninitialised scratch matches a 32-bit tag by chance with probability
  // 2^-32). Word 0 counts the blocks that computed a missing logit themselves, word 1 the calls whose
  // exact picks contradicted the fast bounds; word 2 + 2E is this call's conflict status (0 / 1), read by
  // the launch that writes the output (NaN rows when set).
  struct Route {
    unsigned long long* flag;  // 2 E + 3 words
    const float* x;       // the token [d]
    const float* router;  // [E][d]
    int d, E, renorm, routed, sigmoid, groups_n, groups_top;
    const float* bias;
    float* logits;        // [E]
    int32_t* idx;         // [k]
    float* gates;         // [k]
    int32_t* pos;         // [k]
    int32_t *offsets, *used, *n_used, *perm;  // the dispatch (the launch's read-only views alias these)
    unsigned spin_limit;  // polls of a logit word before the block computes that logit itself
    int no_publish;       // test hook: router blocks do not publish (every block computes every logit)
    int test_corrupt;     // test hook: the fast words carry wrong values under their bounds
    uint32_t logit_tag, fast_tag;  // this call's tags of the exact and fast logit words (nonzero, distinct)
  } route;
  unsigned long long* clear_flag;  // non-null: block 0 of this launch zeroes clear_n words of the flag area
  int clear_n;
};
// One-token layer over d_ff slices (decode, T = 1, a prefill pack present): one launch in which block
// 1 + j * ns + c (ns = d_ff / 64 slices) owns slice c of pick j — the slice's 64 gate and 64 up rows
// (SwiGLU into LDS), then the matching 64 columns of the down projection, streamed as the pack's tiles —
// and writes the slice's partial output part[j][c][0..d); the routing prologue is proj_kernel's fused
// one (block 0: the exact routing record). A second launch sums the partials in fixed order and forms
// the output as the combine does.
struct SliceArgs {
  ProjArgs p;              // route (the fused routing), k, type, ev_start / ev_stop
  const uint8_t* pack_gu;  // the pack's gate/up section [E][ceil(d_ff / 128)][d / 64] tiles
  const uint8_t* pack_dn;  // its down section [E][ceil(d / 256)][d_ff / 64] tiles
  int d, d_ff;
  float* part;             // [k][d_ff / 64][d]
};
bool slices_fit(int type, int d, int d_ff, int E, int k, bool any_size);
int launch_slices(const SliceArgs& a, hipStream_t st);
// out[o] = sum over valid picks j ascending of gates[j] * (sum over slices of part[j][c][o]), then
// (x * scale) + 0; NaN rows when *conflict is set.
// (clear_flag: clear_n words this launch zeroes, the fused routing's logit words, for the next call)
int launch_slice_reduce(const float* part, int ns, int d, int k, const int32_t* idx, const float* gates, float scale,
                        const unsigned long long* conflict, unsigned long long* clear_flag, int clear_n, float* out,
                        hipStream_t st);
// the fused routing's shape limits (the router blocks' and block 0's LDS)
bool fused_route_fits(int type, int d, int E, int k);
constexpr unsigned long long kRouteReady = 0x5e11a7ed0ddba11full;
constexpr int kMaxRouteE = 256;  // experts a fused routing block handles

int launch_projection(const ProjArgs& a, hipStream_t st);

// One-token down projection with the combine fused in (decode, T = 1): out[o] over the token's picks
// (pos / idx / gates of its k slots) and the optional shared expert, in combine_kernel's order.
constexpr int kDown1MaxPicks = 8;
constexpr int kDown1Slots = 512;  // output rows one block owns, at most
struct Down1Args {
  int type;
  const void* w;           // down stack base [E][d][K]
  int64_t expert_stride;
  int d, K, k;
  const float* h;          // [npos][K] dispatch order
  const int32_t* pos;      // [k] slot -> dispatch position (-1: none)
  const int32_t* idx;      // [k]
  const float* gates;      // [k]
  const void* s_w;         // shared expert's down [d][s_K], or null
  int s_K;
  const float* s_h;        // [s_K]
  const float* sg_logit;   // qwen2moe shared-expert gate logit, or null
  float scale;
  float* out;              // [d]
  int nslots;              // set by the launcher
  unsigned long long* clear_flag;
  int clear_n;
  const unsigned long long* conflict;  // the fused routing's conflict word, or null (NaN rows when set)
  hipEvent_t ev_start, ev_stop;
};
bool down1_fits(int type, int d, int K, int k, int s_K);
int launch_down1(const Down1Args& a, hipStream_t st);


// Grouped MFMA GEMM (prefill). Tiles come from `tiles` (pairs expert, first token; *n_tiles valid)
// over expert segments of the dispatch order, or, when tiles is null, cover T rows of one matrix.
struct GemmArgs {
  const _Float16* A;       // activation rows, fp16 [*][K]
  const int32_t* perm;     // non-null: row of sorted position p is perm[p] / k
  int k, T;
  const void* W0;          // gate (or the only) stack
  const void* W1;          // up stack (gated) or null
  int64_t expert_stride;   // bytes between experts' matrices
  int64_t row_bytes;       // bytes of one weight row of K elements
  int type;
  int N, K;
  const int32_t* tiles;
  const int32_t* n_tiles;
  const int32_t* offsets;
  _Float16* out_h;         // gated: silu(gate) * up as fp16 [pos][N]
  float* out_y;            // plain: f32 [pos][N]
  int ksplit;              // plain projections: K split over this many blocks, partial sums to
  int64_t part_stride;     // out_y + s * part_stride (floats), summed in order by the combine
  const uint8_t* Wp;       // non-null: this projection's tiles in the prefill pack (Q8_0, 256-token tiles)
  // Activation range (fp16 operands): A row r holds its values times 2^-a_exp[r] (a_exp indexed as the A
  // rows are: tokens for gate/up, dispatch positions for down; null: unscaled). The gated epilogue
  // undoes the scale before SwiGLU and writes h times 2^-h_exp[p] with h_exp[p] = 2 a_exp (h grows as
  // the product of two projections of x); the plain epilogue multiplies by 2^a_exp. Powers of two:
  // exact.
  const int32_t* a_exp;
  int32_t* h_exp;
  // BF16 weights: bf16 MFMA with A as two bf16 planes, hi = bf16(v) and lo = bf16(v - hi), lo at
  // A + a_plane elements (the products hi * w + lo * w in fp32); the gated epilogue writes h the same
  // way (lo at out_h + h_plane). No range scaling: bf16 has f32's exponent range.
  bool split_bf16;
  int64_t a_plane, h_plane;
  // BF16 weights on the fp16 path (a prefill pack's row exponents): row n of expert e of W0 (W1) enters
  // the MFMAs times 2^-w_exp0[e N + n] (2^-w_exp1[...]), which puts its largest magnitude in [0.5, 1),
  // and the epilogue multiplies that output column by 2^w_exp. Null: unscaled.
  const int16_t* w_exp0;
  const int16_t* w_exp1;
  // ... and per expert the largest w_exp0[n] + w_exp1[n] of its rows: the gated epilogue stores h times
  // 2^-(2 a_exp + w_hexp[e]) (h_exp includes it), so weights far from 1 keep h within fp16's range
  const int16_t* w_hexp;
  // gated projections of dense rows split over K (64-token tiles): raw partial gate / up dots of part s at
  // part_h + (s * part_rows + p) * 2N (+ N for up), finished by a SwiGLU pass
  float* part_h;
  int part_rows;
  // 256-token-tile gate/up (DMA kernels): the work items past the last whole round of `slots` blocks (the
  // tail) split over K into up to tail_parts parts, raw partials at part_h as above (part_rows = T k),
  // finished by gemm_tail_fixup_kernel. tail_parts <= 1: no split.
  int tail_parts, slots;
};
// Parts of the tail split (GemmArgs::tail_parts) for a gated 256-token-tile launch of T k rows against
// N = d_ff columns over K = d: 0 when it does not apply (the partials' size bound); and the resident blocks
// per round (a multiple of 8).
int gemm_tail_parts(int type, bool packed, int rows, int N, int K);
int gemm_slots();
// The prefill pack of a BF16 layer: per weight row the exponent e (int16) that puts the row's largest
// finite magnitude in [0.5, 1) (clamped to [-120, 120]; 0 for a row of zeros), for the routed gate [E][d_ff],
// up [E][d_ff], down [E][d], then per expert the largest gate + up exponent of its rows [E]; then, when the
// shared expert's stacks are BF16 too, its gate [d_ff_shared], up [d_ff_shared], down [d] and gate + up
// maximum [1]; each section 256-byte aligned.
struct Bf16ExpLayout {
  int64_t gate, up, down, hmax, sgate, sup, sdown, shmax, end;  // byte offsets (-1: no section)
};
inline Bf16ExpLayout bf16_exp_layout(int d, int d_ff, int E, int d_ff_shared, bool shared) {
  auto al = [](int64_t v) { return (v + 255) & ~(int64_t)255; };
  Bf16ExpLayout p;
  int64_t o = 0;
  p.gate = o; o = al(o + (int64_t)E * d_ff * 2);
  p.up = o; o = al(o + (int64_t)E * d_ff * 2);
  p.down = o; o = al(o + (int64_t)E * d * 2);
  p.hmax = o; o = al(o + (int64_t)E * 2);
  p.sgate = p.sup = p.sdown = p.shmax = -1;
  if (shared) {
    p.sgate = o; o = al(o + (int64_t)d_ff_shared * 2);
    p.sup = o; o = al(o + (int64_t)d_ff_shared * 2);
    p.sdown = o; o = al(o + (int64_t)d * 2);
    p.shmax = o; o = al(o + 2);
  }
  p.end = o;
  return p;
}
// rows BF16 rows of K elements (row_bytes apart) -> their exponents (Bf16ExpLayout)
int launch_bf16_row_exps(const void* W, int64_t rows, int K, int64_t row_bytes, int16_t* out, hipStream_t st);
// out[e] = max over n < N of ge[e N + n] + ue[e N + n], e < E
int launch_bf16_pair_max(const int16_t* ge, const int16_t* ue, int E, int N, int16_t* out, hipStream_t st);
// Prefill pack (ember_moe_prefill_pack): tiles of 256 weight rows x 64 columns, one tile contiguous;
// the gate/up section [E][ceil(d_ff / 128)][d / 64] (each tile: the 128 gate rows of an n-tile, then
// its 128 up rows), then the down section [E][ceil(d / 256)][d_ff / 64]; rows past a matrix's end
// repeat its last row (as the GEMM's clamped loads would). A row's 64 columns:
//   Q8_0 stacks: the two Q8_0 blocks as they are (68 bytes);
//   Q4_K stacks: 40 bytes = the fp16 factors {a0, m0, a1, m1} of its two 32-element groups, a = d * sc
//     and m = -dmin * mn each rounded to fp16 once (weight = a * q + m), then the 32 nibble bytes of the
//     super-block quarter as they are (low nibbles: group 0, high nibbles: group 1).
constexpr int kPackRowB = 68;
constexpr int kPackRowQ4B = 40;
inline int pack_row_bytes(int type) { return type == EMBER_TYPE_Q4_K ? kPackRowQ4B : kPackRowB; }
inline int64_t pack_tile_bytes(int type) { return (int64_t)256 * pack_row_bytes(type); }
constexpr int64_t kPackTileB = (int64_t)256 * kPackRowB;
struct PackLayout {
  int nt_gu, nk_gu, nt_dn, nk_dn;
  int64_t gu, dn, end;  // byte offsets of the sections, total
};
inline PackLayout pack_layout(int d, int d_ff, int E, int type) {
  PackLayout p;
  p.nt_gu = (d_ff + 127) / 128;
  p.nk_gu = d / 64;
  p.nt_dn = (d + 255) / 256;
  p.nk_dn = d_ff / 64;
  p.gu = 0;
  p.dn = (int64_t)E * p.nt_gu * p.nk_gu * pack_tile_bytes(type);
  p.end = p.dn + (int64_t)E * p.nt_dn * p.nk_dn * pack_tile_bytes(type);
  return p;
}
// Fills one section of the pack from ggml rows of `type` (Q8_0 or Q4_K; W1 non-null: the gate/up section).
int launch_prefill_pack(int type, const void* W0, const void* W1, int64_t expert_stride, int64_t row_bytes, int E,
                        int N, int K, uint8_t* dst, hipStream_t st);
bool gemm_supported(int type, int K);
int gemm_max_tiles(int T, int k, int E);
int launch_gemm(const GemmArgs& g, bool gated, int max_mtiles, hipStream_t st);
// The activation conversion (ActConv) as a launch of its own: one block per row.
int launch_act_conv(const ActConv& c, hipStream_t st);
// rows per tile of the MFMA GEMMs' tile table (DispatchScratch::tile_bm): 64-token or 256-token tiles
int gemm_tile_rows(bool skinny);
// Skinny variant for segments of a few dozen tokens (64-token tiles).
int launch_gemm_skinny(const GemmArgs& g, bool gated, int max_mtiles, hipStream_t st);
int gemm_skinny_max_tiles(int T, int k, int E);
// K split of the skinny path's plain (down) projection: 1..kMaxKSplit, so that the launch has enough
// blocks for the chip when the output is narrow
constexpr int kMaxKSplit = 4;
int gemm_skinny_ksplit(int type, bool packed, int T, int k, int E, int N, int K);
// ... and of a dense projection (the shared expert's T rows) on the 64-token tiles, gated or plain: up to
// kMaxDenseKSplit parts, until the launch has 512 blocks, each part keeps >= 2 K tiles and the partial
// sums (f32) stay within the weights' bytes
constexpr int kMaxDenseKSplit = 16;
int gemm_dense_ksplit(bool gated, int T, int N, int K, int64_t weight_bytes);
// ... and of the 256-token-tile path's (the down launch of a long prefill has few blocks per n-tile row)
int gemm_ksplit(int type, bool packed, int T, int k, int E, int N, int K);
// Whether the DMA tile kernels serve stacks of `type` (packed: with a prefill pack): Q8_0, packed Q4_K.
bool dma_path(int type, bool packed);

int launch_combine(const float* y, int nparts, int64_t part_stride, const float* gates, const int32_t* pos,
                   const float* y_shared, int s_parts, int64_t s_stride, const float* shared_gate_logit, float scale, int T,
                   int k, int d, float* out, hipStream_t st, const unsigned long long* conflict = nullptr);

}  // namespace ember_moe
