// The C ABI of the MoE FFN (include/ember_moe.h): descriptor validation, the scratch layout and the
// launch sequence router -> route -> dispatch -> gate/up(+SwiGLU) -> down -> [shared expert] ->
// combine, all on the caller's stream with no host synchronisation (cuda_kernels.cu:3628-3684 has
// the same shape: router GEMM, routing kernel, expert products, SwiGLU, combine). One-token calls fold
// the first three into the gate/up launch, and with a prefill pack run the slice launch + reduce instead
// (plan(): the launch plan, also reported by ember_moe_path).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <tuple>
#include <cstdlib>
#include <cmath>
#include <string>

#include "moe_internal.hpp"

namespace ember_moe {
namespace {

constexpr int kMaxE = 512;  // route_kernel keeps one bit per (lane, 64-expert stripe) and LDS rows of E
constexpr int kMaxK = 64;   // picks live in a 64-entry LDS array per wave
// Expert-product kernels by tokens per expert (M): the int16-dot GEMV while M is at most a few tokens,
// the skinny MFMA GEMM (64-token tiles) for up to ~100, the 256-token-tile MFMA GEMM beyond.
enum PathMode { kGemv = 0, kSkinny = 1, kGemm = 2 };
int path_mode(int type_in, int K_in, int type_out, int K_out, double avg_m, int E, bool packed = false,
              bool with_shared = false) {
  if (!gemm_supported(type_in, K_in) || !gemm_supported(type_out, K_out)) return kGemv;
  // tuning override: gemv | skinny | gemm (read per call, so a test can select each kernel); the shared
  // expert (E = 1 here) reads EMBER_MOE_SHARED_PATH
  const int forced = [E] {
    const char* v = std::getenv(E == 1 ? "EMBER_MOE_SHARED_PATH" : "EMBER_MOE_PATH");
    if (!v) return -1;
    const std::string s(v);
    return s == "gemv" ? kGemv : s == "skinny" ? kSkinny : s == "gemm" ? kGemm : -1;
  }();
  if (forced >= 0) return forced;
  // Q8_0 (its DMA tile kernels): the GEMV up to 1 token per expert with the prefill pack, 2 without,
  // then the 256-token-tile kernel, which skips the empty 32-row subtiles of a short segment (C2 with the
  // pack, GEMV / 64-token / 256-token tiles: T = 4 253 / 288 / 261 us, T = 5 282 / 280 / 261, T = 6 347
  // / 335 / 305, T = 8 382 / 335 / 308, T = 12 531 / 341 / 311; T = 32 361 vs 387 us on the 64-token
  // tiles. Without it, GEMV / 256-token tiles: T = 6 345 / 403, T = 8 386 / 404, T = 10 458 / 410)
  const bool q8 = type_in == EMBER_TYPE_Q8_0 && type_out == EMBER_TYPE_Q8_0;
  if (q8) return avg_m <= (packed ? 1.0 : 2.0) ? kGemv : kGemm;
  // (packed BF16: row exponents for the fp16 MFMA path, which both tile kernels have; without them BF16 runs
  // the split bf16 MFMA, which only the 64-token-tile kernel implements)
  // The expected tokens per expert HIT, T*k / (E (1 - (1 - 1/E)^(T*k))): the GEMV's cost follows the
  // token passes over the hit experts and the MFMA tiles' the hit experts' weights.
  const double slots = avg_m * E;
  const double hit = slots > 0.0 ? E * (1.0 - std::pow(1.0 - 1.0 / E, slots)) : 0.0;
  const double per_hit = hit > 0.0 ? slots / hit : 0.0;
  // packed Q4_K (the same DMA tile kernels): the GEMV up to 1.55 tokens per hit expert, then the
  // 256-token tiles (Qwen-shaped E = 128, GEMV / 64-token / 256-token tiles: T = 13 (1.47) 114 / 119 / 116
  // us, T = 14 (1.51) 122 / 119 / 114, T = 16 (1.58) 128 / 118 / 115, T = 24 170 / 155 / 150, T = 48 255 /
  // 160 / 159; Mixtral-shaped: T = 4 (1.52) GEMV 182 vs 258 on the 64-token tiles, T = 8 345 (64) vs 278
  // (256))
  if (packed && type_in == EMBER_TYPE_Q4_K && type_out == EMBER_TYPE_Q4_K)
    return per_hit <= 1.55 ? kGemv : kGemm;
  // BF16 / F16: the GEMV up to ~1.55 tokens per hit expert (Qwen-shaped E = 128: T = 12 204 vs 206 us,
  // T = 16 243 vs 210; Mixtral-shaped: T = 4 430 vs 671, T = 8 821 vs 691), up to 1.2 with a shared expert,
  // whose dense MFMA launches then run beside the routed ones on a side stream (C4-shaped, GEMV / 64-token
  // tiles: T = 4 (1.17) 102 / 131 us, T = 5 (1.21) 132 / 128, T = 6 (1.25) 139 / 131, T = 8 166 / 132)
  const bool half = (type_in == EMBER_TYPE_BF16 || type_in == EMBER_TYPE_F16) &&
                    (type_out == EMBER_TYPE_BF16 || type_out == EMBER_TYPE_F16);
  if (half && E > 1) {  // (one matrix, the shared expert: its T rows, the threshold below)
    if (hit <= 0.0 || per_hit <= (with_shared ? 1.2 : 1.55)) return kGemv;
  } else if (avg_m <= 2.0) {
    return kGemv;
  }
  // (one dense matrix, the shared expert: the 64-token tiles, split over K, up to 1024 rows; C4 shape
  // T = 512: 139 vs 201 us on the 256-token tiles, T = 2048: 234 vs 208)
  // packed BF16 routed experts: the 256-token tiles from ~32 tokens per expert (C4-shaped, 64-token /
  // 256-token tiles: T = 256 (24 per expert) 184 / 213 us, T = 512 (48) 270 / 228, T = 1024 426 / 392,
  // T = 2048 716 / 553)
  const bool bf16_packed = packed && type_in == EMBER_TYPE_BF16 && type_out == EMBER_TYPE_BF16 && E > 1;
  if (avg_m <= (E == 1 ? 1024.0 : bf16_packed ? 32.0 : 96.0)) return kSkinny;
  if (type_in == EMBER_TYPE_BF16 && type_out == EMBER_TYPE_BF16 && !packed) return kSkinny;
  return kGemm;
}

// BF16 gate/up and down: the MFMA paths run bf16 MFMA on the weights' own bits with split (hi + lo)
// bf16 activations (GemmArgs::split_bf16); other stacks run fp16 MFMA on row-scaled fp16 activations.
bool split_bf16(int type_in, int type_out) { return type_in == EMBER_TYPE_BF16 && type_out == EMBER_TYPE_BF16; }

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

int64_t row_bytes(int type, int K) {
  switch (type) {
    case EMBER_TYPE_F32: return K % 4 ? -1 : 4 * (int64_t)K;
    case EMBER_TYPE_F16:
    case EMBER_TYPE_BF16: return K % 8 ? -1 : 2 * (int64_t)K;
    case EMBER_TYPE_Q8_0: return K % 64 ? -1 : (int64_t)K / 32 * 34;
    case EMBER_TYPE_Q4_K: return K % 256 ? -1 : (int64_t)K / 256 * 144;
    default: return -2;
  }
}

int check_matrix(const void* p, int type, int K) {
  if (!p) return EMBER_ERR_NULL;
  const int64_t rb = row_bytes(type, K);
  if (rb == -2) return EMBER_ERR_TYPE;
  if (rb < 0) return EMBER_ERR_SHAPE;
  // the decode kernel stages one activation row of K elements per token in LDS
  if ((type_quantizes_activations(type) ? (int64_t)K * 2 + K / 32 * 8 : ((int64_t)K + 63) / 64 * 256) >
      proj_max_row_bytes())
    return EMBER_ERR_SHAPE;
  if (reinterpret_cast<uintptr_t>(p) % 16) return EMBER_ERR_ALIGN;
  return EMBER_OK;
}

bool is_routed(const ember_moe_layer* w) {
  return w->scoring == EMBER_SCORE_SIGMOID || w->selection_bias != nullptr || w->groups_n > 1;
}

bool bf16_stacks(const ember_moe_layer* w) {
  return w->gate_type == EMBER_TYPE_BF16 && w->up_type == EMBER_TYPE_BF16 && w->down_type == EMBER_TYPE_BF16;
}
bool bf16_shared(const ember_moe_layer* w) {
  return w->d_ff_shared > 0 && w->gate_shared_type == EMBER_TYPE_BF16 && w->up_shared_type == EMBER_TYPE_BF16 &&
         w->down_shared_type == EMBER_TYPE_BF16;
}
// The prefill pack serves layers whose three routed stacks are all Q8_0 or all Q4_K (tiles for the DMA
// GEMMs, whole 64-column tiles) or all BF16 (row exponents for the fp16 MFMA path).
bool packable(const ember_moe_layer* w) {
  if (bf16_stacks(w)) return true;
  const int t = w->gate_type;
  return (t == EMBER_TYPE_Q8_0 || t == EMBER_TYPE_Q4_K) && w->up_type == t && w->down_type == t && w->d % 64 == 0 &&
         w->d_ff % 64 == 0;
}
// a BF16 layer's pack: the row exponents (Bf16ExpLayout)
Bf16ExpLayout bf16_exps(const ember_moe_layer* w) {
  return bf16_exp_layout(w->d, w->d_ff, w->E, w->d_ff_shared, bf16_shared(w));
}

int validate(const ember_moe_layer* w) {
  if (!w) return EMBER_ERR_NULL;
  if (w->d <= 0 || w->d_ff <= 0 || w->E <= 0 || w->k <= 0 || w->E > kMaxE || w->k > kMaxK) return EMBER_ERR_SHAPE;
  if (w->scoring != EMBER_SCORE_SOFTMAX && w->scoring != EMBER_SCORE_SIGMOID) return EMBER_ERR_SHAPE;
  if (w->groups_n > 1) {
    // graph_ir.cpp:2696-2700 refuses the same combinations.
    if (w->E % w->groups_n || w->groups_top < 1 || w->groups_top > w->groups_n ||
        w->groups_top * (w->E / w->groups_n) < w->k)
      return EMBER_ERR_SHAPE;
  }
  if (!w->router) return EMBER_ERR_NULL;
  if (reinterpret_cast<uintptr_t>(w->router) % 16 || w->d % 4) return EMBER_ERR_ALIGN;
  int s;
  if ((s = check_matrix(w->gate, w->gate_type, w->d)) || (s = check_matrix(w->up, w->up_type, w->d)) ||
      (s = check_matrix(w->down, w->down_type, w->d_ff)))
    return s;
  if (w->gate_type != w->up_type) return EMBER_ERR_TYPE;  // one fused gate/up kernel per type
  if (w->d_ff % 4) return EMBER_ERR_SHAPE;                // h rows are read as float4
  if (w->d_ff_shared < 0) return EMBER_ERR_SHAPE;
  if (w->d_ff_shared > 0) {
    if ((s = check_matrix(w->gate_shared, w->gate_shared_type, w->d)) ||
        (s = check_matrix(w->up_shared, w->up_shared_type, w->d)) ||
        (s = check_matrix(w->down_shared, w->down_shared_type, w->d_ff_shared)))
      return s;
    if (w->gate_shared_type != w->up_shared_type) return EMBER_ERR_TYPE;
    if (w->d_ff_shared % 4) return EMBER_ERR_SHAPE;
  }
  if (w->shared_gate) {
    if (w->d_ff_shared <= 0) return EMBER_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(w->shared_gate) % 16) return EMBER_ERR_ALIGN;
  }
  if (w->prefill_pack) {
    if (!packable(w)) return EMBER_ERR_TYPE;
    if (reinterpret_cast<uintptr_t>(w->prefill_pack) % 256) return EMBER_ERR_ALIGN;
  }
  return EMBER_OK;
}

// Route/dispatch part of the scratch (also ember_moe_route's whole scratch).
struct RouteLayout {
  size_t rank, chunk_cnt, used, n_used, pos, end;
};
RouteLayout route_layout(int T, int E, int k, size_t base) {
  RouteLayout l;
  const size_t slots = (size_t)T * k, nchunks = (slots + 1023) / 1024;  // dispatch chunks of 1024 slots
  size_t o = base;
  l.rank = o; o = align_up(o + slots * 4);
  l.chunk_cnt = o; o = align_up(o + nchunks * E * 4);
  l.used = o; o = align_up(o + (size_t)E * 4);
  l.n_used = o; o = align_up(o + 4);
  l.pos = o; o = align_up(o + slots * 4);
  l.end = o;
  return l;
}

struct Layout {
  size_t flag;  // the fused routing's flag words (ProjArgs::Route), at a fixed place: offset 0
  size_t logits, idx, gates, offsets, perm, h, y, hs, ys, sg;
  size_t x16, xexp, xb, h16, hexp, hs16, hsexp, tiles, n_tiles;  // MFMA paths
  size_t shpart;                          // the shared expert's partial gate / up dots (K split)
  size_t part;                            // the one-token slice launch's partial outputs
  size_t tailpart;                        // the 256-token gate/up launch's tail partials
  size_t rfast;                           // the proven-picks router's planes, row scales and bounds
  int tail_parts;                         // their parts (0: no tail split)
  int mode, mode_shared;                  // PathMode of the routed experts and of the shared expert
  int ks_sh_gu, ks_sh_dn;                 // K split of the shared expert's 64-token-tile launches
  RouteLayout r;
  size_t end;
};
// Whether a call may take the one-token slice launch (SliceArgs): one token on the decode path, the
// fused routing's limits, a Q8_0 or Q4_K prefill pack, no shared expert; unless any_size, also enough
// slices to give every CU a block (the scratch layout reserves the section whenever the launch can run).
bool slices_possible(const ember_moe_layer* w, int T, int mode, bool any_size) {
  const int t = w->gate_type;
  return T == 1 && mode == kGemv && w->prefill_pack && (t == EMBER_TYPE_Q8_0 || t == EMBER_TYPE_Q4_K) &&
         packable(w) && w->d_ff_shared == 0 && slices_fit(t, w->d, w->d_ff, w->E, w->k, any_size);
}

Layout layout(const ember_moe_layer* w, int T) {
  Layout l;
  const size_t slots = (size_t)T * w->k;
  size_t o = 0;
  l.flag = o; o = align_up(o + (size_t)8 * (2 * w->E + 3));
  l.logits = o; o = align_up(o + (size_t)T * w->E * 4);
  l.idx = o; o = align_up(o + slots * 4);
  l.gates = o; o = align_up(o + slots * 4);
  l.offsets = o; o = align_up(o + (size_t)(w->E + 1) * 4);
  l.perm = o; o = align_up(o + slots * 4);
  l.r = route_layout(T, w->E, w->k, o); o = l.r.end;
  l.rfast = o;
  o = align_up(o + (router_fast_fits(T, w->d, w->E, w->k, w->renorm ? 1 : 0, is_routed(w) ? 1 : 0)
                        ? router_fast_work_bytes(T, w->d, w->E) : 0));
  l.h = o; o = align_up(o + slots * w->d_ff * 4);
  // y holds kMaxKSplit partial sums per row when an MFMA path splits the down projection's K
  l.y = o; o = align_up(o + slots * w->d * 4 * kMaxKSplit);
  l.hs = o; o = align_up(o + (size_t)T * w->d_ff_shared * 4);
  l.sg = o; o = align_up(o + (w->shared_gate ? (size_t)T * 4 : 0));
  l.mode = path_mode(w->gate_type, w->d, w->down_type, w->d_ff, (double)T * w->k / w->E, w->E, w->prefill_pack != nullptr,
                     w->d_ff_shared > 0);
  const bool pack_bf16 = w->prefill_pack && bf16_stacks(w);  // row exponents, also the shared expert's if BF16
  l.mode_shared = w->d_ff_shared > 0 ? path_mode(w->gate_shared_type, w->d, w->down_shared_type, w->d_ff_shared,
                                                 (double)T, 1, pack_bf16 && bf16_shared(w))
                                     : kGemv;
  // a shared expert of the routed experts' types rides in the routed decode launches as one more segment
  // (a few µs), while on its own its T rows make a dense MFMA launch of only d_ff_shared / 128 blocks
  // (C4, T = 4: 205 µs with it on the MFMA path, 100 µs in the routed launches)
  if (w->d_ff_shared > 0 && l.mode == kGemv && w->gate_shared_type == w->gate_type &&
      w->down_shared_type == w->down_type)
    l.mode_shared = kGemv;
  // the shared expert's dense launches on 64-token tiles have d_ff_shared / 128 (gate/up) and d / 256
  // (down) blocks per 64 tokens: split over K until the chip is filled (C4 shape, T = 16: 128 -> 25 us)
  l.ks_sh_gu = l.ks_sh_dn = 1;
  if (w->d_ff_shared > 0 && l.mode_shared == kSkinny) {
    l.ks_sh_gu = gemm_dense_ksplit(true, T, w->d_ff_shared, w->d,
                                   2 * (int64_t)w->d_ff_shared * row_bytes(w->gate_shared_type, w->d));
    l.ks_sh_dn = gemm_dense_ksplit(false, T, w->d, w->d_ff_shared,
                                   (int64_t)w->d * row_bytes(w->down_shared_type, w->d_ff_shared));
  }
  l.ys = o; o = align_up(o + (w->d_ff_shared > 0 ? (size_t)l.ks_sh_dn * T * w->d * 4 : 0));
  l.shpart = o; o = align_up(o + (l.ks_sh_gu > 1 ? (size_t)l.ks_sh_gu * T * 2 * w->d_ff_shared * 4 : 0));
  const size_t tiles = l.mode == kGemm     ? (size_t)gemm_max_tiles(T, w->k, w->E)
                       : l.mode == kSkinny ? (size_t)gemm_skinny_max_tiles(T, w->k, w->E)
                                           : 0;
  const bool mfma = l.mode != kGemv, mfma_sh = w->d_ff_shared > 0 && l.mode_shared != kGemv;
  const bool sp = split_bf16(w->gate_type, w->down_type) && !pack_bf16;
  const bool sp_sh = w->d_ff_shared > 0 && split_bf16(w->gate_shared_type, w->down_shared_type) &&
                     !(pack_bf16 && bf16_shared(w));
  const bool need16 = (mfma && !sp) || (mfma_sh && !sp_sh), needb = (mfma && sp) || (mfma_sh && sp_sh);
  l.x16 = o; o = align_up(o + (need16 ? (size_t)T * w->d * 2 : 0));
  l.xexp = o; o = align_up(o + (need16 ? (size_t)T * 4 : 0));
  l.xb = o; o = align_up(o + (needb ? (size_t)T * w->d * 4 : 0));
  l.h16 = o; o = align_up(o + (mfma ? slots * w->d_ff * (sp ? 4 : 2) : 0));
  l.hexp = o; o = align_up(o + (mfma && !sp ? slots * 4 : 0));
  l.hs16 = o; o = align_up(o + (mfma_sh ? (size_t)T * w->d_ff_shared * (sp_sh ? 4 : 2) : 0));
  l.hsexp = o; o = align_up(o + (mfma_sh && !sp_sh ? (size_t)T * 4 : 0));
  l.tiles = o; o = align_up(o + tiles * 8);
  // the routed gate/up's tail split (256-token tiles): raw partial gate / up dots [parts][T k][2 d_ff]
  l.tail_parts = l.mode == kGemm ? gemm_tail_parts(w->gate_type, w->prefill_pack != nullptr && !pack_bf16,
                                                   (int)slots, w->d_ff, w->d)
                                 : 0;
  l.tailpart = o; o = align_up(o + (size_t)l.tail_parts * slots * 2 * w->d_ff * 4);
  l.n_tiles = o; o = align_up(o + 4);
  // the one-token slice launch's partial outputs [k][d_ff / 64][d]
  l.part = o; o = align_up(o + (slices_possible(w, T, l.mode, true) ? (size_t)w->k * (w->d_ff / 64) * w->d * 4 : 0));
  l.end = o;
  return l;
}

// The launch plan of a call (which kernels run), shared by run_ffn and ember_moe_path.
struct Plan {
  bool fuse_route;  // one token: router, routing and dispatch inside the first expert launch
  bool slices;      // one token: the whole layer in one launch over d_ff slices, plus an ordered reduce
  bool down1;       // one token: the down projection with the combine fused in
};
Plan plan(const ember_moe_layer* w, const Layout& l, int T) {
  static const bool fuse_ok = [] { const char* v = std::getenv("EMBER_FUSE_ROUTE"); return !(v && atoi(v) == 0); }();
  static const bool down1_ok = [] { const char* v = std::getenv("EMBER_MOE_DOWN1"); return !(v && atoi(v) == 0); }();
  // EMBER_MOE_SLICES (read per call): 0 never takes the slice launch, 1 takes it whenever it can run
  const char* sv = std::getenv("EMBER_MOE_SLICES");
  const bool slices_ok = !(sv && atoi(sv) == 0), slices_any = sv && atoi(sv) == 1;
  const int d = w->d, d_ff = w->d_ff, E = w->E, k = w->k;
  Plan p{};
  // (the router blocks are one per expert and must fit the device's CUs: fewer CUs than experts take the
  // unfused launches)
  p.fuse_route = fuse_ok && l.mode == kGemv && T == 1 && fused_route_fits(w->gate_type, d, E, k) && E <= device_cus();
  p.slices = slices_ok && p.fuse_route && slices_possible(w, T, l.mode, slices_any);
  // (the picks of a row run side by side in down1_walk_picks; measured on MI355X against the down launch
  // + combine: C1-shaped layer 17.1 -> 16.7 us, Qwen-shaped top-8 29.0 -> 26.8, DeepSeek-shaped top-6 +
  // shared 54.2 -> 52.0, Mixtral-shaped without a pack even). A shared expert joins when it rides in the
  // routed GEMV launches (same types), as run_ffn then passes it to the down launch.
  const bool shared_gemv = w->d_ff_shared == 0 || (l.mode_shared == kGemv && w->gate_shared_type == w->gate_type &&
                                                    w->down_shared_type == w->down_type);
  p.down1 = !p.slices && down1_ok && l.mode == kGemv && T == 1 && k <= kDown1MaxPicks && shared_gemv &&
            down1_fits(w->down_type, d, d_ff, k, w->d_ff_shared);
  return p;
}

template <class P>
P* at(void* base, size_t off) {
  return reinterpret_cast<P*>(static_cast<char*>(base) + off);
}

DispatchScratch dispatch_scratch(void* scratch, const RouteLayout& r, int32_t* offsets, int32_t* perm) {
  DispatchScratch ds{};
  ds.rank = at<int32_t>(scratch, r.rank);
  ds.chunk_cnt = at<int32_t>(scratch, r.chunk_cnt);
  ds.offsets = offsets;
  ds.used = at<int32_t>(scratch, r.used);
  ds.n_used = at<int32_t>(scratch, r.n_used);
  ds.perm = perm;
  ds.pos = at<int32_t>(scratch, r.pos);
  ds.tiles = ds.n_tiles = nullptr;
  ds.tile_bm = 0;
  return ds;
}

}  // namespace

// Compute units of the current device (cached per device; the table is filled once per device).
int device_cus() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cus[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev >= kMaxDev) {
    int n = 0;
    return hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess ? n : 0;
  }
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0 && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
    cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Blocks per CU of a kernel at a dynamic LDS size on the current device (hipFuncSetAttribute for the
// LDS size, then the occupancy query), cached per (kernel, device, LDS bytes) under a lock.
int blocks_per_cu(const void* fn, int threads, size_t lds, size_t max_lds) {
  static std::mutex mu;
  static std::map<std::tuple<const void*, int, size_t>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> g(mu);
  const auto key = std::make_tuple(fn, dev, lds);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_lds) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, lds) != hipSuccess)
    return 0;
  n = std::max(n, 1);
  cache.emplace(key, n);
  return n;
}

}  // namespace ember_moe

using namespace ember_moe;

extern "C" {

const char* ember_moe_strerror(int status) {
  switch (status) {
    case EMBER_OK: return "ok";
    case EMBER_ERR_SHAPE: return "invalid shape";
    case EMBER_ERR_TYPE: return "unsupported tensor type";
    case EMBER_ERR_SCRATCH: return "scratch buffer missing or too small";
    case EMBER_ERR_NULL: return "null pointer";
    case EMBER_ERR_LAUNCH: return "kernel launch failed";
    case EMBER_ERR_ALIGN: return "pointer or row not 16-byte aligned";
    case EMBER_ERR_FORMAT: return "malformed or unreadable GGUF file";
    case EMBER_ERR_NOT_FOUND: return "no such tensor, key or MoE layer";
    default: return "unknown status";
  }
}

size_t ember_moe_scratch_bytes(const ember_moe_layer* w, int T) {
  if (validate(w) != EMBER_OK || T < 0) return 0;
  return layout(w, std::max(T, 1)).end;
}

namespace {
// Records ev[i] on the stream at phase boundary i when ev is non-null (ember_moe_ffn_timed).
// A side stream and its fork / join events, one set per (host thread, device), created on first use
// (default priority, non-blocking). Null when creation fails: the caller then stays on one stream.
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  bool failed = false;
};
SideStream* side_stream() {
  constexpr int kMaxDev = 64;
  thread_local SideStream tab[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return nullptr;
  SideStream& ss = tab[dev];
  if (!ss.s && !ss.failed) {
    if (hipStreamCreateWithFlags(&ss.s, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ss.join, hipEventDisableTiming) != hipSuccess) {
      ss.failed = true;
      (void)hipGetLastError();
    }
  }
  return ss.failed ? nullptr : &ss;
}

inline void mark(hipEvent_t* ev, int i, hipStream_t st) {
  if (ev) (void)hipEventRecord(ev[i], st);  // a failed record shows up as a failed elapsed-time query
}

// fork_ok: the shared expert's dense launches may run on a side stream (see run_shared)
int run_ffn(const ember_moe_layer* w, const float* x, int T, float* out, void* scratch, size_t scratch_bytes,
            hipStream_t st, hipEvent_t* ev, hipEvent_t* kev = nullptr, int* kev_used = nullptr, bool fork_ok = false) {
  int s = validate(w);
  if (s) return s;
  if (T < 0) return EMBER_ERR_SHAPE;
  if (T == 0) return EMBER_OK;
  if (!x || !out) return EMBER_ERR_NULL;
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(out) % 16) return EMBER_ERR_ALIGN;
  const Layout l = layout(w, T);
  if (!scratch || scratch_bytes < l.end) return EMBER_ERR_SCRATCH;
  if (reinterpret_cast<uintptr_t>(scratch) % 256) return EMBER_ERR_ALIGN;

  const int d = w->d, d_ff = w->d_ff, E = w->E, k = w->k;
  float* logits = at<float>(scratch, l.logits);
  int32_t* idx = at<int32_t>(scratch, l.idx);
  float* gates = at<float>(scratch, l.gates);
  int32_t* offsets = at<int32_t>(scratch, l.offsets);
  int32_t* perm = at<int32_t>(scratch, l.perm);
  DispatchScratch ds = dispatch_scratch(scratch, l.r, offsets, perm);
  if (l.mode != kGemv) {  // the dispatch also writes the MFMA GEMMs' tile table
    ds.tiles = at<int32_t>(scratch, l.tiles);
    ds.n_tiles = at<int32_t>(scratch, l.n_tiles);
    ds.tile_bm = gemm_tile_rows(l.mode == kSkinny);
  }
  float* h = at<float>(scratch, l.h);
  float* y = at<float>(scratch, l.y);
  int ksplit = 1;  // partial sums per y row (K split of the down projection)

  const int groups_n = std::max(w->groups_n, 1), groups_top = std::max(w->groups_top, 1);
  const int renorm = w->renorm ? 1 : 0, routed = is_routed(w) ? 1 : 0;
  const int sigmoid = w->scoring == EMBER_SCORE_SIGMOID ? 1 : 0;
  // one token on the decode path: the router, the routing and the dispatch run inside the gate/up launch
  // (its block 0 publishes them; the other blocks wait), saving two launches on the latency path
  const Plan pl = plan(w, l, T);
  const bool fuse_route = pl.fuse_route;
  const bool shared = w->d_ff_shared > 0;
  const bool shared_mfma = shared && l.mode_shared != kGemv;
  const float out_scale = w->out_scale == 0.0f ? 1.0f : w->out_scale;
  // the shared expert joins the routed decode launches when its type matches (one more segment)
  const bool shared_fused = shared && !shared_mfma && l.mode == kGemv && w->gate_shared_type == w->gate_type &&
                            w->down_shared_type == w->down_type;
  // the activations of the MFMA paths: row-scaled fp16 (x16, xexp) and / or split bf16 planes (xb)
  // BF16 stacks: split bf16 MFMA, or with a prefill pack (row exponents) the fp16 path
  const bool pack_bf16 = w->prefill_pack && bf16_stacks(w);
  const bool pack_bf16_sh = pack_bf16 && bf16_shared(w);
  const Bf16ExpLayout bx = bf16_exps(w);
  auto wexp = [&](int64_t off) {
    return off < 0 ? nullptr : reinterpret_cast<const int16_t*>(static_cast<const uint8_t*>(w->prefill_pack) + off);
  };
  const bool sp = split_bf16(w->gate_type, w->down_type) && !pack_bf16;
  const bool sp_sh = shared && split_bf16(w->gate_shared_type, w->down_shared_type) && !pack_bf16_sh;
  _Float16* x16 = at<_Float16>(scratch, l.x16);
  int32_t* xexp = at<int32_t>(scratch, l.xexp);
  uint16_t* xb = at<uint16_t>(scratch, l.xb);
  // the MFMA paths' activations, converted by extra blocks of the routing launch (or on their own when the
  // routing is fused into the decode launch)
  ActConv conv{};
  conv.x = x;
  conv.rows = T;
  conv.K = d;
  conv.y16 = (l.mode != kGemv && !sp) || (shared_mfma && !sp_sh) ? x16 : nullptr;
  conv.yexp = xexp;
  conv.yb = (l.mode != kGemv && sp) || (shared_mfma && sp_sh) ? xb : nullptr;
  conv.plane = (int64_t)T * d;
  const bool need_conv = conv.y16 || conv.yb;
  auto* flag = at<unsigned long long>(scratch, l.flag);
  mark(ev, 0, st);
  if (!fuse_route && router_fast_fits(T, d, E, k, renorm, routed)) {
    // picks proven from exact-integer fast logits; exact FP64 logits only where the bound leaves a doubt
    if ((s = launch_router_fast(x, T, d, E, k, w->router, logits, idx, gates, at<void>(scratch, l.rfast),
                                need_conv ? &conv : nullptr, st)))
      return s;
    mark(ev, 1, st);
    if ((s = launch_dispatch(idx, T, k, E, ds, st))) return s;
  } else {
    if (!fuse_route && (s = launch_router_logits(x, T, d, E, w->router, logits, st))) return s;
    mark(ev, 1, st);
    if (!fuse_route && (s = launch_route_dispatch(logits, T, E, k, renorm, routed, sigmoid, w->selection_bias,
                                                  groups_n, groups_top, idx, gates, ds, need_conv ? &conv : nullptr,
                                                  st)))
      return s;
  }
  if (fuse_route && need_conv && (s = launch_act_conv(conv, st))) return s;
  mark(ev, 2, st);
  mark(ev, 3, st);

  float* ys = shared ? at<float>(scratch, l.ys) : nullptr;
  float* hs = at<float>(scratch, l.hs);
  // one token on the decode path: the down launch also forms the output rows (combine fused in)
  const bool down1 = pl.down1;
  // qwen2moe's shared-expert gate logit per token: a one-row router (the same FP64 fixed-order dot)
  float* sg = w->shared_gate ? at<float>(scratch, l.sg) : nullptr;
  if (sg && (s = launch_router_logits(x, T, d, 1, w->shared_gate, sg, st))) return s;

  // The shared expert's dense MFMA launches (its T rows) depend only on the converted activations, not
  // on the routed launches: when the caller allows it they run on a side stream, forked here after the
  // routing and joined before the combine, so that their blocks fill the CUs the routed launches leave
  // idle (their tail rounds) instead of running alone on a few hundred blocks.
  auto run_shared = [&](hipStream_t sst) -> int {
    int s = EMBER_OK;
    _Float16* hs16 = at<_Float16>(scratch, l.hs16);
    int32_t* hsexp = at<int32_t>(scratch, l.hsexp);
    GemmArgs g{};
    g.A = sp_sh ? reinterpret_cast<const _Float16*>(xb) : x16;
    g.a_exp = sp_sh ? nullptr : xexp;
    g.h_exp = sp_sh ? nullptr : hsexp;
    g.split_bf16 = sp_sh;
    if (pack_bf16_sh) {
      g.w_exp0 = wexp(bx.sgate);
      g.w_exp1 = wexp(bx.sup);
      g.w_hexp = wexp(bx.shmax);
    }
    g.a_plane = (int64_t)T * d;
    g.h_plane = (int64_t)T * w->d_ff_shared;
    g.T = T;
    g.W0 = w->gate_shared;
    g.W1 = w->up_shared;
    g.type = w->gate_shared_type;
    g.row_bytes = row_bytes(w->gate_shared_type, d);
    g.N = w->d_ff_shared;
    g.K = d;
    g.out_h = hs16;
    const bool skinny = l.mode_shared == kSkinny;  // one dense segment of T rows
    const int mt = skinny ? gemm_skinny_max_tiles(T, 1, 0) : gemm_max_tiles(T, 1, 0);
    g.ksplit = skinny ? l.ks_sh_gu : 1;
    g.part_h = g.ksplit > 1 ? at<float>(scratch, l.shpart) : nullptr;
    g.part_rows = T;
    if ((s = skinny ? launch_gemm_skinny(g, true, mt, sst) : launch_gemm(g, true, mt, sst))) return s;
    g.A = hs16;
    g.a_exp = sp_sh ? nullptr : hsexp;
    g.h_exp = nullptr;
    g.a_plane = (int64_t)T * w->d_ff_shared;
    g.W0 = w->down_shared;
    g.W1 = nullptr;
    g.w_exp0 = pack_bf16_sh ? wexp(bx.sdown) : nullptr;
    g.w_exp1 = nullptr;
    g.w_hexp = nullptr;
    g.type = w->down_shared_type;
    g.row_bytes = row_bytes(w->down_shared_type, w->d_ff_shared);
    g.N = d;
    g.K = w->d_ff_shared;
    g.out_h = nullptr;
    g.out_y = ys;
    g.ksplit = skinny ? l.ks_sh_dn : 1;
    g.part_stride = (int64_t)T * d;
    g.part_h = nullptr;
    if ((s = skinny ? launch_gemm_skinny(g, false, mt, sst) : launch_gemm(g, false, mt, sst))) return s;
    return s;
  };
  SideStream* side = shared_mfma && fork_ok ? side_stream() : nullptr;
  // Once forked, every return joins the side stream back into `st` (on an error return too), so that a
  // capture on `st` never ends with an unjoined fork.
  struct JoinGuard {
    SideStream* side = nullptr;
    hipStream_t st = nullptr;
    ~JoinGuard() {
      if (side) {
        (void)hipEventRecord(side->join, side->s);
        (void)hipStreamWaitEvent(st, side->join, 0);
      }
    }
  } join_guard;
  if (side) {
    if (hipEventRecord(side->fork, st) != hipSuccess || hipStreamWaitEvent(side->s, side->fork, 0) != hipSuccess)
      return EMBER_ERR_LAUNCH;
    join_guard.side = side;
    join_guard.st = st;
    if ((s = run_shared(side->s))) return s;
  }

  if (l.mode != kGemv) {
    const bool skinny = l.mode == kSkinny;
    auto gemm = [&](const GemmArgs& g, bool gated, int mt) {
      return skinny ? launch_gemm_skinny(g, gated, mt, st) : launch_gemm(g, gated, mt, st);
    };
    int32_t* tiles = ds.tiles;
    int32_t* n_tiles = ds.n_tiles;
    _Float16* h16 = at<_Float16>(scratch, l.h16);
    int32_t* hexp = at<int32_t>(scratch, l.hexp);
    GemmArgs g{};
    g.A = sp ? reinterpret_cast<const _Float16*>(xb) : x16;
    g.a_exp = sp ? nullptr : xexp;
    g.h_exp = sp ? nullptr : hexp;
    g.split_bf16 = sp;
    g.a_plane = (int64_t)T * d;
    g.h_plane = (int64_t)T * k * d_ff;
    g.perm = perm;
    g.k = k;
    g.T = T;
    g.W0 = w->gate;
    g.W1 = w->up;
    g.type = w->gate_type;
    g.row_bytes = row_bytes(w->gate_type, d);
    g.expert_stride = g.row_bytes * d_ff;
    g.N = d_ff;
    g.K = d;
    g.tiles = tiles;
    g.n_tiles = n_tiles;
    g.offsets = offsets;
    g.out_h = h16;
    // the prefill pack serves the DMA tile kernels (256- and 64-token tiles alike)
    const PackLayout pl = pack_layout(d, d_ff, E, w->gate_type);
    const uint8_t* pack = pack_bf16 ? nullptr : static_cast<const uint8_t*>(w->prefill_pack);
    g.Wp = pack ? pack + pl.gu : nullptr;
    if (pack_bf16) {
      g.w_exp0 = wexp(bx.gate);
      g.w_exp1 = wexp(bx.up);
      g.w_hexp = wexp(bx.hmax);
    }
    const int mt = skinny ? gemm_skinny_max_tiles(T, k, E) : gemm_max_tiles(T, k, E);
    if (!skinny && l.tail_parts > 1) {  // the tail round's tiles split over K
      g.part_h = at<float>(scratch, l.tailpart);
      g.part_rows = T * k;
      g.tail_parts = l.tail_parts;
      g.slots = gemm_slots();
    }
    if ((s = gemm(g, true, mt))) return s;
    g.part_h = nullptr;
    g.tail_parts = 0;
    mark(ev, 4, st);
    g.A = h16;
    g.perm = nullptr;
    g.a_exp = sp ? nullptr : hexp;
    g.h_exp = nullptr;
    g.a_plane = (int64_t)T * k * d_ff;
    g.W0 = w->down;
    g.W1 = nullptr;
    g.type = w->down_type;
    g.row_bytes = row_bytes(w->down_type, d_ff);
    g.expert_stride = g.row_bytes * d;
    g.N = d;
    g.K = d_ff;
    g.out_h = nullptr;
    g.out_y = y;
    g.Wp = pack ? pack + pl.dn : nullptr;
    g.w_exp0 = pack_bf16 ? wexp(bx.down) : nullptr;
    g.w_exp1 = nullptr;
    g.w_hexp = nullptr;
    g.ksplit = ksplit = skinny ? gemm_skinny_ksplit(g.type, pack != nullptr, T, k, E, d, d_ff)
                               : gemm_ksplit(g.type, pack != nullptr, T, k, E, d, d_ff);
    g.part_stride = (int64_t)T * k * d;
    if ((s = gemm(g, false, mt))) return s;
    mark(ev, 5, st);
  } else {
    // gate/up + SwiGLU (x rows gathered through perm, h in dispatch order), then down (h -> y)
    ProjArgs a{};
    a.type = w->gate_type;
    a.gated = true;
    a.w0 = w->gate;
    a.w1 = w->up;
    a.rows = d_ff;
    a.K = d;
    a.expert_stride = row_bytes(w->gate_type, d) * d_ff;
    a.in = x;
    a.out = h;
    a.offsets = offsets;
    a.used = ds.used;
    a.n_used = ds.n_used;
    a.perm = perm;
    a.k = k;
    a.in_by_perm = true;
    a.max_segments = std::min(E, T * k);
    a.T = T;
    if (shared_fused) {
      a.s_w0 = w->gate_shared;
      a.s_w1 = w->up_shared;
      a.s_rows = w->d_ff_shared;
      a.s_K = d;
      a.s_in = x;
      a.s_out = hs;
    }
    if (kev) {  // per-dispatch timing events of the two expert launches (ember_moe_ffn_timed)
      a.ev_start = kev[0];
      a.ev_stop = kev[1];
      *kev_used = 3;
    }
    if (fuse_route) {
      ProjArgs::Route& r = a.route;
      r.flag = flag;
      r.x = x;
      r.router = w->router;
      r.d = d;
      r.E = E;
      r.renorm = renorm;
      r.routed = routed;
      r.sigmoid = sigmoid;
      r.groups_n = groups_n;
      r.groups_top = groups_top;
      r.bias = w->selection_bias;
      r.logits = logits;
      r.idx = idx;
      r.gates = gates;
      r.pos = ds.pos;
      r.offsets = offsets;
      r.used = ds.used;
      r.n_used = ds.n_used;
      r.perm = perm;
      // A poll is one device-coherent load (an L2 round trip) plus a short sleep; the router blocks
      // publish within a few microseconds, so 4096 polls only run out when a router block is not
      // resident. The test hook makes every block compute every logit itself.
      const char* tv = std::getenv("EMBER_MOE_TEST_ROUTE_NOPUBLISH");  // read per call: tests toggle it
      const bool test_nopub = tv && atoi(tv) != 0;
      r.no_publish = test_nopub ? 1 : 0;
      r.spin_limit = test_nopub ? 4u : 4096u;
      // test hook: the router blocks publish wrong fast values (negated) under tight bounds, a pick-set
      // conflict that block 0 must catch (the output rows are then NaN)
      const char* tc = std::getenv("EMBER_MOE_TEST_FAST_CORRUPT");
      r.test_corrupt = tc && atoi(tc) != 0 ? 1 : 0;
      // per-call tags (a word from an earlier call never matches; under graph capture the replays share
      // the captured tags, and every call's last expert launch clears the words)
      static std::atomic<uint32_t> calls{0};
      const uint32_t c = calls.fetch_add(1, std::memory_order_relaxed) * 0x9e3779b1u;
      r.logit_tag = (0x10617ed5u ^ c) | 1u;    // odd: never 0 (a cleared word)
      r.fast_tag = (0x0fa57106u ^ c) & ~1u;    // even, and nonzero unless the mix cancels it
      if (r.fast_tag == 0) r.fast_tag = 2u;
    }
    if (pl.slices) {
      // one token: the whole layer in one launch over d_ff slices (the prefill pack's tiles), then the
      // ordered reduce of the slices' partial outputs, which also clears the routing words
      SliceArgs sa{};
      sa.p = a;
      const PackLayout pk = pack_layout(d, d_ff, E, w->gate_type);
      const uint8_t* pack = static_cast<const uint8_t*>(w->prefill_pack);
      sa.pack_gu = pack + pk.gu;
      sa.pack_dn = pack + pk.dn;
      sa.d = d;
      sa.d_ff = d_ff;
      sa.part = at<float>(scratch, l.part);
      if (kev) *kev_used = 1;
      if ((s = launch_slices(sa, st))) return s;
      mark(ev, 4, st);
      if ((s = launch_slice_reduce(sa.part, d_ff / 64, d, k, idx, gates, out_scale, routed ? nullptr : flag + 2 + 2 * E,
                                   flag + 2, 2 * E, out, st)))
        return s;
      mark(ev, 5, st);
      mark(ev, 6, st);
      mark(ev, 7, st);
      return EMBER_OK;
    }
    if (down1) {
      // one token: the down projection with the combine fused in (no y rows, no combine launch)
      Down1Args b{};
      b.type = w->down_type;
      b.w = w->down;
      b.expert_stride = row_bytes(w->down_type, d_ff) * d;
      b.d = d;
      b.K = d_ff;
      b.k = k;
      b.h = h;
      b.pos = ds.pos;
      b.idx = idx;
      b.gates = gates;
      if (shared_fused) {
        b.s_w = w->down_shared;
        b.s_K = w->d_ff_shared;
        b.s_h = hs;
      }
      b.sg_logit = sg;
      b.scale = out_scale;
      b.out = out;
      b.clear_flag = fuse_route ? flag + 2 : nullptr;
      b.clear_n = 2 * E;
      b.conflict = fuse_route && !routed ? flag + 2 + 2 * E : nullptr;
      if ((s = launch_projection(a, st))) return s;
      mark(ev, 4, st);
      if (kev) {
        b.ev_start = kev[2];
        b.ev_stop = kev[3];
        *kev_used = 3;
      }
      if ((s = launch_down1(b, st))) return s;
      mark(ev, 5, st);
      mark(ev, 6, st);
      mark(ev, 7, st);
      return EMBER_OK;
    }
    if ((s = launch_projection(a, st))) return s;
    mark(ev, 4, st);
    a.route = ProjArgs::Route{};
    a.clear_flag = fuse_route ? flag + 2 : nullptr;  // the down launch resets the logit words for the next call
    a.clear_n = 2 * E;
    a.type = w->down_type;
    a.gated = false;
    a.w0 = w->down;
    a.w1 = nullptr;
    a.rows = d;
    a.K = d_ff;
    a.expert_stride = row_bytes(w->down_type, d_ff) * d;
    a.in = h;
    a.out = y;
    a.in_by_perm = false;
    if (shared_fused) {
      a.s_w0 = w->down_shared;
      a.s_w1 = nullptr;
      a.s_rows = d;
      a.s_K = w->d_ff_shared;
      a.s_in = hs;
      a.s_out = ys;
    }
    if (kev) {
      a.ev_start = kev[2];
      a.ev_stop = kev[3];
    }
    if ((s = launch_projection(a, st))) return s;
    mark(ev, 5, st);
  }
  if (shared_mfma) {
    if (!side && (s = run_shared(st))) return s;
  } else if (shared && !shared_fused) {
    ProjArgs b{};
    b.gated = true;
    b.type = w->gate_shared_type;
    b.T = T;
    b.s_w0 = w->gate_shared;
    b.s_w1 = w->up_shared;
    b.s_rows = w->d_ff_shared;
    b.s_K = d;
    b.s_in = x;
    b.s_out = hs;
    if ((s = launch_projection(b, st))) return s;
    b.gated = false;
    b.type = w->down_shared_type;
    b.s_w0 = w->down_shared;
    b.s_w1 = nullptr;
    b.s_rows = d;
    b.s_K = w->d_ff_shared;
    b.s_in = hs;
    b.s_out = ys;
    if ((s = launch_projection(b, st))) return s;
  }
  if (side) {
    join_guard.side = nullptr;
    if (hipEventRecord(side->join, side->s) != hipSuccess || hipStreamWaitEvent(st, side->join, 0) != hipSuccess)
      return EMBER_ERR_LAUNCH;
  }
  mark(ev, 6, st);
  const int ys_parts = shared_mfma && l.mode_shared == kSkinny ? l.ks_sh_dn : 1;
  s = launch_combine(y, ksplit, (int64_t)T * k * d, gates, ds.pos, ys, ys_parts, (int64_t)T * d, sg, out_scale, T, k,
                     d, out, st, fuse_route && !routed ? flag + 2 + 2 * E : nullptr);
  mark(ev, 7, st);
  return s;
}
}  // namespace

int ember_moe_ffn(const ember_moe_layer* w, const float* x, int T, float* out, void* scratch, size_t scratch_bytes,
                  hipStream_t st) {
  return run_ffn(w, x, T, out, scratch, scratch_bytes, st, nullptr, nullptr, nullptr, true);
}

}  // extern "C"

// ---- the allocation-free entry point: the library's own scratch in device memory
// The buffer ember_moe_ffn_noalloc runs in. In host code `scratch` names a host-side stand-in, never
// the device address: the address comes from hipGetSymbolAddress, once per device, and only that
// pointer is handed to kernels. It is zero when the code object loads; the fused one-token routing's
// logit words (its first bytes) are zeroed again by every call's last expert launch, as in a caller's
// scratch.
static __device__ __align__(256) uint8_t scratch[EMBER_MOE_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices];  // per device: the device address of `scratch`, or null before set-up

// The device address of this device's copy of `scratch` (set up on the first call on the device).
void* noalloc_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> g(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    g_noalloc_ptr[dev] = p;
  }
  return g_noalloc_ptr[dev];
}
}  // namespace

extern "C" {

int ember_moe_ffn_noalloc(const ember_moe_layer* w, const float* x, int T, float* out, hipStream_t st) {
  int s = validate(w);
  if (s) return s;
  if (T < 0) return EMBER_ERR_SHAPE;
  if (T == 0) return EMBER_OK;
  if (layout(w, T).end > (size_t)EMBER_MOE_NOALLOC_SCRATCH_BYTES) return EMBER_ERR_SCRATCH;
  void* p = noalloc_scratch();
  if (!p) return EMBER_ERR_LAUNCH;
  return run_ffn(w, x, T, out, p, (size_t)EMBER_MOE_NOALLOC_SCRATCH_BYTES, st, nullptr);
}

int ember_moe_ffn_timed(const ember_moe_layer* w, const float* x, int T, float* out, void* scratch,
                        size_t scratch_bytes, hipStream_t st, float* phase_ms) {
  if (!phase_ms) return EMBER_ERR_NULL;
  hipEvent_t ev[12];  // 8 phase boundaries + start / stop of the gate/up and down dispatches
  for (int i = 0; i < 12; ++i)
    if (hipEventCreate(&ev[i]) != hipSuccess) return EMBER_ERR_LAUNCH;
  // The dispatch events are recorded only by the decode path's expert launches; then they replace the
  // event-to-event spans of those two phases (unrecorded events are never queried: a failed query
  // would stay behind as HIP's last error).
  int kev_used = 0;  // bit 0: the gate/up dispatch events were recorded; bit 1: the down dispatch events
  int s = run_ffn(w, x, T, out, scratch, scratch_bytes, st, ev, ev + 8, &kev_used);
  if (s == EMBER_OK && T > 0) {
    if (hipEventSynchronize(ev[7]) != hipSuccess) s = EMBER_ERR_LAUNCH;
    for (int i = 0; i < EMBER_MOE_NPHASES && s == EMBER_OK; ++i)
      if (hipEventElapsedTime(&phase_ms[i], ev[i], ev[i + 1]) != hipSuccess) s = EMBER_ERR_LAUNCH;
    if (s == EMBER_OK && (kev_used & 1) && hipEventElapsedTime(&phase_ms[3], ev[8], ev[9]) != hipSuccess)
      s = EMBER_ERR_LAUNCH;
    if (s == EMBER_OK && (kev_used & 2) && hipEventElapsedTime(&phase_ms[4], ev[10], ev[11]) != hipSuccess)
      s = EMBER_ERR_LAUNCH;
  }
  for (int i = 0; i < 12; ++i) (void)hipEventDestroy(ev[i]);
  return s;
}

int ember_moe_path(const ember_moe_layer* w, int T) {
  const int s = validate(w);
  if (s) return s;
  if (T < 0) return EMBER_ERR_SHAPE;
  if (T == 0) return 0;
  const Layout l = layout(w, T);
  const Plan p = plan(w, l, T);
  int bits = l.mode == kGemv ? EMBER_PATH_GEMV : l.mode == kSkinny ? EMBER_PATH_TILES64 : EMBER_PATH_TILES256;
  if (p.fuse_route) bits |= EMBER_PATH_FUSED_ROUTE;
  if (p.slices) bits |= EMBER_PATH_SLICES;
  if (p.down1) bits |= EMBER_PATH_DOWN1;
  if (w->d_ff_shared > 0 && l.mode_shared != kGemv) bits |= EMBER_PATH_SHARED_MFMA;
  return bits;
}

int ember_moe_scratch_routing(const ember_moe_layer* w, int T, ember_moe_routing_view* v) {
  const int s = validate(w);
  if (s) return s;
  if (T < 0) return EMBER_ERR_SHAPE;
  if (!v) return EMBER_ERR_NULL;
  const Layout l = layout(w, std::max(T, 1));
  v->logits = l.logits;
  v->idx = l.idx;
  v->gates = l.gates;
  v->offsets = l.offsets;
  v->perm = l.perm;
  v->pos = l.r.pos;
  v->used = l.r.used;
  v->n_used = l.r.n_used;
  v->fallbacks = l.flag;
  v->mismatches = l.flag + 8;
  v->conflict = l.flag + 8 * (2 * (size_t)w->E + 2);
  return EMBER_OK;
}

size_t ember_moe_prefill_pack_bytes(const ember_moe_layer* w) {
  if (validate(w) != EMBER_OK || !packable(w)) return 0;
  if (bf16_stacks(w)) return (size_t)bf16_exps(w).end;
  return (size_t)pack_layout(w->d, w->d_ff, w->E, w->gate_type).end;
}

int ember_moe_prefill_pack(const ember_moe_layer* w, void* pack, size_t pack_bytes, hipStream_t st) {
  int s = validate(w);
  if (s) return s;
  if (!packable(w)) return EMBER_ERR_TYPE;
  if (!pack) return EMBER_ERR_NULL;
  if (reinterpret_cast<uintptr_t>(pack) % 256) return EMBER_ERR_ALIGN;
  if (bf16_stacks(w)) {
    const Bf16ExpLayout bx = bf16_exps(w);
    if (pack_bytes < (size_t)bx.end) return EMBER_ERR_SCRATCH;
    uint8_t* p = static_cast<uint8_t*>(pack);
    auto o = [&](int64_t off) { return reinterpret_cast<int16_t*>(p + off); };
    const int64_t rb_gu = row_bytes(EMBER_TYPE_BF16, w->d), rb_dn = row_bytes(EMBER_TYPE_BF16, w->d_ff);
    if ((s = launch_bf16_row_exps(w->gate, (int64_t)w->E * w->d_ff, w->d, rb_gu, o(bx.gate), st)) ||
        (s = launch_bf16_row_exps(w->up, (int64_t)w->E * w->d_ff, w->d, rb_gu, o(bx.up), st)) ||
        (s = launch_bf16_row_exps(w->down, (int64_t)w->E * w->d, w->d_ff, rb_dn, o(bx.down), st)) ||
        (s = launch_bf16_pair_max(o(bx.gate), o(bx.up), w->E, w->d_ff, o(bx.hmax), st)))
      return s;
    if (bx.sgate >= 0) {
      const int64_t rs_gu = row_bytes(EMBER_TYPE_BF16, w->d), rs_dn = row_bytes(EMBER_TYPE_BF16, w->d_ff_shared);
      if ((s = launch_bf16_row_exps(w->gate_shared, w->d_ff_shared, w->d, rs_gu, o(bx.sgate), st)) ||
          (s = launch_bf16_row_exps(w->up_shared, w->d_ff_shared, w->d, rs_gu, o(bx.sup), st)) ||
          (s = launch_bf16_row_exps(w->down_shared, w->d, w->d_ff_shared, rs_dn, o(bx.sdown), st)) ||
          (s = launch_bf16_pair_max(o(bx.sgate), o(bx.sup), 1, w->d_ff_shared, o(bx.shmax), st)))
        return s;
    }
    return EMBER_OK;
  }
  const int t = w->gate_type;
  const PackLayout pl = pack_layout(w->d, w->d_ff, w->E, t);
  if (pack_bytes < (size_t)pl.end) return EMBER_ERR_SCRATCH;
  uint8_t* p = static_cast<uint8_t*>(pack);
  const int64_t rb_gu = row_bytes(t, w->d), rb_dn = row_bytes(t, w->d_ff);
  if ((s = launch_prefill_pack(t, w->gate, w->up, rb_gu * w->d_ff, rb_gu, w->E, w->d_ff, w->d, p + pl.gu, st))) return s;
  return launch_prefill_pack(t, w->down, nullptr, rb_dn * w->d, rb_dn, w->E, w->d, w->d_ff, p + pl.dn, st);
}

int ember_moe_router_logits(const float* x, int T, int d, int E, const float* router, float* logits, hipStream_t st) {
  if (T < 0 || d <= 0 || E <= 0) return EMBER_ERR_SHAPE;
  if (T == 0) return EMBER_OK;
  if (!x || !router || !logits) return EMBER_ERR_NULL;
  return launch_router_logits(x, T, d, E, router, logits, st);
}

size_t ember_moe_route_scratch_bytes(int T, int E, int k) {
  if (T < 0 || E <= 0 || k <= 0) return 0;
  return route_layout(std::max(T, 1), E, k, 0).end;
}

int ember_moe_route(const float* logits, int T, int E, int k, int renorm, int scoring, const float* selection_bias,
                    int groups_n, int groups_top, int32_t* idx, float* gates, int32_t* offsets, int32_t* perm,
                    void* scratch, size_t scratch_bytes, hipStream_t st) {
  if (T < 0 || E <= 0 || k <= 0 || E > kMaxE || k > kMaxK) return EMBER_ERR_SHAPE;
  if (scoring != EMBER_SCORE_SOFTMAX && scoring != EMBER_SCORE_SIGMOID) return EMBER_ERR_SHAPE;
  groups_n = std::max(groups_n, 1);
  groups_top = std::max(groups_top, 1);
  if (groups_n > 1 && (E % groups_n || groups_top > groups_n || groups_top * (E / groups_n) < k))
    return EMBER_ERR_SHAPE;
  if (T == 0) return EMBER_OK;
  if (!logits || !idx || !gates || !offsets || !perm) return EMBER_ERR_NULL;
  const RouteLayout r = route_layout(T, E, k, 0);
  if (!scratch || scratch_bytes < r.end) return EMBER_ERR_SCRATCH;
  const bool routed = scoring == EMBER_SCORE_SIGMOID || selection_bias || groups_n > 1;
  return launch_route_dispatch(logits, T, E, k, renorm ? 1 : 0, routed ? 1 : 0, scoring == EMBER_SCORE_SIGMOID ? 1 : 0,
                               selection_bias, groups_n, groups_top, idx, gates,
                               dispatch_scratch(scratch, r, offsets, perm), nullptr, st);
}

}  // extern "C"
