/* C ABI of the MI355X-native mixture-of-experts FFN (libember_moe.so, HIP / gfx950).
 *
 * Replaces ember.cpp's CUDA operator
 *     size_t moe_ffn_scratch_floats(int T, int d, int d_ff, int E, int k);          cuda_kernels.h:678
 *     void moe_ffn_cuda(cublasHandle_t, const float* x, int T, int d, int d_ff, int E, int k,
 *                       bool renorm, const float* router, const float* gate_exps,
 *                       const float* up_exps, const float* down_exps, float* scratch,
 *                       float* out, cudaStream_t);                                   cuda_kernels.h:691-693
 * and its CPU twins moe_ffn_f32_cpu / moe_ffn_routed_f32_cpu (utils.h:45-51). Same contract as the
 * CUDA operator: caller-owned device weights, input, output and scratch; one stream; no host
 * synchronisation and no allocation inside the call, so it can be captured in a HIP graph; out[T][d]
 * is overwritten. Differences: expert stacks may stay in their GGUF encoding (F32, F16, BF16, Q8_0,
 * Q4_K) instead of being dequantized to F32 at load; the DeepSeek router options of the IR's
 * moe_ffn op (graph_ir.cpp:2689-2709) and a shared expert (graph_ir.cpp:651-657, 919-928) are
 * fields of the layer descriptor; errors are status codes, never exceptions.
 *
 * Layouts (ggml ne order, rows contiguous, blocks along a row):
 *   router        f32 [E][d]                  (ffn_gate_inp)
 *   gate, up      [E][d_ff][d] in `*_type`    (ffn_gate_exps, ffn_up_exps)
 *   down          [E][d][d_ff] in `down_type` (ffn_down_exps)
 *   *_shared      [d_ff_shared][d], [d][d_ff_shared]  (ffn_*_shexp)
 *   x, out        f32 [T][d]
 */
#ifndef EMBER_MOE_H
#define EMBER_MOE_H
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>
#include "ember_moe_host.h"
#include "ember_gguf.h"

#ifdef __cplusplus
extern "C" {
#endif


typedef struct ember_moe_layer {
  int d, d_ff, E, k;
  int renorm;                 /* 1: "renorm" gates (normalised over the k picks); 0: "raw" */
  int scoring;                /* enum ember_moe_scoring */
  const float* selection_bias;/* [E] device, or NULL (IR "selection_bias") */
  int groups_n, groups_top;   /* group-limited routing (IR "groups"); groups_n <= 1: none */
  float out_scale;            /* expert_weights_scale applied to the routed sum; 1: none */
  const float* router;
  const void* gate;  int gate_type;
  const void* up;    int up_type;
  const void* down;  int down_type;
  int d_ff_shared;            /* 0: no shared expert */
  const void* gate_shared; int gate_shared_type;
  const void* up_shared;   int up_shared_type;
  const void* down_shared; int down_shared_type;
  /* Optional (NULL: none): the prefill pack ember_moe_prefill_pack prepared for this layer's stacks
   * (Q8_0 / Q4_K tiles, or BF16 row exponents). Appended last, so descriptors that zero-initialise
   * keep working. */
  const void* prefill_pack;
  /* Optional (NULL: none; requires d_ff_shared > 0): qwen2moe's shared-expert gate ffn_gate_inp_shexp,
   * f32 [d] on the device. The shared expert's output row of token t is scaled by
   * sigmoid(shared_gate · x_t) before it is added (graph_ir.cpp:694-705). Appended last. */
  const float* shared_gate;
} ember_moe_layer;

/* Scratch bytes ember_moe_ffn needs for T tokens of this layer (moe_ffn_scratch_floats' role,
 * cuda_kernels.h:678, in bytes). Returns 0 for an invalid descriptor. */
size_t ember_moe_scratch_bytes(const ember_moe_layer* w, int T);

/* Where ember_moe_ffn leaves its routing in the scratch buffer (byte offsets from its start), for
 * callers and tests that inspect a call's routing after it completes (no reference counterpart; it
 * plays the role of reading back moe_route_sel_kernel's outputs, cuda_kernels.cu:3565-3604):
 *   logits    f32 [T][E]   router logits (with the proven-picks router, EMBER_ROUTER_FAST=1: exact for every
 *                          expert its bound could not rule out, the picks among them, and elsewhere a lower
 *                          bound of the logit that lies strictly below every pick's)
 *   idx       i32 [T][k]   picks, ascending expert ids (-1: none); gates f32 [T][k] their weights
 *   offsets   i32 [E+1]    expert segment starts in the dispatch order; perm i32 [T*k] the slot t*k+j
 *                          at each dispatch position; pos i32 [T*k] slot -> position (-1: no pick)
 *   used      i32 [E]      experts with at least one slot, ascending; n_used i32 their count
 *   fallbacks u64          one-token calls whose routing is fused into the expert launch: the number of
 *                          blocks that stopped waiting for another block's router logit and computed it
 *                          themselves (results are identical either way; a diagnostic that only grows,
 *                          from whatever the buffer held, and is never reset by the library).
 *   mismatches u64         one-token calls with a softmax router: the number of calls whose exact
 *                          routing differed from the pick set the expert launch proved from its fast
 *                          logits (never expected; it only grows, from whatever the buffer held).
 *   conflict  u64          the same event for this call alone: set to 0 by every such call and to 1
 *                          when it happens, in which case that call's output rows are all NaN (a
 *                          pick-set conflict never yields plausible numbers). Meaningful after
 *                          one-token calls with a softmax router; other calls leave it untouched.
 * The same layout holds for every call with this descriptor and T. */
typedef struct ember_moe_routing_view {
  size_t logits, idx, gates, offsets, perm, pos, used, n_used, fallbacks, mismatches, conflict;
} ember_moe_routing_view;
int ember_moe_scratch_routing(const ember_moe_layer* w, int T, ember_moe_routing_view* view);

/* Which kernels a call of this descriptor with T tokens runs (a diagnostic for tests and integrators; no
 * reference counterpart): a bit set of EMBER_PATH_*, or a negative ember_status. Exactly one of GEMV /
 * TILES64 / TILES256 names the routed experts' path; the others add the one-token fusions:
 *   FUSED_ROUTE  router, routing and dispatch run inside the first expert launch;
 *   SLICES       the whole layer in one launch over 64-column slices of d_ff (prefill pack required), plus an
 *                ordered reduce of the slices' partial outputs;
 *   DOWN1        the down projection forms the output rows itself (the combine fused in);
 *   SHARED_MFMA  the shared expert's rows take the MFMA tiles (on a side stream for ember_moe_ffn).
 * The answer can depend on the current device (its CU count) and on the EMBER_* tuning variables. */
#define EMBER_PATH_GEMV 1
#define EMBER_PATH_TILES64 2
#define EMBER_PATH_TILES256 4
#define EMBER_PATH_FUSED_ROUTE 8
#define EMBER_PATH_SLICES 16
#define EMBER_PATH_DOWN1 32
#define EMBER_PATH_SHARED_MFMA 64
int ember_moe_path(const ember_moe_layer* w, int T);

/* Prefill weight packing (no counterpart in the reference, which dequantizes every stack to F32 at
 * load, weight_management.cpp:486-511): a one-time preparation of a layer's routed stacks for the
 * prefill MFMA GEMMs (more than ~1.5-2 tokens per expert), kept beside the stacks, which it never
 * replaces: decode batches stream the ggml rows, except that a one-token call of a Q8_0 / Q4_K layer
 * without a shared expert whose k * d_ff / 64 slices fill the device (EMBER_PATH_SLICES) reads the pack's
 * tiles.
 *   All-Q8_0 layers: each 256-row x 64-column tile contiguous (gate/up: the tile's 128 gate and 128 up
 *     rows; rows past the end repeat the last), 68-byte rows, as large as the three stacks; the GEMM
 *     loads whole tiles and reads them at a bank-conflict-free stride. Same values, same arithmetic:
 *     outputs are bit-identical with or without the pack.
 *   All-Q4_K layers: the same tiles with 40-byte rows (per 32-element group the fp16 factors d * sc and
 *     -dmin * m, then the 32 nibble bytes), 1.11x the stacks; they feed the DMA tile GEMMs, which
 *     without the pack only Q8_0 has.
 *   All-BF16 layers: per weight row an int16 exponent (its largest magnitude lands in [0.5, 1) once
 *     scaled by 2^-e) and per expert the largest gate + up sum, also for a BF16 shared expert (a few KB).
 *     With them the MFMA paths run one fp16 product per weight (rows scaled into fp16's range, the
 *     epilogues scale back exactly) instead of two bf16 products (hi and lo halves of the activations).
 * Q8_0 / Q4_K need d and d_ff multiples of 64; for other layers ember_moe_prefill_pack_bytes returns 0.
 * ember_moe_prefill_pack fills a caller-owned, 256-byte aligned device buffer on `stream`; set the
 * descriptor's prefill_pack to it afterwards. */
size_t ember_moe_prefill_pack_bytes(const ember_moe_layer* w);
int ember_moe_prefill_pack(const ember_moe_layer* w, void* pack, size_t pack_bytes, hipStream_t stream);

/* out[T][d] = the MoE FFN of x[T][d] (moe_ffn_cuda, cuda_kernels.cu:3628-3684; per token the
 * result of moe_ffn_f32_cpu / moe_ffn_routed_f32_cpu, utils.cpp:704-836). T = 0 is a no-op.
 * Returns an ember_status; on error nothing is launched. */
int ember_moe_ffn(const ember_moe_layer* w, const float* x, int T, float* out, void* scratch,
                  size_t scratch_bytes, hipStream_t stream);

/* ember_moe_ffn without a caller scratch buffer, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference (moe_ffn_cuda always takes a caller scratch). It runs exactly ember_moe_ffn's kernels, with
 * identical results, in a library-owned static device buffer of EMBER_MOE_NOALLOC_SCRATCH_BYTES
 * (32 MiB) that each GPU the library runs on holds until the process ends; the call allocates nothing
 * (no hipMalloc / hipFree, no allocating library routine). Calls whose ember_moe_scratch_bytes(w, T)
 * exceeds that size return EMBER_ERR_SCRATCH and launch nothing (decode batches and prefill of a few
 * dozen tokens fit Mixtral-sized layers). Every call on one GPU shares that GPU's buffer: calls that
 * overlap on one GPU (concurrent streams, threads) race and must be serialised by the caller. */
#define EMBER_MOE_NOALLOC_SCRATCH_BYTES (32u << 20)
int ember_moe_ffn_noalloc(const ember_moe_layer* w, const float* x, int T, float* out, hipStream_t stream);

/* ember_moe_ffn with per-phase timing (the role of ember's PrefillOpTimer, model.cpp:1927-1975, which
 * brackets each op with CUDA events). Records HIP events between the launches on `stream`, waits for
 * the last one (this call synchronises the host; it is a profiling entry, not for graph capture) and
 * writes the elapsed milliseconds of the EMBER_MOE_NPHASES phases: router logits, routing, dispatch,
 * gate/up + SwiGLU, down, shared expert, combine. The gate/up and down phases of the decode path are
 * the kernels' own durations (events attached to their dispatch packets), not event-to-event spans. */
#define EMBER_MOE_NPHASES 7
int ember_moe_ffn_timed(const ember_moe_layer* w, const float* x, int T, float* out, void* scratch,
                        size_t scratch_bytes, hipStream_t stream, float* phase_ms);

/* Router logits only: logits[T][E] = (float) of the FP64 fixed-order dot of router row e with x[t]
 * (utils.cpp:707 with cpu_dot.h:12-21) — bit-identical to the reference's CPU logits. */
int ember_moe_router_logits(const float* x, int T, int d, int E, const float* router, float* logits,
                            hipStream_t stream);

/* Routing and dispatch given logits (test / integration entry; no reference counterpart as one
 * call — it isolates moe_route_sel_kernel's role, cuda_kernels.cu:3565-3604, plus the stable
 * counting-sort dispatch). Per token: idx[T][k] ascending expert ids and gates[T][k] exactly as
 * moe_ffn_f32_cpu (scoring softmax, no bias, no groups) or moe_ffn_routed_f32_cpu computes them.
 * offsets[E+1]: per-expert starts in the sorted order; perm[T*k]: the slot t*k+j at each sorted
 * position (a stable sort of the slots by expert). Scratch: ember_moe_route_scratch_bytes. */
size_t ember_moe_route_scratch_bytes(int T, int E, int k);
int ember_moe_route(const float* logits, int T, int E, int k, int renorm, int scoring,
                    const float* selection_bias, int groups_n, int groups_top, int32_t* idx,
                    float* gates, int32_t* offsets, int32_t* perm, void* scratch,
                    size_t scratch_bytes, hipStream_t stream);

/* Device bytes ember_gguf_upload_layer needs for a layer read by ember_gguf_moe_layer (ember_gguf.h),
 * or 0 if the view is incomplete. */
size_t ember_gguf_layer_bytes(const struct ember_gguf_moe* m);
/* Copies the layer's tensors from the mapped file into `dev` (caller-owned device memory, 256-byte
 * aligned, ember_gguf_layer_bytes long) in their GGUF encoding — the expert stacks are not dequantized,
 * unlike the reference's MoE upload (weight_management.cpp:486-511, 1162-1176); only a non-F32 router
 * (F16, BF16, Q8_0) is widened to F32, exactly — and fills *w with device pointers into `dev`, ready for
 * ember_moe_ffn. Synchronises `stream` before returning (the host sources must outlive the copies).
 * EMBER_ERR_TYPE for an encoding the FFN does not run (experts: F32, F16, BF16, Q8_0, Q4_K),
 * EMBER_ERR_SCRATCH if dev_bytes is too small, EMBER_ERR_SHAPE if the descriptor fails validation. */
int ember_gguf_upload_layer(const struct ember_gguf_moe* m, void* dev, size_t dev_bytes, ember_moe_layer* w,
                            hipStream_t stream);
/* Human-readable text for an ember_status. */
const char* ember_moe_strerror(int status);

#ifdef __cplusplus
}
#endif
#endif
