/* GGUF reader for the MoE FFN's tensors (libember_moe_host.so: plain C ABI, no GPU).
 *
 * Replaces, for the expert path, the reference's load_gguf_meta (gguf_parser.h:91-94,
 * gguf_parser.cpp) and the way its loader finds an MoE layer's tensors (weight_management.cpp:
 * 1162-1176: ffn_gate_inp, ffn_{gate,up,down}_exps) and router options (graph_ir.cpp:630-720 for
 * llama / qwen2moe / qwen3moe, 820-930 for deepseek2). The file is memory-mapped; nothing is
 * dequantized: ember_gguf_upload_layer (ember_moe.h) copies the expert stacks to the GPU in their
 * GGUF blocks, where the reference dequantizes them to F32 first (weight_management.cpp:486-511).
 *
 * Supported: GGUF versions 2 and 3, every metadata value type, tensors of any ggml type (sizes are
 * known for F32, F16, BF16, F64, I8-I64, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 and the K-quants);
 * general.alignment (default 32). Every tensor of a known type is checked against the file size.
 */
#ifndef EMBER_GGUF_H
#define EMBER_GGUF_H
#include <stddef.h>
#include <stdint.h>
#include "ember_moe_host.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ember_gguf ember_gguf; /* an open, mapped file */

typedef struct ember_gguf_tensor {
  const char* name;    /* NULL: absent (in ember_gguf_moe) */
  int type;            /* ggml type id */
  int n_dims;
  int64_t ne[4];       /* ggml order: ne[0] is the contiguous dimension; unused dims are 1 */
  uint64_t offset;     /* bytes from the start of the tensor data section */
  uint64_t bytes;      /* size of the data */
  const void* data;    /* the mapped bytes */
} ember_gguf_tensor;

/* Opens and validates `path`. Returns EMBER_OK and *out, or EMBER_ERR_FORMAT (unreadable file, bad
 * magic / version, truncated or inconsistent header, duplicate tensor names, a tensor offset not
 * aligned or a tensor past the end of the file) or EMBER_ERR_NULL. A tensor of a type whose layout
 * is not known here has bytes = 0 (its extent cannot be checked; the MoE path rejects it). */
int ember_gguf_open(const char* path, ember_gguf** out);
void ember_gguf_close(ember_gguf* g);

int ember_gguf_version(const ember_gguf* g);
int64_t ember_gguf_n_tensors(const ember_gguf* g);
/* Tensor i in file order, or by name. EMBER_ERR_NOT_FOUND when out of range / absent. */
int ember_gguf_tensor_at(const ember_gguf* g, int64_t i, ember_gguf_tensor* out);
int ember_gguf_find_tensor(const ember_gguf* g, const char* name, ember_gguf_tensor* out);

/* Scalar metadata as a double (any integer, float or bool type), a string, or general.architecture.
 * meta_number returns EMBER_ERR_NOT_FOUND when the key is absent or not a scalar; meta_string NULL. */
int ember_gguf_meta_number(const ember_gguf* g, const char* key, double* out);
const char* ember_gguf_meta_string(const ember_gguf* g, const char* key);
const char* ember_gguf_arch(const ember_gguf* g);
int ember_gguf_n_layers(const ember_gguf* g); /* {arch}.block_count, or -1 */

/* Mixture-of-experts layer `layer` of the file, as the reference's IR builder reads it:
 *   llama / mistral (Mixtral's layout): softmax, renorm (graph_ir.cpp:681-690);
 *   qwen3moe: softmax, renorm; qwen2moe: softmax, raw gates, and, when the file has
 *     ffn_gate_inp_shexp, the shared expert ffn_{gate,up,down}_shexp scaled per token by
 *     sigmoid(ffn_gate_inp_shexp · h) (graph_ir.cpp:694-705);
 *   deepseek2: expert_gating_func (1 softmax, 2 sigmoid), expert_weights_norm (renorm), expert_weights_scale,
 *     exp_probs_b.bias as the selection bias, expert_group_count / expert_group_used_count, and the
 *     ungated shared expert ffn_{gate,up,down}_shexp (graph_ir.cpp:832-851, 911-928).
 * Shapes are taken from the tensors (router [E][d] = ne {d, E}; gate/up ne {d, d_ff, E}; down
 * ne {d_ff, d, E}; shared gate/up ne {d, d_ff_shared}, down ne {d_ff_shared, d}) and checked against
 * each other and {arch}.expert_count / expert_used_count. Returns EMBER_ERR_NOT_FOUND when the layer
 * has no MoE tensors (e.g. deepseek2's leading dense blocks), EMBER_ERR_SHAPE on inconsistent shapes
 * or options. */
typedef struct ember_gguf_moe {
  int layer;
  int d, d_ff, E, k;
  int renorm, scoring;     /* enum ember_moe_scoring values */
  int groups_n, groups_top;
  float out_scale;
  int d_ff_shared;         /* 0: none */
  ember_gguf_tensor router, gate, up, down;
  ember_gguf_tensor bias;                               /* name NULL: none */
  ember_gguf_tensor gate_shared, up_shared, down_shared; /* name NULL: none */
  ember_gguf_tensor shared_gate;                        /* qwen2moe ffn_gate_inp_shexp ne {d}; name NULL: none */
} ember_gguf_moe;
int ember_gguf_moe_layer(const ember_gguf* g, int layer, ember_gguf_moe* out);

/* Bytes of n elements of ggml type `type` (n a whole number of blocks), or -1 for an unknown type. */
int64_t ember_ggml_nbytes(int type, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
