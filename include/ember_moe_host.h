/* Host-side data utilities for the MI355X MoE FFN (libember_moe_host.so, plain C ABI, no GPU).
 *
 * These write the llama.cpp byte layouts the reference reads: ggml type ids (ggml_types.h:20-40),
 * block_q8_0 {fp16 d; int8 qs[32]} (quantization.h:137-140) and block_q4_K {fp16 d, dmin;
 * u8 scales[12]; u8 qs[128]} (quantization.h:58-63). The reference itself quantizes with gguf-py
 * (tools/quantize_gguf.py:84-86); these quantizers are this project's own, and the reference's
 * dequantizers (quantization.cpp:171-224, 1092-1097) decode their output.
 */
#ifndef EMBER_MOE_HOST_H
#define EMBER_MOE_HOST_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids (ggml_types.h:20-40). */
enum ember_ggml_type {
  EMBER_TYPE_F32 = 0,
  EMBER_TYPE_F16 = 1,
  EMBER_TYPE_Q8_0 = 8,
  EMBER_TYPE_Q4_K = 12,
  EMBER_TYPE_BF16 = 30
};

/* Router scoring of an MoE layer (ember_moe_layer.scoring, ember_gguf_moe.scoring). */
enum ember_moe_scoring {
  EMBER_SCORE_SOFTMAX = 0, /* softmax of the router logits */
  EMBER_SCORE_SIGMOID = 1  /* DeepSeek-V3 sigmoid scores (IR "scoring": "sigmoid") */
};

/* Status codes shared by every entry point: 0 is success, errors are negative. */
enum ember_status {
  EMBER_OK = 0,
  EMBER_ERR_SHAPE = -1,   /* a dimension is out of range or not a multiple of the block width */
  EMBER_ERR_TYPE = -2,    /* unsupported ggml type */
  EMBER_ERR_SCRATCH = -3, /* scratch buffer missing or smaller than ember_moe_scratch_bytes */
  EMBER_ERR_NULL = -4,    /* a required pointer is NULL */
  EMBER_ERR_LAUNCH = -5,  /* a kernel launch failed (hipGetLastError) */
  EMBER_ERR_ALIGN = -6,   /* a weight pointer is not 16-byte aligned */
  EMBER_ERR_FORMAT = -7,  /* a malformed or unreadable GGUF file (ember_gguf.h) */
  EMBER_ERR_NOT_FOUND = -8 /* no such tensor, key or MoE layer in the file */
};

/* n values ~ N(mean, stddev^2) from a counter-based generator: value i depends only on
 * (seed, stream, i), so slices can be generated independently. Deterministic across hosts
 * that share a libm. */
void ember_fill_normal(float* out, int64_t n, uint64_t seed, uint64_t stream, float mean, float stddev);

/* Bytes of one row of n elements of `type` (n must be a whole number of blocks), or -1. */
int64_t ember_row_bytes(int type, int64_t n);

/* Quantize / dequantize n elements (whole blocks) between f32 and `type`. Return ember_status. */
int ember_quantize(int type, const float* x, int64_t n, void* out);
int ember_dequantize(int type, const void* src, int64_t n, float* out);

uint16_t ember_f32_to_f16(float f);
float ember_f16_to_f32(uint16_t h);
uint16_t ember_f32_to_bf16(float f);

#ifdef __cplusplus
}
#endif
#endif
