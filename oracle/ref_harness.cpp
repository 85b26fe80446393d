// ORACLE — TEST INFRASTRUCTURE ONLY. A C-ABI harness around the reference's own CPU MoE sources
// (utils.cpp, quantization.cpp, logger.cpp, graph_ir_ops.cpp under /root/reference, compiled in place by oracle/Makefile
// into oracle/_ref/libref_moe.so). It is used to pin oracle/moe_oracle.cpp and to write golden vectors;
// nothing from the reference is copied into this repository.
#include <omp.h>

#include <cstdint>
#include <vector>
#include "cpu_dot.h"
#include "graph_ir_ops.h"
#include "quantization.h"
#include "utils.h"

extern "C" {

double ref_dot_f32_f64(const float* a, const float* b, int n) { return ember::dot_f32_f64(a, b, n); }
double ref_dot_f32_f64_portable(const float* a, const float* b, int n) { return ember::dot_f32_f64_portable(a, b, n); }

float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h, false); }

// quantization.cpp:1092 dequantize_q8_0_block over nb consecutive 34-byte blocks.
void ref_dequant_q8_0(const void* blocks, int64_t nb, float* out) {
  const block_q8_0* b = static_cast<const block_q8_0*>(blocks);
  for (int64_t i = 0; i < nb; ++i) dequantize_q8_0_block(b + i, out + i * 32);
}

// quantization.cpp:171 dequantize_q4_k_m over nb consecutive 144-byte super-blocks.
void ref_dequant_q4_k(const void* blocks, int64_t nb, float* out) {
  const block_q4_K* b = static_cast<const block_q4_K*>(blocks);
  for (int64_t i = 0; i < nb; ++i) dequantize_q4_k_m(b + i, out + i * 256, 256, false);
}

// utils.cpp:704 moe_ffn_f32_cpu, token by token.
void ref_moe_ffn_f32(const float* x, int T, int d, int d_ff, int E, int k, const float* R, const float* G,
                     const float* U, const float* D, float* out, int renorm) {
  for (int t = 0; t < T; ++t)
    moe_ffn_f32_cpu(x + (size_t)t * d, d, d_ff, E, k, R, G, U, D, out + (size_t)t * d, renorm != 0);
}

// The reference's prefill driver over the same function: an OpenMP static schedule over tokens
// (cpu_batch_processor.cpp:223-231), on nthreads threads (<= 0: OpenMP's default).
void ref_moe_ffn_f32_omp(const float* x, int T, int d, int d_ff, int E, int k, const float* R, const float* G,
                         const float* U, const float* D, float* out, int renorm, int nthreads) {
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : omp_get_max_threads())
  for (int t = 0; t < T; ++t)
    moe_ffn_f32_cpu(x + (size_t)t * d, d, d_ff, E, k, R, G, U, D, out + (size_t)t * d, renorm != 0);
}

// utils.cpp:758 moe_ffn_routed_f32_cpu, token by token.
void ref_moe_ffn_routed_f32(const float* x, int T, int d, int d_ff, int E, int k, const float* R, const float* G,
                            const float* U, const float* D, float* out, int renorm, int sigmoid, const float* bias,
                            int groups_n, int groups_top) {
  for (int t = 0; t < T; ++t)
    moe_ffn_routed_f32_cpu(x + (size_t)t * d, d, d_ff, E, k, R, G, U, D, out + (size_t)t * d, renorm != 0,
                           sigmoid != 0, bias, groups_n, groups_top);
}

// utils.cpp:867 matmul_f32_f32_batch_cpu (the IR's F32 `linear`) and utils.cpp:838 silu_cpu.
void ref_matmul_f32_batch(const float* W, const float* x, float* y, int T, int out_dim, int in_dim) {
  std::vector<float> w(W, W + (size_t)out_dim * in_dim), xv(x, x + (size_t)T * in_dim), yv;
  matmul_f32_f32_batch_cpu(w, xv, yv, T, out_dim, in_dim);
  for (size_t i = 0; i < yv.size(); ++i) y[i] = yv[i];
}
void ref_silu(const float* x, float* y, int64_t n) {
  std::vector<float> xv(x, x + n), yv(n);
  silu_cpu(xv, yv);
  for (int64_t i = 0; i < n; ++i) y[i] = yv[i];
}

// graph_ir_ops.cpp:22 sigmoid and :61 mul_col (the IR ops of qwen2moe's shared-expert gate,
// graph_ir.cpp:704-705).
void ref_sigmoid(const float* x, float* y, int64_t n) { ember_ir::cpu::sigmoid(x, y, (size_t)n); }
void ref_mul_col(const float* x, const float* c, float* y, int T, int w) { ember_ir::cpu::mul_col(x, c, y, T, w); }

}  // extern "C"
