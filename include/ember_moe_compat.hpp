// C++ shim with the signature of ember.cpp's MoE operator, for the engine's call sites.
//
// Replaces (cuda_kernels.h:678, 691-693)
//   size_t moe_ffn_scratch_floats(int T, int d, int d_ff, int E, int k);
//   void moe_ffn_cuda(cublasHandle_t, const float* x, int T, int d, int d_ff, int E, int k, bool renorm,
//                     const float* router, const float* gate_exps, const float* up_exps,
//                     const float* down_exps, float* scratch, float* out, cudaStream_t);
// with the same arguments minus the cuBLAS handle: F32 stacks in llama.cpp's layout, caller-owned
// device scratch of moe_ffn_scratch_floats(T, ...) floats, one stream, no host synchronisation (so
// the decode call can stay inside a captured graph, model.cpp:1246, 1321). Like the reference, a
// failure throws std::runtime_error. moe_ffn_hip_typed takes stacks still in their GGUF encoding.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstddef>

size_t moe_ffn_scratch_floats(int T, int d, int d_ff, int E, int k);

void moe_ffn_hip(const float* x, int T, int d, int d_ff, int E, int k, bool renorm, const float* router,
                 const float* gate_exps, const float* up_exps, const float* down_exps, float* scratch, float* out,
                 hipStream_t stream);

// Quantized / half stacks: `type` is the ggml type id of all three stacks (EMBER_TYPE_*).
size_t moe_ffn_scratch_floats_typed(int T, int d, int d_ff, int E, int k, int type);
void moe_ffn_hip_typed(const float* x, int T, int d, int d_ff, int E, int k, bool renorm, const float* router,
                       const void* gate_exps, const void* up_exps, const void* down_exps, int type, float* scratch,
                       float* out, hipStream_t stream);
