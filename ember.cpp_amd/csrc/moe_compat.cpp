// moe_ffn_hip / moe_ffn_scratch_floats: ember.cpp's operator signature (cuda_kernels.h:678, 691-693)
// over the C ABI. See include/ember_moe_compat.hpp.
#include "ember_moe_compat.hpp"

#include <stdexcept>
#include <string>

#include "ember_moe.h"

namespace {

ember_moe_layer descriptor(int d, int d_ff, int E, int k, bool renorm, const float* router, const void* g,
                           const void* u, const void* dn, int type) {
  ember_moe_layer w{};
  w.d = d;
  w.d_ff = d_ff;
  w.E = E;
  w.k = k;
  w.renorm = renorm ? 1 : 0;
  w.scoring = EMBER_SCORE_SOFTMAX;
  w.groups_n = 1;
  w.groups_top = 1;
  w.out_scale = 1.0f;
  w.router = router;
  w.gate = g;
  w.up = u;
  w.down = dn;
  w.gate_type = w.up_type = w.down_type = type;
  return w;
}

// Stand-in pointers for sizing only: the descriptor checks them for null and 16-byte alignment.
const void* const kSizingPtr = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));

}  // namespace

size_t moe_ffn_scratch_floats_typed(int T, int d, int d_ff, int E, int k, int type) {
  const ember_moe_layer w = descriptor(d, d_ff, E, k, true, static_cast<const float*>(kSizingPtr), kSizingPtr,
                                       kSizingPtr, kSizingPtr, type);
  const size_t bytes = ember_moe_scratch_bytes(&w, T);
  if (bytes == 0) throw std::runtime_error("moe_ffn_scratch_floats: unsupported shape or type");
  return (bytes + sizeof(float) - 1) / sizeof(float);
}

size_t moe_ffn_scratch_floats(int T, int d, int d_ff, int E, int k) {
  return moe_ffn_scratch_floats_typed(T, d, d_ff, E, k, EMBER_TYPE_F32);
}

void moe_ffn_hip_typed(const float* x, int T, int d, int d_ff, int E, int k, bool renorm, const float* router,
                       const void* gate_exps, const void* up_exps, const void* down_exps, int type, float* scratch,
                       float* out, hipStream_t stream) {
  const ember_moe_layer w = descriptor(d, d_ff, E, k, renorm, router, gate_exps, up_exps, down_exps, type);
  const size_t floats = moe_ffn_scratch_floats_typed(T, d, d_ff, E, k, type);
  const int s = ember_moe_ffn(&w, x, T, out, scratch, floats * sizeof(float), stream);
  if (s != EMBER_OK) throw std::runtime_error(std::string("moe_ffn_hip: ") + ember_moe_strerror(s));
}

void moe_ffn_hip(const float* x, int T, int d, int d_ff, int E, int k, bool renorm, const float* router,
                 const float* gate_exps, const float* up_exps, const float* down_exps, float* scratch, float* out,
                 hipStream_t stream) {
  moe_ffn_hip_typed(x, T, d, d_ff, E, k, renorm, router, gate_exps, up_exps, down_exps, EMBER_TYPE_F32, scratch, out,
                    stream);
}
