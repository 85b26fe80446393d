// Upload of one GGUF MoE layer to the GPU in its file encoding (the role of the reference's MoE
// upload, weight_management.cpp:486-511, minus its dequantization of the expert stacks to F32).
#include <hip/hip_runtime.h>

#include <cstring>
#include <vector>

#include "ember_gguf.h"
#include "ember_moe.h"
#include "moe_internal.hpp"

namespace {

constexpr size_t kAlign = 256;
size_t up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

bool expert_type_ok(int t) {
  return t == EMBER_TYPE_F32 || t == EMBER_TYPE_F16 || t == EMBER_TYPE_BF16 || t == EMBER_TYPE_Q8_0 ||
         t == EMBER_TYPE_Q4_K;
}
bool router_type_ok(int t) {
  return t == EMBER_TYPE_F32 || t == EMBER_TYPE_F16 || t == EMBER_TYPE_BF16 || t == EMBER_TYPE_Q8_0;
}
bool present(const ember_gguf_tensor& t) { return t.name != nullptr && t.data != nullptr; }

}  // namespace

extern "C" {

size_t ember_gguf_layer_bytes(const ember_gguf_moe* m) {
  if (!m || !present(m->router) || !present(m->gate) || !present(m->up) || !present(m->down)) return 0;
  size_t n = up((size_t)m->E * m->d * sizeof(float));
  if (present(m->bias)) n += up((size_t)m->E * sizeof(float));
  n += up(m->gate.bytes) + up(m->up.bytes) + up(m->down.bytes);
  if (m->d_ff_shared > 0) n += up(m->gate_shared.bytes) + up(m->up_shared.bytes) + up(m->down_shared.bytes);
  if (m->d_ff_shared > 0 && present(m->shared_gate)) n += up((size_t)m->d * sizeof(float));
  return n;
}

int ember_gguf_upload_layer(const ember_gguf_moe* m, void* dev, size_t dev_bytes, ember_moe_layer* w,
                            hipStream_t stream) {
  if (!m || !dev || !w) return EMBER_ERR_NULL;
  const size_t need = ember_gguf_layer_bytes(m);
  if (need == 0) return EMBER_ERR_NULL;
  if (dev_bytes < need) return EMBER_ERR_SCRATCH;
  if (!router_type_ok(m->router.type) || !expert_type_ok(m->gate.type) || !expert_type_ok(m->up.type) ||
      !expert_type_ok(m->down.type))
    return EMBER_ERR_TYPE;
  if (m->d_ff_shared > 0 && (!present(m->gate_shared) || !present(m->up_shared) || !present(m->down_shared) ||
                             !expert_type_ok(m->gate_shared.type) || !expert_type_ok(m->up_shared.type) ||
                             !expert_type_ok(m->down_shared.type)))
    return EMBER_ERR_TYPE;
  const bool sgate = m->d_ff_shared > 0 && present(m->shared_gate);
  if (sgate && !router_type_ok(m->shared_gate.type)) return EMBER_ERR_TYPE;
  // the descriptor first, so that its own validation (block widths, alignment) runs before any copy
  ember_moe_layer l{};
  l.d = m->d;
  l.d_ff = m->d_ff;
  l.E = m->E;
  l.k = m->k;
  l.renorm = m->renorm;
  l.scoring = m->scoring;
  l.groups_n = m->groups_n;
  l.groups_top = m->groups_top;
  l.out_scale = m->out_scale;
  l.gate_type = m->gate.type;
  l.up_type = m->up.type;
  l.down_type = m->down.type;
  l.d_ff_shared = m->d_ff_shared;
  uint8_t* base = static_cast<uint8_t*>(dev);
  size_t at = 0;
  auto place = [&](size_t bytes) {
    void* p = base + at;
    at += up(bytes);
    return p;
  };
  float* router = static_cast<float*>(place((size_t)m->E * m->d * sizeof(float)));
  float* bias = present(m->bias) ? static_cast<float*>(place((size_t)m->E * sizeof(float))) : nullptr;
  void* gate = place(m->gate.bytes);
  void* upw = place(m->up.bytes);
  void* down = place(m->down.bytes);
  void *gs = nullptr, *us = nullptr, *ds = nullptr;
  if (m->d_ff_shared > 0) {
    gs = place(m->gate_shared.bytes);
    us = place(m->up_shared.bytes);
    ds = place(m->down_shared.bytes);
    l.gate_shared_type = m->gate_shared.type;
    l.up_shared_type = m->up_shared.type;
    l.down_shared_type = m->down_shared.type;
  }
  float* sg = sgate ? static_cast<float*>(place((size_t)m->d * sizeof(float))) : nullptr;
  l.shared_gate = sg;
  l.router = router;
  l.selection_bias = bias;
  l.gate = gate;
  l.up = upw;
  l.down = down;
  l.gate_shared = gs;
  l.up_shared = us;
  l.down_shared = ds;
  if (ember_moe_scratch_bytes(&l, 1) == 0) return EMBER_ERR_SHAPE;

  // the router is F32 on the device: other encodings are dequantized here, exactly (fp16 / bf16
  // widen exactly; a Q8_0 value d * q is exact in f32), as the reference does at load
  std::vector<float> rf;
  const void* rsrc = m->router.data;
  const size_t rbytes = (size_t)m->E * m->d * sizeof(float);
  if (m->router.type != EMBER_TYPE_F32) {
    rf.resize((size_t)m->E * m->d);
    if (ember_dequantize(m->router.type, m->router.data, (int64_t)rf.size(), rf.data()) != EMBER_OK) return EMBER_ERR_TYPE;
    rsrc = rf.data();
  }
  hipError_t e = hipMemcpyAsync(router, rsrc, rbytes, hipMemcpyHostToDevice, stream);
  if (e == hipSuccess && bias) e = hipMemcpyAsync(bias, m->bias.data, (size_t)m->E * sizeof(float), hipMemcpyHostToDevice, stream);
  if (e == hipSuccess) e = hipMemcpyAsync(gate, m->gate.data, m->gate.bytes, hipMemcpyHostToDevice, stream);
  if (e == hipSuccess) e = hipMemcpyAsync(upw, m->up.data, m->up.bytes, hipMemcpyHostToDevice, stream);
  if (e == hipSuccess) e = hipMemcpyAsync(down, m->down.data, m->down.bytes, hipMemcpyHostToDevice, stream);
  if (e == hipSuccess && gs) e = hipMemcpyAsync(gs, m->gate_shared.data, m->gate_shared.bytes, hipMemcpyHostToDevice, stream);
  if (e == hipSuccess && us) e = hipMemcpyAsync(us, m->up_shared.data, m->up_shared.bytes, hipMemcpyHostToDevice, stream);
  if (e == hipSuccess && ds) e = hipMemcpyAsync(ds, m->down_shared.data, m->down_shared.bytes, hipMemcpyHostToDevice, stream);
  // qwen2moe's shared-expert gate row, F32 on the device like the router (widened exactly)
  std::vector<float> gf;
  if (e == hipSuccess && sg) {
    const void* src = m->shared_gate.data;
    if (m->shared_gate.type != EMBER_TYPE_F32) {
      gf.resize((size_t)m->d);
      if (ember_dequantize(m->shared_gate.type, m->shared_gate.data, (int64_t)gf.size(), gf.data()) != EMBER_OK)
        return EMBER_ERR_TYPE;
      src = gf.data();
    }
    e = hipMemcpyAsync(sg, src, (size_t)m->d * sizeof(float), hipMemcpyHostToDevice, stream);
  }
  // the host sources (the mapped file, the dequantized router) must outlive the copies
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return EMBER_ERR_LAUNCH;
  *w = l;
  return EMBER_OK;
}

}  // extern "C"
