// GGUF reader for the MoE FFN's tensors: header, metadata and tensor infos of a memory-mapped file,
// and the MoE layer view the reference's IR builder derives from them. Interface: include/ember_gguf.h.
//
// Format (GGUF v2/v3, as the reference's gguf_parser.cpp reads it): u32 magic "GGUF", u32 version,
// u64 tensor count, u64 metadata count; metadata entries {string key, u32 type, value}; tensor infos
// {string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset}; the data section starts at the
// next multiple of general.alignment (default 32). Strings are {u64 length, bytes}; arrays are
// {u32 element type, u64 count, elements}. Little-endian throughout.
#include "ember_gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace {

enum : uint32_t {
  KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6, KV_BOOL = 7,
  KV_STRING = 8, KV_ARRAY = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12
};

struct Meta {
  uint32_t type = 0;
  double num = 0.0;  // scalar types
  std::string str;   // KV_STRING
};

struct TensorRec {
  std::string name;
  int type = 0;
  int n_dims = 0;
  int64_t ne[4] = {1, 1, 1, 1};
  uint64_t offset = 0;
  uint64_t bytes = 0;
};

// bytes per block and elements per block of the ggml types whose layout is fixed (ggml_types.h:20-40)
bool type_block(int type, int64_t& bsz, int64_t& bel) {
  switch (type) {
    case 0: bsz = 4; bel = 1; return true;     // F32
    case 1: bsz = 2; bel = 1; return true;     // F16
    case 2: bsz = 18; bel = 32; return true;   // Q4_0
    case 3: bsz = 20; bel = 32; return true;   // Q4_1
    case 6: bsz = 22; bel = 32; return true;   // Q5_0
    case 7: bsz = 24; bel = 32; return true;   // Q5_1
    case 8: bsz = 34; bel = 32; return true;   // Q8_0
    case 9: bsz = 36; bel = 32; return true;   // Q8_1
    case 10: bsz = 84; bel = 256; return true;  // Q2_K
    case 11: bsz = 110; bel = 256; return true; // Q3_K
    case 12: bsz = 144; bel = 256; return true; // Q4_K
    case 13: bsz = 176; bel = 256; return true; // Q5_K
    case 14: bsz = 210; bel = 256; return true; // Q6_K
    case 15: bsz = 292; bel = 256; return true; // Q8_K
    case 24: bsz = 1; bel = 1; return true;     // I8
    case 25: bsz = 2; bel = 1; return true;     // I16
    case 26: bsz = 4; bel = 1; return true;     // I32
    case 27: bsz = 8; bel = 1; return true;     // I64
    case 28: bsz = 8; bel = 1; return true;     // F64
    case 30: bsz = 2; bel = 1; return true;     // BF16
    default: return false;
  }
}

// Bounds-checked little-endian cursor over the mapped file.
struct Cursor {
  const uint8_t* p;
  size_t n, at = 0;
  bool ok = true;
  bool need(size_t k) {
    if (!ok || k > n - at) ok = false;
    return ok;
  }
  template <class T>
  T get() {
    T v{};
    if (need(sizeof(T))) {
      std::memcpy(&v, p + at, sizeof(T));
      at += sizeof(T);
    }
    return v;
  }
  std::string str() {
    const uint64_t len = get<uint64_t>();
    if (!ok || len > (1ull << 30) || !need((size_t)len)) {
      ok = false;
      return {};
    }
    std::string s(reinterpret_cast<const char*>(p + at), (size_t)len);
    at += (size_t)len;
    return s;
  }
  // one value of type t; scalars into m (when given); arrays and strings of arrays are skipped over
  void value(uint32_t t, Meta* m, int depth = 0) {
    double v = 0.0;
    switch (t) {
      case KV_U8: v = get<uint8_t>(); break;
      case KV_I8: v = get<int8_t>(); break;
      case KV_U16: v = get<uint16_t>(); break;
      case KV_I16: v = get<int16_t>(); break;
      case KV_U32: v = get<uint32_t>(); break;
      case KV_I32: v = get<int32_t>(); break;
      case KV_F32: v = get<float>(); break;
      case KV_BOOL: v = get<uint8_t>() != 0; break;
      case KV_U64: v = (double)get<uint64_t>(); break;
      case KV_I64: v = (double)get<int64_t>(); break;
      case KV_F64: v = get<double>(); break;
      case KV_STRING: {
        std::string s = str();
        if (m) m->str = std::move(s);
        break;
      }
      case KV_ARRAY: {
        const uint32_t et = get<uint32_t>();
        const uint64_t cnt = get<uint64_t>();
        if (!ok || depth > 4 || et > KV_F64) {
          ok = false;
          return;
        }
        for (uint64_t i = 0; i < cnt && ok; ++i) value(et, nullptr, depth + 1);
        break;
      }
      default: ok = false; return;
    }
    if (m) {
      m->type = t;
      m->num = v;
    }
  }
};

}  // namespace

struct ember_gguf {
  int fd = -1;
  void* map = nullptr;
  size_t size = 0;
  int version = 0;
  std::map<std::string, Meta> meta;
  std::vector<TensorRec> tensors;
  std::map<std::string, size_t> by_name;
  const uint8_t* data = nullptr;  // start of the tensor data section
  std::string arch;
};

extern "C" {

int64_t ember_ggml_nbytes(int type, int64_t n) {
  int64_t bsz, bel;
  if (!type_block(type, bsz, bel) || n < 0 || n % bel) return -1;
  return n / bel * bsz;
}

void ember_gguf_close(ember_gguf* g) {
  if (!g) return;
  if (g->map && g->map != MAP_FAILED) munmap(g->map, g->size);
  if (g->fd >= 0) close(g->fd);
  delete g;
}

int ember_gguf_open(const char* path, ember_gguf** out) {
  if (!path || !out) return EMBER_ERR_NULL;
  *out = nullptr;
  ember_gguf* g = new ember_gguf();
  auto fail = [&](int s) {
    ember_gguf_close(g);
    return s;
  };
  g->fd = open(path, O_RDONLY);
  if (g->fd < 0) return fail(EMBER_ERR_FORMAT);
  struct stat st;
  if (fstat(g->fd, &st) != 0 || st.st_size < 24) return fail(EMBER_ERR_FORMAT);
  g->size = (size_t)st.st_size;
  g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
  if (g->map == MAP_FAILED) return fail(EMBER_ERR_FORMAT);
  Cursor c{static_cast<const uint8_t*>(g->map), g->size};
  if (c.get<uint32_t>() != 0x46554747u) return fail(EMBER_ERR_FORMAT);  // "GGUF"
  g->version = (int)c.get<uint32_t>();
  if (g->version != 2 && g->version != 3) return fail(EMBER_ERR_FORMAT);
  const uint64_t n_tensors = c.get<uint64_t>();
  const uint64_t n_kv = c.get<uint64_t>();
  if (!c.ok || n_tensors > (1ull << 24) || n_kv > (1ull << 24)) return fail(EMBER_ERR_FORMAT);
  for (uint64_t i = 0; i < n_kv && c.ok; ++i) {
    std::string key = c.str();
    const uint32_t t = c.get<uint32_t>();
    Meta m;
    c.value(t, &m);
    if (c.ok) g->meta[key] = std::move(m);
  }
  if (!c.ok) return fail(EMBER_ERR_FORMAT);
  g->tensors.resize((size_t)n_tensors);
  for (uint64_t i = 0; i < n_tensors && c.ok; ++i) {
    TensorRec& r = g->tensors[(size_t)i];
    r.name = c.str();
    const uint32_t nd = c.get<uint32_t>();
    if (!c.ok || nd == 0 || nd > 4) return fail(EMBER_ERR_FORMAT);
    r.n_dims = (int)nd;
    int64_t nel = 1;
    for (uint32_t j = 0; j < nd; ++j) {
      const uint64_t v = c.get<uint64_t>();
      if (v > (1ull << 40)) return fail(EMBER_ERR_FORMAT);
      r.ne[j] = (int64_t)v;
      if (r.ne[j] != 0 && nel > (int64_t(1) << 50) / r.ne[j]) return fail(EMBER_ERR_FORMAT);
      nel *= r.ne[j];
    }
    r.type = (int)c.get<uint32_t>();
    r.offset = c.get<uint64_t>();
    int64_t bsz, bel;
    if (type_block(r.type, bsz, bel)) {
      if (nel % bel) return fail(EMBER_ERR_FORMAT);  // rows must be whole blocks
      r.bytes = (uint64_t)(nel / bel * bsz);
    } else {
      r.bytes = 0;  // a type whose layout this reader does not know
    }
    if (c.ok && !g->by_name.emplace(r.name, (size_t)i).second) return fail(EMBER_ERR_FORMAT);  // duplicate name
  }
  if (!c.ok) return fail(EMBER_ERR_FORMAT);
  uint64_t align = 32;
  auto ai = g->meta.find("general.alignment");
  if (ai != g->meta.end()) {
    if (ai->second.type == KV_STRING || ai->second.num < 1 || ai->second.num > (1 << 20)) return fail(EMBER_ERR_FORMAT);
    align = (uint64_t)ai->second.num;
    if (align & (align - 1)) return fail(EMBER_ERR_FORMAT);
  }
  const uint64_t start = (c.at + align - 1) / align * align;
  if (start > g->size) return fail(EMBER_ERR_FORMAT);
  g->data = static_cast<const uint8_t*>(g->map) + start;
  const uint64_t avail = g->size - start;
  for (const TensorRec& r : g->tensors)
    if (r.offset % align || r.offset > avail || r.bytes > avail - r.offset) return fail(EMBER_ERR_FORMAT);
  auto arch = g->meta.find("general.architecture");
  if (arch != g->meta.end() && arch->second.type == KV_STRING) g->arch = arch->second.str;
  *out = g;
  return EMBER_OK;
}

int ember_gguf_version(const ember_gguf* g) { return g ? g->version : 0; }
int64_t ember_gguf_n_tensors(const ember_gguf* g) { return g ? (int64_t)g->tensors.size() : 0; }

static void fill_tensor(const ember_gguf* g, const TensorRec& r, ember_gguf_tensor* out) {
  out->name = r.name.c_str();
  out->type = r.type;
  out->n_dims = r.n_dims;
  for (int j = 0; j < 4; ++j) out->ne[j] = r.ne[j];
  out->offset = r.offset;
  out->bytes = r.bytes;
  out->data = g->data + r.offset;
}

int ember_gguf_tensor_at(const ember_gguf* g, int64_t i, ember_gguf_tensor* out) {
  if (!g || !out) return EMBER_ERR_NULL;
  if (i < 0 || i >= (int64_t)g->tensors.size()) return EMBER_ERR_NOT_FOUND;
  fill_tensor(g, g->tensors[(size_t)i], out);
  return EMBER_OK;
}

int ember_gguf_find_tensor(const ember_gguf* g, const char* name, ember_gguf_tensor* out) {
  if (!g || !name || !out) return EMBER_ERR_NULL;
  auto it = g->by_name.find(name);
  if (it == g->by_name.end()) return EMBER_ERR_NOT_FOUND;
  fill_tensor(g, g->tensors[it->second], out);
  return EMBER_OK;
}

int ember_gguf_meta_number(const ember_gguf* g, const char* key, double* out) {
  if (!g || !key || !out) return EMBER_ERR_NULL;
  auto it = g->meta.find(key);
  if (it == g->meta.end() || it->second.type == KV_STRING || it->second.type == KV_ARRAY) return EMBER_ERR_NOT_FOUND;
  *out = it->second.num;
  return EMBER_OK;
}

const char* ember_gguf_meta_string(const ember_gguf* g, const char* key) {
  if (!g || !key) return nullptr;
  auto it = g->meta.find(key);
  return it != g->meta.end() && it->second.type == KV_STRING ? it->second.str.c_str() : nullptr;
}

const char* ember_gguf_arch(const ember_gguf* g) { return g ? g->arch.c_str() : nullptr; }

int ember_gguf_n_layers(const ember_gguf* g) {
  double v;
  if (!g || ember_gguf_meta_number(g, (g->arch + ".block_count").c_str(), &v) != EMBER_OK) return -1;
  return (int)v;
}

int ember_gguf_moe_layer(const ember_gguf* g, int layer, ember_gguf_moe* out) {
  if (!g || !out) return EMBER_ERR_NULL;
  std::memset(out, 0, sizeof(*out));
  out->layer = layer;
  const std::string B = "blk." + std::to_string(layer) + ".";
  const std::string& a = g->arch;
  auto num = [&](const char* key, double dflt) {
    double v;
    return ember_gguf_meta_number(g, (a + "." + key).c_str(), &v) == EMBER_OK ? v : dflt;
  };
  auto find = [&](const std::string& name, ember_gguf_tensor* t) { return ember_gguf_find_tensor(g, name.c_str(), t); };
  if (find(B + "ffn_gate_inp.weight", &out->router) || find(B + "ffn_gate_exps.weight", &out->gate))
    return EMBER_ERR_NOT_FOUND;
  if (find(B + "ffn_up_exps.weight", &out->up) || find(B + "ffn_down_exps.weight", &out->down)) return EMBER_ERR_SHAPE;
  const int64_t* ge = out->gate.ne;
  const int64_t d = ge[0], dff = ge[1], E = ge[2];
  auto same = [](const ember_gguf_tensor& t, int64_t a0, int64_t a1, int64_t a2) {
    return t.ne[0] == a0 && t.ne[1] == a1 && t.ne[2] == a2 && t.ne[3] == 1;
  };
  if (d <= 0 || dff <= 0 || E <= 0 || ge[3] != 1 || !same(out->up, d, dff, E) || !same(out->down, dff, d, E) ||
      !same(out->router, d, E, 1))
    return EMBER_ERR_SHAPE;
  const double count = num("expert_count", (double)E), used = num("expert_used_count", -1.0);
  if (count != (double)E || used < 1 || used > (double)E || d > (1 << 20) || dff > (1 << 24) || E > (1 << 16))
    return EMBER_ERR_SHAPE;
  out->d = (int)d;
  out->d_ff = (int)dff;
  out->E = (int)E;
  out->k = (int)used;
  out->scoring = EMBER_SCORE_SOFTMAX;
  out->renorm = 1;
  out->groups_n = out->groups_top = 1;
  out->out_scale = 1.0f;
  if (a == "llama" || a == "mistral" || a == "qwen3moe") {
    // Mixtral's layout and qwen3moe: renorm softmax gates, no shared expert (graph_ir.cpp:681-699)
  } else if (a == "qwen2moe") {
    out->renorm = 0;  // llama.cpp b6000's qwen2moe graph ignores norm_topk_prob (graph_ir.cpp:693-699)
    // the shared expert joins the FFN only when ffn_gate_inp_shexp gates it (graph_ir.cpp:700-706):
    // f = f + sigmoid(ffn_gate_inp_shexp · h2) * shared(h2)
    if (find(B + "ffn_gate_inp_shexp.weight", &out->shared_gate) == EMBER_OK) {
      const ember_gguf_tensor& g = out->shared_gate;
      if (g.ne[0] != d || g.ne[1] != 1 || g.ne[2] != 1 || g.ne[3] != 1) return EMBER_ERR_SHAPE;
      if (find(B + "ffn_gate_shexp.weight", &out->gate_shared) || find(B + "ffn_up_shexp.weight", &out->up_shared) ||
          find(B + "ffn_down_shexp.weight", &out->down_shared))
        return EMBER_ERR_SHAPE;
      const int64_t dfs = out->gate_shared.ne[1];
      if (dfs <= 0 || !same(out->gate_shared, d, dfs, 1) || !same(out->up_shared, d, dfs, 1) ||
          !same(out->down_shared, dfs, d, 1))
        return EMBER_ERR_SHAPE;
      out->d_ff_shared = (int)dfs;
    }
  } else if (a == "deepseek2") {
    double gating = num("expert_gating_func", 1.0);
    if (gating == 0.0) gating = 1.0;
    if (gating != 1.0 && gating != 2.0) return EMBER_ERR_SHAPE;
    out->scoring = gating == 2.0 ? EMBER_SCORE_SIGMOID : EMBER_SCORE_SOFTMAX;
    out->renorm = num("expert_weights_norm", 0.0) != 0.0;
    double s = num("expert_weights_scale", 1.0);
    if (s == 0.0) s = 1.0;
    out->out_scale = (float)s;
    const double gn = num("expert_group_count", 1.0);
    if (gn > 1) {
      out->groups_n = (int)gn;
      out->groups_top = (int)num("expert_group_used_count", 1.0);
      if (out->groups_n > E || E % out->groups_n || out->groups_top < 1 || out->groups_top > out->groups_n)
        return EMBER_ERR_SHAPE;
    }
    if (find(B + "exp_probs_b.bias", &out->bias) == EMBER_OK) {
      if (out->bias.type != EMBER_TYPE_F32 || !same(out->bias, E, 1, 1)) return EMBER_ERR_SHAPE;
    } else {
      std::memset(&out->bias, 0, sizeof(out->bias));
    }
    if (find(B + "ffn_gate_shexp.weight", &out->gate_shared) == EMBER_OK) {
      if (find(B + "ffn_up_shexp.weight", &out->up_shared) || find(B + "ffn_down_shexp.weight", &out->down_shared))
        return EMBER_ERR_SHAPE;
      const int64_t dfs = out->gate_shared.ne[1];
      if (dfs <= 0 || !same(out->gate_shared, d, dfs, 1) || !same(out->up_shared, d, dfs, 1) ||
          !same(out->down_shared, dfs, d, 1))
        return EMBER_ERR_SHAPE;
      out->d_ff_shared = (int)dfs;
    } else {
      std::memset(&out->gate_shared, 0, sizeof(out->gate_shared));
    }
  } else {
    return EMBER_ERR_SHAPE;  // an architecture whose MoE options the reference's builder does not define
  }
  return EMBER_OK;
}

}  // extern "C"
