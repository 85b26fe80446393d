// ORACLE — TEST INFRASTRUCTURE ONLY. A C-ABI harness around the reference's own GGUF reader
// (load_gguf_meta, gguf_parser.cpp:117+ under /root/reference, compiled in place by oracle/Makefile into
// oracle/_ref/libref_gguf.so with logger.cpp and quantization.cpp). It reports what the reference reads
// from a file — header, scalar metadata, tensor infos — as text, so that tests can compare this
// project's reader (csrc/gguf.cpp) with it; nothing from the reference is copied into this repository.
#include <cstdio>
#include <cstring>
#include <sstream>
#include <string>
#include <type_traits>
#include <variant>

#include "gguf_parser.h"

namespace {

void put(char* out, size_t cap, const std::string& s) {
  if (!out || cap == 0) return;
  const size_t n = std::min(cap - 1, s.size());
  std::memcpy(out, s.data(), n);
  out[n] = '\0';
}

}  // namespace

extern "C" {

// Reads `path` with load_gguf_meta (no mmap). On success returns 0 and writes lines
//   H <version> <tensor_count> <metadata_kv_count> <data_alignment>
//   M <key> <value>          numeric and bool scalars as %.17g, strings as S <key> <text>
//   T <name> <type> <n_dims> <dim0> ... <offset> <size_in_bytes>
// in the reference's own order (metadata map order, tensor_infos order). On an exception returns -1 and
// writes its message. Returns -2 when `cap` is too small for the text.
int ref_gguf_dump(const char* path, char* out, size_t cap) {
  std::ostringstream os;
  try {
    GGUFData g = load_gguf_meta(path, false);
    os << "H " << g.header.version << ' ' << g.header.tensor_count << ' ' << g.header.metadata_kv_count << ' '
       << g.data_alignment << '\n';
    for (const auto& [key, val] : g.metadata) {
      std::visit(
          [&](const auto& v) {
            using V = std::decay_t<decltype(v)>;
            if constexpr (std::is_same_v<V, std::string>) {
              os << "S " << key << ' ' << v << '\n';
            } else if constexpr (std::is_arithmetic_v<V>) {
              char buf[64];
              std::snprintf(buf, sizeof buf, "%.17g", static_cast<double>(v));
              os << "M " << key << ' ' << buf << '\n';
            }
          },
          val);
    }
    for (const auto& t : g.tensor_infos) {
      os << "T " << t.name << ' ' << static_cast<int>(t.type) << ' ' << t.shape.size();
      for (uint64_t s : t.shape) os << ' ' << s;
      os << ' ' << t.offset << ' ' << t.size_in_bytes << '\n';
    }
  } catch (const std::exception& e) {
    put(out, cap, e.what());
    return -1;
  }
  const std::string s = os.str();
  if (s.size() + 1 > cap) return -2;
  put(out, cap, s);
  return 0;
}

}  // extern "C"
