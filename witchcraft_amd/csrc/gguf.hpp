// gguf.hpp -- GGUF v2/v3 container reader (host).
//
// Format: written by the reference's quantize-tool through candle gguf_file::write
// (tools/quantize-tool/src/main.rs:33-35, no metadata) and read by
// VarBuilder::from_gguf_buffer (src/quantized_t5.rs:740-743).  Tensor dims are stored
// innermost-first; `shape` below is outermost-first ([rows, cols] for a weight W[N, K]).
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

namespace t5h {

enum GgmlType : uint32_t { GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_K = 12 };

struct GgufTensor {
  std::string name;
  std::vector<uint64_t> shape;  // outermost first
  uint32_t type = 0;
  const uint8_t* data = nullptr;
  size_t nbytes = 0;
  uint64_t rows() const {
    uint64_t r = 1;
    for (size_t i = 0; i + 1 < shape.size(); i++) r *= shape[i];
    return r;
  }
  uint64_t cols() const { return shape.empty() ? 0 : shape.back(); }
};

struct GgufFile {
  uint32_t version = 0;
  std::vector<GgufTensor> tensors;
  const GgufTensor* find(const std::string& name) const {
    for (const auto& t : tensors)
      if (t.name == name) return &t;
    return nullptr;
  }
};

// Parses `buf` (borrowed: tensor data pointers point into it).  Returns false and sets
// `err` on malformed input or unsupported tensor types.
bool parse_gguf(const uint8_t* buf, size_t len, GgufFile& out, std::string& err);

}  // namespace t5h
