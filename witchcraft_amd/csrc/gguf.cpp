// gguf.cpp -- GGUF container reader (see gguf.hpp).
#include "gguf.hpp"

#include <string.h>

namespace t5h {
namespace {

class Cursor {
 public:
  Cursor(const uint8_t* p, size_t n) : p_(p), n_(n) {}
  bool ok() const { return ok_; }
  size_t pos() const { return pos_; }
  template <typename T>
  T get() {
    T v{};
    if (pos_ + sizeof(T) > n_) {
      ok_ = false;
      return v;
    }
    memcpy(&v, p_ + pos_, sizeof(T));
    pos_ += sizeof(T);
    return v;
  }
  std::string str() {
    const uint64_t len = get<uint64_t>();
    if (!ok_ || len > n_ - pos_) {
      ok_ = false;
      return {};
    }
    std::string s(reinterpret_cast<const char*>(p_ + pos_), len);
    pos_ += len;
    return s;
  }
  void skip(uint64_t nbytes) {
    if (nbytes > n_ - pos_) {
      ok_ = false;
      return;
    }
    pos_ += nbytes;
  }
  // Skips one metadata value of GGUF type `t`; returns its u32 value when t == UINT32.
  uint64_t value(uint32_t t, int depth = 0) {
    switch (t) {
      case 0: case 1: case 7: skip(1); return 0;   // u8 i8 bool
      case 2: case 3: skip(2); return 0;           // u16 i16
      case 4: return get<uint32_t>();              // u32
      case 5: case 6: skip(4); return 0;           // i32 f32
      case 10: case 11: case 12: skip(8); return 0;  // u64 i64 f64
      case 8: str(); return 0;                     // string
      case 9: {                                    // array
        const uint32_t et = get<uint32_t>();
        const uint64_t n = get<uint64_t>();
        if (depth > 4 || n > n_) {
          ok_ = false;
          return 0;
        }
        for (uint64_t i = 0; i < n && ok_; i++) value(et, depth + 1);
        return 0;
      }
      default: ok_ = false; return 0;
    }
  }

 private:
  const uint8_t* p_;
  size_t n_, pos_ = 0;
  bool ok_ = true;
};

}  // namespace

bool parse_gguf(const uint8_t* buf, size_t len, GgufFile& out, std::string& err) {
  if (!buf || len < 24) {
    err = "GGUF buffer is empty or truncated";
    return false;
  }
  Cursor c(buf, len);
  if (c.get<uint32_t>() != 0x46554747u) {  // "GGUF"
    err = "not a GGUF file (bad magic)";
    return false;
  }
  out.version = c.get<uint32_t>();
  if (out.version != 2 && out.version != 3) {
    err = "unsupported GGUF version " + std::to_string(out.version);
    return false;
  }
  const uint64_t n_tensors = c.get<uint64_t>();
  const uint64_t n_kv = c.get<uint64_t>();
  uint64_t alignment = 32;
  for (uint64_t i = 0; i < n_kv && c.ok(); i++) {
    const std::string key = c.str();
    const uint32_t t = c.get<uint32_t>();
    const uint64_t v = c.value(t);
    if (key == "general.alignment" && t == 4) alignment = v;
  }
  if (!c.ok() || n_tensors > 1000000 || alignment == 0) {
    err = "malformed GGUF metadata";
    return false;
  }
  struct Info {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type;
    uint64_t offset;
  };
  std::vector<Info> infos(n_tensors);
  for (auto& in : infos) {
    in.name = c.str();
    const uint32_t nd = c.get<uint32_t>();
    if (!c.ok() || nd == 0 || nd > 4) {
      err = "malformed GGUF tensor info";
      return false;
    }
    in.dims.resize(nd);
    for (auto& d : in.dims) d = c.get<uint64_t>();
    in.type = c.get<uint32_t>();
    in.offset = c.get<uint64_t>();
  }
  if (!c.ok()) {
    err = "truncated GGUF tensor table";
    return false;
  }
  const uint64_t data0 = (c.pos() + alignment - 1) / alignment * alignment;
  out.tensors.clear();
  out.tensors.reserve(infos.size());
  for (auto& in : infos) {
    GgufTensor t;
    t.name = in.name;
    t.shape.assign(in.dims.rbegin(), in.dims.rend());
    t.type = in.type;
    uint64_t ne = 1;
    for (auto d : in.dims) ne *= d;
    switch (in.type) {
      case GGML_F32: t.nbytes = ne * 4; break;
      case GGML_F16: t.nbytes = ne * 2; break;
      case GGML_Q4_K:
        if (in.dims[0] % 256) {
          err = "tensor " + in.name + ": Q4_K row length not a multiple of 256";
          return false;
        }
        t.nbytes = ne / 256 * 144;
        break;
      default:
        err = "tensor " + in.name + ": unsupported GGML type " + std::to_string(in.type);
        return false;
    }
    if (data0 + in.offset > len || t.nbytes > len - (data0 + in.offset)) {
      err = "tensor " + in.name + ": data out of range";
      return false;
    }
    t.data = buf + data0 + in.offset;
    out.tensors.push_back(std::move(t));
  }
  return true;
}

}  // namespace t5h
