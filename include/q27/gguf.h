// Drop-in C++ declarations of the reference engine's src/gguf.h (namespace q27): GType, GTensor, GValue and the
// GGUF reader class with the same members and error behaviour (std::runtime_error with the reference's
// messages), implemented on the C ABI of include/q27h.h (q27h_gguf_*). The file stays memory-mapped for the life
// of the GGUF object; GTensor::data points into the mapping.
#pragma once
#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../q27h.h"

namespace q27 {

// src/gguf.h:11-14: ggml type ids of this model's files.
enum class GType : uint32_t {
  F32 = 0, F16 = 1, Q2_K = 10, Q4_K = 12, Q6_K = 14, IQ2_XXS = 16, IQ2_XS = 17, IQ3_XXS = 18,
  IQ3_S = 21, IQ2_S = 22, IQ4_XS = 23, IQ1_M = 29, BF16 = 30,
};
// src/gguf.h:15-19
inline const char* gtype_name(GType t) { return q27h_gtype_name((int)t); }
inline int gtype_block_bytes(GType t) {
  const int b = q27h_gtype_block_bytes((int)t);
  if (b == 0) throw std::runtime_error("unknown ggml type " + std::to_string((uint32_t)t));
  return b;
}
inline int gtype_block_size(GType t) {
  gtype_block_bytes(t);
  return q27h_gtype_block_size((int)t);
}

// src/gguf.h:21-30
struct GTensor {
  std::string name;
  GType type;
  int n_dims = 0;
  int64_t ne[4] = {1, 1, 1, 1};  // ne[0] = row length (K), ne[1] = rows (N)
  uint64_t offset = 0;           // from the start of the data section
  uint64_t nbytes = 0;
  const uint8_t* data = nullptr;  // points into the mapped file
  int64_t rows() const { return ne[1] * ne[2] * ne[3]; }
  int64_t row_bytes() const { return ne[0] / gtype_block_size(type) * gtype_block_bytes(type); }
};

// src/gguf.h:33-41
struct GValue {
  enum Kind { INT, FLOAT, BOOL, STRING, ARR_INT, ARR_FLOAT, ARR_STRING } kind = INT;
  int64_t i = 0;
  double f = 0;
  std::string s;
  std::vector<int64_t> ai;
  std::vector<double> af;
  std::vector<std::string> as;
};

// src/gguf.h:43-70
class GGUF {
 public:
  explicit GGUF(const std::string& path) : path_(path) {
    if (q27h_gguf_open(path.c_str(), &h_) != Q27H_OK) throw std::runtime_error(q27h_last_error());
    try {
      load();
    } catch (...) {
      q27h_gguf_close(h_);  // the destructor does not run for a constructor that throws
      throw;
    }
  }
  ~GGUF() { q27h_gguf_close(h_); }
  GGUF(const GGUF&) = delete;
  GGUF& operator=(const GGUF&) = delete;

 private:
  // Copies the tensor directory and the key / value table out of the handle.
  void load() {
    const int64_t nt = q27h_gguf_n_tensors(h_);
    tensors_.reserve((size_t)nt);
    for (int64_t i = 0; i < nt; i++) {
      q27h_gtensor c;
      if (q27h_gguf_tensor(h_, i, &c) != Q27H_OK) throw std::runtime_error(q27h_last_error());
      GTensor t;
      t.name.assign(c.name, c.name_len);
      t.type = (GType)c.type;
      t.n_dims = c.n_dims;
      for (int d = 0; d < 4; d++) t.ne[d] = c.ne[d];
      t.offset = c.offset;
      t.nbytes = c.nbytes;
      t.data = c.data;
      index_[t.name] = tensors_.size();
      tensors_.push_back(std::move(t));
    }
    const int64_t nk = q27h_gguf_n_kv(h_);
    for (int64_t i = 0; i < nk; i++) {
      const char* kp = nullptr;
      size_t kn = 0;
      q27h_gvalue c;
      if (q27h_gguf_key(h_, i, &kp, &kn) != Q27H_OK || q27h_gguf_kv_at(h_, i, &c) != Q27H_OK)
        throw std::runtime_error(q27h_last_error());
      GValue v;
      v.kind = (GValue::Kind)c.kind;
      v.i = c.i;
      v.f = c.f;
      if (c.kind == Q27H_GV_STRING) v.s.assign(c.s, c.s_len);
      if (c.kind == Q27H_GV_ARR_INT) v.ai.assign(c.ai, c.ai + c.n);
      if (c.kind == Q27H_GV_ARR_FLOAT) v.af.assign(c.af, c.af + c.n);
      if (c.kind == Q27H_GV_ARR_STRING) {
        v.as.reserve(c.n);
        for (uint64_t j = 0; j < c.n; j++) {
          const char* s = nullptr;
          size_t n = 0;
          if (q27h_gguf_kv_str_at(h_, i, j, &s, &n) != Q27H_OK) throw std::runtime_error(q27h_last_error());
          v.as.emplace_back(s, n);
        }
      }
      kv_[std::string(kp, kn)] = std::move(v);
    }
  }

 public:
  const GTensor& tensor(const std::string& name) const {
    const GTensor* t = find(name);
    if (!t) throw std::runtime_error("missing tensor " + name);
    return *t;
  }
  const GTensor* find(const std::string& name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
  }
  const std::vector<GTensor>& tensors() const { return tensors_; }

  bool has(const std::string& key) const { return kv_.count(key) != 0; }
  const GValue& kv(const std::string& key) const {
    auto it = kv_.find(key);
    if (it == kv_.end()) throw std::runtime_error("missing key " + key);
    return it->second;
  }
  // src/gguf.cpp:203-222
  int64_t get_int(const std::string& key) const {
    const GValue& v = kv(key);
    if (v.kind == GValue::INT || v.kind == GValue::BOOL) return v.i;
    if (v.kind == GValue::ARR_INT && v.ai.size() == 1) return v.ai[0];
    throw std::runtime_error("key is not an int: " + key);
  }
  double get_float(const std::string& key) const {
    const GValue& v = kv(key);
    if (v.kind == GValue::FLOAT) return v.f;
    if (v.kind == GValue::INT) return (double)v.i;
    throw std::runtime_error("key is not a float: " + key);
  }
  const std::string& get_str(const std::string& key) const {
    const GValue& v = kv(key);
    if (v.kind != GValue::STRING) throw std::runtime_error("key is not a string: " + key);
    return v.s;
  }

 private:
  std::string path_;
  q27h_gguf* h_ = nullptr;
  std::map<std::string, GValue> kv_;
  std::vector<GTensor> tensors_;
  std::map<std::string, size_t> index_;
};

}  // namespace q27
