// aos_ingest.hpp — reading the artifacts the reference loads: safetensors files (a JSON header and
// one data buffer), MLX-community 4-bit base projections and LoRA adapters.
//
//   safetensors layout        the reference reads it with the Rust crate safetensors 0.7.0 (Cargo.lock);
//                             this restates the format that crate documents: 8-byte little-endian
//                             header length N (at most 100 MB), N bytes of JSON starting with '{'
//                             {name: {dtype, shape, data_offsets: [begin, end]}, "__metadata__": {..}},
//                             then the data buffer, which the offsets index entirely, without holes
//                             or overlaps; each tensor's byte length is numel x dtype size
//   4-bit base projection     "<key>.weight" u32 [out, in/8], "<key>.scales" and optional "<key>.biases"
//                             [out, in/64] (mlx_cpp_wrapper_real.cpp:925-956: a missing bias is zero)
//   LoRA adapter              crates/adapteros-lora-mlx-ffi/src/backend.rs:1017-1210 — target modules
//                             discovered from "lora_a.<m>" or "<m>.lora_A" keys (sorted, unique), the
//                             LoRAConfig defaults otherwise (lora.rs:29-43: rank 4, alpha 16,
//                             q/k/v/o_proj), overridden by metadata "rank"/"lora_rank",
//                             "alpha"/"lora_alpha", "target_modules" (top level or under "metadata");
//                             per module the prefix pair "lora_a.<m>"/"lora_b.<m>" first, then the
//                             suffix pair "<m>.lora_A"/"<m>.lora_B", modules without either skipped;
//                             tensors 2-D, their bytes read as float32 whatever the dtype says
//                             (tensor_to_nested_vec, backend.rs:1371-1410; data is copied, so the
//                             reference's 4-byte alignment requirement does not arise).
//
// Host-only C++17, no HIP dependency. Errors are thrown as IngestError, whose kinds are the
// reference's AosError kinds for the same failures (Parse, Validation, Io).
#pragma once

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace adapteros {
namespace ingest {

class IngestError : public std::runtime_error {
 public:
  enum class Kind { Parse, Validation, Io };
  IngestError(Kind kind, const std::string &msg) : std::runtime_error(msg), kind_(kind) {}
  Kind kind() const { return kind_; }

 private:
  Kind kind_;
};

// ---- JSON (the subset safetensors headers and adapter metadata use) ---------------------------

struct Json {
  enum class Type { Null, Bool, Number, String, Array, Object };
  Type type = Type::Null;
  bool b = false;
  double num = 0.0;
  std::string str;  // String; for Number, the literal text
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;  // in file order

  const Json *get(const std::string &key) const {
    if (type != Type::Object) return nullptr;
    for (const auto &kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

namespace detail {

class JsonParser {
 public:
  JsonParser(const char *s, size_t n) : s_(s), n_(n) {}
  Json parse_document() {
    Json v = value(0);
    ws();
    if (i_ != n_) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const char *why) {
    throw IngestError(IngestError::Kind::Parse, std::string("invalid JSON (") + why + ") at offset " +
                                                     std::to_string(i_));
  }
  void ws() {
    while (i_ < n_ && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
  }
  bool lit(const char *w) {
    const size_t m = strlen(w);
    if (n_ - i_ >= m && memcmp(s_ + i_, w, m) == 0) {
      i_ += m;
      return true;
    }
    return false;
  }
  static void put_utf8(std::string &out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  uint32_t hex4() {
    if (n_ - i_ < 4) fail("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = s_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else fail("bad \\u escape");
    }
    return v;
  }
  std::string string() {
    if (i_ >= n_ || s_[i_] != '"') fail("expected string");
    ++i_;
    std::string out;
    while (true) {
      if (i_ >= n_) fail("unterminated string");
      const char c = s_[i_++];
      if (c == '"') break;
      if ((unsigned char)c < 0x20) fail("control character in string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= n_) fail("unterminated escape");
      const char e = s_[i_++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {
            if (!(n_ - i_ >= 2 && s_[i_] == '\\' && s_[i_ + 1] == 'u')) fail("lone surrogate");
            i_ += 2;
            const uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
    return out;
  }
  Json number() {
    const size_t b = i_;
    if (i_ < n_ && s_[i_] == '-') ++i_;
    if (i_ >= n_) fail("bad number");
    if (s_[i_] == '0') {
      ++i_;
    } else if (s_[i_] >= '1' && s_[i_] <= '9') {
      while (i_ < n_ && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
    } else {
      fail("bad number");
    }
    if (i_ < n_ && s_[i_] == '.') {
      ++i_;
      if (i_ >= n_ || !(s_[i_] >= '0' && s_[i_] <= '9')) fail("bad fraction");
      while (i_ < n_ && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
    }
    if (i_ < n_ && (s_[i_] == 'e' || s_[i_] == 'E')) {
      ++i_;
      if (i_ < n_ && (s_[i_] == '+' || s_[i_] == '-')) ++i_;
      if (i_ >= n_ || !(s_[i_] >= '0' && s_[i_] <= '9')) fail("bad exponent");
      while (i_ < n_ && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
    }
    Json v;
    v.type = Json::Type::Number;
    v.str.assign(s_ + b, i_ - b);
    v.num = strtod(v.str.c_str(), nullptr);
    return v;
  }
  Json value(int depth) {
    if (depth > 64) fail("nesting too deep");
    ws();
    if (i_ >= n_) fail("unexpected end");
    Json v;
    const char c = s_[i_];
    if (c == '{') {
      ++i_;
      v.type = Json::Type::Object;
      ws();
      if (i_ < n_ && s_[i_] == '}') {
        ++i_;
        return v;
      }
      while (true) {
        ws();
        std::string k = string();
        ws();
        if (i_ >= n_ || s_[i_] != ':') fail("expected ':'");
        ++i_;
        v.obj.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (i_ < n_ && s_[i_] == ',') {
          ++i_;
          continue;
        }
        if (i_ < n_ && s_[i_] == '}') {
          ++i_;
          break;
        }
        fail("expected ',' or '}'");
      }
    } else if (c == '[') {
      ++i_;
      v.type = Json::Type::Array;
      ws();
      if (i_ < n_ && s_[i_] == ']') {
        ++i_;
        return v;
      }
      while (true) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (i_ < n_ && s_[i_] == ',') {
          ++i_;
          continue;
        }
        if (i_ < n_ && s_[i_] == ']') {
          ++i_;
          break;
        }
        fail("expected ',' or ']'");
      }
    } else if (c == '"') {
      v.type = Json::Type::String;
      v.str = string();
    } else if (lit("true")) {
      v.type = Json::Type::Bool;
      v.b = true;
    } else if (lit("false")) {
      v.type = Json::Type::Bool;
    } else if (lit("null")) {
      v.type = Json::Type::Null;
    } else {
      v = number();
    }
    return v;
  }

  const char *s_;
  size_t n_;
  size_t i_ = 0;
};

// float32 -> float16 bit pattern, round to nearest even (IEEE 754 binary16), NaN kept quiet.
inline uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // |f| >= 65520 rounds to infinity
  const uint32_t e = ax >> 23;
  uint32_t m, shift, h;
  if (e >= 113) {  // normal half: |f| >= 2^-14
    m = ax & 0x7FFFFFu;
    h = ((e - 112) << 10) | (m >> 13);
    m &= 0x1FFFu;
    shift = 13;
  } else {  // subnormal half (or zero): units of 2^-24
    if (e < 101) return (uint16_t)sign;  // |f| < 2^-25 (or a float32 denormal): rounds to zero
    const uint32_t mm = (ax & 0x7FFFFFu) | 0x800000u;
    shift = 126 - e;  // 14..25
    h = mm >> shift;
    m = mm & ((1u << shift) - 1u);
  }
  const uint32_t half = 1u << (shift - 1);
  if (m > half || (m == half && (h & 1u))) ++h;  // a carry into the exponent is the right result
  return (uint16_t)(sign | h);
}

}  // namespace detail

inline Json parse_json(const std::string &text) { return detail::JsonParser(text.data(), text.size()).parse_document(); }

// ---- safetensors ---------------------------------------------------------------------------------

struct TensorView {
  std::string dtype;            // "F32", "F16", "BF16", "U32", ...
  std::vector<size_t> shape;
  const uint8_t *data = nullptr;
  size_t nbytes = 0;
  size_t numel() const {  // the parser has checked that the product does not overflow
    size_t n = 1;
    for (size_t d : shape) n *= d;
    return n;
  }
};

// Element count of a shape, or false when it overflows size_t.
inline bool checked_numel(const std::vector<size_t> &shape, size_t &n) {
  n = 1;
  for (size_t d : shape)
    if (__builtin_mul_overflow(n, d, &n)) return false;
  return true;
}

inline size_t dtype_size(const std::string &dt) {
  if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
  if (dt == "F32" || dt == "I32" || dt == "U32") return 4;
  if (dt == "F16" || dt == "BF16" || dt == "I16" || dt == "U16") return 2;
  if (dt == "I8" || dt == "U8" || dt == "BOOL" || dt == "F8_E4M3" || dt == "F8_E5M2") return 1;
  return 0;
}

// A parsed safetensors buffer; views point into the caller's bytes, which must outlive it.
class SafeTensors {
 public:
  static SafeTensors parse(const uint8_t *bytes, size_t len) {
    auto bad = [](const std::string &why) { return IngestError(IngestError::Kind::Parse, "safetensors: " + why); };
    if (len < 8) throw bad("shorter than the 8-byte header length");
    uint64_t n = 0;
    for (int k = 7; k >= 0; --k) n = (n << 8) | bytes[k];
    if (n > 100000000ull) throw bad("header length " + std::to_string(n) + " exceeds the 100 MB limit");
    if (n > len - 8) throw bad("header length " + std::to_string(n) + " exceeds the buffer");
    if (n == 0 || bytes[8] != '{') throw bad("header does not start with '{'");
    const Json h = detail::JsonParser((const char *)bytes + 8, (size_t)n).parse_document();
    if (h.type != Json::Type::Object) throw bad("header is not a JSON object");
    SafeTensors st;
    const uint8_t *buf = bytes + 8 + n;
    const size_t buflen = len - 8 - (size_t)n;
    std::vector<std::pair<size_t, size_t>> spans;  // [begin, end) per tensor
    for (const auto &kv : h.obj) {
      if (kv.first == "__metadata__") {
        if (kv.second.type != Json::Type::Object) throw bad("__metadata__ is not an object");
        for (const auto &m : kv.second.obj) {
          if (m.second.type != Json::Type::String) throw bad("__metadata__ values must be strings");
          st.metadata_[m.first] = m.second.str;
        }
        continue;
      }
      const Json &t = kv.second;
      const Json *dt = t.get("dtype"), *sh = t.get("shape"), *off = t.get("data_offsets");
      if (!dt || dt->type != Json::Type::String || !sh || sh->type != Json::Type::Array || !off ||
          off->type != Json::Type::Array || off->arr.size() != 2)
        throw bad("tensor '" + kv.first + "' lacks dtype/shape/data_offsets");
      TensorView v;
      v.dtype = dt->str;
      for (const Json &d : sh->arr) {
        // dimensions are used as int extents downstream: larger ones are rejected here
        if (d.type != Json::Type::Number || d.num < 0 || d.num != std::floor(d.num) || d.num > 2147483647.0)
          throw bad("tensor '" + kv.first + "' has a bad shape");
        v.shape.push_back((size_t)d.num);
      }
      const Json &b = off->arr[0], &e = off->arr[1];
      if (b.type != Json::Type::Number || e.type != Json::Type::Number || b.num < 0 || e.num < b.num ||
          b.num != std::floor(b.num) || e.num != std::floor(e.num) || e.num > (double)buflen)
        throw bad("tensor '" + kv.first + "' has bad data_offsets");
      const size_t es = dtype_size(v.dtype);
      if (es == 0) throw bad("tensor '" + kv.first + "' has unsupported dtype " + v.dtype);
      v.data = buf + (size_t)b.num;
      v.nbytes = (size_t)e.num - (size_t)b.num;
      size_t count = 0, want = 0;
      if (!checked_numel(v.shape, count) || __builtin_mul_overflow(count, es, &want))
        throw bad("tensor '" + kv.first + "' has a shape whose size overflows");
      if (v.nbytes != want) throw bad("tensor '" + kv.first + "' size does not match its shape");
      if (st.tensors_.count(kv.first)) throw bad("duplicate tensor '" + kv.first + "'");
      st.tensors_[kv.first] = v;
      st.order_.push_back(kv.first);
      spans.emplace_back((size_t)b.num, (size_t)e.num);
    }
    // the data buffer is indexed entirely, without holes or overlaps
    std::sort(spans.begin(), spans.end());
    size_t at = 0;
    for (const auto &sp : spans) {
      if (sp.first != at) throw bad("tensor data is not contiguous");
      at = sp.second;
    }
    if (at != buflen) throw bad("tensor data does not cover the buffer");
    return st;
  }

  const TensorView *tensor(const std::string &name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
  }
  const std::vector<std::string> &names() const { return order_; }
  const std::map<std::string, std::string> &metadata() const { return metadata_; }

 private:
  std::map<std::string, TensorView> tensors_;
  std::vector<std::string> order_;
  std::map<std::string, std::string> metadata_;
};

// A file mapped read-only (safetensors model shards run to gigabytes).
class MappedFile {
 public:
  explicit MappedFile(const std::string &path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw IngestError(IngestError::Kind::Io, "cannot open " + path + ": " + strerror(errno));
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
      ::close(fd);
      throw IngestError(IngestError::Kind::Io, "cannot stat " + path);
    }
    size_ = (size_t)sb.st_size;
    if (size_ > 0) {
      void *p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
      if (p == MAP_FAILED) {
        ::close(fd);
        throw IngestError(IngestError::Kind::Io, "cannot map " + path + ": " + strerror(errno));
      }
      data_ = (const uint8_t *)p;
    }
    ::close(fd);
  }
  ~MappedFile() {
    if (data_) munmap((void *)data_, size_);
  }
  MappedFile(const MappedFile &) = delete;
  MappedFile &operator=(const MappedFile &) = delete;
  const uint8_t *data() const { return data_; }
  size_t size() const { return size_; }

 private:
  const uint8_t *data_ = nullptr;
  size_t size_ = 0;
};

// ---- LoRA adapter (backend.rs:1017-1210) ---------------------------------------------------------

struct AdapterModule {
  std::string name;
  int rank = 0;                   // rows of A
  int in_features = 0, out_features = 0;
  std::vector<float> A, B;        // A [rank, in], B [out, rank], row-major
  std::string problem;            // non-empty: shapes that no projection can use
};

struct AdapterSpec {
  uint64_t rank = 4;              // config rank (scale = alpha / rank)
  float alpha = 16.0f;
  std::vector<std::string> target_modules;
  std::vector<AdapterModule> modules;  // target modules found in the file, in target order
  float scale() const { return alpha / (float)rank; }  // backend.rs:462
};

namespace detail {

inline const Json *metadata_value_any(const Json &md, const std::vector<std::string> &keys) {
  for (const auto &k : keys) {
    if (const Json *v = md.get(k)) return v;
    if (const Json *inner = md.get("metadata"))
      if (const Json *v = inner->get(k)) return v;
  }
  return nullptr;
}

inline std::string trim(const std::string &s) {
  size_t b = 0, e = s.size();
  while (b < e && (s[b] == ' ' || s[b] == '\t' || s[b] == '\n' || s[b] == '\r')) ++b;
  while (e > b && (s[e - 1] == ' ' || s[e - 1] == '\t' || s[e - 1] == '\n' || s[e - 1] == '\r')) --e;
  return s.substr(b, e - b);
}

// parse_rank (backend.rs:1181-1190): a positive integer, as a JSON integer (serde's as_u64) or a
// string that Rust's usize parser accepts (digits with an optional leading '+')
inline bool parse_rank(const Json &v, uint64_t &out) {
  std::string t;
  if (v.type == Json::Type::Number) {
    if (v.str.find_first_of(".eE-") != std::string::npos) return false;
    t = v.str;
  } else if (v.type == Json::Type::String) {
    t = trim(v.str);
    if (!t.empty() && t[0] == '+') t = t.substr(1);
  } else {
    return false;
  }
  if (t.empty() || t.find_first_not_of("0123456789") != std::string::npos) return false;
  errno = 0;
  const unsigned long long r = strtoull(t.c_str(), nullptr, 10);
  if (errno == ERANGE || r == 0) return false;
  out = (uint64_t)r;
  return true;
}

// parse_alpha (backend.rs:1192-1205): finite and positive, as a number or a string (f32)
inline bool parse_alpha(const Json &v, float &out) {
  float a;
  if (v.type == Json::Type::Number) {
    a = (float)v.num;
  } else if (v.type == Json::Type::String) {
    const std::string t = trim(v.str);
    if (t.empty()) return false;
    if (t.find_first_of("xX") != std::string::npos) return false;  // Rust's f32 parser has no hex form
    char *end = nullptr;
    a = strtof(t.c_str(), &end);
    if (end != t.c_str() + t.size()) return false;
  } else {
    return false;
  }
  if (!std::isfinite(a) || !(a > 0.0f)) return false;
  out = a;
  return true;
}

// metadata_target_modules_override (backend.rs:1120-1164): an array of strings, a JSON-array
// string or a comma-separated string; trimmed, empties dropped, first occurrences kept
inline bool parse_targets(const Json &v, std::vector<std::string> &out) {
  std::vector<std::string> mods;
  if (v.type == Json::Type::Array) {
    for (const Json &it : v.arr)
      if (it.type == Json::Type::String) {
        const std::string m = trim(it.str);
        if (!m.empty()) mods.push_back(m);
      }
  } else if (v.type == Json::Type::String) {
    const std::string t = trim(v.str);
    if (!t.empty() && t[0] == '[') {
      Json arr;
      try {
        arr = parse_json(t);
      } catch (const IngestError &) {
        return false;
      }
      if (arr.type != Json::Type::Array) return false;
      for (const Json &it : arr.arr) {
        if (it.type != Json::Type::String) return false;
        const std::string m = trim(it.str);
        if (!m.empty()) mods.push_back(m);
      }
    } else {
      size_t b = 0;
      while (b <= t.size()) {
        size_t e = t.find(',', b);
        if (e == std::string::npos) e = t.size();
        const std::string m = trim(t.substr(b, e - b));
        if (!m.empty()) mods.push_back(m);
        b = e + 1;
      }
    }
  } else {
    return false;
  }
  if (mods.empty()) return false;
  out.clear();
  for (const auto &m : mods) {
    bool seen = false;
    for (const auto &o : out) seen = seen || o == m;
    if (!seen) out.push_back(m);
  }
  return true;
}

// tensor_to_nested_vec (backend.rs:1371-1410): a 2-D tensor whose bytes are float32
inline std::vector<float> f32_matrix(const TensorView &t, size_t &rows, size_t &cols) {
  if (t.shape.size() != 2) {
    std::string s = "[";
    for (size_t k = 0; k < t.shape.size(); ++k) s += (k ? ", " : "") + std::to_string(t.shape[k]);
    throw IngestError(IngestError::Kind::Parse, "Expected 2D tensor, got shape " + s + "]");
  }
  rows = t.shape[0];
  cols = t.shape[1];
  if (t.nbytes % 4 != 0)
    throw IngestError(IngestError::Kind::Parse, "Tensor data length " + std::to_string(t.nbytes) +
                                                    " is not a multiple of f32 size (4)");
  if (t.nbytes / 4 != rows * cols)
    throw IngestError(IngestError::Kind::Parse, "Data size mismatch: expected " + std::to_string(rows * cols) +
                                                    " elements, got " + std::to_string(t.nbytes / 4));
  std::vector<float> v(rows * cols);
  memcpy(v.data(), t.data, t.nbytes);
  return v;
}

}  // namespace detail

inline void read_modules(const SafeTensors &st, AdapterSpec &spec);

// The adapter in a safetensors buffer; metadata (may be null) as the reference's JSON value.
inline AdapterSpec read_adapter(const SafeTensors &st, const Json *metadata) {
  AdapterSpec spec;
  std::vector<std::string> found;
  for (const auto &name : st.names()) {
    std::string m;
    if (name.rfind("lora_a.", 0) == 0) m = name.substr(7);
    else if (name.size() > 7 && name.compare(name.size() - 7, 7, ".lora_A") == 0) m = name.substr(0, name.size() - 7);
    else continue;
    found.push_back(m);
  }
  std::sort(found.begin(), found.end());
  found.erase(std::unique(found.begin(), found.end()), found.end());
  spec.target_modules = found.empty() ? std::vector<std::string>{"q_proj", "k_proj", "v_proj", "o_proj"} : found;
  if (metadata) {
    uint64_t r;
    float a;
    std::vector<std::string> t;
    if (const Json *v = detail::metadata_value_any(*metadata, {"rank", "lora_rank"}))
      if (detail::parse_rank(*v, r)) spec.rank = r;
    if (const Json *v = detail::metadata_value_any(*metadata, {"alpha", "lora_alpha"}))
      if (detail::parse_alpha(*v, a)) spec.alpha = a;
    if (const Json *v = detail::metadata_value_any(*metadata, {"target_modules"}))
      if (detail::parse_targets(*v, t)) spec.target_modules = t;
  }
  read_modules(st, spec);
  return spec;
}

// LoRAAdapter::load (crates/adapteros-lora-mlx-ffi/src/lora.rs:154-216): the file at path read with
// a given config (no discovery, no metadata). An unreadable file is an Io error; every other
// failure, the safetensors parse included, is a Validation error there.
inline AdapterSpec load_lora(const std::string &path, AdapterSpec config) {
  std::unique_ptr<MappedFile> f;
  try {
    f.reset(new MappedFile(path));
  } catch (const IngestError &e) {
    throw IngestError(IngestError::Kind::Io, std::string("Failed to read LoRA file ") + path + ": " + e.what());
  }
  config.modules.clear();
  try {
    const SafeTensors st = SafeTensors::parse(f->data(), f->size());
    read_modules(st, config);
  } catch (const IngestError &e) {
    throw IngestError(IngestError::Kind::Validation, e.what());
  }
  return config;
}

// The modules of spec.target_modules that st holds, appended to spec.modules: the prefix pair
// "lora_a.<m>"/"lora_b.<m>" if both are present, else the suffix pair, else the module is skipped.
inline void read_modules(const SafeTensors &st, AdapterSpec &spec) {
  for (const auto &m : spec.target_modules) {
    const TensorView *ta = st.tensor("lora_a." + m), *tb = st.tensor("lora_b." + m);
    if (!(ta && tb)) {
      ta = st.tensor(m + ".lora_A");
      tb = st.tensor(m + ".lora_B");
      if (!(ta && tb)) continue;
    }
    AdapterModule mod;
    mod.name = m;
    size_t ar, ac, br, bc;
    mod.A = detail::f32_matrix(*ta, ar, ac);
    mod.B = detail::f32_matrix(*tb, br, bc);
    if (bc != ar)
      mod.problem = "A has " + std::to_string(ar) + " rows but B has " + std::to_string(bc) + " columns";
    mod.rank = (int)ar;
    mod.in_features = (int)ac;
    mod.out_features = (int)br;
    spec.modules.push_back(std::move(mod));
  }
}

// ---- 4-bit base projection (mlx_cpp_wrapper_real.cpp:925-956) -------------------------------------

struct BaseProjection {
  int out_features = 0, in_features = 0;
  std::vector<uint32_t> packed;       // [out, in / 8]
  std::vector<uint16_t> scales_f16;   // [out, in / 64]
  std::vector<uint16_t> biases_f16;   // [out, in / 64]
};

namespace detail {
inline std::vector<uint16_t> to_f16(const TensorView &t, const std::string &what) {
  std::vector<uint16_t> out(t.numel());
  if (t.dtype == "F16") {
    memcpy(out.data(), t.data, t.nbytes);
  } else if (t.dtype == "BF16") {
    for (size_t k = 0; k < out.size(); ++k) {
      uint16_t b;
      memcpy(&b, t.data + 2 * k, 2);
      const uint32_t u = (uint32_t)b << 16;
      float f;
      memcpy(&f, &u, 4);
      out[k] = f32_to_f16_bits(f);
    }
  } else if (t.dtype == "F32") {
    for (size_t k = 0; k < out.size(); ++k) {
      float f;
      memcpy(&f, t.data + 4 * k, 4);
      out[k] = f32_to_f16_bits(f);
    }
  } else {
    throw IngestError(IngestError::Kind::Validation, what + " must be F16, BF16 or F32, not " + t.dtype);
  }
  return out;
}
}  // namespace detail

// "<key>.weight" (U32 [out, in/8]), "<key>.scales", "<key>.biases" (zero when absent). Returns
// false when "<key>.weight" is absent; throws when it is present but not a 4-bit group-64 layout.
inline bool read_base(const SafeTensors &st, const std::string &key, BaseProjection &bp) {
  const TensorView *w = st.tensor(key + ".weight");
  if (!w) return false;
  const TensorView *s = st.tensor(key + ".scales"), *b = st.tensor(key + ".biases");
  auto bad = [&](const std::string &why) { return IngestError(IngestError::Kind::Validation, key + ": " + why); };
  if (!s) throw bad("not quantized (no .scales): only 4-bit group-64 projections are supported");
  if (w->dtype != "U32" || w->shape.size() != 2) throw bad(".weight must be a 2-D U32 array of packed nibbles");
  const size_t out = w->shape[0], in = w->shape[1] * 8;
  if (s->shape.size() != 2 || s->shape[0] != out || s->shape[1] * 64 != in)
    throw bad(".scales shape does not match 4-bit group-64 packing of .weight");
  if (b && (b->shape.size() != 2 || b->shape[0] != out || b->shape[1] * 64 != in))
    throw bad(".biases shape does not match .scales");
  bp.out_features = (int)out;
  bp.in_features = (int)in;
  bp.packed.resize(out * in / 8);
  memcpy(bp.packed.data(), w->data, w->nbytes);
  bp.scales_f16 = detail::to_f16(*s, key + ".scales");
  bp.biases_f16 = b ? detail::to_f16(*b, key + ".biases") : std::vector<uint16_t>(bp.scales_f16.size(), 0);
  return true;
}

}  // namespace ingest
}  // namespace adapteros
