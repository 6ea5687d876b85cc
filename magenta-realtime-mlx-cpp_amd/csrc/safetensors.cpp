#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cstring>

#include "common.hpp"

namespace mrt {

const HostTensor& TensorSource::tensor(const std::string& key) const {
  auto it = map_.find(key);
  if (it == map_.end()) throw Error(4, "weight bundle " + label_ + ": missing key \"" + key + "\"");
  return it->second;
}

std::vector<std::string> TensorSource::keys() const {
  std::vector<std::string> out;
  for (auto& kv : map_) out.push_back(kv.first);
  return out;
}

void TensorList::add(const std::string& name, const float* data, std::vector<int64_t> shape) {
  int64_t n = 1;
  for (int64_t d : shape)
    if (d < 0 || __builtin_mul_overflow(n, d, &n)) throw Error(1, "host tensor " + name + ": bad shape");
  HostTensor t;
  t.shape = std::move(shape);
  t.data = data;
  map_[name] = t;
  label_ = "<host tensors>";
}

namespace {

// A JSON value restricted to what a safetensors header holds.
struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  double num = 0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
};

class JParser {
 public:
  JParser(const char* p, const char* e) : p_(p), e_(e) {}
  JVal parse() {
    JVal v = value();
    ws();
    return v;
  }

 private:
  const char* p_;
  const char* e_;
  [[noreturn]] void fail(const char* what) { throw Error(5, std::string("safetensors header: ") + what); }
  void ws() {
    while (p_ < e_ && std::isspace(static_cast<unsigned char>(*p_))) ++p_;
  }
  char peek() {
    ws();
    if (p_ >= e_) fail("unexpected end");
    return *p_;
  }
  void expect(char c) {
    if (peek() != c) fail("unexpected character");
    ++p_;
  }
  JVal value() {
    char c = peek();
    if (c == '{') return object();
    if (c == '[') return array();
    if (c == '"') {
      JVal v;
      v.kind = JVal::Str;
      v.str = string();
      return v;
    }
    if (c == 't' || c == 'f' || c == 'n') {
      JVal v;
      const char* words[] = {"true", "false", "null"};
      for (const char* w : words) {
        size_t n = std::strlen(w);
        if ((size_t)(e_ - p_) >= n && std::strncmp(p_, w, n) == 0) {
          p_ += n;
          v.kind = (w[0] == 'n') ? JVal::Null : JVal::Bool;
          return v;
        }
      }
      fail("bad literal");
    }
    JVal v;
    v.kind = JVal::Num;
    const char* s = p_;
    while (p_ < e_ && (std::isdigit(static_cast<unsigned char>(*p_)) || *p_ == '-' || *p_ == '+' ||
                       *p_ == '.' || *p_ == 'e' || *p_ == 'E'))
      ++p_;
    if (s == p_) fail("bad number");
    v.num = std::stod(std::string(s, p_));
    return v;
  }
  std::string string() {
    expect('"');
    std::string out;
    while (p_ < e_ && *p_ != '"') {
      if (*p_ == '\\') {
        ++p_;
        if (p_ >= e_) fail("bad escape");
        char c = *p_;
        if (c == 'u') {
          if (e_ - p_ < 5) fail("bad escape");
          unsigned cp = std::stoul(std::string(p_ + 1, p_ + 5), nullptr, 16);
          if (cp < 0x80) out.push_back(static_cast<char>(cp));
          else out.push_back('?');
          p_ += 4;
        } else {
          out.push_back(c == 'n' ? '\n' : c == 't' ? '\t' : c);
        }
        ++p_;
      } else {
        out.push_back(*p_++);
      }
    }
    if (p_ >= e_) fail("unterminated string");
    ++p_;
    return out;
  }
  JVal array() {
    JVal v;
    v.kind = JVal::Arr;
    expect('[');
    if (peek() == ']') {
      ++p_;
      return v;
    }
    for (;;) {
      v.arr.push_back(value());
      char c = peek();
      ++p_;
      if (c == ']') break;
      if (c != ',') fail("expected , or ]");
    }
    return v;
  }
  JVal object() {
    JVal v;
    v.kind = JVal::Obj;
    expect('{');
    if (peek() == '}') {
      ++p_;
      return v;
    }
    for (;;) {
      if (peek() != '"') fail("expected key");
      std::string k = string();
      expect(':');
      v.obj.emplace_back(std::move(k), value());
      char c = peek();
      ++p_;
      if (c == '}') break;
      if (c != ',') fail("expected , or }");
    }
    return v;
  }
};

const JVal* field(const JVal& o, const char* name) {
  for (auto& kv : o.obj)
    if (kv.first == name) return &kv.second;
  return nullptr;
}

}  // namespace

FileMapping::~FileMapping() {
  if (base) ::munmap(base, len);
}

namespace {

// A JSON number that is a non-negative integer no larger than `max`.
bool as_count(const JVal& v, double max, uint64_t* out) {
  if (v.kind != JVal::Num || !(v.num >= 0.0) || v.num > max || v.num != static_cast<double>(static_cast<uint64_t>(v.num)))
    return false;
  *out = static_cast<uint64_t>(v.num);
  return true;
}

constexpr double kMaxDim = 1099511627776.0;  // 2^40 elements along one axis

}  // namespace

SafetensorsFile::SafetensorsFile(const std::string& path) {
  label_ = path;
  int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) throw Error(4, "weight bundle: not a file: " + path);
  struct stat st;
  if (::fstat(fd, &st) != 0 || st.st_size < 8) {
    ::close(fd);
    throw Error(5, "weight bundle: too small: " + path);
  }
  const size_t map_len = static_cast<size_t>(st.st_size);
  void* mapped = ::mmap(nullptr, map_len, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (mapped == MAP_FAILED) throw Error(5, "weight bundle: mmap failed: " + path);
  map_file_.base = mapped;
  map_file_.len = map_len;
  const uint8_t* base = static_cast<const uint8_t*>(mapped);
  uint64_t hlen = 0;
  for (int i = 0; i < 8; ++i) hlen |= static_cast<uint64_t>(base[i]) << (8 * i);
  if (hlen > map_len - 8) throw Error(5, "weight bundle: bad header length: " + path);
  JParser jp(reinterpret_cast<const char*>(base + 8), reinterpret_cast<const char*>(base + 8 + hlen));
  JVal root = jp.parse();
  if (root.kind != JVal::Obj) throw Error(5, "weight bundle: header is not an object");
  const uint8_t* data = base + 8 + hlen;
  const size_t data_len = map_len - 8 - hlen;
  for (auto& kv : root.obj) {
    if (kv.first == "__metadata__") continue;
    const JVal* dt = field(kv.second, "dtype");
    const JVal* sh = field(kv.second, "shape");
    const JVal* off = field(kv.second, "data_offsets");
    if (!dt || !sh || !off || dt->kind != JVal::Str || sh->kind != JVal::Arr || off->kind != JVal::Arr ||
        off->arr.size() != 2)
      throw Error(5, "weight bundle: bad entry " + kv.first);
    size_t esz = 0;
    if (dt->str == "F32") esz = 4;
    else if (dt->str == "BF16" || dt->str == "F16") esz = 2;
    else throw Error(5, "weight bundle: unsupported dtype " + dt->str + " for " + kv.first);
    HostTensor t;
    uint64_t n = 1;
    for (auto& d : sh->arr) {
      uint64_t dim = 0;
      if (!as_count(d, kMaxDim, &dim)) throw Error(5, "weight bundle: bad dimension in shape of " + kv.first);
      if (__builtin_mul_overflow(n, dim, &n)) throw Error(5, "weight bundle: element count overflows for " + kv.first);
      t.shape.push_back(static_cast<int64_t>(dim));
    }
    uint64_t b0 = 0, b1 = 0, bytes = 0;
    if (!as_count(off->arr[0], static_cast<double>(data_len), &b0) ||
        !as_count(off->arr[1], static_cast<double>(data_len), &b1) || b1 < b0)
      throw Error(5, "weight bundle: offsets out of range for " + kv.first);
    if (__builtin_mul_overflow(n, static_cast<uint64_t>(esz), &bytes) || bytes != b1 - b0)
      throw Error(5, "weight bundle: size mismatch " + kv.first);
    const uint8_t* src = data + b0;
    if (esz == 4) {
      if (reinterpret_cast<uintptr_t>(src) % 4 == 0) {
        t.data = reinterpret_cast<const float*>(src);
      } else {
        auto buf = std::make_unique<std::vector<float>>(n);
        std::memcpy(buf->data(), src, n * 4);
        t.data = buf->data();
        widened_.push_back(std::move(buf));
      }
    } else {
      auto buf = std::make_unique<std::vector<float>>(n);
      for (uint64_t i = 0; i < n; ++i) {
        uint16_t h;
        std::memcpy(&h, src + 2 * i, 2);
        (*buf)[i] = dt->str == "BF16" ? bf2f(h) : h2f_host(h);
      }
      t.data = buf->data();
      widened_.push_back(std::move(buf));
    }
    map_[kv.first] = t;
  }
}

}  // namespace mrt
