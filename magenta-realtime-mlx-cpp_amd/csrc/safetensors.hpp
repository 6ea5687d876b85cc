// Minimal ``.safetensors`` reader: 8-byte little-endian header length, JSON
// header {name: {dtype, shape, data_offsets}}, raw little-endian buffer.
// Replaces ``mx::load_safetensors`` behind ``WeightBundle`` (weights.cpp:118-133).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace mrt {

struct HostTensor {
  std::vector<int64_t> shape;
  const float* data = nullptr;  // fp32 view (owned by the source)
  int64_t numel() const {
    int64_t n = 1;
    for (auto d : shape) n *= d;
    return n;
  }
};

// Name -> fp32 host tensor.  ``tensor`` throws Error(4, "missing key ...")
// for an absent key, mirroring WeightBundle::tensor (weights.cpp:126-133).
class TensorSource {
 public:
  virtual ~TensorSource() = default;
  const HostTensor& tensor(const std::string& key) const;
  bool contains(const std::string& key) const { return map_.count(key) != 0; }
  std::vector<std::string> keys() const;

 protected:
  std::map<std::string, HostTensor> map_;
  std::string label_;
};

// A read-only file mapping, unmapped by its destructor (so also when the
// reader's constructor throws after mapping).
struct FileMapping {
  void* base = nullptr;
  size_t len = 0;
  FileMapping() = default;
  FileMapping(const FileMapping&) = delete;
  FileMapping& operator=(const FileMapping&) = delete;
  ~FileMapping();
};

// Memory-maps a bundle file; F32 tensors are used in place, BF16/F16 are
// widened to fp32 copies.  Every entry is validated before use: dtype known,
// each dimension an integer in [0, 2^40], the element count and its byte size
// free of overflow, and the byte size equal to the entry's data_offsets span,
// which must lie inside the file.
class SafetensorsFile : public TensorSource {
 public:
  explicit SafetensorsFile(const std::string& path);

 private:
  FileMapping map_file_;
  std::vector<std::unique_ptr<std::vector<float>>> widened_;
};

// Caller-owned fp32 arrays (no copy).
class TensorList : public TensorSource {
 public:
  void add(const std::string& name, const float* data, std::vector<int64_t> shape);
};

}  // namespace mrt
