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

// Memory-maps a bundle file; F32 tensors are used in place, BF16/F16 are
// widened to fp32 copies.
class SafetensorsFile : public TensorSource {
 public:
  explicit SafetensorsFile(const std::string& path);
  ~SafetensorsFile() override;

 private:
  void* map_base_ = nullptr;
  size_t map_len_ = 0;
  std::vector<std::unique_ptr<std::vector<float>>> widened_;
};

// Caller-owned fp32 arrays (no copy).
class TensorList : public TensorSource {
 public:
  void add(const std::string& name, const float* data, std::vector<int64_t> shape);
};

}  // namespace mrt
