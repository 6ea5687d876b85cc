// Shared helpers for the Depthformer HIP backend (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

namespace mrt {

// Storage dtypes of the model (weights, KV caches, activations).
enum class DType : int { F32 = 0, BF16 = 1 };

inline const char* dtype_name(DType d) { return d == DType::F32 ? "fp32" : "bf16"; }
inline size_t dtype_size(DType d) { return d == DType::F32 ? 4 : 2; }

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define MRT_HIP_CHECK(expr)                                                       \
  do {                                                                            \
    hipError_t _e = (expr);                                                       \
    if (_e != hipSuccess)                                                         \
      throw ::mrt::Error(3, std::string("HIP error at " __FILE__ ":") +           \
                                std::to_string(__LINE__) + " " #expr ": " +       \
                                hipGetErrorString(_e));                           \
  } while (0)

#define MRT_REQUIRE(cond, msg)                                                    \
  do {                                                                            \
    if (!(cond)) throw ::mrt::Error(1, std::string(msg));                         \
  } while (0)

// bf16 is stored as its raw 16 bits; conversions are round-to-nearest-even.
using bf16 = uint16_t;

__host__ __device__ inline float bf2f(bf16 v) {
#ifdef __HIP_DEVICE_COMPILE__
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
#else
  uint32_t u = static_cast<uint32_t>(v) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
#endif
}

__host__ __device__ inline bf16 f2bf(float f) {
#ifdef __HIP_DEVICE_COMPILE__
  // v_cvt_pk_bf16_f32: round-to-nearest-even in hardware.
  return __builtin_bit_cast(bf16, static_cast<__bf16>(f));
#else
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16>(0x7fc0);  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16>(u >> 16);
#endif
}

// Per-storage-type traits: load as float, store from float, and round a float
// to the precision the storage type holds (identity for fp32).
template <typename T>
struct St;

template <>
struct St<float> {
  static constexpr int kVec = 4;  // elements per 16-byte load
  __device__ __forceinline__ static float ld(float v) { return v; }
  __device__ __forceinline__ static float st(float f) { return f; }
  __device__ __forceinline__ static float rnd(float f) { return f; }
};

template <>
struct St<bf16> {
  static constexpr int kVec = 8;
  __device__ __forceinline__ static float ld(bf16 v) { return bf2f(v); }
  __device__ __forceinline__ static bf16 st(float f) { return f2bf(f); }
  __device__ __forceinline__ static float rnd(float f) { return bf2f(f2bf(f)); }
};

}  // namespace mrt
