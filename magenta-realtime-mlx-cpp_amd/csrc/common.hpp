// Shared helpers for the Depthformer HIP backend (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

namespace mrt {

// Storage dtypes of the model (weights, KV caches, activations).
enum class DType : int { F32 = 0, BF16 = 1, F16 = 2 };

inline const char* dtype_name(DType d) { return d == DType::F32 ? "fp32" : d == DType::BF16 ? "bf16" : "fp16"; }
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

// fp16 (IEEE binary16) storage.  Device code converts with v_cvt_f16_f32 /
// v_cvt_f32_f16 (round-to-nearest-even, subnormals kept); host code only moves
// the raw 16 bits and converts with the bit-level routines below.
using f16 = _Float16;

// binary16 bits -> float (exact).
inline float h2f_host(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, u;
  if (e == 0x1f) {
    u = sign | 0x7f800000u | (m << 13);  // inf / NaN (payload kept)
  } else if (e != 0) {
    u = sign | ((e + 112u) << 23) | (m << 13);
  } else if (m == 0) {
    u = sign;
  } else {  // subnormal: m * 2^-24, normalised
    int sh = 0;
    while ((m & 0x400u) == 0) {
      m <<= 1;
      ++sh;
    }
    u = sign | ((113u - sh) << 23) | ((m & 0x3ffu) << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// float -> nearest binary16 bits, ties to even; overflow to inf, NaN kept quiet.
inline uint16_t f2h_host(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  const uint16_t sign = static_cast<uint16_t>((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;
  if (a >= 0x477ff000u) return sign | 0x7c00u;  // >= 65520 rounds to inf
  if (a >= 0x38800000u) {                        // normal half (>= 2^-14)
    const uint32_t r = a + 0xfffu + ((a >> 13) & 1u);
    return sign | static_cast<uint16_t>((r - 0x38000000u) >> 13);
  }
  if (a < 0x33000000u) return sign;  // below half the smallest subnormal (2^-25)
  // subnormal half: the value is mant * 2^(e-150), i.e. (mant >> (126-e)) units of 2^-24
  const uint32_t e = a >> 23, mant = (a & 0x7fffffu) | 0x800000u;
  const uint32_t shift = 126u - e;
  const uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
  const uint32_t r = q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
  return sign | static_cast<uint16_t>(r);
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

// 16-bit types also expose their raw bits, for packing two elements a word.
template <>
struct St<bf16> {
  static constexpr int kVec = 8;
  __device__ __forceinline__ static float ld(bf16 v) { return bf2f(v); }
  __device__ __forceinline__ static bf16 st(float f) { return f2bf(f); }
  __device__ __forceinline__ static float rnd(float f) { return bf2f(f2bf(f)); }
  __device__ __forceinline__ static uint32_t bits(float f) { return f2bf(f); }
  __device__ __forceinline__ static float unbits(uint32_t u) { return bf2f(static_cast<bf16>(u)); }
};

template <>
struct St<f16> {
  static constexpr int kVec = 8;
  __device__ __forceinline__ static float ld(f16 v) { return static_cast<float>(v); }
  __device__ __forceinline__ static f16 st(float f) { return static_cast<f16>(f); }
  __device__ __forceinline__ static float rnd(float f) { return static_cast<float>(static_cast<f16>(f)); }
  __device__ __forceinline__ static uint32_t bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<f16>(f));
  }
  __device__ __forceinline__ static float unbits(uint32_t u) {
    return static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(u)));
  }
};

// Runs the statements that follow with `T` naming the storage type of `dt`.
#define MRT_DTYPE_DISPATCH(dt, ...)                    \
  do {                                                 \
    switch (dt) {                                      \
      case ::mrt::DType::F32: {                        \
        using T = float;                               \
        __VA_ARGS__;                                   \
        break;                                         \
      }                                                \
      case ::mrt::DType::BF16: {                       \
        using T = ::mrt::bf16;                         \
        __VA_ARGS__;                                   \
        break;                                         \
      }                                                \
      case ::mrt::DType::F16: {                        \
        using T = ::mrt::f16;                          \
        __VA_ARGS__;                                   \
        break;                                         \
      }                                                \
    }                                                  \
  } while (0)

}  // namespace mrt
