// Device-side helpers: wave reductions, the tanh-GELU with per-op rounding,
// and the Philox-4x32-10 counter-based generator used for sampling.
#pragma once

#include "common.hpp"

// Address-space qualifiers: global memory and LDS.
#define MRT_GLOBAL __attribute__((address_space(1)))
#define MRT_LDS __attribute__((address_space(3)))

namespace mrt {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal hint: weights are read once per step)
// through a global-address-space pointer (global_load, not flat_load).
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
  const u32x4_t v =
      __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4_t*)(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Plain 16-byte global load.
__device__ __forceinline__ uint4 ld_g16(const void* p) {
  const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t*)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Plain global load of one element.
template <typename T>
__device__ __forceinline__ T ld_g(const T* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// gelu_approx (nn_ops.h:66-84): 0.5*x*(1+tanh(sqrt(2/pi)*x*(1+0.044715*x^2)))
// with every intermediate materialised in the model dtype, as the compiled
// MLX body does (scalar literals cast to the model dtype first).
template <typename T>
__device__ __forceinline__ float gelu_t(float x) {
  using S = St<T>;
  const float half = S::rnd(0.5f), one = S::rnd(1.0f);
  const float c0 = S::rnd(0.7978845608028654f), c1 = S::rnd(0.044715f);
  const float x2 = S::rnd(x * x);
  float t = S::rnd(c1 * x2);
  t = S::rnd(one + t);
  t = S::rnd(x * t);
  const float inner = S::rnd(c0 * t);
  const float th = S::rnd(tanhf(inner));
  t = S::rnd(one + th);
  t = S::rnd(x * t);
  return S::rnd(half * t);
}

// Philox-4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as
// easy as 1, 2, 3", SC'11).  Returns the first output word.
__device__ __forceinline__ uint32_t philox_x0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                              uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return c0;
}

// Polls of the persistent kernels give up (and flag an error for the host)
// after this many rounds, so no wait can hang the device.
constexpr uint32_t kSpinLimit = 1u << 20;

constexpr uint32_t kSampleStreamTag = 0x4D525444u;

// Gumbel(0,1) noise for candidate ``i`` of draw (frame, level):
// counter (i, level, frame, tag), key = seed; u = ((x >> 9) + 0.5) * 2^-23
// lies strictly inside (0, 1); g = -log(-log(u)).
__device__ __forceinline__ float gumbel(uint64_t seed, int frame, int level, int i) {
  const uint32_t x = philox_x0((uint32_t)i, (uint32_t)level, (uint32_t)frame, kSampleStreamTag,
                               (uint32_t)(seed & 0xffffffffu), (uint32_t)(seed >> 32));
  const float u = ((float)(x >> 9) + 0.5f) * 1.1920928955078125e-07f;
  return -logf(-logf(u));
}

// Order-preserving map of a float to uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t float_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

}  // namespace mrt
