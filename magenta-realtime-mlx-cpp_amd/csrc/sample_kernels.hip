// On-device CFG + level-masked top-k temperature sampling and token feedback
// for one RVQ level (decode.cpp:71-148, 458-484).
//
// One 64-lane wave per stream; the level's C logits (C <= 1024) live in
// registers, 16 per lane.  The top-k threshold (the k-th largest value,
// counting ties, i.e. min(topk(x, k)) of decode.cpp:119-120) is found by a
// 32-step bitwise radix select over order-preserving float keys; the draw is
// Gumbel-max over the kept entries with Philox-4x32-10 noise.
#include <cmath>

#include "device_utils.hpp"
#include "kernels.hpp"

namespace mrt {
namespace {

constexpr int kMaxPerLane = 16;  // C <= 1024

// argmax with the first index winning ties (mx::argmax semantics).
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(i, o, 64);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
}

// Block b draws for stream b: logits rows (2b, 2b + 1), seed p.seed[b], token
// slots slot + b * tstride; frame < 0 reads the frame index from *frame_ptr.
template <typename T>
__global__ __launch_bounds__(64) void k_sample(const float* __restrict__ logits, SampleParams p,
                                               int frame, const int* __restrict__ frame_ptr, int level, int slot,
                                               int tstride, const int* __restrict__ teacher,
                                               int* __restrict__ tokens, int* __restrict__ drawn,
                                               const T* __restrict__ emb, int D, T* __restrict__ next_in,
                                               T* __restrict__ fsum, T* __restrict__ fmean) {
  using S = St<T>;
  const int lane = threadIdx.x;
  const int stream = blockIdx.x;
  const int C = p.codebook;
  if (frame_ptr != nullptr) {
    frame = *frame_ptr;
    slot += frame * p.rvq_depth;
  }
  slot += stream * tstride;
  const float* l0 = logits + (size_t)(2 * stream) * C;
  const float* l1 = l0 + C;
  const float wc = 1.0f + p.guidance_weight;  // decode.cpp:255-256
  const float wu = p.guidance_weight;

  float v[kMaxPerLane];
#pragma unroll
  for (int t = 0; t < kMaxPerLane; ++t) {
    const int c = lane + 64 * t;
    // (1+w)*cond - w*uncond, each product rounded separately (decode.cpp:83-84).
    v[t] = (c < C) ? __fsub_rn(__fmul_rn(wc, l0[c]), __fmul_rn(wu, l1[c])) : -INFINITY;
  }

  if (p.temperature != 0.0f) {
#pragma unroll
    for (int t = 0; t < kMaxPerLane; ++t)
      if (lane + 64 * t < C) v[t] = __fdiv_rn(v[t], p.temperature);
    if (p.top_k > 0 && p.top_k < C) {
      uint32_t key[kMaxPerLane];
#pragma unroll
      for (int t = 0; t < kMaxPerLane; ++t) key[t] = (lane + 64 * t < C) ? float_key(v[t]) : 0u;
      uint32_t prefix = 0;
      for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = prefix | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int t = 0; t < kMaxPerLane; ++t) cnt += key[t] >= cand ? 1 : 0;
        cnt = wave_sum_i(cnt);
        if (cnt >= p.top_k) prefix = cand;
      }
      const float thr = key_float(prefix);
#pragma unroll
      for (int t = 0; t < kMaxPerLane; ++t)
        if (v[t] < thr) v[t] = -INFINITY;  // decode.cpp:121
    }
    const uint64_t seed = p.seed[stream];
#pragma unroll
    for (int t = 0; t < kMaxPerLane; ++t) {
      const int c = lane + 64 * t;
      if (c < C && v[t] != -INFINITY) v[t] = v[t] + gumbel(seed, frame, level, c);
    }
  }
  float best = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int t = 0; t < kMaxPerLane; ++t) {
    const int c = lane + 64 * t;
    if (c < C && (v[t] > best || bi == 0x7fffffff)) {  // c ascends: first max wins
      best = v[t];
      bi = c;
    }
  }
  wave_argmax(best, bi);

  const int L = p.rvq_depth;
  const int drawn_id = p.codec_offset + level * C + bi;
  const int fed = teacher ? teacher[slot] : drawn_id;
  if (lane == 0) {
    tokens[slot] = fed;
    if (drawn) drawn[slot] = drawn_id;
  }
  // Token feedback (decode.cpp:476-484): both CFG rows take emb(fed); the
  // frame sum accumulates in the model dtype; at the last level the mean is
  // the sum divided by L in the model dtype.
  const T* e = emb + (size_t)fed * D;
  const float Lf = S::rnd((float)L);
  T* ni = next_in + (size_t)(2 * stream) * D;
  T* fs = fsum + (size_t)(2 * stream) * D;
  T* fm = fmean + (size_t)(2 * stream) * D;
  for (int d = lane; d < D; d += 64) {
    const T ev = e[d];
    const float sum = (level == 0) ? S::ld(ev) : S::rnd(S::ld(fs[d]) + S::ld(ev));
    ni[d] = ev;
    ni[D + d] = ev;
    fs[d] = S::st(sum);
    fs[D + d] = S::st(sum);
    if (level == L - 1) {
      const T m = S::st(sum / Lf);
      fm[d] = m;
      fm[D + d] = m;
    }
  }
}

}  // namespace

void sample_level(DType dt, const float* logits, const SampleParams& p, int frame, int level, int slot,
                  const int* teacher, int* tokens, int* drawn, const void* emb, int D,
                  void* next_in, void* fsum, void* frame_mean, hipStream_t s) {
  sample_levels(dt, 1, logits, p, frame, nullptr, level, slot, 0, teacher, tokens, drawn, emb, D, next_in, fsum,
                frame_mean, s);
}

void sample_levels(DType dt, int streams, const float* logits, const SampleParams& p, int frame,
                   const int* frame_ptr, int level, int slot, int tstride, const int* teacher, int* tokens,
                   int* drawn, const void* emb, int D, void* next_in, void* fsum, void* frame_mean, hipStream_t s) {
  MRT_REQUIRE(p.codebook >= 1 && p.codebook <= 64 * kMaxPerLane, "sample: codebook must be <= 1024");
  MRT_REQUIRE(streams >= 1, "sample: no streams");
  if (dt == DType::F32)
    hipLaunchKernelGGL(k_sample<float>, dim3(streams), dim3(64), 0, s, logits, p, frame, frame_ptr, level, slot,
                       tstride, teacher, tokens, drawn, (const float*)emb, D, (float*)next_in, (float*)fsum,
                       (float*)frame_mean);
  else
    hipLaunchKernelGGL(k_sample<bf16>, dim3(streams), dim3(64), 0, s, logits, p, frame, frame_ptr, level, slot,
                       tstride, teacher, tokens, drawn, (const bf16*)emb, D, (bf16*)next_in, (bf16*)fsum,
                       (bf16*)frame_mean);
  MRT_HIP_CHECK(hipGetLastError());
}

}  // namespace mrt
