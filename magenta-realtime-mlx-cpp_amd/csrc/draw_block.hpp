// Block-wide exact draw of one level slice (CFG, temperature, top-k, Gumbel-max)
// over 256 threads, shared by the frame kernel (persist_kernels.hip) and the
// per-level sampling kernel (sample_kernels.hip), with the wave reductions it
// uses.
#pragma once

#include <cstdint>

#include "device_utils.hpp"
#include "kernels.hpp"

namespace mrt {

constexpr int kDrawThreads = 256;
constexpr int kDrawPer = 1024 / kDrawThreads;  // candidates (and d_model elements) per thread
constexpr int kDrawChainSteps = 3;             // restricted-argmax steps of a draw before its radix select
constexpr int kDrawHistWords = 3 * 4 * 256;    // 3 rotating buffers x 4 per-wave 256-bin histograms

// ---- DPP wave reductions (all 64 lanes active; result is wave-uniform) -----------

__device__ __forceinline__ float dpp_max(float v) {
  const int ninf = __float_as_int(-INFINITY);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0xB1, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x4E, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x114, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x118, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x142, 0xa, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x143, 0xc, 0xf, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Inclusive prefix sum over the 64 lanes (lane 0 first): Hillis-Steele
// within each 16-lane row, then row 0 -> 1, 2 -> 3 and rows 0-1 -> 2-3.
__device__ __forceinline__ unsigned dpp_prefix_sum(unsigned v) {
  v += __builtin_amdgcn_update_dpp(0u, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0u, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0u, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0u, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0u, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

__device__ __forceinline__ int dpp_min_i(int v) {
  const int big = 0x7fffffff;
  v = min(v, __builtin_amdgcn_update_dpp(big, v, 0xB1, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(big, v, 0x4E, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(big, v, 0x114, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(big, v, 0x118, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(big, v, 0x142, 0xa, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(big, v, 0x143, 0xc, 0xf, false));
  return __builtin_amdgcn_readlane(v, 63);
}

// Loads of a draw that do not depend on the logits (issued before the gather).
struct DrawPrefetch {
  float gn[kDrawPer];  // Gumbel noise of this thread's candidates
  int teacher_id;
};

__device__ __forceinline__ void draw_prefetch(int C, const float* noise, const int* teacher, int slot,
                                              DrawPrefetch& d) {
#pragma unroll
  for (int t = 0; t < kDrawPer; ++t) {
    const int c = threadIdx.x + kDrawThreads * t;
    d.gn[t] = c < C ? ld_g(noise + c) : 0.f;
  }
  d.teacher_id = teacher ? ld_g(teacher + slot) : 0;
}

// Zeroes the histogram buffers of the first two radix passes of the next draw
// (the caller orders this before the draw with a barrier).
__device__ __forceinline__ void draw_clear(unsigned* hist) {
  for (int i = threadIdx.x; i < 2 * 4 * 256; i += kDrawThreads) hist[i] = 0u;
}

// Block argmax of w (ties to the smallest candidate index), candidate c =
// tid + 256 t.  One barrier; wres[0..7] is written.
__device__ __forceinline__ int block_argmax(const float (&w)[kDrawPer], int C, int* wres) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  float best = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int t = 0; t < kDrawPer; ++t) {
    const int c = tid + kDrawThreads * t;
    if (c < C && (w[t] > best || bi == 0x7fffffff)) {
      best = w[t];
      bi = c;
    }
  }
  const float wmx = dpp_max(best);
  const int warg = dpp_min_i(best == wmx ? bi : 0x7fffffff);
  if (lane == 0) {
    wres[wid] = __float_as_int(wmx);
    wres[4 + wid] = warg;
  }
  __syncthreads();
  float mx = __int_as_float(wres[0]);
  int arg = wres[4];
#pragma unroll
  for (int q = 1; q < 4; ++q) {
    const float m = __int_as_float(wres[q]);
    const int ix = wres[4 + q];
    if (m > mx || (m == mx && ix < arg)) {
      mx = m;
      arg = ix;
    }
  }
  return arg;
}

// Threshold key of the top-k set: the k-th largest key of the candidates
// (ties counted), or a smaller key with no candidate key between the two (so
// {key >= threshold} is the same set), by a most-significant-
// byte-first radix select: each pass counts the candidates into per-wave
// 256-bin LDS histograms, and after one barrier every wave scans the four
// histograms itself, so the selected digit needs no broadcast.  Pass p uses
// buffer p % 3; buffer (p + 2) % 3, last read before this pass's barrier, is
// cleared for pass p + 2.  Buffers 0 and 1 must be zero on entry.
template <class TP>
__device__ __forceinline__ uint32_t radix_select(const uint32_t (&key)[kDrawPer], int C, int k, unsigned* hist,
                                                 TP&& tpoint) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  uint32_t prefix = 0, mask = 0;
  int need = k;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    unsigned* hb = hist + (pass % 3) * 1024;
#pragma unroll
    for (int t = 0; t < kDrawPer; ++t)
      if (tid + kDrawThreads * t < C && (key[t] & mask) == prefix)
        atomicAdd(&hb[wid * 256 + ((key[t] >> shift) & 255u)], 1u);
    __syncthreads();
    if (pass < 2) {  // buffer of pass + 2 (pass 2: buffer 2, pass 3: buffer 0)
      unsigned* hc = hist + ((pass + 2) % 3) * 1024;
      for (int i = tid; i < 1024; i += kDrawThreads) hc[i] = 0u;
    }
    // lane l holds the bins of group g = 63 - l (bins 4g..4g+3, top group in
    // lane 0), summed over the waves; a prefix sum over lanes then counts the
    // keys in this group and every group above it.
    const int g = 63 - lane;
    unsigned cs[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 h4 = *reinterpret_cast<const uint4*>(hb + q * 256 + 4 * g);
      cs[0] += h4.x;
      cs[1] += h4.y;
      cs[2] += h4.z;
      cs[3] += h4.w;
    }
    const unsigned own = cs[0] + cs[1] + cs[2] + cs[3];
    unsigned above = dpp_prefix_sum(own) - own;  // keys in the groups above
    int bin = -1, before = 0, count = 0;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
      if (bin < 0 && above < (unsigned)need && above + cs[i] >= (unsigned)need) {
        bin = 4 * g + i;
        before = (int)above;
        count = (int)cs[i];
      }
      above += cs[i];
    }
    // exactly one lane finds the bin (the counts sum to >= need)
    const uint64_t hit = __ballot(bin >= 0);
    const int src = hit ? (int)__builtin_ctzll(hit) : 0;
    prefix |= (uint32_t)__builtin_amdgcn_readlane(bin, src) << shift;
    mask |= 255u << shift;
    need -= __builtin_amdgcn_readlane(before, src);
    tpoint(5 + pass);
    // When the selected bin holds exactly the remaining rank, every key in it
    // belongs to the set, so {key >= prefix} (lower digits zero) is the set
    // {key >= k-th largest key}: the remaining passes are skipped.  The
    // threshold this prefix gives must be finite, and the +0 key is left to
    // the full select so that -0 compares equal to it exactly as there.  The
    // decision is the same in every wave (same histograms, lane-uniform
    // values).
    if (pass < 3 && __builtin_amdgcn_readlane(count, src) == need && prefix != 0x80000000u &&
        __builtin_isfinite(key_float(prefix)))
      return prefix;
  }
  return prefix;
}

// Block-wide CFG + temperature/top-k Gumbel-max draw (decode.cpp:71-148,
// 465-474) for one level: `lg` holds the two logit rows of the level slice in
// LDS.  The reference masks every logit below the k-th largest (ties kept) and
// takes the argmax of logit + Gumbel noise, ties to the smallest index.  Fast
// path: A = argmax of v + g over all candidates is that answer whenever A is
// in the top-k set, i.e. fewer than k values are strictly greater than v_A
// (every candidate of the set is a candidate of the full argmax, and A is the
// smallest index attaining its maximum).  Otherwise up to kDrawChainSteps
// restricted argmaxes (below), and only then the k-th largest value by radix
// select and the masked argmax.  Returns the winning candidate index (the same
// in every thread).  kDrawThreads threads; `hist` (kDrawHistWords) must have
// its buffers 0 and 1 zeroed, and has them zeroed again on return; `wres`
// holds 12 ints; tpoint(i) marks the draw's phases (0: guided logits, 1:
// argmax, 2: count, 3: after a radix select, 5 + pass: each radix pass).
template <class TP>
__device__ __forceinline__ int block_draw(const SampleParams& p, const DrawPrefetch& pf, const float* lg,
                                          unsigned* hist, int* wres, TP&& tpoint) {
  constexpr int kPer = kDrawPer;
  const int tid = threadIdx.x, wid = tid >> 6;
  const int C = p.codebook;
  const float wc = 1.0f + p.guidance_weight, wu = p.guidance_weight;
  // (1+w)*cond - w*uncond with both products rounded (decode.cpp:83-84): no
  // fused multiply-add.
  auto guided = [&](int c) {
#pragma clang fp contract(off)
    return wc * lg[c] - wu * lg[C + c];
  };
  float v[kPer];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int c = tid + kDrawThreads * t;
    v[t] = (c < C) ? guided(c) : -INFINITY;
  }
  tpoint(0);
  int arg;
  if (p.temperature == 0.0f) {
    arg = block_argmax(v, C, wres);
  } else {
#pragma unroll
    for (int t = 0; t < kPer; ++t)
      if (tid + kDrawThreads * t < C) v[t] = __fdiv_rn(v[t], p.temperature);
    float w[kPer];
#pragma unroll
    for (int t = 0; t < kPer; ++t) w[t] = v[t] != -INFINITY ? v[t] + pf.gn[t] : -INFINITY;
    arg = block_argmax(w, C, wres);
    tpoint(1);
    if (p.top_k > 0 && p.top_k < C) {
      const float va = __fdiv_rn(guided(arg), p.temperature);
      int n = 0;
#pragma unroll
      for (int t = 0; t < kPer; ++t) n += __popcll(__ballot(tid + kDrawThreads * t < C && v[t] > va));
      if ((tid & 63) == 0) wres[8 + wid] = n;
      __syncthreads();
      int greater = wres[8] + wres[9] + wres[10] + wres[11];
      tpoint(2);
      // Chain steps: while the winner B is outside the top-k set (at least k
      // values are strictly greater than v_B, so the k-th largest value is
      // too), the set lies within {v > v_B}, and the winner over that subset
      // is the answer as soon as it is in the set itself (the smallest index
      // attaining the maximum over a superset that lies in the set).  Each
      // step strictly shrinks the subset; after kDrawChainSteps the radix select
      // below finds the threshold instead.
      for (int step = 0; step < kDrawChainSteps && greater >= p.top_k; ++step) {
        const float vb = __fdiv_rn(guided(arg), p.temperature);
#pragma unroll
        for (int t = 0; t < kPer; ++t) w[t] = v[t] > vb ? v[t] + pf.gn[t] : -INFINITY;
        arg = block_argmax(w, C, wres);
        const float vn = __fdiv_rn(guided(arg), p.temperature);
        int m = 0;
#pragma unroll
        for (int t = 0; t < kPer; ++t) m += __popcll(__ballot(tid + kDrawThreads * t < C && v[t] > vn));
        if ((tid & 63) == 0) wres[8 + wid] = m;
        __syncthreads();
        greater = wres[8] + wres[9] + wres[10] + wres[11];
      }
      if (greater >= p.top_k) {  // the winner is still outside the top-k set
        uint32_t key[kPer];
#pragma unroll
        for (int t = 0; t < kPer; ++t) key[t] = (tid + kDrawThreads * t < C) ? float_key(v[t]) : 0u;
        const float thr = key_float(radix_select(key, C, p.top_k, hist, tpoint));
#pragma unroll
        for (int t = 0; t < kPer; ++t) w[t] = (v[t] >= thr && v[t] != -INFINITY) ? v[t] + pf.gn[t] : -INFINITY;
        arg = block_argmax(w, C, wres);
        for (int i = tid; i < 2 * 4 * 256; i += kDrawThreads) hist[i] = 0u;  // buffers 0 / 1 for the next draw
        tpoint(3);
      }
    }
  }
  return arg;
}

}  // namespace mrt
