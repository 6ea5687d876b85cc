// On-device CFG + level-masked top-k temperature sampling and token feedback
// for one RVQ level (decode.cpp:71-148, 458-484).
//
// One workgroup per stream; its first wave draws, with the level's C logits
// (C <= 1024) in registers, 16 per lane.  The draw is Gumbel-max over the kept entries with
// Philox-4x32-10 noise.  When the winner over every candidate is itself in the
// top-k set it is the answer; else up to 3 winners over {v > v_previous
// winner} are tried the same way; otherwise the top-k threshold (the k-th largest
// value, counting ties, i.e. min(topk(x, k)) of decode.cpp:119-120) is found
// by a bitwise radix select over order-preserving float keys (at most 32
// steps, each counting with a DPP wave sum; it stops once exactly k keys lie
// at or above the prefix).
#include <cmath>
#include <mutex>

#include "device_utils.hpp"
#include "kernels.hpp"
#include "draw_block.hpp"

namespace mrt {
namespace {

constexpr int kMaxPerLane = 16;  // C <= 1024
constexpr int kChainSteps = 3;   // restricted-argmax steps of a draw before its radix select
constexpr int kFeedPer = 8;      // d_model elements per thread in the feedback (d_model <= 2048)
constexpr int kQkvPer = 8;       // q (k, v) table elements per thread (heads x 64 <= 2048)

// Sum over the 64 lanes with DPP (row shifts and broadcasts, no LDS
// crossbar); every lane active; the result is wave-uniform.
__device__ __forceinline__ int dpp_sum_i(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, true);   // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, true);   // quad_perm [2,3,0,1]
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, true);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, true);  // row_bcast:31
  return __builtin_amdgcn_readlane(v, 63);
}

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

// One draw by one wave (lane = threadIdx.x < 64) over the level's C entries
// of the CFG rows l0 (conditioned) / l1 (unconditioned); nz: the draw's
// tabulated noise row, or null to compute gumbel(seed, frame, level, i).
// Returns the winning index.
__device__ __forceinline__ int wave_draw_rows(const float* __restrict__ l0, const float* __restrict__ l1,
                                              const float* __restrict__ nz, uint64_t seed, const SampleParams& p,
                                              int frame, int level) {
  const int lane = threadIdx.x;
  const int C = p.codebook;
  const float wc = 1.0f + p.guidance_weight;  // decode.cpp:255-256
  const float wu = p.guidance_weight;

  // Loads are unconditional (indices clamped into range) and all issued
  // before the first use; entries past C are masked afterwards.
  float a0[kMaxPerLane], a1[kMaxPerLane], gn[kMaxPerLane];
#pragma unroll
  for (int t = 0; t < kMaxPerLane; ++t) {
    const int c = min(lane + 64 * t, C - 1);
    a0[t] = l0[c];
    a1[t] = l1[c];
  }
  if (p.temperature != 0.0f && nz != nullptr) {
#pragma unroll
    for (int t = 0; t < kMaxPerLane; ++t) gn[t] = nz[min(lane + 64 * t, C - 1)];
  }
  float v[kMaxPerLane];
  {
    // (1+w)*cond - w*uncond, each product rounded separately (decode.cpp:83-84):
    // no fused multiply-add here.
#pragma clang fp contract(off)
#pragma unroll
    for (int t = 0; t < kMaxPerLane; ++t) v[t] = lane + 64 * t < C ? wc * a0[t] - wu * a1[t] : -INFINITY;
  }

  bool done = false;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  if (p.temperature != 0.0f) {
#pragma unroll
    for (int t = 0; t < kMaxPerLane; ++t)
      if (lane + 64 * t < C) v[t] = __fdiv_rn(v[t], p.temperature);
    if (nz == nullptr) {
      const uint64_t seed0 = seed;
#pragma unroll
      for (int t = 0; t < kMaxPerLane; ++t) {
        const int c = lane + 64 * t;
        gn[t] = c < C ? gumbel(seed0, frame, level, c) : 0.f;
      }
    }
    if (p.top_k > 0 && p.top_k < C) {
      // The Gumbel-max winner A over every candidate is the winner over the
      // top-k set whenever A is in it, i.e. when fewer than k scaled logits
      // exceed v_A (ties at the k-th value are kept); only otherwise is the
      // threshold needed.
#pragma unroll
      for (int t = 0; t < kMaxPerLane; ++t) {
        const int c = lane + 64 * t;
        const float w = v[t] + gn[t];
        if (c < C && (w > best || bi == 0x7fffffff)) {
          best = w;
          bi = c;
        }
      }
      wave_argmax(best, bi);
      float va = 0.f;
#pragma unroll
      for (int t = 0; t < kMaxPerLane; ++t)
        if (lane + 64 * t == bi) va = v[t];
      va = __shfl(va, bi & 63, 64);
      int above = 0;
#pragma unroll
      for (int t = 0; t < kMaxPerLane; ++t) above += (lane + 64 * t < C && v[t] > va) ? 1 : 0;
      done = dpp_sum_i(above) < p.top_k;
      // Restricted steps: while the winner is outside the top-k set, the set
      // lies within {v > v_winner}; the winner over that subset is the answer
      // once it is in the set (it maximises over a superset of the set,
      // smallest index first).  Each step shrinks the subset strictly.
      for (int step = 0; step < kChainSteps && !done; ++step) {
        best = -INFINITY;
        bi = 0x7fffffff;
#pragma unroll
        for (int t = 0; t < kMaxPerLane; ++t) {
          const int c = lane + 64 * t;
          const float w = v[t] + gn[t];
          if (c < C && v[t] > va && (w > best || bi == 0x7fffffff)) {
            best = w;
            bi = c;
          }
        }
        wave_argmax(best, bi);
        va = 0.f;
#pragma unroll
        for (int t = 0; t < kMaxPerLane; ++t)
          if (lane + 64 * t == bi) va = v[t];
        va = __shfl(va, bi & 63, 64);
        above = 0;
#pragma unroll
        for (int t = 0; t < kMaxPerLane; ++t) above += (lane + 64 * t < C && v[t] > va) ? 1 : 0;
        done = dpp_sum_i(above) < p.top_k;
      }
    }
    if (!done && p.top_k > 0 && p.top_k < C) {
      uint32_t key[kMaxPerLane];
#pragma unroll
      for (int t = 0; t < kMaxPerLane; ++t) key[t] = (lane + 64 * t < C) ? float_key(v[t]) : 0u;
      uint32_t prefix = 0;
      for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = prefix | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int t = 0; t < kMaxPerLane; ++t) cnt += key[t] >= cand ? 1 : 0;
        const int n = dpp_sum_i(cnt);
        if (n >= p.top_k) prefix = cand;
        // exactly k keys at or above cand: {key >= cand} is already the top-k
        // set (no tie straddles it), so the lower bits are not needed; the
        // threshold must be finite and not +0 (-0 compares equal to +0)
        if (n == p.top_k && cand != 0x80000000u && __builtin_isfinite(key_float(cand))) break;
      }
      const float thr = key_float(prefix);
#pragma unroll
      for (int t = 0; t < kMaxPerLane; ++t)
        if (v[t] < thr) v[t] = -INFINITY;  // decode.cpp:121
    }
    if (!done) {
#pragma unroll
      for (int t = 0; t < kMaxPerLane; ++t) {
        const int c = lane + 64 * t;
        if (c < C && v[t] != -INFINITY) v[t] = v[t] + gn[t];
      }
    }
  }
  if (!done) {
    best = -INFINITY;
    bi = 0x7fffffff;
#pragma unroll
    for (int t = 0; t < kMaxPerLane; ++t) {
      const int c = lane + 64 * t;
      if (c < C && (v[t] > best || bi == 0x7fffffff)) {  // c ascends: first max wins
        best = v[t];
        bi = c;
      }
    }
    wave_argmax(best, bi);
  }

  return bi;
}

// Every level of one frame drawn at once (block l draws level l from logit
// rows 2l, 2l + 1; the speculative verification pass): drawn[l] = the LLM id.
__global__ __launch_bounds__(64) void k_draw_levels(const float* __restrict__ logits, SampleParams p, int frame,
                                                    int* __restrict__ drawn) {
  const int l = blockIdx.x, C = p.codebook;
  const float* l0 = logits + (size_t)(2 * l) * C;
  const float* nz = p.noise != nullptr ? p.noise + ((size_t)frame * p.rvq_depth + l) * C : nullptr;
  const uint64_t seed = p.seed != nullptr ? p.seed[0] : p.seed_value;
  const int bi = wave_draw_rows(l0, l0 + C, nz, p.temperature != 0.0f ? seed : 0, p, frame, l);
  if (threadIdx.x == 0) drawn[l] = p.codec_offset + l * C + bi;
}

// Block b draws for stream b: logits rows (2b, 2b + 1), seed p.seed[b], token
// slots slot + b * tstride; a non-null frame_ptr supplies the frame index.
// The whole block draws (block_draw, the frame kernel's draw) from the two
// logit rows staged in LDS, then writes the token's embedding to both rows of
// next_in and updates the frame sum (whose rows it loads before the draw).
template <typename T>
__global__ __launch_bounds__(kDrawThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_sample(
    const float* __restrict__ logits, SampleParams p, int frame, const int* __restrict__ frame_ptr, int level,
    int slot, int tstride, const int* __restrict__ teacher, int* __restrict__ tokens, int* __restrict__ drawn,
    const T* __restrict__ emb, int D, T* __restrict__ next_in, T* __restrict__ fsum, T* __restrict__ fmean,
    QkvFeed feed) {
  using S = St<T>;
  constexpr int kRowsPer = 2 * 1024 / kDrawThreads;  // logit-row elements per thread (codebook <= 1024)
  __shared__ float lg[2 * 1024];
  __shared__ __align__(16) unsigned hist[kDrawHistWords];
  __shared__ int wres[16];
  const int tid = threadIdx.x;
  const int stream = blockIdx.x;
  const int C = p.codebook, L = p.rvq_depth;
  if (frame_ptr != nullptr) {
    frame = *frame_ptr;
    slot += frame * L;
  }
  slot += stream * tstride;
  T* ni = next_in + (size_t)(2 * stream) * D;
  if (p.decided != nullptr && *p.decided >= level) {
    // the level's token is already known: only feed it to the next depth step
    // (the frame sum is not kept on this path)
    const T* e = emb + (size_t)tokens[slot] * D;
    for (int d = tid; d < D; d += kDrawThreads) {
      ni[d] = e[d];
      ni[D + d] = e[d];
    }
    return;
  }
  T* fs = fsum + (size_t)(2 * stream) * D;
  T* fm = fmean + (size_t)(2 * stream) * D;
  // Every load that does not depend on the token, issued before the first
  // store: the frame sum rows, the level slice's two logit rows, the draw's
  // noise (tabulated, or computed from the seed) and the teacher id.
  T fv[kFeedPer];
#pragma unroll
  for (int i = 0; i < kFeedPer; ++i) fv[i] = fs[min(tid + kDrawThreads * i, D - 1)];  // unused at level 0
  const float* l0 = logits + (size_t)(2 * stream) * C;
  float lv[kRowsPer];
#pragma unroll
  for (int i = 0; i < kRowsPer; ++i) lv[i] = l0[min(tid + kDrawThreads * i, 2 * C - 1)];
  const float* nz = p.noise != nullptr
                        ? p.noise + (((size_t)stream * p.noise_frames + frame) * p.rvq_depth + level) * C
                        : nullptr;
  const uint64_t seed = p.seed != nullptr ? p.seed[stream] : p.seed_value;
  DrawPrefetch pf;
#pragma unroll
  for (int t = 0; t < kDrawPer; ++t) {
    const int c = tid + kDrawThreads * t;
    pf.gn[t] = (c < C && p.temperature != 0.0f) ? (nz != nullptr ? nz[c] : gumbel(seed, frame, level, c)) : 0.f;
  }
  pf.teacher_id = teacher ? teacher[slot] : 0;
#pragma unroll
  for (int i = 0; i < kRowsPer; ++i)
    if (tid + kDrawThreads * i < 2 * C) lg[tid + kDrawThreads * i] = lv[i];
  draw_clear(hist);
  __syncthreads();
  const int bi = block_draw(p, pf, lg, hist, wres, [](int) {});
  const int drawn_id = p.codec_offset + level * C + bi;
  const int fed = teacher ? pf.teacher_id : drawn_id;
  if (tid == 0) {
    tokens[slot] = fed;
    if (drawn) drawn[slot] = drawn_id;
  }
  // Token feedback (decode.cpp:476-484): both CFG rows take emb(fed); the
  // frame sum accumulates in the model dtype; at the last level the mean is
  // the sum divided by L in the model dtype.  With a q/k/v feed, the fed
  // token's table row (the next level's depth layer-0 q | k | v) is written
  // for both rows too.  Every load of the token's rows is issued before the
  // first store: the stores could alias them as far as the compiler knows, so
  // interleaved they would serialise the round trips.
  const T* e = emb + (size_t)fed * D;
  const float Lf = S::rnd((float)L);
  T ev[kFeedPer];
#pragma unroll
  for (int i = 0; i < kFeedPer; ++i) ev[i] = e[min(tid + 256 * i, D - 1)];
  const int row = fed - feed.offset;
  const bool fed_qkv = feed.table != nullptr && level + 1 < L && row >= 0 && row < feed.rows;
  const int HD = feed.HD;
  T qv[3][kQkvPer];  // q, k, v: elements tid + 256 i of each
  if (fed_qkv) {
    const T* src = static_cast<const T*>(feed.table) + (size_t)row * 3 * HD;
#pragma unroll
    for (int w = 0; w < 3; ++w)
#pragma unroll
      for (int i = 0; i < kQkvPer; ++i)
        if (tid + 256 * i < HD) qv[w][i] = src[w * HD + tid + 256 * i];
  }
#pragma unroll
  for (int i = 0; i < kFeedPer; ++i) {
    const int d = tid + 256 * i;
    if (d >= D) continue;
    const float sum = (level == 0) ? S::ld(ev[i]) : S::rnd(S::ld(fv[i]) + S::ld(ev[i]));
    ni[d] = ev[i];
    ni[D + d] = ev[i];
    fs[d] = S::st(sum);
    fs[D + d] = S::st(sum);
    if (level == L - 1) {
      const T m = S::st(sum / Lf);
      fm[d] = m;
      fm[D + d] = m;
    }
  }
  if (fed_qkv) {
    T* q = static_cast<T*>(feed.q);
    T* kc = static_cast<T*>(feed.kc);
    T* vc = static_cast<T*>(feed.vc);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const size_t m = 2 * stream + b;
#pragma unroll
      for (int i = 0; i < kQkvPer; ++i) {
        const int nn = tid + 256 * i;
        if (nn >= HD) continue;
        const size_t slot = ((m * feed.H + (nn >> 6)) * feed.Lmax + level + 1) * 64 + (nn & 63);
        q[m * HD + nn] = qv[0][i];
        kc[slot] = qv[1][i];
        vc[slot] = qv[2][i];
      }
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

void draw_levels(const float* logits, const SampleParams& p, int frame, int levels, int* drawn, hipStream_t s) {
  MRT_REQUIRE(p.codebook >= 1 && p.codebook <= 64 * kMaxPerLane, "draw: codebook must be <= 1024");
  hipLaunchKernelGGL(k_draw_levels, dim3(levels), dim3(64), 0, s, logits, p, frame, drawn);
  MRT_HIP_CHECK(hipGetLastError());
}

void sample_levels(DType dt, int streams, const float* logits, const SampleParams& p, int frame,
                   const int* frame_ptr, int level, int slot, int tstride, const int* teacher, int* tokens,
                   int* drawn, const void* emb, int D, void* next_in, void* fsum, void* frame_mean, hipStream_t s,
                   const QkvFeed* feed) {
  MRT_REQUIRE(p.codebook >= 1 && p.codebook <= 64 * kMaxPerLane, "sample: codebook must be <= 1024");
  MRT_REQUIRE(streams >= 1, "sample: no streams");
  MRT_REQUIRE(D >= 1 && D <= 256 * kFeedPer, "sample: d_model must be in [1, 2048]");
  const QkvFeed fd = feed != nullptr ? *feed : QkvFeed{};
  if (fd.table != nullptr)
    MRT_REQUIRE(fd.q && fd.kc && fd.vc && fd.HD == fd.H * 64 && fd.HD <= 256 * kQkvPer &&
                    fd.Lmax >= p.rvq_depth && fd.rows >= 0,
                "sample: bad q/k/v feed");
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_sample<T>, dim3(streams), dim3(kDrawThreads), 0, s, logits, p, frame, frame_ptr,
                                            level, slot, tstride, teacher, tokens, drawn, (const T*)emb, D,
                                            (T*)next_in, (T*)fsum, (T*)frame_mean, fd));
  MRT_HIP_CHECK(hipGetLastError());
}

// ---- the draw without library allocations ---------------------------------------------
namespace {

// Scratch of sample_level_noalloc on each device: the three feedback row
// pairs k_sample writes (next depth input, frame sum, frame mean: 2 x d_model
// elements each, model dtype) from offset 256 (the first 256 bytes are
// unused).  The caller discards them; the seed travels by value in the
// kernel arguments, so calls that overlap on one device still draw their own
// tokens.  Every call on a device shares its copy, which keeps the last
// call's contents.
constexpr size_t kNoAllocBytes = 32 * 1024;
constexpr size_t kNoAllocRows = 256;
__device__ __align__(256) unsigned char scratch[kNoAllocBytes];

constexpr int kMaxNoAllocDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kMaxNoAllocDevices];  // device address of `scratch`, per device

}  // namespace

size_t noalloc_scratch_bytes() { return kNoAllocBytes; }

// The device address of `scratch` on `device` (the current device), looked up
// once per device.  The host-side name of a __device__ array is not its device
// address, so kernels only ever receive this pointer.
static unsigned char* scratch_on(int device) {
  MRT_REQUIRE(device >= 0 && device < kMaxNoAllocDevices, "sample_noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    MRT_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    g_scratch_ptr[device] = static_cast<unsigned char*>(ptr);
  }
  return g_scratch_ptr[device];
}

void sample_level_noalloc(DType dt, int device, const void* emb, int D, const float* logits, const SampleParams& p,
                          uint64_t seed, int frame, int level, int* token, hipStream_t s) {
  const size_t esz = dtype_size(dt);
  const size_t need = kNoAllocRows + 3 * 2 * static_cast<size_t>(D) * esz;
  if (need > kNoAllocBytes)
    throw Error(1, "sample_noalloc: d_model " + std::to_string(D) + " needs " + std::to_string(need) +
                       " bytes of scratch, more than the fixed " + std::to_string(kNoAllocBytes));
  unsigned char* base = scratch_on(device);
  unsigned char* rows = base + kNoAllocRows;
  const size_t row_pair = 2 * static_cast<size_t>(D) * esz;
  SampleParams sp = p;
  sp.seed = nullptr;
  sp.seed_value = seed;
  sp.noise = nullptr;
  sp.decided = nullptr;
  sample_level(dt, logits, sp, frame, level, 0, nullptr, token, nullptr, emb, D, rows, rows + row_pair,
               rows + 2 * row_pair, s);
}

}  // namespace mrt
