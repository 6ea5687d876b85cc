// Persistent step kernels for gfx950: one launch runs a whole depth_step
// (4 decoder layers + decoder_norm + level-sliced lm_head + CFG/top-k sampling
// + token feedback) or a whole temporal_step (20 layers with cross attention).
//
// Grid = H * bph workgroups (one per CU: 256 on MI355X), 4 waves each.  The
// phases of a step hand data to each other through 64-bit words {payload,
// tag} written and read with agent-scope (sc1) atomics, which are coherent
// across the 8 XCDs without cache maintenance.  A consumer polls the words it
// needs until each carries the tag of the producing phase of this launch
// (tag = launch epoch << 10 | phase code), so a hand-off costs one store ->
// load propagation and needs no counters, barriers or store drains.  The
// epoch is a device counter that workgroup 0 advances once it has seen data
// from every workgroup, so graph replays never match stale words.
//
// Every buffer is rewritten only after all of its readers have consumed it:
// each phase's inputs depend on outputs of every workgroup of the previous
// phase, which those workgroups produce only after finishing their reads.
//
// Weights are read exactly once with 16-byte non-temporal loads issued as
// soon as the previous phase's outputs are stored, so their HBM latency
// overlaps the wait for the next phase's inputs.
//
// Work split per phase (H=16, bph=16, G=256):
//   QKV:   workgroup (h, j) owns rows 4j..4j+3 of head h's q, k and v
//          (3 rows per wave); workgroup (h, 0) then runs head h's attention
//          over the ring (<= 64 keys).
//   O / FFN-down / cross-O / head: ceil(N / G) rows per workgroup.
//   FFN-up: ceil(d_ff / G) gate/up row pairs per workgroup.
//   cross:  workgroup (h, j) owns head h's q rows 4j.., then computes the
//          softmax partial of key block j (ceil(S / bph) keys); workgroup
//          (h, 0) combines the bph partials.
#include <cmath>

#include "device_utils.hpp"
#include "persist.hpp"

#define MRT_GLOBAL __attribute__((address_space(1)))

namespace mrt {
namespace {

// ---- memory helpers ---------------------------------------------------------------

template <typename W>
__device__ __forceinline__ W aload(const W* p) {
  return __hip_atomic_load((const MRT_GLOBAL W*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename W>
__device__ __forceinline__ void astore(W* p, W v) {
  __hip_atomic_store((MRT_GLOBAL W*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_g(T* p, T v) {
  *(MRT_GLOBAL T*)(p) = v;
}

__device__ __forceinline__ bool spin_failed(uint32_t& spins, int* err) {
  if ((++spins & 255u) == 0) {
    if (aload(err) != 0 || spins > kSpinLimit) {
      astore(err, 1);
      return true;
    }
  }
  return false;
}

// Plain (rows 0/1) pair of one element: bf16 -> 32 bits, fp32 -> 64 bits.
template <typename T>
struct PairT;
template <>
struct PairT<bf16> {
  using W = uint32_t;
  __device__ static float lo(W w) { return bf2f(static_cast<bf16>(w & 0xffffu)); }
  __device__ static float hi(W w) { return bf2f(static_cast<bf16>(w >> 16)); }
  __device__ static W pack(float a, float b) { return (W)f2bf(a) | ((W)f2bf(b) << 16); }
};
template <>
struct PairT<float> {
  using W = uint64_t;
  __device__ static float lo(W w) { return __uint_as_float(static_cast<uint32_t>(w)); }
  __device__ static float hi(W w) { return __uint_as_float(static_cast<uint32_t>(w >> 32)); }
  __device__ static W pack(float a, float b) {
    return (W)__float_as_uint(a) | ((W)__float_as_uint(b) << 32);
  }
};

// ---- tagged words -------------------------------------------------------------------

__device__ __forceinline__ uint64_t ll_word(uint32_t payload, uint32_t tag) {
  return ((uint64_t)tag << 32) | payload;
}
__device__ __forceinline__ uint32_t ll_tag(uint64_t w) { return static_cast<uint32_t>(w >> 32); }

// Element k (both rows) of a tagged vector: bf16 -> one word, fp32 -> one
// word per row (row 1 at +kMaxPersistK).
template <typename T>
struct LL;
template <>
struct LL<bf16> {
  static constexpr int kWords = 1;
  __device__ static int idx(int k, int) { return k; }
  __device__ static void put(uint64_t* b, int k, float v0, float v1, uint32_t tag) {
    astore(b + k, ll_word((uint32_t)f2bf(v0) | ((uint32_t)f2bf(v1) << 16), tag));
  }
  __device__ static float get(const uint64_t (&w)[1], int r) {
    return bf2f(static_cast<bf16>((static_cast<uint32_t>(w[0]) >> (16 * r)) & 0xffffu));
  }
};
template <>
struct LL<float> {
  static constexpr int kWords = 2;
  __device__ static int idx(int k, int r) { return r * kMaxPersistK + k; }
  __device__ static void put(uint64_t* b, int k, float v0, float v1, uint32_t tag) {
    astore(b + k, ll_word(__float_as_uint(v0), tag));
    astore(b + kMaxPersistK + k, ll_word(__float_as_uint(v1), tag));
  }
  __device__ static float get(const uint64_t (&w)[2], int r) { return __uint_as_float(static_cast<uint32_t>(w[r])); }
};

// A residual value fetched alongside a vector: element `row` from a tagged
// buffer, or from the launch's plain input pairs when `plain` is set.
struct Side {
  const uint64_t* ll;
  const void* plain;
  uint32_t tag;
  int row;  // -1: nothing for this thread
};

// Polls elements k = tid + 256 i (k < K) of a tagged vector until each word
// carries `tag` and stores both rows to xs[k], xs[kMaxPersistK + k]; the
// side element (if any) is returned in r0/r1.  All loads of one round are
// issued before any is waited for.
template <typename T>
__device__ void ll_load_vec(const uint64_t* src, int K, uint32_t tag, float* xs, const Side& sd, float& r0,
                            float& r1, int* err) {
  using PT = PairT<T>;
  constexpr int kPer = kMaxPersistK / kPersistThreads;
  constexpr int NW = LL<T>::kWords;
  const int tid = threadIdx.x;
  uint64_t w[kPer][NW];
  uint64_t sw[NW];
  uint32_t pend = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (src != nullptr && tid + i * kPersistThreads < K) pend |= 1u << i;
  bool side_pend = sd.row >= 0 && sd.plain == nullptr;
  if (sd.row >= 0 && sd.plain != nullptr) {
    const typename PT::W p = ld_g(static_cast<const typename PT::W*>(sd.plain) + sd.row);
    r0 = PT::lo(p);
    r1 = PT::hi(p);
  }
  uint32_t spins = 0;
  while (pend != 0 || side_pend) {
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if ((pend >> i) & 1u)
#pragma unroll
        for (int r = 0; r < NW; ++r) w[i][r] = aload(src + LL<T>::idx(tid + i * kPersistThreads, r));
    if (side_pend)
#pragma unroll
      for (int r = 0; r < NW; ++r) sw[r] = aload(sd.ll + LL<T>::idx(sd.row, r));
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      if ((pend >> i) & 1u) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < NW; ++r) ok = ok && ll_tag(w[i][r]) == tag;
        if (ok) {
          const int k = tid + i * kPersistThreads;
          xs[k] = LL<T>::get(w[i], 0);
          xs[kMaxPersistK + k] = LL<T>::get(w[i], 1);
          pend &= ~(1u << i);
        }
      }
    }
    if (side_pend) {
      bool ok = true;
#pragma unroll
      for (int r = 0; r < NW; ++r) ok = ok && ll_tag(sw[r]) == sd.tag;
      if (ok) {
        r0 = LL<T>::get(sw, 0);
        r1 = LL<T>::get(sw, 1);
        side_pend = false;
      }
    }
    if (pend == 0 && !side_pend) break;
    if (spin_failed(spins, err)) break;
    __builtin_amdgcn_s_sleep(1);
  }
}

// RMS normalisation of both rows in xs with weight g (modules.cpp:72-84).
template <typename T>
__device__ void norm_rows(int K, const T* g, float eps, float* xs, float* red) {
  using S = St<T>;
  float s0 = 0.f, s1 = 0.f;
  for (int k = threadIdx.x; k < K; k += kPersistThreads) {
    s0 = fmaf(xs[k], xs[k], s0);
    s1 = fmaf(xs[kMaxPersistK + k], xs[kMaxPersistK + k], s1);
  }
  s0 = wave_sum(s0);
  s1 = wave_sum(s1);
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[wid] = s0;
    red[4 + wid] = s1;
  }
  __syncthreads();
  const float inv0 = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + eps);
  const float inv1 = 1.0f / sqrtf((red[4] + red[5] + red[6] + red[7]) / (float)K + eps);
  for (int k = threadIdx.x; k < K; k += kPersistThreads) {
    const float gk = S::ld(ld_g(g + k));
    xs[k] = S::rnd(S::rnd(xs[k] * inv0) * gk);
    xs[kMaxPersistK + k] = S::rnd(S::rnd(xs[kMaxPersistK + k] * inv1) * gk);
  }
}

// Loads the activation vector of a phase into xs (tagged, or the launch's
// plain input pairs), with an optional side element and RMS norm.
__device__ __forceinline__ void trace_point(uint64_t* trace, int slot);

template <typename T>
__device__ void load_act(const uint64_t* ll, const void* plain, int K, uint32_t tag, const T* g, float* xs,
                         float* red, const Side& sd, float& r0, float& r1, int* err, uint64_t* trace = nullptr,
                         int* tp = nullptr) {
  using PT = PairT<T>;
  if (tp) trace_point(trace, (*tp)++);
  if (plain != nullptr) {
    constexpr int kPer = kMaxPersistK / kPersistThreads;
    typename PT::W w[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int k = threadIdx.x + i * kPersistThreads;
      if (k < K) w[i] = ld_g(static_cast<const typename PT::W*>(plain) + k);
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int k = threadIdx.x + i * kPersistThreads;
      if (k < K) {
        xs[k] = PT::lo(w[i]);
        xs[kMaxPersistK + k] = PT::hi(w[i]);
      }
    }
    ll_load_vec<T>(nullptr, 0, 0, xs, sd, r0, r1, err);
  } else {
    ll_load_vec<T>(ll, K, tag, xs, sd, r0, r1, err);
  }
  if (tp) trace_point(trace, (*tp)++);
  __syncthreads();
  if (g != nullptr) {
    norm_rows<T>(K, g, 1e-6f, xs, red);
    __syncthreads();
  }
  if (tp) trace_point(trace, (*tp)++);
}

// ---- GEMV machinery ---------------------------------------------------------------

template <typename T>
constexpr int nbuf() {
  return 6 * ((1024 + St<T>::kVec * 64 - 1) / (St<T>::kVec * 64));  // 6 rows of K <= 1024
}

// Loads the rows of one batch (R rows of P parts) into registers.
template <typename T, int NV, int P, class RowOf>
__device__ __forceinline__ void fetch_batch(uint4 (&buf)[nbuf<T>()], const T* W, int K, int b0, int nb,
                                            RowOf row_of) {
  constexpr int V = St<T>::kVec;
  constexpr int R = nbuf<T>() / (P * NV);
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r < nb) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const T* row = W + (size_t)row_of(b0 + r, p) * K;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int c = lane + 64 * i;
          if (c * V < K) buf[(r * P + p) * NV + i] = ld_nt16(row + (size_t)c * V);
        }
      }
    }
  }
}

// Dots of a batch against the two activation rows xs[0..K), xs[kMax..kMax+K),
// reduced across the wave; epi(index, acc[P][2]) runs on every lane.
template <typename T, int NV, int P, class Epi>
__device__ __forceinline__ void dot_batch(const uint4 (&buf)[nbuf<T>()], int K, int b0, int nb, const float* xs,
                                          Epi epi) {
  constexpr int V = St<T>::kVec;
  constexpr int R = nbuf<T>() / (P * NV);
  const int lane = threadIdx.x & 63;
  float acc[R][P][2];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p) acc[r][p][0] = acc[r][p][1] = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    if (c * V < K) {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float x0 = xs[c * V + e], x1 = xs[kMaxPersistK + c * V + e];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r < nb) {
#pragma unroll
            for (int p = 0; p < P; ++p) {
              const float w = St<T>::ld(reinterpret_cast<const T*>(&buf[(r * P + p) * NV + i])[e]);
              acc[r][p][0] = fmaf(w, x0, acc[r][p][0]);
              acc[r][p][1] = fmaf(w, x1, acc[r][p][1]);
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r < nb) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        acc[r][p][0] = wave_sum(acc[r][p][0]);
        acc[r][p][1] = wave_sum(acc[r][p][1]);
      }
      epi(b0 + r, acc[r]);
    }
  }
}

// Runs a wave's nw rows in batches; the first batch is already in buf.
template <typename T, int NV, int P, class RowOf, class Epi>
__device__ __forceinline__ void gemv_rows(uint4 (&buf)[nbuf<T>()], const T* W, int K, int nw, RowOf row_of,
                                          const float* xs, Epi epi) {
  constexpr int R = nbuf<T>() / (P * NV);
  for (int b0 = 0; b0 < nw; b0 += R) {
    const int nb = min(R, nw - b0);
    if (b0 > 0) fetch_batch<T, NV, P>(buf, W, K, b0, nb, row_of);
    dot_batch<T, NV, P>(buf, K, b0, nb, xs, epi);
  }
}

// Rows [blk * rpb, ...) of an N-row matrix; wave w takes local rows w, w+4, ...
struct RowSplit {
  int first, count;  // block range
  __device__ RowSplit(int N, int G, int blk) {
    const int rpb = (N + G - 1) / G;
    first = blk * rpb;
    count = max(0, min(N, first + rpb) - first);
  }
  __device__ int nw(int wid) const { return count > wid ? (count - wid + 3) / 4 : 0; }
  __device__ int row(int wid, int t) const { return first + wid + 4 * t; }
};

__device__ __forceinline__ int geglu_row(int j, int p) { return (j >> 5) * 64 + (j & 31) + 32 * p; }

// Polls `n` (<= 256) tagged elements src[i] into LDS floats dst0[i], dst1[i].
template <typename T>
__device__ void ll_load_small(const uint64_t* src, int n, uint32_t tag, float* dst0, float* dst1, int* err) {
  constexpr int NW = LL<T>::kWords;
  const int tid = threadIdx.x;
  if (tid >= n) return;
  uint64_t w[NW];
  uint32_t spins = 0;
  for (;;) {
#pragma unroll
    for (int r = 0; r < NW; ++r) w[r] = aload(src + LL<T>::idx(tid, r));
    bool ok = true;
#pragma unroll
    for (int r = 0; r < NW; ++r) ok = ok && ll_tag(w[r]) == tag;
    if (ok || spin_failed(spins, err)) break;
    __builtin_amdgcn_s_sleep(1);
  }
  dst0[tid] = LL<T>::get(w, 0);
  dst1[tid] = LL<T>::get(w, 1);
}

// Self attention of head h over ring slots 0..pos (scale 1.0, bias
// table[bucket[pos - j], h]; modules.cpp:243-295).  Slots before pos were
// written by earlier launches (plain loads); q and slot pos come as tagged
// words of this launch.
template <typename T>
__device__ void self_attention_head(const StepArgs& a, const LayerDev& L, int h, uint32_t tag, uint32_t out_tag,
                                    float* sm) {
  using S = St<T>;
  constexpr int V = S::kVec;
  float* qs = sm;        // [2][64]
  float* ks = sm + 128;  // [2][64]  slot pos, then the output
  float* vs = sm + 256;  // [2][64]  slot pos
  float* ps = sm + 384;  // [2][64]
  __shared__ float sl[2];
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  if (wid < 3) {  // waves 0, 1, 2 fetch q, k, v of head h
    const uint64_t* src = (wid == 0 ? a.ll.q : wid == 1 ? a.ll.k : a.ll.v) + h * 64;
    float* d = sm + wid * 128;
    constexpr int NW = LL<T>::kWords;
    uint64_t w[NW];
    uint32_t spins = 0;
    for (;;) {
#pragma unroll
      for (int r = 0; r < NW; ++r) w[r] = aload(src + LL<T>::idx(lane, r));
      bool ok = true;
#pragma unroll
      for (int r = 0; r < NW; ++r) ok = ok && ll_tag(w[r]) == tag;
      if (ok || spin_failed(spins, a.ll.err)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    d[lane] = LL<T>::get(w, 0);
    d[64 + lane] = LL<T>::get(w, 1);
  }
  __syncthreads();
  const int len = a.pos + 1;
  float o = 0.f;
  if (wid < 2) {
    const int b = wid;
    const T* Kp = static_cast<const T*>(L.kc) + ((size_t)(b * a.H + h) * a.Lmax) * 64;
    float sc = -INFINITY;
    if (lane < a.pos) {
      const T* kr = Kp + (size_t)lane * 64;
      uint4 kv[64 / V];
#pragma unroll
      for (int i = 0; i < 64 / V; ++i) kv[i] = ld_g16(kr + i * V);
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 64 / V; ++i) {
        const T* ke = reinterpret_cast<const T*>(&kv[i]);
#pragma unroll
        for (int e = 0; e < V; ++e) acc = fmaf(qs[b * 64 + i * V + e], S::ld(ke[e]), acc);
      }
      sc = acc;
    } else if (lane == a.pos) {
      float acc = 0.f;
#pragma unroll 16
      for (int d = 0; d < 64; ++d) acc = fmaf(qs[b * 64 + d], ks[b * 64 + d], acc);
      sc = acc;
    }
    if (lane < len) sc += S::ld(ld_g(static_cast<const T*>(a.bias_tab) + ld_g(a.buckets + a.pos - lane) * a.H + h));
    const float m = wave_max(sc);
    const float p = lane < len ? expf(sc - m) : 0.f;
    const float l = wave_sum(p);
    ps[b * 64 + lane] = p;
    if (lane == 0) sl[b] = l;
  }
  __syncthreads();
  if (wid < 2) {
    const int b = wid;
    const T* Vp = static_cast<const T*>(L.vc) + ((size_t)(b * a.H + h) * a.Lmax) * 64 + lane;
    float vv[kMaxPersistLen];
#pragma unroll
    for (int j = 0; j < kMaxPersistLen; ++j)
      if (j < a.pos) vv[j] = S::ld(ld_g(Vp + (size_t)j * 64));
    o = ps[b * 64 + a.pos] * vs[b * 64 + lane];
#pragma unroll
    for (int j = 0; j < kMaxPersistLen; ++j)
      if (j < a.pos) o = fmaf(ps[b * 64 + j], vv[j], o);
    o = o / sl[b];
  }
  __syncthreads();  // every read of ks is done before it is reused
  if (wid < 2) ks[wid * 64 + lane] = o;
  __syncthreads();
  if (tid < 64) LL<T>::put(a.ll.at, h * 64 + tid, ks[tid], ks[64 + tid], out_tag);
}

// Softmax partial of cross attention: head h, key block j, both rows; the
// cross K/V were written by the encoder launch (plain loads).
template <typename T>
__device__ void cross_partial(const StepArgs& a, const LayerDev& L, int h, int j, uint32_t q_tag, uint32_t out_tag,
                              float* sm) {
  using S = St<T>;
  constexpr int V = S::kVec;
  float* qs = sm;        // [2][64]
  float* ps = sm + 128;  // [4][64]
  float* wo = sm + 384;  // [4][64]
  __shared__ float wm[4], wl[4];
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  ll_load_small<T>(a.ll.q + h * 64, 64, q_tag, qs, qs + 64, a.ll.err);
  __syncthreads();
  const int chunk = (a.S + a.bph - 1) / a.bph;
  const int half = (chunk + 1) / 2;
  const int b = wid >> 1;
  const int kb = j * chunk + (wid & 1) * half;
  const int ke = min(min(a.S, j * chunk + chunk), kb + half);
  const int nk = max(0, ke - kb);
  const T* Kp = static_cast<const T*>(L.ck) + ((size_t)(b * a.H + h) * a.S) * 64;
  const T* Vp = static_cast<const T*>(L.cv) + ((size_t)(b * a.H + h) * a.S) * 64;
  float sc = -INFINITY;
  if (lane < nk) {
    const T* kr = Kp + (size_t)(kb + lane) * 64;
    uint4 kv[64 / V];
#pragma unroll
    for (int i = 0; i < 64 / V; ++i) kv[i] = ld_nt16(kr + i * V);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 64 / V; ++i) {
      const T* ke_ = reinterpret_cast<const T*>(&kv[i]);
#pragma unroll
      for (int e = 0; e < V; ++e) acc = fmaf(qs[b * 64 + i * V + e], S::ld(ke_[e]), acc);
    }
    sc = acc;
  }
  const float m = wave_max(sc);
  const float p = (lane < nk) ? expf(sc - m) : 0.f;
  const float l = wave_sum(p);
  ps[wid * 64 + lane] = p;
  __syncthreads();
  float vv[64];
#pragma unroll
  for (int t = 0; t < 64; ++t)
    if (t < nk) vv[t] = S::ld(ld_g(Vp + (size_t)(kb + t) * 64 + lane));
  float o = 0.f;
#pragma unroll
  for (int t = 0; t < 64; ++t)
    if (t < nk) o = fmaf(ps[wid * 64 + t], vv[t], o);
  wo[wid * 64 + lane] = o;
  if (lane == 0) {
    wm[wid] = nk > 0 ? m : -INFINITY;
    wl[wid] = l;
  }
  __syncthreads();
  if (tid < 128) {
    const int bb = tid >> 6, d = tid & 63;
    const int w0 = 2 * bb, w1 = 2 * bb + 1;
    const float M = fmaxf(wm[w0], wm[w1]);
    const float c0 = wm[w0] == -INFINITY ? 0.f : expf(wm[w0] - M);
    const float c1 = wm[w1] == -INFINITY ? 0.f : expf(wm[w1] - M);
    uint64_t* dst = a.ll.part + ((size_t)(h * a.bph + j) * 2 + bb) * 66;
    astore(dst + 2 + d, ll_word(__float_as_uint(wo[w0 * 64 + d] * c0 + wo[w1 * 64 + d] * c1), out_tag));
    if (d == 0) {
      astore(dst, ll_word(__float_as_uint(M), out_tag));
      astore(dst + 1, ll_word(__float_as_uint(wl[w0] * c0 + wl[w1] * c1), out_tag));
    }
  }
  __syncthreads();  // sm is reused by the caller
}

// Combines the bph partials of head h into its attention output.
template <typename T>
__device__ void cross_combine(const StepArgs& a, int h, uint32_t tag, uint32_t out_tag, float* sm) {
  float* os = sm;  // [2][64]
  const int tid = threadIdx.x;
  if (tid < 128) {
    const int b = tid >> 6, d = tid & 63;
    uint64_t wm[kMaxBph], wl[kMaxBph], wv[kMaxBph];
    uint32_t pend = (1u << a.bph) - 1u;
    uint32_t spins = 0;
    while (pend != 0) {
#pragma unroll
      for (int j = 0; j < kMaxBph; ++j) {
        if ((pend >> j) & 1u) {
          const uint64_t* src = a.ll.part + ((size_t)(h * a.bph + j) * 2 + b) * 66;
          wm[j] = aload(src);
          wl[j] = aload(src + 1);
          wv[j] = aload(src + 2 + d);
        }
      }
#pragma unroll
      for (int j = 0; j < kMaxBph; ++j)
        if (((pend >> j) & 1u) && ll_tag(wm[j]) == tag && ll_tag(wl[j]) == tag && ll_tag(wv[j]) == tag)
          pend &= ~(1u << j);
      if (pend == 0 || spin_failed(spins, a.ll.err)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < kMaxBph; ++j)
      if (j < a.bph) M = fmaxf(M, __uint_as_float(static_cast<uint32_t>(wm[j])));
    float Lt = 0.f, O = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxBph; ++j) {
      if (j < a.bph) {
        const float m = __uint_as_float(static_cast<uint32_t>(wm[j]));
        if (m != -INFINITY) {
          const float c = expf(m - M);
          Lt = fmaf(__uint_as_float(static_cast<uint32_t>(wl[j])), c, Lt);
          O = fmaf(__uint_as_float(static_cast<uint32_t>(wv[j])), c, O);
        }
      }
    }
    os[b * 64 + d] = O / Lt;
  }
  __syncthreads();
  if (tid < 64) LL<T>::put(a.ll.at, h * 64 + tid, os[tid], os[64 + tid], out_tag);
}

// CFG + temperature/top-k Gumbel-max draw and token feedback (decode.cpp:
// 71-148, 458-484), run by wave 0; `lg` holds the two logit rows in LDS.
template <typename T>
__device__ void sample_and_feed(const StepArgs& a, const float* lg) {
  using PT = PairT<T>;
  using W = typename PT::W;
  using S = St<T>;
  constexpr int kPer = 16;
  const int lane = threadIdx.x & 63;
  const SampleParams& p = a.sp;
  const int C = p.codebook;
  const float wc = 1.0f + p.guidance_weight, wu = p.guidance_weight;
  float v[kPer];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int c = lane + 64 * t;
    v[t] = (c < C) ? __fsub_rn(__fmul_rn(wc, lg[c]), __fmul_rn(wu, lg[C + c])) : -INFINITY;
  }
  if (p.temperature != 0.0f) {
#pragma unroll
    for (int t = 0; t < kPer; ++t)
      if (lane + 64 * t < C) v[t] = __fdiv_rn(v[t], p.temperature);
    if (p.top_k > 0 && p.top_k < C) {
      uint32_t key[kPer];
#pragma unroll
      for (int t = 0; t < kPer; ++t) key[t] = (lane + 64 * t < C) ? float_key(v[t]) : 0u;
      uint32_t prefix = 0;
      for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = prefix | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int t = 0; t < kPer; ++t) cnt += key[t] >= cand ? 1 : 0;
        if (wave_sum_i(cnt) >= p.top_k) prefix = cand;
      }
      const float thr = key_float(prefix);
#pragma unroll
      for (int t = 0; t < kPer; ++t)
        if (v[t] < thr) v[t] = -INFINITY;
    }
    const uint64_t seed = ld_g(p.seed);
#pragma unroll
    for (int t = 0; t < kPer; ++t) {
      const int c = lane + 64 * t;
      if (c < C && v[t] != -INFINITY) v[t] = v[t] + gumbel(seed, a.frame, a.level, c);
    }
  }
  float best = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int c = lane + 64 * t;
    if (c < C && (v[t] > best || bi == 0x7fffffff)) {
      best = v[t];
      bi = c;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  const int drawn_id = p.codec_offset + a.level * C + bi;
  const int fed = a.teacher ? ld_g(a.teacher + a.slot) : drawn_id;
  if (lane == 0) {
    st_g(a.tokens + a.slot, fed);
    if (a.drawn) st_g(a.drawn + a.slot, drawn_id);
  }
  // Token feedback: both rows take emb(fed); the frame sum accumulates in the
  // model dtype; the last level's sum / L is the next temporal input.
  constexpr int kDPer = 1024 / 64;
  const T* e = static_cast<const T*>(a.emb) + (size_t)fed * a.D;
  const W* fs_in = static_cast<const W*>(a.fsum);
  float ev[kDPer], fv[kDPer];
#pragma unroll
  for (int t = 0; t < kDPer; ++t) {
    const int d = lane + 64 * t;
    if (d < a.D) {
      ev[t] = S::ld(ld_g(e + d));
      fv[t] = a.level == 0 ? 0.f : PT::lo(ld_g(fs_in + d));
    }
  }
  const float Lf = S::rnd((float)p.rvq_depth);
  W* ni = static_cast<W*>(a.next_in);
  W* fs = static_cast<W*>(a.fsum);
  W* fm = static_cast<W*>(a.fmean);
#pragma unroll
  for (int t = 0; t < kDPer; ++t) {
    const int d = lane + 64 * t;
    if (d < a.D) {
      const float sum = (a.level == 0) ? ev[t] : S::rnd(fv[t] + ev[t]);
      st_g(ni + d, PT::pack(ev[t], ev[t]));
      st_g(fs + d, PT::pack(sum, sum));
      if (a.level == p.rvq_depth - 1) {
        const float m = S::rnd(sum / Lf);
        st_g(fm + d, PT::pack(m, m));
      }
    }
  }
}

__device__ __forceinline__ void trace_point(uint64_t* trace, int slot) {
  if (trace != nullptr && blockIdx.x == 0 && threadIdx.x == 0 && slot < kTraceSlots) trace[slot] = wall_clock64();
}

// Phase codes of the tags (per layer: code = 16 * layer + phase).
enum : int { kPhQKV = 0, kPhAtt = 1, kPhO = 2, kPhCQ = 3, kPhCP = 4, kPhCC = 5, kPhCO = 6, kPhUp = 7, kPhDn = 8 };
constexpr int kPhHead = 1000;

template <typename T, bool CROSS>
__global__ __launch_bounds__(kPersistThreads) void k_step(StepArgs a) {
  using PT = PairT<T>;
  using W = typename PT::W;
  using S = St<T>;
  constexpr int V = S::kVec;
  constexpr int NVD = (1024 + V * 64 - 1) / (V * 64);  // K <= 1024
  constexpr int NVF = 3 * NVD;                         // K <= 3072
  __shared__ float xs[2 * kMaxPersistK];
  __shared__ float red[8];
  __shared__ float sm[640];
  __shared__ float kvst[2][2][8];  // [k|v][row][d within this workgroup's slice]

  if (aload(a.ll.err) != 0) return;  // a previous launch failed: do nothing
  const uint32_t ep = aload(a.ll.seq);
  auto tag = [&](int code) { return (ep << 10) | (uint32_t)code; };
  const int G = gridDim.x, blk = blockIdx.x, wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int D = a.D, HD = a.HD, H = a.H, F = a.F, bph = a.bph;
  const int h = blk / bph, jpart = blk % bph, rps = 64 / bph;
  uint4 buf[nbuf<T>()];
  int tp = 0;  // trace slot
  trace_point(a.trace, kTraceStart);

  const RowSplit sD(D, G, blk), sF(F, G, blk);
  // QKV rows of this wave: local t = wid + 4i < 3*rps -> (segment t / rps, row t % rps).
  const int nqkv = (3 * rps > wid) ? (3 * rps - wid + 3) / 4 : 0;
  auto qkv_row = [&](int t, int) {
    const int lt = wid + 4 * t;
    return (lt / rps) * HD + h * 64 + jpart * rps + (lt % rps);
  };
  const int ncq = (rps > wid) ? (rps - wid + 3) / 4 : 0;
  auto cq_row = [&](int t, int) { return h * 64 + jpart * rps + wid + 4 * t; };
  auto rowD = [&](int t, int) { return sD.row(wid, t); };
  auto rowF = [&](int t, int p) { return geglu_row(sF.row(wid, t), p); };
  // residual element of the wave's D-row `lane` (lanes < nw)
  auto side_x = [&](const uint64_t* ll, const void* plain, uint32_t tg) {
    Side s{ll, plain, tg, lane < sD.nw(wid) ? sD.row(wid, lane) : -1};
    return s;
  };
  const Side no_side{nullptr, nullptr, 0u, -1};
  float r0 = 0.f, r1 = 0.f;

  uint32_t x_tag = 0;  // tag of the current residual stream (layer >= 1)
  if (a.nlayers > 0)
    fetch_batch<T, NVD, 1>(buf, static_cast<const T*>(a.layers[0].wqkv), D, 0, min(nbuf<T>() / NVD, nqkv), qkv_row);
  for (int li = 0; li < a.nlayers; ++li) {
    const LayerDev& L = a.layers[li];
    const bool first = li == 0;
    const int base = 16 * li;
    // ---- QKV of head h's slice (weights already in flight)
    load_act<T>(a.ll.x, first ? a.in : nullptr, D, x_tag, static_cast<const T*>(L.norm_sa), xs, red, no_side, r0,
                r1, a.ll.err, a.trace, &tp);
    gemv_rows<T, NVD, 1>(buf, static_cast<const T*>(L.wqkv), D, nqkv, qkv_row, xs,
                         [&](int t, const float (&acc)[1][2]) {
                           const int lt = wid + 4 * t, seg = lt / rps, r = lt % rps;
                           const int n = h * 64 + jpart * rps + r;
                           const float v0 = S::rnd(acc[0][0]), v1 = S::rnd(acc[0][1]);
                           if (lane == 0) {
                             uint64_t* dst = seg == 0 ? a.ll.q : seg == 1 ? a.ll.k : a.ll.v;
                             LL<T>::put(dst, n, v0, v1, tag(base + kPhQKV));
                             if (seg > 0) {
                               kvst[seg - 1][0][r] = v0;
                               kvst[seg - 1][1][r] = v1;
                             }
                           }
                         });
    __syncthreads();
    // plain ring slot (read by later launches): 4 elements per 8-byte store
    if (threadIdx.x < 2 * 2 * (rps / 4)) {
      const int g4 = threadIdx.x % (rps / 4), rb = (threadIdx.x / (rps / 4)) % 2, kv = threadIdx.x / (rps / 2);
      T* cache = static_cast<T*>(kv == 0 ? L.kc : L.vc);
      T* dst = cache + (((size_t)rb * H + h) * a.Lmax + a.pos) * 64 + jpart * rps + 4 * g4;
      const float* v = &kvst[kv][rb][4 * g4];
      if constexpr (sizeof(T) == 2) {
        st_g(reinterpret_cast<uint64_t*>(dst), (uint64_t)f2bf(v[0]) | ((uint64_t)f2bf(v[1]) << 16) |
                                                   ((uint64_t)f2bf(v[2]) << 32) | ((uint64_t)f2bf(v[3]) << 48));
      } else {
        st_g(reinterpret_cast<uint64_t*>(dst), (uint64_t)__float_as_uint(v[0]) | ((uint64_t)__float_as_uint(v[1]) << 32));
        st_g(reinterpret_cast<uint64_t*>(dst) + 1,
             (uint64_t)__float_as_uint(v[2]) | ((uint64_t)__float_as_uint(v[3]) << 32));
      }
    }
    // next phase's weights, then head h's attention in workgroup (h, 0)
    fetch_batch<T, NVD, 1>(buf, static_cast<const T*>(L.wo), HD, 0, min(nbuf<T>() / NVD, sD.nw(wid)), rowD);
    if (jpart == 0) self_attention_head<T>(a, L, h, tag(base + kPhQKV), tag(base + kPhAtt), sm);
    // ---- attention output projection + residual
    load_act<T>(a.ll.at, nullptr, HD, tag(base + kPhAtt), nullptr, xs, red,
                side_x(a.ll.x, first ? a.in : nullptr, x_tag), r0, r1, a.ll.err, a.trace, &tp);
    auto resid_put = [&](int t, const float (&acc)[1][2], int code) {
      const float x0 = __shfl(r0, t, 64), x1 = __shfl(r1, t, 64);
      if (lane == 0)
        LL<T>::put(a.ll.x, sD.row(wid, t), S::rnd(x0 + S::rnd(acc[0][0])), S::rnd(x1 + S::rnd(acc[0][1])),
                   tag(base + code));
    };
    gemv_rows<T, NVD, 1>(buf, static_cast<const T*>(L.wo), HD, sD.nw(wid), rowD, xs,
                         [&](int t, const float (&acc)[1][2]) { resid_put(t, acc, kPhO); });
    x_tag = tag(base + kPhO);
    if constexpr (CROSS) {
      // ---- cross attention: q rows of head h, key-block partials, combine
      fetch_batch<T, NVD, 1>(buf, static_cast<const T*>(L.wq_c), D, 0, min(nbuf<T>() / NVD, ncq), cq_row);
      load_act<T>(a.ll.x, nullptr, D, x_tag, static_cast<const T*>(L.norm_ca), xs, red, no_side, r0, r1, a.ll.err, a.trace, &tp);
        gemv_rows<T, NVD, 1>(buf, static_cast<const T*>(L.wq_c), D, ncq, cq_row, xs,
                           [&](int t, const float (&acc)[1][2]) {
                             if (lane == 0)
                               LL<T>::put(a.ll.q, cq_row(t, 0), S::rnd(acc[0][0]), S::rnd(acc[0][1]),
                                          tag(base + kPhCQ));
                           });
      fetch_batch<T, NVD, 1>(buf, static_cast<const T*>(L.wo_c), HD, 0, min(nbuf<T>() / NVD, sD.nw(wid)), rowD);
      cross_partial<T>(a, L, h, jpart, tag(base + kPhCQ), tag(base + kPhCP), sm);
      if (jpart == 0) cross_combine<T>(a, h, tag(base + kPhCP), tag(base + kPhCC), sm);
      load_act<T>(a.ll.at, nullptr, HD, tag(base + kPhCC), nullptr, xs, red, side_x(a.ll.x, nullptr, x_tag), r0, r1,
                  a.ll.err, a.trace, &tp);
        gemv_rows<T, NVD, 1>(buf, static_cast<const T*>(L.wo_c), HD, sD.nw(wid), rowD, xs,
                           [&](int t, const float (&acc)[1][2]) { resid_put(t, acc, kPhCO); });
      x_tag = tag(base + kPhCO);
    }
    // ---- gated-GELU up projection
    fetch_batch<T, NVD, 2>(buf, static_cast<const T*>(L.w01), D, 0, min(nbuf<T>() / (2 * NVD), sF.nw(wid)), rowF);
    load_act<T>(a.ll.x, nullptr, D, x_tag, static_cast<const T*>(L.norm_ff), xs, red, no_side, r0, r1, a.ll.err, a.trace, &tp);
    gemv_rows<T, NVD, 2>(buf, static_cast<const T*>(L.w01), D, sF.nw(wid), rowF, xs,
                         [&](int t, const float (&acc)[2][2]) {
                           if (lane == 0) {
                             const float g0 = gelu_t<T>(S::rnd(acc[0][0])), g1 = gelu_t<T>(S::rnd(acc[0][1]));
                             LL<T>::put(a.ll.h, sF.row(wid, t), S::rnd(g0 * S::rnd(acc[1][0])),
                                        S::rnd(g1 * S::rnd(acc[1][1])), tag(base + kPhUp));
                           }
                         });
    // ---- down projection + residual
    fetch_batch<T, NVF, 1>(buf, static_cast<const T*>(L.wo2), F, 0, min(nbuf<T>() / NVF, sD.nw(wid)), rowD);
    load_act<T>(a.ll.h, nullptr, F, tag(base + kPhUp), nullptr, xs, red, side_x(a.ll.x, nullptr, x_tag), r0, r1,
                a.ll.err, a.trace, &tp);
    const bool last = li + 1 == a.nlayers;
    if (CROSS && last) {
      // The temporal step's output leaves as plain pairs (no final norm).
      if (blk == 0 && threadIdx.x == 0) astore(a.ll.seq, ep + 1u);  // every workgroup has started
      gemv_rows<T, NVF, 1>(buf, static_cast<const T*>(L.wo2), F, sD.nw(wid), rowD, xs,
                           [&](int t, const float (&acc)[1][2]) {
                             const float x0 = __shfl(r0, t, 64), x1 = __shfl(r1, t, 64);
                             if (lane == 0)
                               st_g(static_cast<W*>(a.out) + sD.row(wid, t),
                                    PT::pack(S::rnd(x0 + S::rnd(acc[0][0])), S::rnd(x1 + S::rnd(acc[0][1]))));
                           });
    } else {
      gemv_rows<T, NVF, 1>(buf, static_cast<const T*>(L.wo2), F, sD.nw(wid), rowD, xs,
                           [&](int t, const float (&acc)[1][2]) { resid_put(t, acc, kPhDn); });
    }
    x_tag = tag(base + kPhDn);
    if (!last)
      fetch_batch<T, NVD, 1>(buf, static_cast<const T*>(a.layers[li + 1].wqkv), D, 0, min(nbuf<T>() / NVD, nqkv),
                             qkv_row);
  }

  if constexpr (!CROSS) {
    // ---- decoder_norm + lm_head rows (model.cpp:652-653)
    const RowSplit sH(a.head_rows, G, blk);
    auto rowH = [&](int t, int) { return sH.row(wid, t); };
    fetch_batch<T, NVD, 1>(buf, static_cast<const T*>(a.head_w), D, 0, min(nbuf<T>() / NVD, sH.nw(wid)), rowH);
    load_act<T>(a.ll.x, nullptr, D, x_tag, static_cast<const T*>(a.dec_norm), xs, red, no_side, r0, r1, a.ll.err, a.trace, &tp);
    if (blk == 0 && threadIdx.x == 0) astore(a.ll.seq, ep + 1u);  // every workgroup has started
    gemv_rows<T, NVD, 1>(buf, static_cast<const T*>(a.head_w), D, sH.nw(wid), rowH, xs,
                         [&](int t, const float (&acc)[1][2]) {
                           if (lane == 0) {
                             const int n = sH.row(wid, t);
                             astore(a.ll.logit + n, ll_word(__float_as_uint(S::rnd(acc[0][0])), tag(kPhHead)));
                             astore(a.ll.logit + a.head_rows + n,
                                    ll_word(__float_as_uint(S::rnd(acc[0][1])), tag(kPhHead)));
                           }
                         });
    if (blk == 0) {
      // ---- gather the logits, copy them out, sample
      float* lg = xs;  // 2 * head_rows floats when head_rows <= kMaxPersistK
      const int n2 = 2 * a.head_rows;
      const uint32_t tg = tag(kPhHead);
      uint32_t spins = 0;
      __syncthreads();  // xs is no longer read by the head GEMV
      for (int base_i = 0; base_i < n2; base_i += kPersistThreads * 8) {
        uint64_t w[8];
        uint32_t pend = 0;
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (base_i + (int)threadIdx.x + u * kPersistThreads < n2) pend |= 1u << u;
        while (pend != 0) {
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if ((pend >> u) & 1u) w[u] = aload(a.ll.logit + base_i + threadIdx.x + u * kPersistThreads);
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            if (((pend >> u) & 1u) && ll_tag(w[u]) == tg) {
              const int i = base_i + threadIdx.x + u * kPersistThreads;
              const float v = __uint_as_float(static_cast<uint32_t>(w[u]));
              if (i < 2 * kMaxPersistK) lg[i] = v;
              if (a.logits) st_g(a.logits + i, v);
              if (a.rec_slice) st_g(a.rec_slice + i, v);
              pend &= ~(1u << u);
            }
          }
          if (pend == 0 || spin_failed(spins, a.ll.err)) break;
          __builtin_amdgcn_s_sleep(1);
        }
      }
      __syncthreads();
      trace_point(a.trace, kTraceEnd);
      if (a.do_sample && wid == 0) sample_and_feed<T>(a, lg);
    }
  } else {
    trace_point(a.trace, kTraceEnd);
  }
  trace_point(a.trace, kTraceDone);
}

template <typename T>
__global__ void k_rows_to_pairs(const T* __restrict__ rows, int D, typename PairT<T>::W* __restrict__ pairs) {
  for (int d = blockIdx.x * blockDim.x + threadIdx.x; d < D; d += gridDim.x * blockDim.x)
    pairs[d] = PairT<T>::pack(St<T>::ld(rows[d]), St<T>::ld(rows[D + d]));
}

template <typename T>
__global__ void k_pairs_to_rows(const typename PairT<T>::W* __restrict__ pairs, int D, T* __restrict__ rows) {
  for (int d = blockIdx.x * blockDim.x + threadIdx.x; d < D; d += gridDim.x * blockDim.x) {
    const auto w = pairs[d];
    rows[d] = St<T>::st(PairT<T>::lo(w));
    rows[D + d] = St<T>::st(PairT<T>::hi(w));
  }
}

template <typename T>
__global__ void k_embed_pairs(const T* __restrict__ emb, int D, int id, typename PairT<T>::W* __restrict__ pairs) {
  for (int d = blockIdx.x * blockDim.x + threadIdx.x; d < D; d += gridDim.x * blockDim.x) {
    const float e = St<T>::ld(emb[(size_t)id * D + d]);
    pairs[d] = PairT<T>::pack(e, e);
  }
}

}  // namespace

int persist_grid(int H, int num_cu, int* bph_out) {
  int bph = kMaxBph;
  while (bph > 1 && H * bph > num_cu) bph /= 2;
  if (bph < 8 || H * bph > num_cu) return 0;
  if (bph_out) *bph_out = bph;
  return H * bph;
}

void launch_step(DType dt, const StepArgs& a, int grid, hipStream_t s) {
  if (dt == DType::F32) {
    if (a.cross)
      hipLaunchKernelGGL((k_step<float, true>), dim3(grid), dim3(kPersistThreads), 0, s, a);
    else
      hipLaunchKernelGGL((k_step<float, false>), dim3(grid), dim3(kPersistThreads), 0, s, a);
  } else {
    if (a.cross)
      hipLaunchKernelGGL((k_step<bf16, true>), dim3(grid), dim3(kPersistThreads), 0, s, a);
    else
      hipLaunchKernelGGL((k_step<bf16, false>), dim3(grid), dim3(kPersistThreads), 0, s, a);
  }
  MRT_HIP_CHECK(hipGetLastError());
}

void rows_to_pairs(DType dt, const void* rows, int D, void* pairs, hipStream_t s) {
  const int blocks = (D + 255) / 256;
  if (dt == DType::F32)
    hipLaunchKernelGGL(k_rows_to_pairs<float>, dim3(blocks), dim3(256), 0, s, (const float*)rows, D,
                       (uint64_t*)pairs);
  else
    hipLaunchKernelGGL(k_rows_to_pairs<bf16>, dim3(blocks), dim3(256), 0, s, (const bf16*)rows, D,
                       (uint32_t*)pairs);
  MRT_HIP_CHECK(hipGetLastError());
}

void pairs_to_rows(DType dt, const void* pairs, int D, void* rows, hipStream_t s) {
  const int blocks = (D + 255) / 256;
  if (dt == DType::F32)
    hipLaunchKernelGGL(k_pairs_to_rows<float>, dim3(blocks), dim3(256), 0, s, (const uint64_t*)pairs, D,
                       (float*)rows);
  else
    hipLaunchKernelGGL(k_pairs_to_rows<bf16>, dim3(blocks), dim3(256), 0, s, (const uint32_t*)pairs, D,
                       (bf16*)rows);
  MRT_HIP_CHECK(hipGetLastError());
}

void embed_pairs(DType dt, const void* emb, int D, int id, void* pairs, hipStream_t s) {
  const int blocks = (D + 255) / 256;
  if (dt == DType::F32)
    hipLaunchKernelGGL(k_embed_pairs<float>, dim3(blocks), dim3(256), 0, s, (const float*)emb, D, id,
                       (uint64_t*)pairs);
  else
    hipLaunchKernelGGL(k_embed_pairs<bf16>, dim3(blocks), dim3(256), 0, s, (const bf16*)emb, D, id,
                       (uint32_t*)pairs);
  MRT_HIP_CHECK(hipGetLastError());
}

}  // namespace mrt
