// Persistent step kernels for gfx950: one launch runs a whole depth_step
// (4 decoder layers + decoder_norm + level-sliced lm_head + CFG/top-k sampling
// + token feedback) or a whole temporal_step (20 layers with cross attention).
//
// Grid = H * bph workgroups (one per CU: 256 on MI355X), 4 waves each.  The
// phases of a step hand data to each other through 64-bit words {payload,
// tag} written and read with agent-scope atomics, which are coherent across
// the 8 XCDs without cache maintenance.  A consumer polls the words it needs
// until each carries the tag of the producing phase of this launch (tag =
// launch epoch << 12 | phase code), so a hand-off costs one store -> load
// propagation and needs no counters, barriers or store drains.  The epoch is
// a device counter that workgroup 0 advances once it has seen data from every
// workgroup, so graph replays never match stale words.
//
// Every buffer is rewritten only after all of its readers have consumed it:
// each phase's inputs depend on outputs of every workgroup of the previous
// phase, which those workgroups produce only after finishing their reads.
//
// Latency hiding:
//   * weights of the next phase are loaded into registers (16-byte loads)
//     as soon as the current phase's outputs are stored, so HBM latency
//     overlaps the wait for the next phase's inputs;
//   * every weight, norm and cache address is a scalar function of the kernel
//     arguments (stacked per-kind layer layout), so no load waits on a
//     pointer fetched from memory;
//   * the self-attention ring history and the cross-attention K/V block of a
//     layer are copied global -> LDS with direct (register-less) 16-byte
//     loads at the start of the layer, long before they are read;
//   * cross-lane sums and maxima use DPP row operations, top-k counting uses
//     wave ballots.
// Temporal weights (streamed once per frame) use non-temporal loads so that
// they do not displace the depth stack, which every depth step re-reads,
// from the last-level cache.
//
// Work split per phase (H=16, bph=16, G=256):
//   QKV:   workgroup (h, j) owns rows 4j..4j+3 of head h's q, k and v;
//          workgroup (h, 0) then runs head h's attention over the ring.
//   O / FFN-down / cross-O / head: ceil(N / G) rows per workgroup.
//   FFN-up: ceil(d_ff / G) gate/up row pairs per workgroup.
//   cross:  workgroup (h, j) owns head h's q rows 4j.., then computes the
//          softmax partial of key block j (ceil(S / bph) keys); workgroup
//          (h, 0) combines the bph partials.
#include <mutex>
#include <algorithm>
#include <cmath>

#include "device_utils.hpp"
#include "persist.hpp"
#include "draw_block.hpp"


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

// 16-byte weight load: non-temporal for the temporal stack.
template <bool NT>
__device__ __forceinline__ uint4 ld_w16(const void* p) {
  if constexpr (NT)
    return ld_nt16(p);
  else
    return ld_g16(p);
}

// Direct global -> LDS copy: lane l's 16 bytes from `g` land at lds + 16 l.
__device__ __forceinline__ void lds_copy16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds((const MRT_GLOBAL void*)g, (MRT_LDS void*)lds, 16, 0, 0);
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Selects one of three values.  Taking the operands by value keeps the
// selection off member addresses of the kernel arguments, which would force
// a private-memory copy of the argument block.
template <typename P>
__device__ __forceinline__ P pick3(int i, P p0, P p1, P p2) {
  return i == 0 ? p0 : i == 1 ? p1 : p2;
}

// Waits n rounds of s_sleep(1) (64 clocks each) before a hand-off's first poll:
// polls issued before the producers' stores can have landed only congest the
// memory side and delay the words they wait for.
__device__ __forceinline__ void poll_wait(int n) {
  for (int i = 0; i < n; ++i) __builtin_amdgcn_s_sleep(1);
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

// ---- DPP wave reductions (all 64 lanes active; result is wave-uniform) -----------

__device__ __forceinline__ float dpp_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, true));   // quad [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, true));   // quad [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, true));  // row_shr:4
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, true));  // row_shr:8
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, true));  // row_bcast:15
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, true));  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ---- transposed wave sums ----------------------------------------------------------
//
// N values per lane are summed over the 64 lanes by a butterfly that halves
// the value list at each lane bit (5, 4, 3, 2, 1, 0) while it doubles the
// lanes each partial covers: lanes with the bit clear keep the first half,
// lanes with it set the second half (the list padded with zeros to an even
// length), and each adds what its partner across the bit sends.  Once one
// value is left, the remaining bits add the partner's copy.  N values cost
// about N + log2(64) exchanges instead of 6 N, and the exchanges of one step
// are independent.  Bits 5 and 4 exchange with v_permlane32_swap /
// v_permlane16_swap, bits 3..0 with DPP (row mirror, half-row mirror, quad
// permutes); every DPP source lane lies in the same 16-lane row.

// Lane bit M's partner value (M <= 8).
template <int M>
__device__ __forceinline__ float dpp_partner(float v) {
  constexpr int ctrl = M == 8 ? 0x140 : M == 4 ? 0x141 : M == 2 ? 0x4E : 0xB1;
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xf, 0xf, false));
}

// For M = 32 or 16: a[l] + a[l ^ M] on lanes whose bit M is clear, b[l ^ M] +
// b[l] on the others (with a == b: the pair sum on every lane).
template <int M>
__device__ __forceinline__ float swap_add(float a, float b) {
  if constexpr (M == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    static_assert(M == 16, "swap_add: lane bit 5 or 4");
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// One butterfly step over lane bit M on a list of L values.
template <int M, int L, int NMAX>
__device__ __forceinline__ void tsum_step(float (&v)[NMAX]) {
  if constexpr (L == 1) {
    if constexpr (M >= 16)
      v[0] = swap_add<M>(v[0], v[0]);
    else
      v[0] += dpp_partner<M>(v[0]);
  } else {
    constexpr int H = (L + 1) / 2;
    const bool hi = (threadIdx.x & M) != 0;
#pragma unroll
    for (int j = 0; j < H; ++j) {
      const float a = v[j], b = j + H < L ? v[j + H] : 0.f;
      if constexpr (M >= 16) {
        v[j] = swap_add<M>(a, b);
      } else {
        const float keep = hi ? b : a, send = hi ? a : b;
        v[j] = keep + dpp_partner<M>(send);
      }
    }
  }
}

constexpr int half_up(int n) { return (n + 1) / 2; }

// Sums each of v[0..N) over the wave; on return v[0] of every lane is the
// total of one value slot (or of padding, zero); tsum_lane locates slot s.
template <int N, int NMAX>
__device__ __forceinline__ void tsum(float (&v)[NMAX]) {
  constexpr int L1 = half_up(N), L2 = half_up(L1), L3 = half_up(L2), L4 = half_up(L3), L5 = half_up(L4);
  tsum_step<32, N>(v);
  tsum_step<16, L1>(v);
  tsum_step<8, L2>(v);
  tsum_step<4, L3>(v);
  tsum_step<2, L4>(v);
  tsum_step<1, L5>(v);
}

// A lane that holds the total of value slot s (s < N) after tsum<N>: the
// halves are taken greedily, so the lane never lands on padding.
template <int N>
__host__ __device__ constexpr int tsum_lane(int s) {
  int l = 0, n = N;
  for (int m = 32; m >= 1; m >>= 1) {
    if (n > 1) {
      const int h = (n + 1) / 2;
      if (s >= h) {
        s -= h;
        l |= m;
      }
      n = h;
    }
  }
  return l;
}

// 1/sqrt(x) for x > 0: the hardware estimate refined by one Newton-Raphson
// step, y (1.5 - x y^2 / 2), to about 1 ulp.
__device__ __forceinline__ float rsqrt_nr(float x) {
  const float y = __builtin_amdgcn_rsqf(x);
  return y * fmaf(-0.5f * x * y, y, 1.5f);
}

// Value of `v` held by lane `src` (src - lane is wave-uniform): the lane's own
// value when they coincide (no LDS round trip), else a lane shuffle.
__device__ __forceinline__ float from_lane(float v, int src) {
  if (uniform(src - (int)(threadIdx.x & 63)) == 0) return v;
  return __shfl(v, src & 63, 64);
}

// ---- tagged words -------------------------------------------------------------------

__device__ __forceinline__ uint64_t ll_word(uint32_t payload, uint32_t tag) {
  return ((uint64_t)tag << 32) | payload;
}
__device__ __forceinline__ uint32_t ll_tag(uint64_t w) { return static_cast<uint32_t>(w >> 32); }

// Element k (both rows) of a tagged vector: 16-bit types -> one word (row r
// in payload bits 16r..16r+15), fp32 -> one word per row (row 1 at
// +kMaxPersistK).
template <typename T>
struct LL {
  static_assert(sizeof(T) == 2, "16-bit storage types");
  static constexpr int kWords = 1;
  __device__ static int idx(int k, int) { return k; }
  __device__ static void put(uint64_t* b, int k, float v0, float v1, uint32_t tag) {
    astore(b + k, ll_word(St<T>::bits(v0) | (St<T>::bits(v1) << 16), tag));
  }
  __device__ static float get(const uint64_t (&w)[1], int r) {
    return St<T>::unbits((static_cast<uint32_t>(w[0]) >> (16 * r)) & 0xffffu);
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
  const void* plain;  // (2, stride) model-dtype rows
  uint32_t tag;
  int row;  // -1: nothing for this thread
  int stride;
};

// Activation rows in LDS, stored in the model dtype (row 1 at +kMaxPersistK
// elements): 16-bit rows feed v_dot2_f32_bf16 / v_dot2_f32_f16 directly.
template <typename T>
struct Act {
  __device__ static void put(float* xs, int k, float v0, float v1) {
    T* x = reinterpret_cast<T*>(xs);
    x[k] = St<T>::st(v0);
    x[kMaxPersistK + k] = St<T>::st(v1);
  }
  __device__ static float get(const float* xs, int r, int k) {
    return St<T>::ld(reinterpret_cast<const T*>(xs)[r * kMaxPersistK + k]);
  }
};

// Polls elements k = tid + 256 i (i < NPER, k < K) of a tagged vector until
// each word carries `tag`.  KEEP: both rows of element i go to v0[i] / v1[i];
// otherwise they are stored to activation element k in LDS as they arrive.
// The side element (if any) is returned in r0/r1.  All loads of one round are
// issued before any is waited for.
template <typename T, int NPER, bool KEEP>
__device__ __forceinline__ void ll_load_vec(const uint64_t* src, int K, uint32_t tag, float* xs,
                                            float (&v0)[NPER], float (&v1)[NPER], const Side& sd, float& r0,
                                            float& r1, int* err, int delay) {
  constexpr int NW = LL<T>::kWords;
  const int tid = threadIdx.x;
  uint64_t w[NPER][NW];
  uint64_t sw[NW];
  uint32_t pend = 0;
#pragma unroll
  for (int i = 0; i < NPER; ++i)
    if (src != nullptr && tid + i * kPersistThreads < K) pend |= 1u << i;
  bool side_pend = sd.row >= 0 && sd.plain == nullptr;
  if (sd.row >= 0 && sd.plain != nullptr) {
    const T* p = static_cast<const T*>(sd.plain);
    r0 = St<T>::ld(ld_g(p + sd.row));
    r1 = St<T>::ld(ld_g(p + sd.stride + sd.row));
  }
  uint32_t spins = 0;
  if (pend != 0 || side_pend) poll_wait(delay);
  while (pend != 0 || side_pend) {
#pragma unroll
    for (int i = 0; i < NPER; ++i)
      if ((pend >> i) & 1u)
#pragma unroll
        for (int r = 0; r < NW; ++r) w[i][r] = aload(src + LL<T>::idx(tid + i * kPersistThreads, r));
    if (side_pend)
#pragma unroll
      for (int r = 0; r < NW; ++r) sw[r] = aload(sd.ll + LL<T>::idx(sd.row, r));
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      if ((pend >> i) & 1u) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < NW; ++r) ok = ok && ll_tag(w[i][r]) == tag;
        if (ok) {
          if constexpr (KEEP) {
            v0[i] = LL<T>::get(w[i], 0);
            v1[i] = LL<T>::get(w[i], 1);
          } else {
            Act<T>::put(xs, tid + i * kPersistThreads, LL<T>::get(w[i], 0), LL<T>::get(w[i], 1));
          }
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

constexpr int kLoadTrace = 400;  // start of the first 16 activation loads
constexpr int kWaveTrace = 420;  // per-wave poll completion of the first 16 loads
constexpr int kDrawTrace = 490;  // 7 points inside a draw

__device__ __forceinline__ void trace_point(uint64_t* trace, int slot) {
  if (trace != nullptr && blockIdx.x == 0 && threadIdx.x == 0 && slot < kLoadTrace) trace[slot] = wall_clock64();
}

// Norm weights of the elements a thread owns in load_act (k = tid + 256 i),
// loaded into registers ahead of the weight prefetch of the phase that uses
// them and kept raw (model dtype) so that nothing waits for the load before
// the norm; elements past K are masked there.
template <typename T, int NPER>
struct Gamma {
  T g[NPER];
  __device__ float get(int i, int K) const {
    return threadIdx.x + i * kPersistThreads < K ? St<T>::ld(g[i]) : 0.f;
  }
};

template <typename T, int NPER>
__device__ __forceinline__ void load_gamma(const T* g, int K, Gamma<T, NPER>& out) {
#pragma unroll
  for (int i = 0; i < NPER; ++i) out.g[i] = ld_g(g + min((int)threadIdx.x + i * kPersistThreads, K - 1));
}

// Loads the activation vector of a phase (K <= 256 * NPER elements; tagged,
// or plain input rows) into LDS, with an optional side element.
// NORM: RMS norm with the weights gk (modules.cpp:72-84): the sum of squares
// is taken from the polled values in registers, and each element is written
// to LDS once, normalised (zero past K, where the GEMV meets zero weights).
template <typename T, int NPER, bool NORM>
__device__ __forceinline__ void load_act(const uint64_t* ll, const void* plain, int K, uint32_t tag,
                                         const Gamma<T, NPER>& gk, float* xs, float* red, const Side& sd, float& r0,
                                         float& r1, int* err, int delay, uint64_t* trace, int& tp, int& lc, int stride) {
  using S = St<T>;
  const int tid = threadIdx.x;
  if (trace != nullptr && blockIdx.x == 0 && tid == 0 && lc < 16) trace[kLoadTrace + lc] = wall_clock64();
  trace_point(trace, tp++);
  float v0[NPER], v1[NPER];
#pragma unroll
  for (int i = 0; i < NPER; ++i) v0[i] = v1[i] = 0.f;
  if (plain != nullptr) {  // two model-dtype rows, row 1 at +stride (0: the same row twice)
    const T* p = static_cast<const T*>(plain);
    T w0[NPER], w1[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const int k = min(tid + i * kPersistThreads, K - 1);
      w0[i] = ld_g(p + k);
      w1[i] = ld_g(p + stride + k);
    }
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const bool in = tid + i * kPersistThreads < K;
      v0[i] = in ? S::ld(w0[i]) : 0.f;
      v1[i] = in ? S::ld(w1[i]) : 0.f;
      if constexpr (!NORM) Act<T>::put(xs, tid + i * kPersistThreads, v0[i], v1[i]);
    }
    ll_load_vec<T, NPER, NORM>(nullptr, 0, 0, xs, v0, v1, sd, r0, r1, err, delay);
  } else {
    ll_load_vec<T, NPER, NORM>(ll, K, tag, xs, v0, v1, sd, r0, r1, err, delay);
  }
  if (trace != nullptr && blockIdx.x == 0 && (tid & 63) == 0 && lc < 16) trace[kWaveTrace + 4 * lc + (tid >> 6)] = wall_clock64();
  ++lc;
  trace_point(trace, tp++);
  if constexpr (NORM) {
    const float inv_k = 1.0f / (float)K;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < NPER; ++i) {  // zero past K
      s0 = fmaf(v0[i], v0[i], s0);
      s1 = fmaf(v1[i], v1[i], s1);
    }
    // both rows' wave sums at once: row 0's total in lanes 0..31, row 1's in 32..63
    float t[2] = {s0, s1};
    tsum<2>(t);
    const int wid = tid >> 6;
    if ((tid & 31) == 0) red[4 * ((tid >> 5) & 1) + wid] = t[0];
    __syncthreads();
    const float4 ra = *reinterpret_cast<const float4*>(red);
    const float4 rb = *reinterpret_cast<const float4*>(red + 4);
    const float inv0 = rsqrt_nr((ra.x + ra.y + ra.z + ra.w) * inv_k + 1e-6f);
    const float inv1 = rsqrt_nr((rb.x + rb.y + rb.z + rb.w) * inv_k + 1e-6f);
#pragma unroll
    for (int i = 0; i < NPER; ++i) {  // gamma is zero past K
      const float g = gk.get(i, K);
      Act<T>::put(xs, tid + i * kPersistThreads, S::rnd(S::rnd(v0[i] * inv0) * g), S::rnd(S::rnd(v1[i] * inv1) * g));
    }
  }
  __syncthreads();
  trace_point(trace, tp++);
}

// ---- GEMV machinery ---------------------------------------------------------------

constexpr int kNBuf = 12;  // 16-byte weight registers per thread

// Loads the rows of one batch (R rows of P parts; row indices wave-uniform)
// into registers; 16-byte chunks past the end of a row are zero.  (The zero
// fill makes the compiler wait for older memory operations of the wave before
// each row -- the previous phase's result stores too, a store round trip --
// so at most a few loads per wave are in flight at a time.  Unconditional
// loads with no such waits measured slower: with vmcnt in order, the next
// poll then queues behind every weight load of the phase.)
template <typename T, int NV, int P, bool NT, class RowOf>
__device__ __forceinline__ void fetch_batch(uint4 (&buf)[kNBuf], const T* W, int K, int b0, int nb, RowOf row_of) {
  constexpr int V = St<T>::kVec;
  constexpr int R = kNBuf / (P * NV);
  const int lane = threadIdx.x & 63;
  const int nch = K / V;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r < nb) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const T* row = W + (size_t)row_of(b0 + r, p) * K;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int c = lane + 64 * i;
          uint4 v = make_uint4(0u, 0u, 0u, 0u);
          if (c < nch) v = ld_w16<NT>(row + (size_t)c * V);
          buf[(r * P + p) * NV + i] = v;
        }
      }
    }
  }
}

// acc += w . x over one 16-byte chunk (8 16-bit or 4 fp32 elements).
template <typename T>
struct Dot;
template <>
struct Dot<bf16> {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  __device__ static float d2(uint32_t w, uint32_t x, float a) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, w), __builtin_bit_cast(bf2, x), a, false);
  }
  __device__ static float acc(float a, const uint4& w, const uint4& x) {
    a = d2(w.x, x.x, a);
    a = d2(w.y, x.y, a);
    a = d2(w.z, x.z, a);
    return d2(w.w, x.w, a);
  }
};
template <>
struct Dot<f16> {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  __device__ static float d2(uint32_t w, uint32_t x, float a) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w), __builtin_bit_cast(h2, x), a, false);
  }
  __device__ static float acc(float a, const uint4& w, const uint4& x) {
    a = d2(w.x, x.x, a);
    a = d2(w.y, x.y, a);
    a = d2(w.z, x.z, a);
    return d2(w.w, x.w, a);
  }
};
template <>
struct Dot<float> {
  __device__ static float acc(float a, const uint4& w, const uint4& x) {
    a = fmaf(__uint_as_float(w.x), __uint_as_float(x.x), a);
    a = fmaf(__uint_as_float(w.y), __uint_as_float(x.y), a);
    a = fmaf(__uint_as_float(w.z), __uint_as_float(x.z), a);
    return fmaf(__uint_as_float(w.w), __uint_as_float(x.w), a);
  }
};

// Dots of a batch against the two activation rows (model dtype in LDS; the
// weight chunks are zero past every row's end, where they meet finite
// activations).  epi(t, active, sums[P][2]) runs once on every lane: lane r
// holds the sums of the batch's row r (wave-local row index t = b0 + r) and
// is active when that row exists.
template <typename T, int NV, int P, class Epi>
__device__ __forceinline__ void dot_batch(const uint4 (&buf)[kNBuf], int b0, int nb, const float* xs, Epi epi) {
  constexpr int V = St<T>::kVec;
  constexpr int R = kNBuf / (P * NV);
  const int lane = threadIdx.x & 63;
  const T* xt = reinterpret_cast<const T*>(xs);
  float acc[R][P][2];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p) acc[r][p][0] = acc[r][p][1] = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    const uint4 x0 = *reinterpret_cast<const uint4*>(xt + c * V);
    const uint4 x1 = *reinterpret_cast<const uint4*>(xt + kMaxPersistK + c * V);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r < nb) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const uint4& w = buf[(r * P + p) * NV + i];
          acc[r][p][0] = Dot<T>::acc(acc[r][p][0], w, x0);
          acc[r][p][1] = Dot<T>::acc(acc[r][p][1], w, x1);
        }
      }
    }
  }
  // Row r's sums go to lane r, so the epilogue runs once for all rows.  The
  // 2P sums of every row are reduced together (transposed), value k = (r P +
  // p) 2 + c; rows past nb hold zeros.  A single row reduces its 2P values only.
  float v[P][2];
  if (nb == 1) {
    float t[2 * P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      t[2 * p] = acc[0][p][0];
      t[2 * p + 1] = acc[0][p][1];
    }
    tsum<2 * P>(t);
    // each total sits in a known lane: read it into a scalar, no LDS round trip
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        v[p][c] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[0]), tsum_lane<2 * P>(2 * p + c)));
  } else {
    constexpr int N = 2 * P * R;
    float t[N];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        t[(r * P + p) * 2] = acc[r][p][0];
        t[(r * P + p) * 2 + 1] = acc[r][p][1];
      }
    tsum<N>(t);
    const int row = min(lane, R - 1);
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int c = 0; c < 2; ++c) v[p][c] = __shfl(t[0], tsum_lane<N>((row * P + p) * 2 + c), 64);
  }
  epi(b0 + lane, lane < nb, v);
}

// Runs a wave's nw rows in batches; the first batch is already in buf.
template <typename T, int NV, int P, bool NT, class RowOf, class Epi>
__device__ __forceinline__ void gemv_rows(uint4 (&buf)[kNBuf], const T* W, int K, int nw, RowOf row_of,
                                          const float* xs, Epi epi) {
  constexpr int R = kNBuf / (P * NV);
  for (int b0 = 0; b0 < nw; b0 += R) {
    const int nb = min(R, nw - b0);
    if (b0 > 0) fetch_batch<T, NV, P, NT>(buf, W, K, b0, nb, row_of);
    dot_batch<T, NV, P>(buf, b0, nb, xs, epi);
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
__device__ __forceinline__ void ll_load_small(const uint64_t* src, int n, uint32_t tag, float* dst0, float* dst1,
                                              int* err, int delay) {
  constexpr int NW = LL<T>::kWords;
  const int tid = threadIdx.x;
  if (tid >= n) return;
  uint64_t w[NW];
  uint32_t spins = 0;
  poll_wait(delay);
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

// ---- attention ------------------------------------------------------------------

// LDS staging of one layer's attention operands, raw model dtype:
// region (kind, row) = 64 slots x 64 elements, kind 0 = K, 1 = V.
constexpr int kRegion = 64 * 64;

// K slots are kept in LDS rotated by 16-byte chunk: chunk c of slot j sits at
// chunk (c + j) mod kChunks<T>, so the lanes of a score loop (lane = slot)
// reading their chunk i at the same step hit different banks.
template <typename T>
constexpr int kChunks = 64 * (int)sizeof(T) / 16;  // 16-byte chunks per slot
template <typename T>
__device__ __forceinline__ int krot(int slot, int chunk) {
  return (chunk + slot) & (kChunks<T> - 1);
}

// Copies `n` (<= 64) consecutive 64-element slots starting at `src` into an
// LDS region with the calling wave; `lim` bytes from src are readable.  ROT:
// store the slots rotated (K).  The LDS destination of a lane is fixed by the
// instruction (16 bytes per lane), so the rotation picks the source chunk.
// Lanes past the n slots do not copy, so the region from slot n on is left
// as it is (the attention writes the current slot there meanwhile).
template <typename T, bool ROT>
__device__ __forceinline__ void stage_slots(const T* src, int n, long lim, T* region) {
  constexpr int kRow = 64 * (int)sizeof(T);
  const int lane = threadIdx.x & 63;
  const int bytes = n * kRow;
  for (int off = 0; off < bytes; off += 1024) {
    long o = off + lane * 16;
    if (o < bytes) {
      if constexpr (ROT) {
        const int j = (int)(o / kRow), pch = (int)(o % kRow) / 16;  // slot, stored chunk
        o = (long)j * kRow + ((pch - j) & (kChunks<T> - 1)) * 16;
      }
      o = min(o, lim - 16);
      lds_copy16(reinterpret_cast<const char*>(src) + o, reinterpret_cast<char*>(region) + off);
    }
  }
}

// sum_{j < n} p[j] * v[64 j] + init: four independent partial sums over
// float4 reads of p, so eight LDS loads are in flight per step.
template <typename T>
__device__ __forceinline__ float pv_sum(const float* p, const T* v, int n, float init) {
  using S = St<T>;
  float o0 = init, o1 = 0.f, o2 = 0.f, o3 = 0.f;
  int j = 0;
  for (; j + 8 <= n; j += 8) {
    const float4 pa = *reinterpret_cast<const float4*>(p + j);
    const float4 pb = *reinterpret_cast<const float4*>(p + j + 4);
    float w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = S::ld(v[(j + u) * 64]);
    o0 = fmaf(pa.x, w[0], o0);
    o1 = fmaf(pa.y, w[1], o1);
    o2 = fmaf(pa.z, w[2], o2);
    o3 = fmaf(pa.w, w[3], o3);
    o0 = fmaf(pb.x, w[4], o0);
    o1 = fmaf(pb.y, w[5], o1);
    o2 = fmaf(pb.z, w[6], o2);
    o3 = fmaf(pb.w, w[7], o3);
  }
  for (; j < n; ++j) o0 = fmaf(p[j], S::ld(v[j * 64]), o0);
  return (o0 + o1) + (o2 + o3);
}

// Self attention of head h over ring slots 0..pos (scale 1.0, additive bias;
// modules.cpp:243-295).  q and slot pos come as tagged words of this launch;
// slots before pos are in LDS, region (kind, row) = `cap` slots x 64 at hist
// + (kind * 2 + row) * cap * 64 (kind 0 = K, 1 = V).  They were staged there
// from the global ring (slots written by earlier launches) or, `resident`,
// written by this function at earlier steps of the same launch.  Slot pos is
// written there too, so every key is read the same way.  `pbias`: lane j's
// bias for key j (j <= pos) in waves 0 and 1, loaded ahead (attn_bias).
// `qkv_row` non-null: q, k and v of both rows are that table row's (the
// layer-0 projection of a known token), loaded instead of polled, and slot
// pos of the global ring (`ring`: this layer's K, V at +eRing) is written here.
template <typename T>
__device__ __forceinline__ void self_attention_head(const StepArgs& a, int pos, int h, uint32_t tag, uint32_t out_tag,
                                                    T* hist, int cap, bool resident, float pbias, float* sm,
                                                    const T* qkv_row = nullptr, T* ring = nullptr,
                                                    size_t eRing = 0) {
  using S = St<T>;
  constexpr int V = S::kVec;
  float* qs = sm;        // [2][64]
  float* ps = sm + 384;  // [2][64]
  float* os = sm + 512;  // [2][64]
  const int tid = threadIdx.x, wid = uniform(tid >> 6), lane = tid & 63;
  const int len = pos + 1, rs = cap * 64;
  if (wid < 3) {  // waves 0, 1, 2 fetch q, k, v of head h
    float* d = sm + wid * 128;
    float v0, v1;
    if (qkv_row != nullptr) {
      const T e = ld_g(qkv_row + wid * a.HD + h * 64 + lane);
      v0 = v1 = S::ld(e);
      if (wid > 0) {  // the global ring slot of both rows (read by later launches)
        T* slot = ring + (wid - 1) * eRing + ((size_t)h * a.Lmax + pos) * 64 + lane;
        st_g(slot, e);
        st_g(slot + (size_t)a.H * a.Lmax * 64, e);
      }
    } else {
      const uint64_t* src = pick3<const uint64_t*>(wid, a.ll.q, a.ll.k, a.ll.v) + h * 64;
      constexpr int NW = LL<T>::kWords;
      uint64_t w[NW];
      uint32_t spins = 0;
      poll_wait(a.ll.delay[kPollAttn]);
      for (;;) {
#pragma unroll
        for (int r = 0; r < NW; ++r) w[r] = aload(src + LL<T>::idx(lane, r));
        bool ok = true;
#pragma unroll
        for (int r = 0; r < NW; ++r) ok = ok && ll_tag(w[r]) == tag;
        if (ok || spin_failed(spins, a.ll.err)) break;
        __builtin_amdgcn_s_sleep(1);
      }
      v0 = LL<T>::get(w, 0);
      v1 = LL<T>::get(w, 1);
    }
    if (wid == 0) {
      d[lane] = v0;
      d[64 + lane] = v1;
    } else {  // slot pos of K (wave 1, rotated) / V (wave 2), read below and, resident, by later steps
      const int e = wid == 1 ? krot<T>(pos, lane / V) * V + lane % V : lane;
      T* slot = hist + ((wid - 1) * 2) * rs + pos * 64 + e;
      slot[0] = S::st(v0);
      slot[rs] = S::st(v1);
    }
  }
  if (!resident) __builtin_amdgcn_s_waitcnt(0);  // this wave's history copies have landed
  __syncthreads();
  if (wid < 2) {
    const int b = wid;
    float sc = -INFINITY;
    if (lane < len) {
      const T* kr = hist + b * rs + lane * 64;
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 64 / V; ++i) {
        const uint4 kv = *reinterpret_cast<const uint4*>(kr + krot<T>(lane, i) * V);
        const T* ke = reinterpret_cast<const T*>(&kv);
#pragma unroll
        for (int e = 0; e < V; ++e) acc = fmaf(qs[b * 64 + i * V + e], S::ld(ke[e]), acc);
      }
      sc = acc + pbias;
    }
    const float m = dpp_max(sc);
    const float p = lane < len ? expf(sc - m) : 0.f;
    const float l = dpp_sum(p);
    ps[b * 64 + lane] = p;
    // the same wave reads ps back: LDS operations of a wave complete in order
    const float o = pv_sum<T>(ps + b * 64, hist + (2 + b) * rs + lane, len, 0.f);
    os[b * 64 + lane] = o / l;
  }
  __syncthreads();
  if (tid < 64) LL<T>::put(a.ll.at, h * 64 + tid, os[tid], os[64 + tid], out_tag);
}

// Softmax partial of cross attention: head h, key block j (staged in `cst`),
// both rows.  Waves 2b, 2b+1 take the two halves of row b's keys.
template <typename T>
__device__ __forceinline__ void cross_partial(const StepArgs& a, int h, int j, uint32_t q_tag, uint32_t out_tag,
                                              const T* cst, float* sm) {
  using S = St<T>;
  constexpr int V = S::kVec;
  float* qs = sm;        // [2][64]
  float* ps = sm + 128;  // [4][64]
  float* wo = sm + 384;  // [4][64]
  float* wm = sm + 640;  // [4]
  float* wl = sm + 644;  // [4]
  const int tid = threadIdx.x, wid = uniform(tid >> 6), lane = tid & 63;
  ll_load_small<T>(a.ll.q + h * 64, 64, q_tag, qs, qs + 64, a.ll.err, a.ll.delay[kPollCrossPart]);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's K/V copies have landed
  __syncthreads();
  const int chunk = (a.S + a.bph - 1) / a.bph;
  const int nk = max(0, min(chunk, a.S - j * chunk));
  const int h0 = (nk + 1) / 2;
  const int b = wid >> 1, half = wid & 1;
  const int klo = half ? h0 : 0;
  const int nkh = half ? nk - h0 : h0;
  float sc = -INFINITY;
  if (lane < nkh) {
    const T* kr = cst + b * kRegion + (klo + lane) * 64;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 64 / V; ++i) {
      const uint4 kv = *reinterpret_cast<const uint4*>(kr + krot<T>(klo + lane, i) * V);
      const T* ke = reinterpret_cast<const T*>(&kv);
#pragma unroll
      for (int e = 0; e < V; ++e) acc = fmaf(qs[b * 64 + i * V + e], S::ld(ke[e]), acc);
    }
    sc = acc;
  }
  const float m = dpp_max(sc);
  const float p = (lane < nkh) ? expf(sc - m) : 0.f;
  const float l = dpp_sum(p);
  ps[wid * 64 + lane] = p;
  wo[wid * 64 + lane] = pv_sum<T>(ps + wid * 64, cst + (2 + b) * kRegion + klo * 64 + lane, nkh, 0.f);
  if (lane == 0) {
    wm[wid] = nkh > 0 ? m : -INFINITY;
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
__device__ __forceinline__ void cross_combine(const StepArgs& a, int h, uint32_t tag, uint32_t out_tag, float* sm) {
  float* os = sm;  // [2][64]
  const int tid = threadIdx.x;
  if (tid < 128) {
    const int b = tid >> 6, d = tid & 63;
    uint64_t wm[kMaxBph], wl[kMaxBph], wv[kMaxBph];
    uint32_t pend = (1u << a.bph) - 1u;
    uint32_t spins = 0;
    poll_wait(a.ll.delay[kPollCrossComb]);
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

// ---- sampling -------------------------------------------------------------------

static_assert(kPersistThreads == kDrawThreads, "the frame kernel's draw runs on its whole workgroup");

// The frame kernel's draw of one level (block_draw), then the fed token
// written to `tokens` / `drawn` and published (`tok_word`, tagged, when
// non-null) as soon as it is known.  Returns the fed token (the same in every
// thread).
template <typename T>
__device__ __forceinline__ int sample_block(const SampleParams& p, int level, int slot, const DrawPrefetch& pf,
                                            bool teacher, int* tokens, int* drawn, uint64_t* tok_word,
                                            uint32_t tok_tag, const float* lg, unsigned* hist, int* wres,
                                            uint64_t* trace) {
  const int tid = threadIdx.x;
  auto tpoint = [&](int i) {
    if (trace != nullptr && tid == 0) trace[kDrawTrace + i] = wall_clock64();
  };
  const int arg = block_draw(p, pf, lg, hist, wres, tpoint);
  const int drawn_id = p.codec_offset + level * p.codebook + arg;
  const int fed = teacher ? pf.teacher_id : drawn_id;
  if (tid == 0) {
    if (tok_word != nullptr) astore(tok_word, ll_word((uint32_t)fed, tok_tag));
    st_g(tokens + slot, fed);
    if (drawn) st_g(drawn + slot, drawn_id);
  }
  tpoint(4);
  return fed;
}

// Running frame sum of the fed embeddings in the model dtype (decode.cpp:263-273,
// 476-484): fs = emb(tok) at level 0, else rnd(fs + emb(tok)); thread tid owns
// elements tid + 256 t.
template <typename T>
__device__ __forceinline__ void frame_sum_add(float (&fs)[kDrawPer], const T* emb, int tok, int D, bool first) {
  using S = St<T>;
  const T* e = emb + (size_t)tok * D;
  float ev[kDrawPer];
#pragma unroll
  for (int t = 0; t < kDrawPer; ++t) {
    const int d = threadIdx.x + kPersistThreads * t;
    ev[t] = d < D ? S::ld(ld_g(e + d)) : 0.f;
  }
#pragma unroll
  for (int t = 0; t < kDrawPer; ++t) fs[t] = first ? ev[t] : S::rnd(fs[t] + ev[t]);
}

// Frame mean fs / L on both rows: the next temporal input (decode.cpp:484).
template <typename T>
__device__ __forceinline__ void frame_mean_store(const float (&fs)[kDrawPer], int L, T* fmean, int D) {
  using S = St<T>;
  const float Lf = S::rnd((float)L);
#pragma unroll
  for (int t = 0; t < kDrawPer; ++t) {
    const int d = threadIdx.x + kPersistThreads * t;
    if (d < D) {
      const T m = S::st(fs[t] / Lf);
      st_g(fmean + d, m);
      st_g(fmean + D + d, m);
    }
  }
}

__global__ void k_gumbel_table(const uint64_t* __restrict__ seed_p, int frames, int L, int C, float* __restrict__ out) {
  const uint64_t seed = *seed_p;
  const int n = frames * L * C;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const int c = i % C, fl = i / C;
    out[i] = gumbel(seed, fl / L, fl % L, c);
  }
}

// Phase codes of the tags: code = stack base + 16 * layer + phase.
enum : int { kPhQKV = 0, kPhAtt = 1, kPhO = 2, kPhCQ = 3, kPhCP = 4, kPhCC = 5, kPhCO = 6, kPhUp = 7, kPhDn = 8 };
enum : int { kPhLogit = 0, kPhToken = 1 };  // after a depth stack: base + 16 * nlayers + ...

// LDS and per-thread state of one persistent workgroup.
template <typename T>
struct Ctx {
  // Activation rows, double-buffered by phase: a wave that starts polling the
  // next phase writes the other buffer while slower waves still read this one.
  float (*xsb)[2 * kMaxPersistK];
  int xsel;
  float* red;
  float* sm;
  float (*kvst)[2][16];  // [k|v][row][d within this workgroup's slice]
  Gamma<T, 4> gq;        // norm weights of the next QKV / head input
  unsigned* sel_hist;
  int* sel_res;
  T* dyn;                // attention staging (4 regions of kRegion)
  uint4 buf[kNBuf];      // weights of the next phase
  uint32_t ep;
  int tp, lcnt;
  int G, blk, wid, lane, h, jpart, rps;
  __device__ float* next_xs() {
    xsel ^= 1;
    return xsb[xsel];
  }
  __device__ uint32_t tag(int code) const { return (ep << kTagShift) | (uint32_t)code; }
};

// Input and output of a decoder stack.
struct StackIO {
  const void* in_plain;  // layer-0 input as plain rows (nullptr: tagged x words)
  int in_stride;         // row stride of in_plain (0: both rows are the same row)
  uint32_t in_tag;       // tag of the tagged layer-0 input
  void* out_plain;       // optional plain (2, D) copy of the output
  bool out_tagged;       // leave the output as tagged x words
  int code_base;
  bool resident;         // self-attention history kept in LDS across the steps of one launch
  int cap;               // LDS slots per (K|V, row) region
  int pos;               // ring slot written by this step
  uint64_t* trace;       // timeline of workgroup 0, or nullptr
  const void* qkv_row;   // layer 0's q | k | v (3 HD model-dtype values, both rows), or nullptr: computed
  bool qkv_ready;        // c.buf holds layer 0's first QKV batch (prefetch_qkv)
};

// Rows of wave `wid` for the QKV phase: local t = wid + 4i < 3*rps ->
// (segment t / rps, row t % rps) of head h's rows owned by workgroup (h, j).
template <typename T>
__device__ __forceinline__ int qkv_rows(const Ctx<T>& c) {
  return (3 * c.rps > c.wid) ? (3 * c.rps - c.wid + 3) / 4 : 0;
}

// Prefetches the self-attention norm weights (c.gq) and the first QKV batch
// (c.buf) of layer `li` of a stack.
template <typename T, bool NT>
__device__ __forceinline__ void prefetch_qkv(Ctx<T>& c, const StepArgs& a, int li) {
  constexpr int V = St<T>::kVec;
  constexpr int NVD = (1024 + V * 64 - 1) / (V * 64);
  const int HD = a.HD, D = a.D, h = c.h, jpart = c.jpart, rps = c.rps, wid = c.wid;
  load_gamma<T, 4>(static_cast<const T*>(a.st.norm_sa) + (size_t)li * D, D, c.gq);
  auto qkv_row = [&](int t, int) {
    const int lt = wid + 4 * t;
    return (lt / rps) * HD + h * 64 + jpart * rps + (lt % rps);
  };
  const T* w = static_cast<const T*>(a.st.wqkv) + (size_t)li * 3 * HD * D;
  fetch_batch<T, NVD, 1, NT>(c.buf, w, D, 0, min(kNBuf / NVD, qkv_rows(c)), qkv_row);
}

// Decoder stack of a.nlayers layers at ring position io.pos (modules.cpp:384-408):
// pre-norm self attention (+ cross attention) + gated-GELU FFN, residuals.
// On entry c.buf holds layer 0's first QKV batch.  Returns the tag of the
// output x words (when io.out_tagged).
template <typename T, bool CROSS>
__device__ __forceinline__ uint32_t run_stack(Ctx<T>& c, const StepArgs& a, const StackIO& io) {
  using S = St<T>;
  constexpr int V = S::kVec;
  constexpr bool NT = CROSS;
  constexpr int NVD = (1024 + V * 64 - 1) / (V * 64);  // K <= 1024
  constexpr int NVF = 3 * NVD;                         // K <= 3072
  const int G = c.G, blk = c.blk, wid = c.wid, lane = c.lane, h = c.h, jpart = c.jpart, rps = c.rps;
  const int D = a.D, HD = a.HD, H = a.H, F = a.F, bph = a.bph;
  const size_t eQKV = (size_t)3 * HD * D, eO = (size_t)D * HD, eQc = (size_t)HD * D, e01 = (size_t)2 * F * D,
               eO2 = (size_t)D * F;
  const size_t eRing = (size_t)2 * H * a.Lmax * 64, eCross = (size_t)2 * H * a.S * 64;
  const T* wqkv0 = static_cast<const T*>(a.st.wqkv);
  float* xs = c.xsb[c.xsel];
  float* red = c.red;
  float* sm = c.sm;
  T* hist = c.dyn;
  T* cst = c.dyn;
#define MRT_TP trace_point(io.trace, c.tp++)

  const RowSplit sD(D, G, blk), sF(F, G, blk);
  const int nqkv = qkv_rows(c);
  auto qkv_row = [&](int t, int) {
    const int lt = wid + 4 * t;
    return (lt / rps) * HD + h * 64 + jpart * rps + (lt % rps);
  };
  const int ncq = (rps > wid) ? (rps - wid + 3) / 4 : 0;
  auto cq_row = [&](int t, int) { return h * 64 + jpart * rps + wid + 4 * t; };
  auto rowD = [&](int t, int) { return sD.row(wid, t); };
  auto rowF = [&](int t, int p) { return geglu_row(sF.row(wid, t), p); };
  auto side_x = [&](const uint64_t* ll, const void* plain, uint32_t tg, int stride) {
    Side s{ll, plain, tg, lane < sD.nw(wid) ? sD.row(wid, lane) : -1, stride};
    return s;
  };
  const Side no_side{nullptr, nullptr, 0u, -1, 0};
  float r0 = 0.f, r1 = 0.f;
  // lane t holds the residual element of the wave's row t (side_x)
  auto resid_put = [&](int t, bool act, const float (&s)[1][2], uint32_t tg) {
    const float x0 = from_lane(r0, t), x1 = from_lane(r1, t);
    if (act) LL<T>::put(a.ll.x, sD.row(wid, t), S::rnd(x0 + S::rnd(s[0][0])), S::rnd(x1 + S::rnd(s[0][1])), tg);
  };

  // the attention workgroups' bias of key j = lane (the same for every layer
  // of the step), loaded ahead so that no dependent load sits in the attention
  float pbias = 0.f;
  if (jpart == 0 && wid < 2 && lane <= io.pos) {
    const T* row = a.bias_row != nullptr ? static_cast<const T*>(a.bias_row)
                                         : static_cast<const T*>(a.bias_rows) + (size_t)H * io.pos * (io.pos + 1) / 2;
    pbias = S::ld(ld_g(row + h * (io.pos + 1) + lane));
  }
  uint32_t x_tag = io.in_tag;
  for (int li = 0; li < a.nlayers; ++li) {
    const bool first = li == 0, last = li + 1 == a.nlayers;
    const int base = io.code_base + 16 * li;
    auto tag = [&](int code) { return c.tag(code); };
    T* ring_k = static_cast<T*>(a.st.ring) + 2 * li * eRing;
    const void* in_plain = first ? io.in_plain : nullptr;
    const int in_stride = io.in_stride;
    // ---- stage the ring history and cross K/V block of this layer in LDS
    T* lhist = io.resident ? hist + (size_t)li * 4 * io.cap * 64 : hist;
    // ring slots 0..pos-1 of layer lj (written by earlier launches) into the
    // history regions, by the attention workgroups
    auto stage_hist = [&](int lj) {
      const int kind = wid >> 1, b = wid & 1;
      const T* src = static_cast<const T*>(a.st.ring) + (2 * lj + kind) * eRing + (size_t)(b * H + h) * a.Lmax * 64;
      const long lim = (long)a.Lmax * 64 * sizeof(T);
      if (kind == 0)
        stage_slots<T, true>(src, io.pos, lim, hist + wid * kRegion);
      else
        stage_slots<T, false>(src, io.pos, lim, hist + wid * kRegion);
    };
    // with cross attention, layers after the first were staged at the end of
    // the previous layer's cross attention
    if (!io.resident && jpart == 0 && io.pos > 0 && (!CROSS || first)) stage_hist(li);
    auto stage_cross = [&]() {
      const int chunk = (a.S + bph - 1) / bph, kb0 = jpart * chunk;
      const int nk = max(0, min(chunk, a.S - kb0));
      if (nk > 0) {
        const int kind = wid >> 1, b = wid & 1;
        const T* src = static_cast<const T*>(a.st.cross) + (2 * li + kind) * eCross +
                       ((size_t)(b * H + h) * a.S + kb0) * 64;
        const long lim = (long)(a.S - kb0) * 64 * sizeof(T);
        if (kind == 0)
          stage_slots<T, true>(src, nk, lim, cst + wid * kRegion);
        else
          stage_slots<T, false>(src, nk, lim, cst + wid * kRegion);
      }
    };
    // ---- QKV of head h's slice (weights already in flight), unless layer 0's
    // q/k/v come from a table row: the attention workgroups then read their
    // head's slice there and the others go on to the output projection.
    const bool tbl = first && io.qkv_row != nullptr;
    if (tbl) {
      MRT_TP;  // the QKV phase's four trace points, so a timeline keeps its layout
      MRT_TP;
      MRT_TP;
      MRT_TP;
    } else {
    if (first && !io.qkv_ready) prefetch_qkv<T, NT>(c, a, 0);
    xs = c.next_xs();
    load_act<T, 4, true>(a.ll.x, in_plain, D, x_tag, c.gq, xs, red, no_side, r0, r1, a.ll.err, a.ll.delay[kPollQKV], io.trace, c.tp,
                         c.lcnt, in_stride);
    gemv_rows<T, NVD, 1, NT>(c.buf, wqkv0 + li * eQKV, D, nqkv, qkv_row, xs,
                             [&](int t, bool act, const float (&s)[1][2]) {
      const int lt = wid + 4 * t, seg = lt / rps, r = lt % rps;
      const int n = h * 64 + jpart * rps + r;
      const float v0 = S::rnd(s[0][0]), v1 = S::rnd(s[0][1]);
      if (act) {
        uint64_t* dst = pick3<uint64_t*>(seg, a.ll.q, a.ll.k, a.ll.v);
        LL<T>::put(dst, n, v0, v1, tag(base + kPhQKV));
        if (seg > 0) {
          c.kvst[seg - 1][0][r] = v0;
          c.kvst[seg - 1][1][r] = v1;
        }
      }
    });
    MRT_TP;
    __syncthreads();
    // plain ring slot (read by later launches): 4 elements per thread
    if (threadIdx.x < 2 * 2 * (rps / 4)) {
      const int g4 = threadIdx.x % (rps / 4), rb = (threadIdx.x / (rps / 4)) % 2, kv = threadIdx.x / (rps / 2);
      T* dst = ring_k + kv * eRing + (((size_t)rb * H + h) * a.Lmax + io.pos) * 64 + jpart * rps + 4 * g4;
      const float* v = &c.kvst[kv][rb][4 * g4];
      if constexpr (sizeof(T) == 2) {
        st_g(reinterpret_cast<uint64_t*>(dst), (uint64_t)St<T>::bits(v[0]) | ((uint64_t)St<T>::bits(v[1]) << 16) |
                                                   ((uint64_t)St<T>::bits(v[2]) << 32) |
                                                   ((uint64_t)St<T>::bits(v[3]) << 48));
      } else {
        st_g(reinterpret_cast<uint64_t*>(dst), (uint64_t)__float_as_uint(v[0]) | ((uint64_t)__float_as_uint(v[1]) << 32));
        st_g(reinterpret_cast<uint64_t*>(dst) + 1,
             (uint64_t)__float_as_uint(v[2]) | ((uint64_t)__float_as_uint(v[3]) << 32));
      }
    }
    }  // QKV phase
    // The cross K/V block of a workgroup that runs no self attention: after the
    // QKV poll (which would otherwise wait for these copies), while the heads'
    // attention runs.
    if (CROSS && jpart != 0) stage_cross();
    // Head h's attention in workgroup (h, 0), then the next phase's weights:
    // its polls would otherwise also wait for those loads.
    const T* wo = static_cast<const T*>(a.st.wo) + li * eO;
    if (jpart == 0) {
      self_attention_head<T>(a, io.pos, h, tag(base + kPhQKV), tag(base + kPhAtt), lhist, io.resident ? io.cap : 64,
                             io.resident, pbias, sm, tbl ? static_cast<const T*>(io.qkv_row) : nullptr, ring_k, eRing);
      MRT_TP;
      if (CROSS) stage_cross();  // the history has been read (barrier above)
    }
    fetch_batch<T, NVD, 1, NT>(c.buf, wo, HD, 0, min(kNBuf / NVD, sD.nw(wid)), rowD);
    // ---- attention output projection + residual
    xs = c.next_xs();
    load_act<T, 4, false>(a.ll.at, nullptr, HD, tag(base + kPhAtt), c.gq, xs, red,
                          side_x(a.ll.x, in_plain, x_tag, in_stride), r0, r1, a.ll.err, a.ll.delay[kPollO], io.trace, c.tp, c.lcnt, 0);
    gemv_rows<T, NVD, 1, NT>(c.buf, wo, HD, sD.nw(wid), rowD, xs,
                             [&](int t, bool act, const float (&s)[1][2]) { resid_put(t, act, s, tag(base + kPhO)); });
    MRT_TP;
    x_tag = tag(base + kPhO);
    if constexpr (CROSS) {
      // ---- cross attention: q rows of head h, key-block partials, combine
      const T* wqc = static_cast<const T*>(a.st.wq_c) + li * eQc;
      const T* woc = static_cast<const T*>(a.st.wo_c) + li * eO;
      Gamma<T, 4> gc;
      load_gamma<T, 4>(static_cast<const T*>(a.st.norm_ca) + (size_t)li * D, D, gc);
      fetch_batch<T, NVD, 1, NT>(c.buf, wqc, D, 0, min(kNBuf / NVD, ncq), cq_row);
      xs = c.next_xs();
      load_act<T, 4, true>(a.ll.x, nullptr, D, x_tag, gc, xs, red, no_side, r0, r1, a.ll.err, a.ll.delay[kPollCrossQ], io.trace, c.tp,
                           c.lcnt, 0);
      gemv_rows<T, NVD, 1, NT>(c.buf, wqc, D, ncq, cq_row, xs, [&](int t, bool act, const float (&s)[1][2]) {
        if (act) LL<T>::put(a.ll.q, cq_row(t, 0), S::rnd(s[0][0]), S::rnd(s[0][1]), tag(base + kPhCQ));
      });
      MRT_TP;
      fetch_batch<T, NVD, 1, NT>(c.buf, woc, HD, 0, min(kNBuf / NVD, sD.nw(wid)), rowD);
      cross_partial<T>(a, h, jpart, tag(base + kPhCQ), tag(base + kPhCP), cst, sm);
      MRT_TP;
      if (jpart == 0) {
        cross_combine<T>(a, h, tag(base + kPhCP), tag(base + kPhCC), sm);
        MRT_TP;
        // the staged cross K/V has been read (barrier in cross_partial): the
        // next layer's history copies go out now, so that its QKV poll does
        // not wait for them
        if (!io.resident && !last && io.pos > 0) stage_hist(li + 1);
      }
      xs = c.next_xs();
      load_act<T, 4, false>(a.ll.at, nullptr, HD, tag(base + kPhCC), c.gq, xs, red,
                            side_x(a.ll.x, nullptr, x_tag, 0), r0, r1, a.ll.err, a.ll.delay[kPollCrossO], io.trace, c.tp, c.lcnt, 0);
      gemv_rows<T, NVD, 1, NT>(c.buf, woc, HD, sD.nw(wid), rowD, xs,
                               [&](int t, bool act, const float (&s)[1][2]) { resid_put(t, act, s, tag(base + kPhCO)); });
      MRT_TP;
      x_tag = tag(base + kPhCO);
    }
    // ---- gated-GELU up projection
    const T* w01 = static_cast<const T*>(a.st.w01) + li * e01;
    const T* wo2 = static_cast<const T*>(a.st.wo2) + li * eO2;
    Gamma<T, 4> gf;
    load_gamma<T, 4>(static_cast<const T*>(a.st.norm_ff) + (size_t)li * D, D, gf);
    fetch_batch<T, NVD, 2, NT>(c.buf, w01, D, 0, min(kNBuf / (2 * NVD), sF.nw(wid)), rowF);
    xs = c.next_xs();
    load_act<T, 4, true>(a.ll.x, nullptr, D, x_tag, gf, xs, red, no_side, r0, r1, a.ll.err, a.ll.delay[kPollUp], io.trace, c.tp,
                         c.lcnt, 0);
    gemv_rows<T, NVD, 2, NT>(c.buf, w01, D, sF.nw(wid), rowF, xs, [&](int t, bool act, const float (&s)[2][2]) {
      const float g0 = gelu_t<T>(S::rnd(s[0][0])), g1 = gelu_t<T>(S::rnd(s[0][1]));
      if (act)
        LL<T>::put(a.ll.h, sF.row(wid, t), S::rnd(g0 * S::rnd(s[1][0])), S::rnd(g1 * S::rnd(s[1][1])),
                   tag(base + kPhUp));
    });
    MRT_TP;
    // ---- down projection + residual
    fetch_batch<T, NVF, 1, NT>(c.buf, wo2, F, 0, min(kNBuf / NVF, sD.nw(wid)), rowD);
    xs = c.next_xs();
    const Gamma<T, kMaxPersistK / kPersistThreads> nog{};  // no norm
    load_act<T, kMaxPersistK / kPersistThreads, false>(a.ll.h, nullptr, F, tag(base + kPhUp), nog, xs, red,
                                                       side_x(a.ll.x, nullptr, x_tag, 0), r0, r1, a.ll.err, a.ll.delay[kPollDown], io.trace,
                                                       c.tp, c.lcnt, 0);
    const bool tagged_out = !last || io.out_tagged;
    gemv_rows<T, NVF, 1, NT>(c.buf, wo2, F, sD.nw(wid), rowD, xs, [&](int t, bool act, const float (&s)[1][2]) {
      const float x0 = from_lane(r0, t), x1 = from_lane(r1, t);
      const float y0 = S::rnd(x0 + S::rnd(s[0][0])), y1 = S::rnd(x1 + S::rnd(s[0][1]));
      if (act) {
        const int n = sD.row(wid, t);
        if (tagged_out) LL<T>::put(a.ll.x, n, y0, y1, tag(base + kPhDn));
        if (last && io.out_plain != nullptr) {
          T* o = static_cast<T*>(io.out_plain) + n;
          st_g(o, S::st(y0));
          st_g(o + D, S::st(y1));
        }
      }
    });
    MRT_TP;
    x_tag = tag(base + kPhDn);
    if (!last) prefetch_qkv<T, NT>(c, a, li + 1);
    if (!io.resident) __syncthreads();  // LDS staging regions are rewritten by the next layer
  }
#undef MRT_TP
  return x_tag;
}

// decoder_norm + lm_head rows of one level (model.cpp:652-653): every
// workgroup computes ceil(head_rows / G) rows and publishes them as tagged
// fp32 words; c.buf holds the first head batch on entry.
template <typename T>
__device__ __forceinline__ void run_head(Ctx<T>& c, const StepArgs& a, const T* hw, uint32_t x_tag, uint32_t out_tag,
                                         uint64_t* trace) {
  using S = St<T>;
  constexpr int V = S::kVec;
  constexpr int NVD = (1024 + V * 64 - 1) / (V * 64);
  const int wid = c.wid;
  const RowSplit sH(a.head_rows, c.G, c.blk);
  auto rowH = [&](int t, int) { return sH.row(wid, t); };
  const Side no_side{nullptr, nullptr, 0u, -1, 0};
  float r0 = 0.f, r1 = 0.f;
  float* xs = c.next_xs();
  load_act<T, 4, true>(a.ll.x, nullptr, a.D, x_tag, c.gq, xs, c.red, no_side, r0, r1, a.ll.err, a.ll.delay[kPollHead], trace, c.tp,
                       c.lcnt, 0);
  gemv_rows<T, NVD, 1, false>(c.buf, hw, a.D, sH.nw(wid), rowH, xs, [&](int t, bool act, const float (&s)[1][2]) {
    if (act) {
      const int n = sH.row(wid, t);
      astore(a.ll.logit + n, ll_word(__float_as_uint(S::rnd(s[0][0])), out_tag));
      astore(a.ll.logit + a.head_rows + n, ll_word(__float_as_uint(S::rnd(s[0][1])), out_tag));
    }
  });
}

template <typename T>
__device__ __forceinline__ void prefetch_head(Ctx<T>& c, const StepArgs& a, const T* hw) {
  constexpr int V = St<T>::kVec;
  constexpr int NVD = (1024 + V * 64 - 1) / (V * 64);
  const RowSplit sH(a.head_rows, c.G, c.blk);
  const int wid = c.wid;
  load_gamma<T, 4>(static_cast<const T*>(a.dec_norm), a.D, c.gq);
  fetch_batch<T, NVD, 1, false>(c.buf, hw, a.D, 0, min(kNBuf / NVD, sH.nw(wid)), [&](int t, int) { return sH.row(wid, t); });
}

// Workgroup 0 gathers the 2 x head_rows tagged logits into LDS (and copies
// them to `logits` / `rec`, when set).
template <typename T>
__device__ __forceinline__ void gather_logits(const StepArgs& a, uint32_t tg, float* lg, float* logits, float* rec) {
  const int n2 = 2 * a.head_rows;
  uint32_t spins = 0;
  for (int base_i = 0; base_i < n2; base_i += kPersistThreads * 8) {
    uint64_t w[8];
    uint32_t pend = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (base_i + (int)threadIdx.x + u * kPersistThreads < n2) pend |= 1u << u;
    if (base_i == 0) poll_wait(a.ll.delay[kPollLogits]);
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
          if (logits) st_g(logits + i, v);
          if (rec) st_g(rec + i, v);
          pend &= ~(1u << u);
        }
      }
      if (pend == 0 || spin_failed(spins, a.ll.err)) break;
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
}

#define MRT_DECLARE_LDS(T)                                                                    \
  __shared__ float xsb[2][2 * kMaxPersistK];                                                  \
  __shared__ __align__(16) float red[8];                                                      \
  __shared__ __align__(16) float sm[704];                                                     \
  __shared__ float kvst[2][2][16];                                                            \
  __shared__ __align__(16) unsigned sel_hist[kDrawHistWords];                                     \
  __shared__ int sel_res[16];                                                                 \
  extern __shared__ __align__(16) unsigned char dyn_lds[];                                    \
  Ctx<T> c;                                                                                   \
  c.xsb = xsb;                                                                                \
  c.xsel = 0;                                                                                 \
  c.red = red;                                                                                \
  c.sm = sm;                                                                                  \
  c.kvst = kvst;                                                                              \
  c.sel_hist = sel_hist;                                                                      \
  c.sel_res = sel_res;                                                                        \
  c.dyn = reinterpret_cast<T*>(dyn_lds);                                                      \
  c.tp = 0;                                                                                   \
  c.lcnt = 0;                                                                                 \
  c.G = gridDim.x;                                                                            \
  c.blk = blockIdx.x;                                                                         \
  c.wid = uniform(threadIdx.x >> 6);                                                          \
  c.lane = threadIdx.x & 63

// Per-launch start of a persistent kernel: reads the error flag and the
// epoch first (their loads must not queue behind the weight prefetch), zeroes
// the activation buffers (elements past a vector's end meet zero weights).
// Returns false if a previous launch failed.
template <typename T>
__device__ __forceinline__ bool start(Ctx<T>& c, const LLBufs& ll, int bph) {
  c.h = c.blk / bph;
  c.jpart = c.blk % bph;
  c.rps = 64 / bph;
  const int err = aload(ll.err);
  c.ep = aload(ll.seq);
  float4* z = reinterpret_cast<float4*>(&c.xsb[0][0]);
  for (int k = threadIdx.x; k < 2 * 2 * kMaxPersistK / 4; k += kPersistThreads) z[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  return err == 0;
}

// One step launch (the temporal_step / depth_step API): a decoder stack, then
// for depth the level-sliced head with the logits copied to a.logits.
template <typename T, bool CROSS, bool TRACE>
__global__ __launch_bounds__(kPersistThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_step(StepArgs a) {
  MRT_DECLARE_LDS(T);
  // the timeline of workgroup 0 exists only in the TRACE instance
  uint64_t* const trace = TRACE ? a.trace : nullptr;
  const bool ok = start<T>(c, a.ll, a.bph);
  if (a.nlayers > 0) prefetch_qkv<T, CROSS>(c, a, 0);
  __syncthreads();
  if (!ok) return;  // a previous launch failed: do nothing
  if (!CROSS && a.sp.decided != nullptr && *a.sp.decided >= a.pos) {
    // speculative decoding already has this level's token: only the epoch advances
    __builtin_amdgcn_s_waitcnt(0);
    if (c.blk == 0 && threadIdx.x == 0) astore(a.ll.seq, c.ep + 1u);
    return;
  }
  if (trace != nullptr && c.blk == 0 && threadIdx.x == 0) trace[kTraceStart] = wall_clock64();
  StackIO io{a.in, a.D, 0u, CROSS ? a.out : nullptr, !CROSS, 0, false, 64, a.pos, trace, nullptr, true};
  const uint32_t x_tag = run_stack<T, CROSS>(c, a, io);
  if constexpr (!CROSS) {
    const T* hw = static_cast<const T*>(a.head_w);
    prefetch_head<T>(c, a, hw);
    const uint32_t tg = c.tag(16 * a.nlayers + kPhLogit);
    run_head<T>(c, a, hw, x_tag, tg, trace);
    if (c.blk == 0 && threadIdx.x == 0) astore(a.ll.seq, c.ep + 1u);  // every workgroup has started
    if (c.blk == 0) {
      __syncthreads();
      gather_logits<T>(a, tg, c.xsb[c.xsel ^ 1], a.logits, a.rec_slice);
    }
  } else {
    if (c.blk == 0 && threadIdx.x == 0) astore(a.ll.seq, c.ep + 1u);  // every workgroup has read the epoch
  }
  if (trace != nullptr && c.blk == 0 && threadIdx.x == 0) trace[kTraceEnd] = trace[kTraceDone] = wall_clock64();
}

// One frame of the decode loop in one launch (decode.cpp:339-486): the
// temporal step (input a.t.in, the previous frame's mean), then `levels`
// depth steps each ending in a draw by workgroup 0, which publishes the fed
// token as a tagged word; every workgroup then reads that token's embedding
// row as the next depth input.  The depth K/V history stays in the LDS of the
// attention workgroups; ring slots are still written to memory.
template <typename T, bool TRACE>
__global__ __launch_bounds__(kPersistThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_frame(FrameArgs fa) {
  MRT_DECLARE_LDS(T);
  const StepArgs& at = fa.t;
  const StepArgs& ad = fa.d;
  // the timelines of workgroup 0 exist only in the TRACE instance
  uint64_t* const t_trace = TRACE ? at.trace : nullptr;
  uint64_t* const d_trace = TRACE ? ad.trace : nullptr;
  const bool ok = start<T>(c, at.ll, at.bph);
  prefetch_qkv<T, true>(c, at, 0);
  __syncthreads();
  if (!ok) return;
  if (t_trace != nullptr && c.blk == 0 && threadIdx.x == 0) t_trace[kTraceStart] = wall_clock64();
  // phase stamps of workgroup 0 (fa.prof): start, temporal done, draw ticks
  const bool prof = fa.prof != nullptr && c.blk == 0;
  uint64_t p_start = 0, p_temporal = 0, p_draw = 0;
  if (prof) p_start = wall_clock64();
  // ---- temporal step
  StackIO tio{at.in, at.D, 0u, fa.rec_temporal, true, 0, false, 64, at.pos, t_trace, nullptr, true};
  uint32_t x_tag = run_stack<T, true>(c, at, tio);
  if (t_trace != nullptr && c.blk == 0 && threadIdx.x == 0) t_trace[kTraceEnd] = t_trace[kTraceDone] = wall_clock64();
  if (prof) p_temporal = wall_clock64();
  // ---- depth steps
  const int L = fa.levels, C = fa.codebook, D = ad.D;
  const int code0 = 16 * (at.nlayers + 1), per_step = 16 * (ad.nlayers + 1);
  float fs[kDrawPer] = {};  // frame sum (workgroup 0)
  DrawPrefetch pf{};        // noise of the next draw (workgroup 0), loaded a level ahead
  if (c.blk == 0) {
    draw_clear(c.sel_hist);  // ordered before the first draw by the gather's barriers
    draw_prefetch(C, ad.noise, ad.teacher, ad.frame * L, pf);
  }
  int tok = 0;
  prefetch_qkv<T, false>(c, ad, 0);
  for (int l = 0; l < L; ++l) {
    uint64_t* trace = l == 1 ? d_trace : nullptr;  // timeline of level 1
    if (l == 1) {
      c.tp = 0;
      c.lcnt = 0;
      if (trace != nullptr && c.blk == 0 && threadIdx.x == 0) trace[kTraceStart] = wall_clock64();
    }
    const int base = code0 + l * per_step;
    StackIO io{nullptr, 0, x_tag, nullptr, true, base, true, L, l, trace, nullptr, true};
    if (l > 0) {
      io.in_plain = static_cast<const T*>(ad.emb) + (size_t)tok * D;  // both rows: emb(token)
      io.in_stride = 0;
      // layer 0's q/k/v of the fed token from the table (no QKV weights were
      // prefetched for it); a token outside level l - 1 takes the computed path
      const int cb = tok - ad.sp.codec_offset - C * (l - 1);
      io.qkv_ready = fa.qkv_table == nullptr;
      if (fa.qkv_table != nullptr && cb >= 0 && cb < C)
        io.qkv_row = static_cast<const T*>(fa.qkv_table) + ((size_t)(l - 1) * C + cb) * 3 * ad.HD;
    }
    x_tag = run_stack<T, false>(c, ad, io);
    const T* hw = static_cast<const T*>(ad.head_w) + (size_t)l * C * D;
    prefetch_head<T>(c, ad, hw);
    const uint32_t tg_logit = c.tag(base + 16 * ad.nlayers + kPhLogit);
    const uint32_t tg_tok = c.tag(base + 16 * ad.nlayers + kPhToken);
    run_head<T>(c, ad, hw, x_tag, tg_logit, trace);
    if (c.blk != 0 && l + 1 < L && fa.qkv_table == nullptr) prefetch_qkv<T, false>(c, ad, 0);
    if (c.blk == 0) {
      // Nothing is loaded between the head and the gather: a wave's memory
      // operations retire in order, so the gather's polls would wait for them.
      if (l + 1 == L && threadIdx.x == 0) astore(ad.ll.seq, c.ep + 1u);  // every workgroup has started
      const int slot = ad.frame * L + l;
      __syncthreads();
      float* lg = c.xsb[c.xsel ^ 1];
      gather_logits<T>(ad, tg_logit, lg, nullptr, fa.rec_slices ? fa.rec_slices + (size_t)l * 2 * C : nullptr);
      if (trace != nullptr && threadIdx.x == 0) trace[kTraceEnd] = wall_clock64();
      const uint64_t p_gathered = prof ? wall_clock64() : 0;
      if (l + 1 < L && fa.qkv_table == nullptr) prefetch_qkv<T, false>(c, ad, 0);  // lands during the draw
      tok = sample_block<T>(ad.sp, l, slot, pf, ad.teacher != nullptr, ad.tokens, ad.drawn,
                            l + 1 < L ? ad.ll.tok : nullptr, tg_tok, lg, c.sel_hist, c.sel_res, trace);
      if (trace != nullptr && threadIdx.x == 0) trace[kTraceDone] = wall_clock64();
      // this level's token joins the frame sum (the embedding row is the next
      // level's input too), and the next draw's noise is loaded a level ahead
      frame_sum_add<T>(fs, static_cast<const T*>(ad.emb), tok, D, l == 0);
      if (l + 1 < L)
        draw_prefetch(C, ad.noise + (size_t)(l + 1) * C, ad.teacher, slot + 1, pf);
      else
        frame_mean_store<T>(fs, L, static_cast<T*>(ad.fmean), D);
      if (prof) p_draw += wall_clock64() - p_gathered;
    } else if (l + 1 < L) {
      // every workgroup waits for the draw (one word, polled by one lane)
      __shared__ int tok_s;
      if (threadIdx.x == 0) {
        uint32_t spins = 0;
        uint64_t w;
        poll_wait(ad.ll.delay[kPollToken]);
        for (;;) {
          w = aload(ad.ll.tok);
          if (ll_tag(w) == tg_tok || spin_failed(spins, ad.ll.err)) break;
          __builtin_amdgcn_s_sleep(1);
        }
        // after a failed poll (error flagged) any in-range row keeps the reads in bounds
        tok_s = ll_tag(w) == tg_tok ? (int)static_cast<uint32_t>(w) : 0;
      }
      __syncthreads();
      tok = tok_s;
    }
  }
  if (prof && threadIdx.x == 0) {
    uint64_t* o = fa.prof + 4 * ad.frame;
    st_g(o, p_start);
    st_g(o + 1, p_temporal);
    st_g(o + 2, (uint64_t)wall_clock64());
    st_g(o + 3, p_draw);
  }
}

// The levels after a speculative verification pass, in one launch
// (decode.cpp:429-446: the depth loop resumes after the first rejected draft).
// Levels 0..n are decided, n = *d.sp.decided (written before this launch, the
// same for every workgroup), tokens[frame * levels + n] the last of them; each
// level n + 1 .. levels - 1 is a depth step on emb(previous token), the
// level's head slice and workgroup 0's draw, as in k_frame.  The attention
// workgroups first copy the decided levels' K/V (ring slots 0..n, written by
// the verification pass in earlier launches) into their LDS history; the
// levels of this launch then keep theirs in LDS, as k_frame does (ring slots
// written in this launch are not read back in it: the caches of the XCDs are
// coherent only between launches).  With every level decided the launch does
// nothing: no word is tagged and the epoch stays.  The frame mean is left to
// the caller.
template <typename T>
__global__ __launch_bounds__(kPersistThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_levels(FrameArgs fa) {
  MRT_DECLARE_LDS(T);
  const StepArgs& ad = fa.d;
  const int L = fa.levels, C = fa.codebook, D = ad.D;
  const int n = *ad.sp.decided;
  const bool ok = start<T>(c, ad.ll, ad.bph);
  if (n < 0 || n + 1 >= L) return;
  const bool tbl = fa.qkv_table != nullptr;
  if (!tbl) prefetch_qkv<T, false>(c, ad, 0);
  if (c.jpart == 0) {
    // wave w copies region (kind w / 2, row w % 2) of every layer: slots 0..n
    const int kind = c.wid >> 1, b = c.wid & 1;
    const size_t eRing = (size_t)2 * ad.H * ad.Lmax * 64;
    const long lim = (long)ad.Lmax * 64 * sizeof(T);
    for (int li = 0; li < ad.nlayers; ++li) {
      const T* src = static_cast<const T*>(ad.st.ring) + (2 * li + kind) * eRing + (size_t)(b * ad.H + c.h) * ad.Lmax * 64;
      T* region = c.dyn + (size_t)li * 4 * L * 64 + (size_t)c.wid * L * 64;
      if (kind == 0)
        stage_slots<T, true>(src, n + 1, lim, region);
      else
        stage_slots<T, false>(src, n + 1, lim, region);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's history copies have landed
  }
  __syncthreads();
  if (!ok) return;
  const int per_step = 16 * (ad.nlayers + 1);
  SampleParams sp = ad.sp;
  sp.decided = nullptr;  // every level drawn here is open
  DrawPrefetch pf{};
  if (c.blk == 0) {
    draw_clear(c.sel_hist);
    draw_prefetch(C, ad.noise + (size_t)(n + 1) * C, ad.teacher, ad.frame * L + n + 1, pf);
  }
  int tok = ad.tokens[(size_t)ad.frame * L + n];
  uint32_t x_tag = 0;
  for (int l = n + 1; l < L; ++l) {
    const int base = l * per_step;
    StackIO io{static_cast<const T*>(ad.emb) + (size_t)tok * D, 0, x_tag, nullptr, true, base, true, L, l,
               nullptr, nullptr, !tbl};
    const int cb = tok - ad.sp.codec_offset - C * (l - 1);
    if (tbl && cb >= 0 && cb < C) io.qkv_row = static_cast<const T*>(fa.qkv_table) + ((size_t)(l - 1) * C + cb) * 3 * ad.HD;
    x_tag = run_stack<T, false>(c, ad, io);
    const T* hw = static_cast<const T*>(ad.head_w) + (size_t)l * C * D;
    prefetch_head<T>(c, ad, hw);
    const uint32_t tg_logit = c.tag(base + 16 * ad.nlayers + kPhLogit);
    const uint32_t tg_tok = c.tag(base + 16 * ad.nlayers + kPhToken);
    run_head<T>(c, ad, hw, x_tag, tg_logit, nullptr);
    if (c.blk != 0 && l + 1 < L && !tbl) prefetch_qkv<T, false>(c, ad, 0);
    if (c.blk == 0) {
      if (l + 1 == L && threadIdx.x == 0) astore(ad.ll.seq, c.ep + 1u);  // every workgroup has started
      const int slot = ad.frame * L + l;
      __syncthreads();
      float* lg = c.xsb[c.xsel ^ 1];
      gather_logits<T>(ad, tg_logit, lg, nullptr, fa.rec_slices ? fa.rec_slices + (size_t)l * 2 * C : nullptr);
      if (l + 1 < L && !tbl) prefetch_qkv<T, false>(c, ad, 0);
      tok = sample_block<T>(sp, l, slot, pf, ad.teacher != nullptr, ad.tokens, ad.drawn, l + 1 < L ? ad.ll.tok : nullptr,
                            tg_tok, lg, c.sel_hist, c.sel_res, nullptr);
      if (l + 1 < L) draw_prefetch(C, ad.noise + (size_t)(l + 1) * C, ad.teacher, slot + 1, pf);
    } else if (l + 1 < L) {
      __shared__ int tok_s;
      if (threadIdx.x == 0) {
        uint32_t spins = 0;
        uint64_t w;
        poll_wait(ad.ll.delay[kPollToken]);
        for (;;) {
          w = aload(ad.ll.tok);
          if (ll_tag(w) == tg_tok || spin_failed(spins, ad.ll.err)) break;
          __builtin_amdgcn_s_sleep(1);
        }
        tok_s = ll_tag(w) == tg_tok ? (int)static_cast<uint32_t>(w) : 0;
      }
      __syncthreads();
      tok = tok_s;
    }
  }
}

template <typename T>
size_t lds_bytes() {
  return 4 * static_cast<size_t>(kRegion) * sizeof(T);
}

bool allow_lds(const void* fn, size_t dyn, int device) {
  hipFuncAttributes attr{};
  MRT_HIP_CHECK(hipFuncGetAttributes(&attr, fn));
  int max_lds = 0;
  MRT_HIP_CHECK(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeSharedMemPerBlockOptin, device));
  if (max_lds <= 0) MRT_HIP_CHECK(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device));
  if (attr.sharedSizeBytes + dyn > static_cast<size_t>(max_lds)) return false;
  MRT_HIP_CHECK(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(dyn)));
  // Every workgroup of the grid polls words that other workgroups write, so all
  // of them must be resident at once: at least one workgroup with this LDS and
  // these registers per CU (the grid is at most one per CU).
  int per_cu = 0;
  MRT_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kPersistThreads, dyn));
  return per_cu >= 1;
}

template <typename T, bool TRACE>
const void* persist_fn(PersistKernel kind) {
  return kind == PersistKernel::Temporal ? reinterpret_cast<const void*>(&k_step<T, true, TRACE>)
         : kind == PersistKernel::Depth  ? reinterpret_cast<const void*>(&k_step<T, false, TRACE>)
         : kind == PersistKernel::Levels ? reinterpret_cast<const void*>(&k_levels<T>)
                                         : reinterpret_cast<const void*>(&k_frame<T, TRACE>);
}

template <typename T>
size_t prepare(PersistKernel kind, int device) {
  const size_t n = lds_bytes<T>();
  // both the plain and the traced instance must fit (the traced one runs with MRT_TRACE_PHASES)
  return allow_lds(persist_fn<T, false>(kind), n, device) && allow_lds(persist_fn<T, true>(kind), n, device) ? n : 0;
}

}  // namespace

namespace {

constexpr int kMaxGateDevices = 64;
struct DeviceGate {
  std::mutex mu;
  hipEvent_t last = nullptr;  // end of the device's latest persistent unit; kept until the process ends
};
DeviceGate g_gates[kMaxGateDevices];

}  // namespace

PersistSection::PersistSection(int device, hipStream_t stream) : device_(device), stream_(stream) {
  MRT_REQUIRE(device >= 0 && device < kMaxGateDevices, "persistent kernels: device index out of range");
  DeviceGate& g = g_gates[device];
  g.mu.lock();
  try {
    if (!g.last) MRT_HIP_CHECK(hipEventCreateWithFlags(&g.last, hipEventDisableTiming));
    MRT_HIP_CHECK(hipStreamWaitEvent(stream, g.last, 0));
  } catch (...) {
    g.mu.unlock();
    throw;
  }
}

PersistSection::~PersistSection() {
  DeviceGate& g = g_gates[device_];
  (void)hipEventRecord(g.last, stream_);
  g.mu.unlock();
}

int persist_grid(int H, int num_cu, int* bph_out) {
  int bph = kMaxBph;
  while (bph > 1 && H * bph > num_cu) bph /= 2;
  if (bph < 8 || H * bph > num_cu) return 0;
  if (bph_out) *bph_out = bph;
  return H * bph;
}

size_t persist_prepare(DType dt, PersistKernel kind, int device) {
  size_t r = 0;
  MRT_DTYPE_DISPATCH(dt, r = prepare<T>(kind, device));
  return r;
}

void launch_step(DType dt, const StepArgs& a, int grid, size_t lds, hipStream_t s) {
  const bool tr = a.trace != nullptr;
  MRT_DTYPE_DISPATCH(dt, {
    if (a.cross && tr)
      hipLaunchKernelGGL((k_step<T, true, true>), dim3(grid), dim3(kPersistThreads), lds, s, a);
    else if (a.cross)
      hipLaunchKernelGGL((k_step<T, true, false>), dim3(grid), dim3(kPersistThreads), lds, s, a);
    else if (tr)
      hipLaunchKernelGGL((k_step<T, false, true>), dim3(grid), dim3(kPersistThreads), lds, s, a);
    else
      hipLaunchKernelGGL((k_step<T, false, false>), dim3(grid), dim3(kPersistThreads), lds, s, a);
  });
  MRT_HIP_CHECK(hipGetLastError());
}

void launch_frame(DType dt, const FrameArgs& a, int grid, size_t lds, hipStream_t s) {
  const bool tr = a.t.trace != nullptr || a.d.trace != nullptr;
  MRT_DTYPE_DISPATCH(dt, {
    if (tr)
      hipLaunchKernelGGL((k_frame<T, true>), dim3(grid), dim3(kPersistThreads), lds, s, a);
    else
      hipLaunchKernelGGL((k_frame<T, false>), dim3(grid), dim3(kPersistThreads), lds, s, a);
  });
  MRT_HIP_CHECK(hipGetLastError());
}

void launch_levels(DType dt, const FrameArgs& a, int grid, size_t lds, hipStream_t s) {
  MRT_REQUIRE(a.d.sp.decided != nullptr && a.d.tokens != nullptr && a.d.noise != nullptr,
              "levels launch: the decided count, the token and the noise buffers are required");
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL((k_levels<T>), dim3(grid), dim3(kPersistThreads), lds, s, a));
  MRT_HIP_CHECK(hipGetLastError());
}

void gumbel_table(const uint64_t* seed, int frames, int L, int C, float* out, hipStream_t s) {
  const int n = frames * L * C;
  const int blocks = std::min((n + 255) / 256, 1024);
  hipLaunchKernelGGL(k_gumbel_table, dim3(blocks), dim3(256), 0, s, seed, frames, L, C, out);
  MRT_HIP_CHECK(hipGetLastError());
}

}  // namespace mrt
