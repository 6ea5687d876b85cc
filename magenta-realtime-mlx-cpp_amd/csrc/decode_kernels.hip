// Batch-1 (2 CFG rows) decode kernels for gfx950: GEMVs with fused RMSNorm
// prologue and fused epilogues, ring-KV self-attention with the T5 relative
// position bias, split-key cross-attention, embedding gathers.
//
// Every weight byte is read exactly once per call with 16-byte vector loads
// (one 1 KiB coalesced segment per wave instruction); the work per byte is 2
// FMAs (2 CFG rows), so these kernels are HBM/MALL-bandwidth bound.
#include <algorithm>
#include <cmath>

#include "device_utils.hpp"
#include "kernels.hpp"

namespace mrt {
namespace {

constexpr int kGemvThreads = 256;
constexpr int kMaxSelfLen = 1024;
constexpr int kMaxCrossChunk = 256;

// ---- epilogues ----------------------------------------------------------------

template <typename T, int NB>
struct EpiStore {
  T* y;
  int ldy;
  __device__ void operator()(int n, const float (&a)[1][NB]) const {
#pragma unroll
    for (int b = 0; b < NB; ++b) y[(size_t)b * ldy + n] = St<T>::st(a[0][b]);
  }
};

template <typename T, int NB>
struct EpiF32 {
  float* y;
  int ldy;
  __device__ void operator()(int n, const float (&a)[1][NB]) const {
#pragma unroll
    for (int b = 0; b < NB; ++b) y[(size_t)b * ldy + n] = St<T>::rnd(a[0][b]);
  }
};

template <typename T, int NB>
struct EpiResid {
  T* r;
  int ldr;
  __device__ void operator()(int n, const float (&a)[1][NB]) const {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      T* p = r + (size_t)b * ldr + n;
      *p = St<T>::st(St<T>::ld(*p) + St<T>::rnd(a[0][b]));
    }
  }
};

template <typename T, int NB>
struct EpiQKV {
  T* q;
  T* kc;
  T* vc;
  int HD, H, Lmax, pos;
  __device__ void operator()(int n, const float (&a)[1][NB]) const {
    const int which = n / HD;
    const int nn = n - which * HD;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const T v = St<T>::st(a[0][b]);
      if (which == 0) {
        q[(size_t)b * HD + nn] = v;
      } else {
        const int h = nn >> 6, d = nn & 63;
        T* c = which == 1 ? kc : vc;
        c[(((size_t)b * H + h) * Lmax + pos) * 64 + d] = v;
      }
    }
  }
};

template <typename T, int NB>
struct EpiGeglu {
  T* h;
  int ldh;
  __device__ void operator()(int j, const float (&a)[2][NB]) const {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float g = gelu_t<T>(St<T>::rnd(a[0][b]));
      h[(size_t)b * ldh + j] = St<T>::st(g * St<T>::rnd(a[1][b]));
    }
  }
};

// ---- GEMV ---------------------------------------------------------------------
// Block = 4 waves; each wave owns R consecutive outputs.  P = 1: output n is
// weight row n.  P = 2: output j reads the gate/up row pair of the 32-row
// packed wi_0/wi_1 matrix.  Lane l covers 16-byte chunks l, l+64, ... of each
// row, so one wave instruction streams a contiguous 1 KiB of the row.
template <typename T, int NB, int R, int P, class Epi>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(const T* __restrict__ W, int nout, int K,
                                                     const T* __restrict__ X, int ldx,
                                                     const T* __restrict__ g, float eps, Epi epi) {
  using S = St<T>;
  constexpr int V = S::kVec;
  extern __shared__ float xs[];  // NB * K activations (normalised when g != null)
  __shared__ float red[4][NB];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;

  float ss[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    ss[b] = 0.f;
    for (int k = tid; k < K; k += kGemvThreads) {
      const float v = S::ld(X[(size_t)b * ldx + k]);
      xs[b * K + k] = v;
      ss[b] += v * v;
    }
  }
  if (g != nullptr) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float t = wave_sum(ss[b]);
      if (lane == 0) red[wid][b] = t;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float tot = red[0][b] + red[1][b] + red[2][b] + red[3][b];
      const float inv = 1.0f / sqrtf(tot / (float)K + eps);
      for (int k = tid; k < K; k += kGemvThreads)
        xs[b * K + k] = S::rnd(S::rnd(xs[b * K + k] * inv) * S::ld(g[k]));
    }
  }
  __syncthreads();

  const int o0 = (blockIdx.x * 4 + wid) * R;
  if (o0 >= nout) return;  // no barrier below this point
  const T* wrow[R][P];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int o = (o0 + r < nout) ? o0 + r : o0;
    if constexpr (P == 1) {
      wrow[r][0] = W + (size_t)o * K;
    } else {
      const size_t gr = (size_t)(o >> 5) * 64 + (o & 31);
      wrow[r][0] = W + gr * K;
      wrow[r][1] = W + (gr + 32) * K;
    }
  }
  float acc[R][P][NB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[r][p][b] = 0.f;

  const int nch = K / V;
  for (int c = lane; c < nch; c += 64) {
    uint4 wv[R][P];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p)
        wv[r][p] = ld_nt16(wrow[r][p] + (size_t)c * V);
    float xv[NB][V];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int e = 0; e < V; ++e) xv[b][e] = xs[b * K + c * V + e];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const T* we = reinterpret_cast<const T*>(&wv[r][p]);
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float w = S::ld(we[e]);
#pragma unroll
          for (int b = 0; b < NB; ++b) acc[r][p][b] = fmaf(w, xv[b][e], acc[r][p][b]);
        }
      }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[r][p][b] = wave_sum(acc[r][p][b]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (o0 + r < nout) epi(o0 + r, acc[r]);
  }
}

template <typename T, int NB, int P, class Epi>
void launch_gemv_t(const void* W, int nout, int K, const void* X, int ldx, NormArg norm, Epi epi,
                   hipStream_t s) {
  MRT_REQUIRE(K % St<T>::kVec == 0, "gemv: K must be a multiple of the vector width");
  const size_t lds = (size_t)NB * K * sizeof(float);
  MRT_REQUIRE(lds <= 64 * 1024, "gemv: activation tile exceeds 64 KiB of LDS");
  auto go = [&](auto rtag) {
    constexpr int R = decltype(rtag)::value;
    const int blocks = (nout + 4 * R - 1) / (4 * R);
    hipLaunchKernelGGL((k_gemv<T, NB, R, P, Epi>), dim3(blocks), dim3(kGemvThreads), lds, s,
                       static_cast<const T*>(W), nout, K, static_cast<const T*>(X), ldx,
                       static_cast<const T*>(norm.g), norm.eps, epi);
  };
  // Aim for >= 256 workgroups (one per CU) while keeping >= 2 rows in flight
  // per wave on the larger matrices.
  if (nout >= 8192 * P)
    go(std::integral_constant<int, 4>{});
  else if (nout >= 2048)
    go(std::integral_constant<int, 2>{});
  else
    go(std::integral_constant<int, 1>{});
  MRT_HIP_CHECK(hipGetLastError());
}

}  // namespace

// The public launchers spell out the (dtype, nb) dispatch explicitly.
#define MRT_NB_DISPATCH(nb, BODY)                                          \
  switch (nb) {                                                            \
    case 1: { constexpr int NB = 1; BODY; break; }                         \
    case 2: { constexpr int NB = 2; BODY; break; }                         \
    case 4: { constexpr int NB = 4; BODY; break; }                         \
    default: throw Error(1, "decode kernels support nb in {1, 2, 4}");      \
  }

void gemv_store(DType dt, int nb, const void* W, int N, int K, const void* X, int ldx,
                NormArg norm, void* Y, int ldy, hipStream_t s) {
  MRT_DTYPE_DISPATCH(dt, MRT_NB_DISPATCH(nb, (launch_gemv_t<T, NB, 1>(W, N, K, X, ldx, norm,
                                                                      EpiStore<T, NB>{static_cast<T*>(Y), ldy}, s))));
}

void gemv_f32(DType dt, int nb, const void* W, int N, int K, const void* X, int ldx,
              NormArg norm, float* Y, int ldy, hipStream_t s) {
  MRT_DTYPE_DISPATCH(dt, MRT_NB_DISPATCH(nb, (launch_gemv_t<T, NB, 1>(W, N, K, X, ldx, norm,
                                                                      EpiF32<T, NB>{Y, ldy}, s))));
}

void gemv_resid(DType dt, int nb, const void* W, int N, int K, const void* X, int ldx,
                NormArg norm, void* R, int ldr, hipStream_t s) {
  MRT_DTYPE_DISPATCH(dt, MRT_NB_DISPATCH(nb, (launch_gemv_t<T, NB, 1>(W, N, K, X, ldx, norm,
                                                                      EpiResid<T, NB>{static_cast<T*>(R), ldr}, s))));
}

void gemv_qkv(DType dt, int nb, const void* W, int HD, int K, const void* X, int ldx,
              NormArg norm, void* Q, void* Kc, void* Vc, int H, int Lmax, int pos,
              hipStream_t s) {
  MRT_REQUIRE(HD == H * 64, "gemv_qkv: head dim must be 64");
  MRT_REQUIRE(pos >= 0 && pos < Lmax, "gemv_qkv: ring position out of range");
  MRT_DTYPE_DISPATCH(dt, MRT_NB_DISPATCH(nb, (launch_gemv_t<T, NB, 1>(
                                                 W, 3 * HD, K, X, ldx, norm,
                                                 EpiQKV<T, NB>{static_cast<T*>(Q), static_cast<T*>(Kc),
                                                               static_cast<T*>(Vc), HD, H, Lmax, pos},
                                                 s))));
}

void gemv_geglu(DType dt, int nb, const void* W01, int F, int K, const void* X, int ldx,
                NormArg norm, void* Hout, int ldh, hipStream_t s) {
  MRT_REQUIRE(F % 32 == 0, "gemv_geglu: d_ff must be a multiple of 32");
  MRT_DTYPE_DISPATCH(dt, MRT_NB_DISPATCH(nb, (launch_gemv_t<T, NB, 2>(W01, F, K, X, ldx, norm,
                                                                      EpiGeglu<T, NB>{static_cast<T*>(Hout), ldh}, s))));
}

// ---- self-attention over the ring KV ----------------------------------------------
namespace {

// qpos_ptr non-null: the query position is read from it and len = qpos + 1.
// pos_rows > 0: query row b is position b / pos_rows of ring row b % pos_rows
// (all positions of one frame at once, causal: len = position + 1).
template <typename T>
__global__ __launch_bounds__(64) void k_self_attn(const T* __restrict__ Q, const T* __restrict__ Kc,
                                                  const T* __restrict__ Vc, int H, int Lmax, int len,
                                                  int qpos, const int* __restrict__ qpos_ptr, int pos_rows,
                                                  const T* __restrict__ bias_tab,
                                                  const int* __restrict__ buckets, const T* __restrict__ bias_row,
                                                  T* __restrict__ out) {
  using S = St<T>;
  constexpr int V = S::kVec;
  const int bh = blockIdx.x, b = bh / H, h = bh - b * H, lane = threadIdx.x;
  if (qpos_ptr != nullptr) {
    qpos = *qpos_ptr;
    len = qpos + 1;
  }
  int rb = b;  // ring row
  if (pos_rows > 0) {
    rb = b % pos_rows;
    qpos = b / pos_rows;
    len = qpos + 1;
  }
  const int HD = H * 64;
  __shared__ float qs[64];
  __shared__ float ps[kMaxSelfLen];
  const T* Kp = Kc + ((size_t)rb * H + h) * Lmax * 64;
  const T* Vp = Vc + ((size_t)rb * H + h) * Lmax * 64;
  if (len <= 64) {
    // One key per lane: the bias, K row and V row of key j = lane are all
    // requested before any is used (one round trip), V goes to LDS, and the
    // sums run in the order of the general path below (identical results).
    __shared__ __align__(16) T vs[64 * 64];
    const int j = lane;
    const bool live = j < len;
    const int jc = min(j, len - 1);
    const float qv = S::ld(Q[(size_t)b * HD + h * 64 + lane]);
    int bk = 0;
    float bias = 0.f;
    if (bias_row != nullptr)
      bias = S::ld(bias_row[h * len + jc]);
    else
      bk = buckets[qpos - jc];
    uint4 kv[64 / V], vv[64 / V];
#pragma unroll
    for (int i = 0; i < 64 / V; ++i) {
      kv[i] = *reinterpret_cast<const uint4*>(Kp + (size_t)jc * 64 + i * V);
      vv[i] = *reinterpret_cast<const uint4*>(Vp + (size_t)jc * 64 + i * V);
    }
    if (bias_row == nullptr) bias = S::ld(bias_tab[bk * H + h]);
    qs[lane] = qv;
#pragma unroll
    for (int i = 0; i < 64 / V; ++i) *reinterpret_cast<uint4*>(vs + j * 64 + i * V) = vv[i];
    __syncthreads();
    float sc = 0.f;
#pragma unroll
    for (int i = 0; i < 64 / V; ++i) {
      const T* ke = reinterpret_cast<const T*>(&kv[i]);
#pragma unroll
      for (int e = 0; e < V; ++e) sc = fmaf(qs[i * V + e], S::ld(ke[e]), sc);
    }
    sc += bias;
    const float m = wave_max(live ? sc : -INFINITY);
    const float pj = live ? expf(sc - m) : 0.f;
    ps[j] = pj;
    const float sum = wave_sum(pj);
    __syncthreads();
    float o = 0.f;
    for (int t = 0; t < len; ++t) o = fmaf(ps[t], S::ld(vs[t * 64 + lane]), o);
    out[(size_t)b * HD + h * 64 + lane] = S::st(o / sum);
    return;
  }
  qs[lane] = S::ld(Q[(size_t)b * HD + h * 64 + lane]);
  __syncthreads();
  float mx = -INFINITY;
  for (int j = lane; j < len; j += 64) {
    const T* kr = Kp + (size_t)j * 64;
    float sc = 0.f;
#pragma unroll
    for (int d = 0; d < 64; d += V) {
      const uint4 kv = *reinterpret_cast<const uint4*>(kr + d);
      const T* ke = reinterpret_cast<const T*>(&kv);
#pragma unroll
      for (int e = 0; e < V; ++e) sc = fmaf(qs[d + e], S::ld(ke[e]), sc);
    }
    sc += bias_row != nullptr ? S::ld(bias_row[h * len + j]) : S::ld(bias_tab[buckets[qpos - j] * H + h]);
    ps[j] = sc;
    mx = fmaxf(mx, sc);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  for (int j = lane; j < len; j += 64) {
    const float p = expf(ps[j] - mx);
    ps[j] = p;
    sum += p;
  }
  sum = wave_sum(sum);
  __syncthreads();
  float o = 0.f;
  for (int j = 0; j < len; ++j) o = fmaf(ps[j], S::ld(Vp[(size_t)j * 64 + lane]), o);
  out[(size_t)b * HD + h * 64 + lane] = S::st(o / sum);
}

// Full-sequence self attention (depth_forward_full, model.cpp:243-268): one
// 64-lane block per (row m = b*K + i, head h); lane j scores key j, lane d
// then sums dimension d of the softmax-weighted values.
template <typename T>
__global__ __launch_bounds__(64) void k_full_attn(const T* __restrict__ qkv, int K, int H,
                                                  const T* __restrict__ explicit_bias,
                                                  const T* __restrict__ bias_tab, const int* __restrict__ buckets,
                                                  int causal, T* __restrict__ out) {
  using S = St<T>;
  const int mh = blockIdx.x, m = mh / H, h = mh - m * H, lane = threadIdx.x;
  const int b = m / K, i = m - b * K;
  const int HD = H * 64, ld = 3 * HD;
  __shared__ float qs[64];
  __shared__ float ps[64];
  qs[lane] = S::ld(qkv[(size_t)m * ld + h * 64 + lane]);
  __syncthreads();
  const int len = causal ? i + 1 : K;
  float sc = -INFINITY;
  if (lane < len) {
    const T* kr = qkv + (size_t)(b * K + lane) * ld + HD + h * 64;
    float acc = 0.f;
    for (int d = 0; d < 64; ++d) acc = fmaf(qs[d], S::ld(kr[d]), acc);
    const float bias = explicit_bias != nullptr ? S::ld(explicit_bias[((size_t)h * K + i) * K + lane])
                                                : S::ld(bias_tab[buckets[max(i - lane, 0)] * H + h]);
    sc = acc + bias;
  }
  const float mx = wave_max(sc);
  const float p = lane < len ? expf(sc - mx) : 0.f;
  const float sum = wave_sum(p);
  ps[lane] = p;
  __syncthreads();
  float o = 0.f;
  for (int j = 0; j < len; ++j) o = fmaf(ps[j], S::ld(qkv[(size_t)(b * K + j) * ld + 2 * HD + h * 64 + lane]), o);
  out[(size_t)m * HD + h * 64 + lane] = S::st(o / sum);
}

// Partial softmax-attention of one (row, head) over one block of keys.
template <typename T>
__global__ __launch_bounds__(64) void k_cross_part(const T* __restrict__ Q, const T* __restrict__ Kc,
                                                   const T* __restrict__ Vc, int H, int S, int nsplit,
                                                   float* __restrict__ part) {
  using St_ = St<T>;
  constexpr int V = St_::kVec;
  const int blk = blockIdx.x, bh = blk / nsplit, sp = blk - bh * nsplit;
  const int b = bh / H, h = bh - b * H, lane = threadIdx.x;
  const int HD = H * 64;
  const int chunk = (S + nsplit - 1) / nsplit;
  const int j0 = sp * chunk, j1 = min(S, j0 + chunk);
  __shared__ float qs[64];
  __shared__ float ps[kMaxCrossChunk];
  qs[lane] = St_::ld(Q[(size_t)b * HD + h * 64 + lane]);
  __syncthreads();
  const T* Kp = Kc + (size_t)bh * S * 64;
  const T* Vp = Vc + (size_t)bh * S * 64;
  float mx = -INFINITY;
  for (int j = j0 + lane; j < j1; j += 64) {
    const T* kr = Kp + (size_t)j * 64;
    float sc = 0.f;
#pragma unroll
    for (int d = 0; d < 64; d += V) {
      const uint4 kv = ld_nt16(kr + d);
      const T* ke = reinterpret_cast<const T*>(&kv);
#pragma unroll
      for (int e = 0; e < V; ++e) sc = fmaf(qs[d + e], St_::ld(ke[e]), sc);
    }
    ps[j - j0] = sc;
    mx = fmaxf(mx, sc);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  for (int j = j0 + lane; j < j1; j += 64) {
    const float p = expf(ps[j - j0] - mx);
    ps[j - j0] = p;
    sum += p;
  }
  sum = wave_sum(sum);
  __syncthreads();
  float o = 0.f;
  for (int j = j0; j < j1; ++j) o = fmaf(ps[j - j0], St_::ld(Vp[(size_t)j * 64 + lane]), o);
  float* dst = part + (size_t)blk * 66;
  if (lane == 0) {
    dst[0] = mx;
    dst[1] = sum;
  }
  dst[2 + lane] = o;
}

template <typename T>
__global__ __launch_bounds__(64) void k_cross_combine(const float* __restrict__ part, int H, int nsplit,
                                                      T* __restrict__ out) {
  const int bh = blockIdx.x, b = bh / H, h = bh - b * H, lane = threadIdx.x;
  const float* p = part + (size_t)bh * nsplit * 66;
  float M = -INFINITY;
  for (int i = 0; i < nsplit; ++i) M = fmaxf(M, p[i * 66]);
  float L = 0.f, O = 0.f;
  for (int i = 0; i < nsplit; ++i) {
    const float m = p[i * 66];
    if (m == -INFINITY) continue;
    const float c = expf(m - M);
    L = fmaf(p[i * 66 + 1], c, L);
    O = fmaf(p[i * 66 + 2 + lane], c, O);
  }
  out[(size_t)b * H * 64 + h * 64 + lane] = St<T>::st(O / L);
}

template <typename T>
__global__ void k_embed_rows(const T* __restrict__ emb, int D, const int* __restrict__ ids,
                             T* __restrict__ out) {
  const int r = blockIdx.x;
  const T* src = emb + (size_t)ids[r] * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) out[(size_t)r * D + d] = src[d];
}

__global__ void k_copy16(uint4* __restrict__ dst, const uint4* __restrict__ src, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

__global__ void k_copy1(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

template <typename T>
__global__ void k_embed_fill(const T* __restrict__ emb, int D, int id, T* __restrict__ out) {
  const int r = blockIdx.x;
  const T* src = emb + (size_t)id * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) out[(size_t)r * D + d] = src[d];
}

}  // namespace

void self_attn(DType dt, int nb, const void* Q, const void* Kc, const void* Vc, int H, int Lmax,
               int len, int qpos, const void* bias_tab, const int* buckets, void* out,
               hipStream_t s, const void* bias_row) {
  MRT_REQUIRE(len >= 1 && len <= kMaxSelfLen && len <= Lmax, "self_attn: bad cache length");
  MRT_REQUIRE(qpos >= len - 1, "self_attn: query precedes keys");
  self_attn_at(dt, nb, Q, Kc, Vc, H, Lmax, len, qpos, nullptr, bias_tab, buckets, out, s, 0, bias_row);
}

void self_attn_at(DType dt, int nb, const void* Q, const void* Kc, const void* Vc, int H, int Lmax, int len,
                  int qpos, const int* qpos_ptr, const void* bias_tab, const int* buckets, void* out,
                  hipStream_t s, int pos_rows, const void* bias_row) {
  MRT_REQUIRE(qpos_ptr == nullptr || Lmax <= kMaxSelfLen, "self_attn: ring longer than the kernel's score buffer");
  MRT_REQUIRE(pos_rows == 0 || (nb % pos_rows == 0 && nb / pos_rows <= Lmax && Lmax <= kMaxSelfLen),
              "self_attn: positions exceed the ring");
  MRT_REQUIRE(bias_row == nullptr || (qpos_ptr == nullptr && pos_rows == 0),
              "self_attn: an explicit bias needs a host-known query position");
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_self_attn<T>, dim3(nb * H), dim3(64), 0, s, (const T*)Q, (const T*)Kc,
                                            (const T*)Vc, H, Lmax, len, qpos, qpos_ptr, pos_rows,
                                            (const T*)bias_tab, buckets, (const T*)bias_row, (T*)out));
  MRT_HIP_CHECK(hipGetLastError());
}

namespace {

// Step f's bias rows (H, f + 1) at element H * f * (f + 1) / 2:
// out[..][h][j] = table[bucket[f - j], h] for j <= f.
template <typename T>
__global__ void k_bias_rows(const T* __restrict__ table, const int* __restrict__ buckets, int H, int n,
                            T* __restrict__ out) {
  const int f = blockIdx.x;
  T* o = out + (size_t)H * f * (f + 1) / 2;
  for (int e = threadIdx.x; e < H * (f + 1); e += blockDim.x) {
    const int h = e / (f + 1), j = e - h * (f + 1);
    o[e] = table[buckets[f - j] * H + h];
  }
}

}  // namespace

void bias_rows(DType dt, const void* table, const int* buckets, int H, int n, void* out, hipStream_t s) {
  MRT_REQUIRE(n >= 1 && H >= 1, "bias_rows: empty request");
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_bias_rows<T>, dim3(n), dim3(256), 0, s, (const T*)table, buckets, H, n,
                                            (T*)out));
  MRT_HIP_CHECK(hipGetLastError());
}

void full_attn(DType dt, int nb, int K, int H, const void* qkv, const void* explicit_bias, const void* bias_tab,
               const int* buckets, bool causal, void* out, hipStream_t s) {
  MRT_REQUIRE(nb >= 1 && K >= 1 && K <= 64, "full_attn: K must be in [1, 64]");
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_full_attn<T>, dim3(nb * K * H), dim3(64), 0, s, (const T*)qkv, K, H,
                                            (const T*)explicit_bias, (const T*)bias_tab, buckets, causal ? 1 : 0,
                                            (T*)out));
  MRT_HIP_CHECK(hipGetLastError());
}

int cross_attn_splits(int S) {
  int n = (S + 63) / 64;
  return n < 1 ? 1 : n;
}

void cross_attn(DType dt, int nb, const void* Q, const void* Kc, const void* Vc, int H, int S,
                void* out, float* part, int nsplit, hipStream_t s) {
  MRT_REQUIRE(S >= 1, "cross_attn: empty encoder output");
  MRT_REQUIRE((S + nsplit - 1) / nsplit <= kMaxCrossChunk, "cross_attn: key block too large");
  MRT_DTYPE_DISPATCH(dt, {
    hipLaunchKernelGGL(k_cross_part<T>, dim3(nb * H * nsplit), dim3(64), 0, s, (const T*)Q, (const T*)Kc,
                       (const T*)Vc, H, S, nsplit, part);
    hipLaunchKernelGGL(k_cross_combine<T>, dim3(nb * H), dim3(64), 0, s, part, H, nsplit, (T*)out);
  });
  MRT_HIP_CHECK(hipGetLastError());
}

void embed_rows(DType dt, const void* emb, int D, const int* ids, int rows, void* out,
                hipStream_t s) {
  if (rows <= 0) return;
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_embed_rows<T>, dim3(rows), dim3(256), 0, s, (const T*)emb, D, ids,
                                            (T*)out));
  MRT_HIP_CHECK(hipGetLastError());
}

void copy_dev(void* dst, const void* src, size_t bytes, hipStream_t s) {
  if (bytes == 0 || dst == src) return;
  const bool aligned = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) | bytes) & 15) == 0;
  if (aligned) {
    const size_t n = bytes / 16;
    const int blocks = (int)std::min<size_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(k_copy16, dim3(blocks), dim3(256), 0, s, static_cast<uint4*>(dst),
                       static_cast<const uint4*>(src), n);
  } else {
    const int blocks = (int)std::min<size_t>((bytes + 255) / 256, 1024);
    hipLaunchKernelGGL(k_copy1, dim3(blocks), dim3(256), 0, s, static_cast<uint8_t*>(dst),
                       static_cast<const uint8_t*>(src), bytes);
  }
  MRT_HIP_CHECK(hipGetLastError());
}

void embed_fill(DType dt, const void* emb, int D, int id, int rows, void* out, hipStream_t s) {
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_embed_fill<T>, dim3(rows), dim3(256), 0, s, (const T*)emb, D, id,
                                            (T*)out));
  MRT_HIP_CHECK(hipGetLastError());
}

}  // namespace mrt
