// Batched-stream decode kernels for gfx950: B independent streams decoded
// together, R = 2B activation rows (both CFG rows of every stream), R <= 64.
//
// At R = 64 every weight row meets 64 activation rows, so the projections are
// skinny GEMMs and run on the matrix cores: v_mfma_f32_16x16x32_bf16, one
// block per 16 output columns, the 8 waves of a block splitting K and summing
// their partial tiles through LDS in a fixed order (deterministic).  The
// activations (R x K, at most 360 KB) are read by every block from L2; the
// weights stream from HBM/MALL once per step.
#include <algorithm>
#include <type_traits>

#include "batch.hpp"
#include "device_utils.hpp"
#include "kernels.hpp"

namespace mrt {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBgCols = 16;   // output columns per block
constexpr int kBgChunk = 1;   // k-steps (of 32) per loop step of a wave: fewer live registers (per 32-stream chunk: 8: 243.6 ms, 4: 238.7, 2: 234.2, 1: 232.2)
constexpr int kBgWaves = 8;   // waves per block, splitting K
constexpr int kBgThreads = 64 * kBgWaves;

// ---- epilogues: op(m, n, v[P]) with v the fp32 sums of output (m, n) ---------------

struct BStore {
  bf16* y;
  int ldy;
  __device__ void operator()(int m, int n, const float (&v)[1]) const { y[(size_t)m * ldy + n] = St<bf16>::st(v[0]); }
};

struct BF32 {
  float* y;
  int ldy;
  __device__ void operator()(int m, int n, const float (&v)[1]) const { y[(size_t)m * ldy + n] = St<bf16>::rnd(v[0]); }
};

// Residual update; the residual values are read at the start of the kernel
// (pre), so the epilogue does not wait for them.  `ssq` non-null: the sum of
// squares of each updated row over the block's 16 columns goes to
// ssq[m * ntiles + tile], the partials a normalised consumer reads (BNorm).
struct BResid {
  bf16* r;
  int ldr;
  float* ssq;
  static constexpr bool kPre = true;
  __device__ float pre(int m, int n) const { return St<bf16>::ld(r[(size_t)m * ldr + n]); }
  __device__ float operator()(int m, int n, const float (&v)[1], float x) const {
    const bf16 y = St<bf16>::st(x + St<bf16>::rnd(v[0]));
    r[(size_t)m * ldr + n] = y;
    return St<bf16>::ld(y);
  }
};

// n < HD: q; else k / v into ring slot pos (fixed, or *pos_ptr) of the caches
// laid out (R, H, Lmax, 64).
struct BQKV {
  bf16* q;
  bf16* kc;
  bf16* vc;
  int HD, H, Lmax, pos;
  const int* pos_ptr;
  __device__ void operator()(int m, int n, const float (&v)[1]) const {
    const bf16 o = St<bf16>::st(v[0]);
    const int which = n / HD, nn = n - which * HD;
    if (which == 0) {
      q[(size_t)m * HD + nn] = o;
    } else {
      const int p = pos_ptr ? *pos_ptr : pos;
      bf16* c = which == 1 ? kc : vc;
      c[(((size_t)m * H + (nn >> 6)) * Lmax + p) * 64 + (nn & 63)] = o;
    }
  }
};

// Rows m = P * pos + r (the positions of one frame, rows r = 0..P-1 each):
// q -> Q row m; k / v -> ring slot pos of ring row r, caches (P, H, Lmax, 64).
struct BQKVPos {
  bf16* q;
  bf16* kc;
  bf16* vc;
  int HD, H, Lmax, P;
  __device__ void operator()(int m, int n, const float (&v)[1]) const {
    const bf16 o = St<bf16>::st(v[0]);
    const int which = n / HD, nn = n - which * HD;
    if (which == 0) {
      q[(size_t)m * HD + nn] = o;
    } else {
      const int r = m % P, pos = m / P;
      bf16* c = which == 1 ? kc : vc;
      c[(((size_t)r * H + (nn >> 6)) * Lmax + pos) * 64 + (nn & 63)] = o;
    }
  }
};

struct BGeglu {
  bf16* h;
  int ldh;
  __device__ void operator()(int m, int j, const float (&v)[2]) const {
    const float g = gelu_t<bf16>(St<bf16>::rnd(v[0]));
    h[(size_t)m * ldh + j] = St<bf16>::st(g * St<bf16>::rnd(v[1]));
  }
};

__device__ __forceinline__ int bg_geglu_row(int j, int p) { return (j >> 5) * 64 + (j & 31) + 32 * p; }

// Y (M x nout) = X (M x K) . W^T with epilogue.  P = 1: output n reads weight
// row n; P = 2: output j reads the gate / up rows of the 32-row packed wi_0 /
// wi_1 matrix.  Operand fragments of the 16x16x32 MFMA: lane l holds row
// (l % 16) of A and column (l % 16) of B over k = 8 (l / 16) .. + 7 of the
// step; the 4 accumulators of lane l hold column l % 16, rows 4 (l / 16) + i.
// Wave w of the 8 takes k-steps w, w + 8, ...; the 8 partial tiles are summed
// in wave order.  Rows past M are zero, columns past nout re-read the last row
// and are not stored.
// RMSNorm of the activation rows applied as they are loaded (modules.cpp
// RMSNorm, as rmsnorm_rows): row m of X is the raw residual, its sum of squares
// the `parts` partials at ssq + m * parts (summed in order), element k scaled
// to bf16(bf16(x * inv) * g[k]) with inv = 1 / sqrt(ss / K + eps).
struct BNormDev {
  const bf16* g;
  const float* ssq;
  int parts;
  float eps;
};

// Sum over each 16-lane row of a wave, complete in the row's last lane.
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, true));   // quad [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, true));   // quad [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, true));  // row_shr:4
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, true));  // row_shr:8
  return v;
}

// Eight bf16 activations scaled by the row's inverse RMS and the norm weights.
__device__ __forceinline__ uint4 norm8(uint4 x, uint4 g, float inv) {
  const bf16* xe = reinterpret_cast<const bf16*>(&x);
  const bf16* ge = reinterpret_cast<const bf16*>(&g);
  uint4 out;
  bf16* oe = reinterpret_cast<bf16*>(&out);
#pragma unroll
  for (int e = 0; e < 8; ++e) oe[e] = St<bf16>::st(St<bf16>::rnd(St<bf16>::ld(xe[e]) * inv) * St<bf16>::ld(ge[e]));
  return out;
}

template <class Epi, class = void>
struct HasPre {
  static constexpr bool value = false;
};
template <class Epi>
struct HasPre<Epi, decltype((void)Epi::kPre)> {
  static constexpr bool value = Epi::kPre;
};

// Block (tile, ms) of the grid computes output columns [16 tile, +16) for the
// MT row tiles [MT ms, +MT) of 16 rows: blocks sharing a column tile are
// tile + ntiles * ms, on the same XCD when ntiles % 8 == 0 (blocks are dealt to
// the 8 XCDs in turn), so the weight tile comes from HBM once and from that
// XCD's L2 for the others.
template <int P, int MT, bool NORM, class Epi>
__global__ __launch_bounds__(kBgThreads) void k_bgemm(const bf16* __restrict__ X, int M, int K,
                                                      const bf16* __restrict__ W, int nout, int ntiles, Epi epi,
                                                      long w_group_stride, BNormDev nrm) {
  // blockIdx.y = group g (grouped launch): rows [g M, g M + M) of X against
  // W + g * w_group_stride, outputs at rows g M + m
  const int grow = blockIdx.y * M;
  X += (size_t)grow * K;
  W += blockIdx.y * w_group_stride;
  constexpr int kRows = 16 * MT;
  constexpr int kOut = kRows * kBgCols;                        // outputs of the block
  constexpr int kPer = (kOut + kBgThreads - 1) / kBgThreads;  // epilogue outputs per thread
  __shared__ float part[kBgWaves][kRows][kBgCols + 1];  // one part (gate / up) at a time
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int tile = blockIdx.x % ntiles, m0 = (blockIdx.x / ntiles) * kRows;
  const int j0 = tile * kBgCols;
  const int c16 = lane & 15, kg = lane >> 4;
  const bf16* wrow[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int j = min(j0 + c16, nout - 1);
    wrow[p] = W + (size_t)(P == 1 ? j : bg_geglu_row(j, p)) * K + kg * 8;
  }
  const bf16* xrow[MT];
  bool xin[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = m0 + 16 * t + c16;
    xin[t] = m < M;
    xrow[t] = X + (size_t)min(m, M - 1) * K + kg * 8;
  }
  float inv[MT];
  const bf16* grow_g = nullptr;
  if constexpr (NORM) {
    // eight lanes per row: with 64 partials lane q sums [8 q, 8 q + 8) in
    // order (other counts: lane 0 sums them all), and the eight sums meet by
    // lane exchange (the same total in each lane)
    __shared__ float inv_s[kRows];
    const int r = tid >> 3, q = tid & 7;
    float ss = 0.f;
    if (r < kRows) {
      const float* sp = nrm.ssq + (size_t)(grow + min(m0 + r, M - 1)) * nrm.parts;
      if (nrm.parts == 64) {
        const float4 u = *reinterpret_cast<const float4*>(sp + 8 * q);
        const float4 w = *reinterpret_cast<const float4*>(sp + 8 * q + 4);
        ss = ((((((u.x + u.y) + u.z) + u.w) + w.x) + w.y) + w.z) + w.w;
      } else if (q == 0) {
        for (int t = 0; t < nrm.parts; ++t) ss += sp[t];
      }
    }
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 4);
    if (r < kRows && q == 0) inv_s[r] = 1.0f / sqrtf(ss / (float)K + nrm.eps);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < MT; ++t) inv[t] = inv_s[16 * t + c16];
    grow_g = nrm.g + kg * 8;
  }
  float pre[kPer];
  if constexpr (HasPre<Epi>::value) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = tid + kBgThreads * i, m = m0 + idx / kBgCols, n = j0 + idx % kBgCols;
      pre[i] = (idx < kOut && m < M && n < nout) ? epi.pre(grow + m, n) : 0.f;
    }
  }
  f32x4_t acc[P][MT];
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[p][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nks = K / 32;
  for (int s0 = wid; s0 < nks; s0 += kBgWaves * kBgChunk) {
    uint4 b[kBgChunk][P], a[kBgChunk][MT], gk[NORM ? kBgChunk : 1];
#pragma unroll
    for (int c = 0; c < kBgChunk; ++c) {
      const int ks = s0 + kBgWaves * c;
      if (ks < nks) {
#pragma unroll
        for (int p = 0; p < P; ++p) b[c][p] = ld_g16(wrow[p] + ks * 32);
#pragma unroll
        for (int t = 0; t < MT; ++t) a[c][t] = xin[t] ? ld_g16(xrow[t] + ks * 32) : make_uint4(0u, 0u, 0u, 0u);
        if constexpr (NORM) gk[c] = ld_g16(grow_g + ks * 32);
      }
    }
#pragma unroll
    for (int c = 0; c < kBgChunk; ++c) {
      if (s0 + kBgWaves * c < nks) {
        if constexpr (NORM) {
#pragma unroll
          for (int t = 0; t < MT; ++t) a[c][t] = norm8(a[c][t], gk[c], inv[t]);
        }
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int t = 0; t < MT; ++t)
            acc[p][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[c][t]),
                                                                __builtin_bit_cast(bf16x8_t, b[c][p]), acc[p][t], 0, 0, 0);
      }
    }
  }
  float v[kPer][P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    if (p > 0) __syncthreads();  // the previous part has been read
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[wid][16 * t + 4 * kg + i][c16] = acc[p][t][i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = min(tid + kBgThreads * i, kOut - 1), m = idx / kBgCols, n = idx % kBgCols;
      float a = part[0][m][n];
#pragma unroll
      for (int w = 1; w < kBgWaves; ++w) a += part[w][m][n];
      v[i][p] = a;
    }
  }
  if constexpr (std::is_same<Epi, BResid>::value) {
    // lanes 16 r .. 16 r + 15 of a wave hold the 16 columns of one output row
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = tid + kBgThreads * i, m = m0 + idx / kBgCols, n = idx % kBgCols;
      const bool ok = idx < kOut && m < M && j0 + n < nout;
      const float y = ok ? epi(grow + m, j0 + n, v[i], pre[i]) : 0.f;
      if (epi.ssq != nullptr) {
        const float ss = row16_sum(y * y);
        if (ok && n == kBgCols - 1) epi.ssq[(size_t)(grow + m) * ntiles + tile] = ss;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = tid + kBgThreads * i, m = m0 + idx / kBgCols, n = idx % kBgCols;
      if (idx >= kOut || m >= M || j0 + n >= nout) continue;
      if constexpr (HasPre<Epi>::value)
        epi(grow + m, j0 + n, v[i], pre[i]);
      else
        epi(grow + m, j0 + n, v[i]);
    }
  }
}

// Row tiles per block: grids of fewer than 128 column tiles (the d_model-wide
// outputs) split the rows until there are 256 blocks, one per CU; wider
// outputs keep all rows in a block (measured faster: each block then reads the
// activations once for twice the columns' work).
template <int P, bool NORM, class Epi>
void launch_bgemm_t(const bf16* X, int M, int K, const bf16* W, int nout, const Epi& epi, hipStream_t s, int groups,
                    long w_group_stride, const BNormDev& nrm) {
  const int ntiles = (nout + kBgCols - 1) / kBgCols, mtiles = (M + 15) / 16;
  int ms = 1;
  while (ntiles < 128 && ms < 4 && ms < mtiles && ntiles * ms < 256) ms *= 2;
  const dim3 grid(ntiles * ms, groups), block(kBgThreads);
  if (ms == 1)
    hipLaunchKernelGGL((k_bgemm<P, 4, NORM, Epi>), grid, block, 0, s, X, M, K, W, nout, ntiles, epi, w_group_stride,
                       nrm);
  else if (ms == 2)
    hipLaunchKernelGGL((k_bgemm<P, 2, NORM, Epi>), grid, block, 0, s, X, M, K, W, nout, ntiles, epi, w_group_stride,
                       nrm);
  else
    hipLaunchKernelGGL((k_bgemm<P, 1, NORM, Epi>), grid, block, 0, s, X, M, K, W, nout, ntiles, epi, w_group_stride,
                       nrm);
  MRT_HIP_CHECK(hipGetLastError());
}

// nrm.g non-null: X holds raw residual rows normalised on load (BNormDev),
// their sums of squares the K / 16 partials per row a BResid GEMM of width K
// wrote.
template <int P, class Epi>
void launch_bgemm(const bf16* X, int M, int K, const bf16* W, int nout, const Epi& epi, hipStream_t s, int groups = 1,
                  long w_group_stride = 0, const BNorm& norm = {}) {
  MRT_REQUIRE(M >= 1 && M <= kBatchRows, "batched GEMM: rows must be in [1, 64]");
  MRT_REQUIRE(K % 32 == 0 && K >= 32, "batched GEMM: K must be a multiple of 32");
  MRT_REQUIRE(nout >= 1 && groups >= 1, "batched GEMM: no outputs");
  if (norm.g != nullptr) {
    MRT_REQUIRE(norm.ssq != nullptr && groups == 1, "batched GEMM: a normalised input needs its row partials");
    const BNormDev d{static_cast<const bf16*>(norm.g), norm.ssq, K / kBgCols, norm.eps};
    launch_bgemm_t<P, true>(X, M, K, W, nout, epi, s, groups, w_group_stride, d);
  } else {
    launch_bgemm_t<P, false>(X, M, K, W, nout, epi, s, groups, w_group_stride, BNormDev{nullptr, nullptr, 0, 0.f});
  }
}

// Cross attention of one (row, head) over all S encoder keys (no bias, no
// mask, scale 1.0: modules.cpp:243-295), one 256-thread block per pair.  A
// wave reads 8 whole K (then V) rows per 16-byte load instruction: thread t
// owns the 8-dim slice t % 8 of keys t / 8, t / 8 + 32, ...; scores are
// reduced over the 8 slices with lane shuffles and kept in LDS; the softmax
// weights then scale V the same way and the 32 key groups are summed in a
// fixed order.
constexpr int kCrossMaxS = 1024;

__global__ __launch_bounds__(256) void k_cross_attn_b(const bf16* __restrict__ Q, const bf16* __restrict__ Kc,
                                                      const bf16* __restrict__ Vc, int H, int S, bf16* __restrict__ out) {
  __shared__ float qs[64];
  __shared__ float ps[kCrossMaxS];
  __shared__ float red[32][65];
  __shared__ float wred[2][4];
  const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int d8 = tid & 7, kg = tid >> 3;
  const int HD = H * 64;
  if (tid < 64) qs[tid] = St<bf16>::ld(Q[(size_t)b * HD + h * 64 + tid]);
  __syncthreads();
  float q[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) q[e] = qs[8 * d8 + e];
  const bf16* Kp = Kc + (size_t)bh * S * 64 + 8 * d8;
  const bf16* Vp = Vc + (size_t)bh * S * 64 + 8 * d8;
  float mx = -INFINITY;
  for (int j0 = 0; j0 < S; j0 += 4 * 32) {
    uint4 kv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + kg + 32 * u;
      kv[u] = j < S ? ld_nt16(Kp + (size_t)j * 64) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bf16* ke = reinterpret_cast<const bf16*>(&kv[u]);
      float sc = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) sc = fmaf(q[e], St<bf16>::ld(ke[e]), sc);
      sc += __shfl_xor(sc, 1, 64);
      sc += __shfl_xor(sc, 2, 64);
      sc += __shfl_xor(sc, 4, 64);
      const int j = j0 + kg + 32 * u;
      if (j < S) {
        if (d8 == 0) ps[j] = sc;
        mx = fmaxf(mx, sc);
      }
    }
  }
  mx = wave_max(mx);
  if (lane == 0) wred[0][wid] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wred[0][0], wred[0][1]), fmaxf(wred[0][2], wred[0][3]));
  float sum = 0.f;
  for (int j = tid; j < S; j += 256) {
    const float e = expf(ps[j] - mx);
    ps[j] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  if (lane == 0) wred[1][wid] = sum;
  __syncthreads();
  sum = (wred[1][0] + wred[1][1]) + (wred[1][2] + wred[1][3]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < S; j0 += 4 * 32) {
    uint4 vv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + kg + 32 * u;
      vv[u] = j < S ? ld_nt16(Vp + (size_t)j * 64) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + kg + 32 * u;
      const float pj = j < S ? ps[j] : 0.f;
      const bf16* ve = reinterpret_cast<const bf16*>(&vv[u]);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(pj, St<bf16>::ld(ve[e]), acc[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[kg][8 * d8 + e] = acc[e];
  __syncthreads();
  if (tid < 64) {
    float o = 0.f;
    for (int g = 0; g < 32; ++g) o += red[g][tid];
    out[(size_t)b * HD + h * 64 + tid] = St<bf16>::st(o / sum);
  }
}

// Gumbel noise of every draw of a chunk for every stream: out (B, frames, L, C)
// = gumbel(seeds[b], frame, level, i), the values the sampler would compute.
__global__ void k_gumbel_tables(const uint64_t* __restrict__ seeds, int frames, int L, int C, int n,
                                float* __restrict__ out) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const int c = i % C, r = i / C, level = r % L, r2 = r / L, frame = r2 % frames, b = r2 / frames;
    out[i] = gumbel(seeds[b], frame, level, c);
  }
}

__global__ void k_set_counter(int* p, int v) { *p = v; }
__global__ void k_advance_counter(int* p) { *p = *p + 1; }

}  // namespace

void gumbel_tables(const uint64_t* seeds, int streams, int frames, int L, int C, float* out, hipStream_t s) {
  const long n = (long)streams * frames * L * C;
  MRT_REQUIRE(n > 0 && n < (1L << 31), "gumbel tables: size out of range");
  const int blocks = (int)std::min<long>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(k_gumbel_tables, dim3(blocks), dim3(256), 0, s, seeds, frames, L, C, (int)n, out);
  MRT_HIP_CHECK(hipGetLastError());
}

void set_counter(int* p, int v, hipStream_t s) {
  hipLaunchKernelGGL(k_set_counter, dim3(1), dim3(1), 0, s, p, v);
  MRT_HIP_CHECK(hipGetLastError());
}

void advance_counter(int* p, hipStream_t s) {
  hipLaunchKernelGGL(k_advance_counter, dim3(1), dim3(1), 0, s, p);
  MRT_HIP_CHECK(hipGetLastError());
}

void cross_attn_rows(const void* Q, const void* Kc, const void* Vc, int rows, int H, int S, void* out, hipStream_t s) {
  MRT_REQUIRE(S >= 1 && S <= kCrossMaxS, "batched cross attention: encoder length must be in [1, 1024]");
  hipLaunchKernelGGL(k_cross_attn_b, dim3(rows * H), dim3(256), 0, s, static_cast<const bf16*>(Q),
                     static_cast<const bf16*>(Kc), static_cast<const bf16*>(Vc), H, S, static_cast<bf16*>(out));
  MRT_HIP_CHECK(hipGetLastError());
}

void bgemm_store(const void* X, int M, int K, const void* W, int N, void* Y, int ldy, hipStream_t s, const BNorm& norm) {
  launch_bgemm<1>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W), N, BStore{static_cast<bf16*>(Y), ldy},
                  s, 1, 0, norm);
}

void bgemm_f32(const void* X, int M, int K, const void* W, int N, float* Y, int ldy, hipStream_t s, const BNorm& norm) {
  launch_bgemm<1>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W), N, BF32{Y, ldy}, s, 1, 0, norm);
}

void bgemm_resid(const void* X, int M, int K, const void* W, int N, void* R, int ldr, hipStream_t s, float* ssq) {
  MRT_REQUIRE(ssq == nullptr || N % kBgCols == 0, "batched GEMM: row partials need whole 16-column tiles");
  launch_bgemm<1>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W), N,
                  BResid{static_cast<bf16*>(R), ldr, ssq}, s);
}

void bgemm_qkv(const void* X, int M, int K, const void* W, int HD, void* Q, void* Kc, void* Vc, int H, int Lmax, int pos,
               const int* pos_ptr, hipStream_t s, const BNorm& norm) {
  BQKV e{static_cast<bf16*>(Q), static_cast<bf16*>(Kc), static_cast<bf16*>(Vc), HD, H, Lmax, pos, pos_ptr};
  launch_bgemm<1>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W), 3 * HD, e, s, 1, 0, norm);
}

void bgemm_qkv_pos(const void* X, int M, int K, const void* W, int HD, void* Q, void* Kc, void* Vc, int H, int Lmax,
                   int P, hipStream_t s) {
  MRT_REQUIRE(P >= 1 && M % P == 0 && M / P <= Lmax, "batched GEMM: positions exceed the ring");
  BQKVPos e{static_cast<bf16*>(Q), static_cast<bf16*>(Kc), static_cast<bf16*>(Vc), HD, H, Lmax, P};
  launch_bgemm<1>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W), 3 * HD, e, s);
}

void bgemm_f32_grouped(const void* X, int rows, int K, const void* W, long w_group_stride, int N, float* Y, int ldy,
                       int groups, hipStream_t s) {
  launch_bgemm<1>(static_cast<const bf16*>(X), rows, K, static_cast<const bf16*>(W), N, BF32{Y, ldy}, s, groups,
                  w_group_stride);
}

void bgemm_geglu(const void* X, int M, int K, const void* W01, int F, void* Hout, int ldh, hipStream_t s,
                 const BNorm& norm) {
  MRT_REQUIRE(F % 32 == 0, "batched GEMM: d_ff must be a multiple of 32 (packed gate/up groups)");
  launch_bgemm<2>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W01), F,
                  BGeglu{static_cast<bf16*>(Hout), ldh}, s, 1, 0, norm);
}

}  // namespace mrt
