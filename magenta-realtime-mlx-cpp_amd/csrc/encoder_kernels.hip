// Once-per-chunk encoder prefill kernels for gfx950 (model.cpp:226-241,
// modules.cpp:339-358) and the cross-attention K/V projection of every
// temporal layer (modules.cpp:448-455) as one wide GEMM.
//
// GEMM operands are both K-contiguous ("NT": activations (M, K) row-major,
// weights (N, K) row-major as the bundle stores them).  bf16 and fp16 use
// v_mfma_f32_32x32x16_{bf16,f16} with LDS-double-buffered tiles; fp32 uses a
// VALU tile (parity mode).
#include <atomic>
#include <cmath>
#include <mutex>
#include <set>
#include <utility>

#include "device_utils.hpp"
#include "kernels.hpp"

namespace mrt {
namespace {

// ---- embedding + position embedding ------------------------------------------
template <typename T>
__global__ void k_encoder_embed(const T* __restrict__ emb, const T* __restrict__ pe,
                                const int* __restrict__ tok, int S, int D, T* __restrict__ x) {
  const int r = blockIdx.x, s = r % S;
  const T* e = emb + (size_t)tok[r] * D;
  const T* p = pe + (size_t)s * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x)
    x[(size_t)r * D + d] = St<T>::st(St<T>::ld(e[d]) + St<T>::ld(p[d]));
}

// Rows of up to 256 * kNormPer elements: each thread keeps its elements in
// registers between the sum of squares and the scaling (one read of x).
constexpr int kNormPer = 8;

template <typename T>
__global__ __launch_bounds__(256) void k_rmsnorm_rows_reg(const T* __restrict__ x, const T* __restrict__ g,
                                                          float eps, int D, T* __restrict__ y) {
  using S = St<T>;
  __shared__ float red[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const T* xr = x + (size_t)r * D;
  float v[kNormPer];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kNormPer; ++i) {
    const int d = tid + 256 * i;
    v[i] = d < D ? S::ld(xr[d]) : 0.f;
    ss += v[i] * v[i];
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)D + eps);
#pragma unroll
  for (int i = 0; i < kNormPer; ++i) {
    const int d = tid + 256 * i;
    if (d < D) y[(size_t)r * D + d] = S::st(S::rnd(v[i] * inv) * S::ld(g[d]));
  }
}

// One wave per row of D = 64 V NV elements (V per 16-byte chunk): a lane keeps
// its NV chunks in registers between the sum of squares and the scaling, and
// the row's sum is one wave reduction (no LDS, no barrier); four rows per block.
template <typename T, int NV>
__global__ __launch_bounds__(256) void k_rmsnorm_rows_wave(const T* __restrict__ x, const T* __restrict__ g,
                                                           float eps, int M, int D, T* __restrict__ y) {
  using S = St<T>;
  constexpr int V = S::kVec;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);  // wave-uniform
  if (r >= M) return;
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)r * D);
  const uint4* gr = reinterpret_cast<const uint4*>(g);
  uint4 v[NV], gv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = xr[lane + 64 * i];
#pragma unroll
  for (int i = 0; i < NV; ++i) gv[i] = gr[lane + 64 * i];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const T* e = reinterpret_cast<const T*>(&v[i]);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float f = S::ld(e[k]);
      ss += f * f;
    }
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
  uint4* yr = reinterpret_cast<uint4*>(y + (size_t)r * D);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const T* e = reinterpret_cast<const T*>(&v[i]);
    const T* ge = reinterpret_cast<const T*>(&gv[i]);
    uint4 o;
    T* oe = reinterpret_cast<T*>(&o);
#pragma unroll
    for (int k = 0; k < V; ++k) oe[k] = S::st(S::rnd(S::ld(e[k]) * inv) * S::ld(ge[k]));
    yr[lane + 64 * i] = o;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const T* __restrict__ x, const T* __restrict__ g,
                                                      float eps, int D, T* __restrict__ y) {
  using S = St<T>;
  __shared__ float red[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const T* xr = x + (size_t)r * D;
  float ss = 0.f;
  for (int d = tid; d < D; d += 256) {
    const float v = S::ld(xr[d]);
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)D + eps);
  for (int d = tid; d < D; d += 256)
    y[(size_t)r * D + d] = S::st(S::rnd(S::ld(xr[d]) * inv) * S::ld(g[d]));
}

// ---- GEMM epilogue ----------------------------------------------------------------
template <typename T>
struct GemmOut {
  GemmEpiArgs a;
  int N;
  __device__ __forceinline__ void put(int m, int n, float acc) const {
    using S = St<T>;
    T* C = static_cast<T*>(a.C);
    if (a.kind == GemmEpi::Store) {
      C[(size_t)m * N + n] = S::st(acc);
    } else if (a.kind == GemmEpi::Resid) {
      T* p = C + (size_t)m * N + n;
      *p = S::st(S::ld(*p) + S::rnd(acc));
    } else if (a.kind == GemmEpi::StoreF32) {
      static_cast<float*>(a.C)[(size_t)m * N + n] = S::rnd(acc);
    } else {  // CrossKV
      const int lk = n / a.HD, nn = n - lk * a.HD;
      const int h = nn >> 6, d = nn & 63;
      const int b = m / a.S, s = m - b * a.S;
      C[((((size_t)lk * a.nb + b) * a.H + h) * a.S + s) * 64 + d] = S::st(acc);
    }
  }
  // Gated-GELU pair: packed column n (gate, n % 64 < 32) and n + 32 (up).
  __device__ __forceinline__ void put_geglu(int m, int n, float g, float u) const {
    using S = St<T>;
    T* C = static_cast<T*>(a.C);
    const int j = (n >> 6) * 32 + (n & 31);
    const float gl = gelu_t<T>(S::rnd(g));
    C[(size_t)m * (N / 2) + j] = S::st(gl * S::rnd(u));
  }
};

// ---- VALU tiled GEMM (fp32 parity path; also the 16-bit fallback) -----------------
// 64x64 tile, BK 16, 256 threads, 4x4 outputs per thread at rows ty+16i and
// columns tx+16j, so columns j and j+2 form a packed gate/up pair.
template <typename T>
__global__ __launch_bounds__(256) void k_gemm_valu(const T* __restrict__ A, const T* __restrict__ B,
                                                   int M, int N, int K, GemmOut<T> out) {
  using S = St<T>;
  __shared__ float As[16][64 + 4];
  __shared__ float Bs[16][64 + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i, r = idx >> 4, c = idx & 15;
      const int gm = m0 + r, gn = n0 + r, gk = k0 + c;
      As[c][r] = (gm < M && gk < K) ? S::ld(A[(size_t)gm * K + gk]) : 0.f;
      Bs[c][r] = (gn < N && gk < K) ? S::ld(B[(size_t)gn * K + gk]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty + 16 * i;
    if (m >= M) continue;
    if (out.a.kind == GemmEpi::Geglu) {
#pragma unroll
      for (int j = 0; j < 2; ++j) out.put_geglu(m, n0 + tx + 16 * j, acc[i][j], acc[i][j + 2]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + tx + 16 * j;
        if (n < N) out.put(m, n, acc[i][j]);
      }
    }
  }
}

// ---- 16-bit MFMA GEMM ----------------------------------------------------------------
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x8_t __attribute__((ext_vector_type(8)));

// The 32x32x16 matrix instruction of each 16-bit storage type (fp32 accumulators).
template <typename T>
struct Mfma;
template <>
struct Mfma<bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static f32x16_t mma(v8 a, v8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<f16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static f32x16_t mma(v8 a, v8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kBN = 128, kBK = 64, kStages = 2;

// LDS rows of a tile are 64 elements = 8 chunks of 16 bytes; chunk c of row r is
// stored at chunk c ^ swz(r), so the 32 rows x 2 chunks of an MFMA fragment
// read (and 16 consecutive lanes of any ds_read_b128) fall in distinct banks.
__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

// s_waitcnt immediate waiting for vmcnt <= n (expcnt and lgkmcnt left alone).
constexpr int vm_wait_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// Workgroup barrier of the global -> LDS rings: every LDS read this wave has
// issued has returned (so another wave may refill that stage after the
// barrier), then the waves meet.  Unlike __syncthreads() it does not wait for
// this wave's loads still in flight to later stages (a release fence would
// wait for every outstanding LDS write, direct-to-LDS loads included): the
// stage about to be read is awaited with an explicit vmcnt before it.  The
// asm is a compiler barrier for memory operations.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Epilogue of the MFMA GEMMs.  Accumulator r of tile (i, j) of a lane holds
// row mb + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4 and column
// nb + 32 j + lane % 32 (j = 2p / 2p + 1: gate / up columns of gated-GELU pair p).
// The kind is resolved once per tile, and the residual epilogue loads every
// residual before it stores anything: with the loads and stores of one
// element interleaved, each load would wait for the previous element's store.
template <typename T, int MI, int NJ = 2>
__device__ __forceinline__ void mfma_epilogue(const GemmOut<T>& out, const f32x16_t (&acc)[MI][NJ], int M, int mb,
                                              int nb) {
  using St_ = St<T>;
  const int lane = threadIdx.x & 63, col = lane & 31, rl = 4 * (lane >> 5);
  const int N = out.N;
  T* C = static_cast<T*>(out.a.C);
  auto row = [&](int i, int r) { return mb + 32 * i + 8 * (r >> 2) + rl + (r & 3); };
  switch (out.a.kind) {
    case GemmEpi::Geglu:
      if constexpr (NJ % 2 == 0) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int pj = 0; pj < NJ / 2; ++pj)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (row(i, r) < M) out.put_geglu(row(i, r), nb + 64 * pj + col, acc[i][2 * pj][r], acc[i][2 * pj + 1][r]);
      }
      break;
    case GemmEpi::Resid:
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          T old[16];  // rows past M load row M - 1 (unconditional loads, issued together)
#pragma unroll
          for (int r = 0; r < 16; ++r) old[r] = C[(size_t)min(row(i, r), M - 1) * N + nb + 32 * j + col];
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (row(i, r) < M)
              C[(size_t)row(i, r) * N + nb + 32 * j + col] = St_::st(St_::ld(old[r]) + St_::rnd(acc[i][j][r]));
        }
      break;
    case GemmEpi::Store:
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (row(i, r) < M) C[(size_t)row(i, r) * N + nb + 32 * j + col] = St_::st(acc[i][j][r]);
      break;
    case GemmEpi::StoreF32:
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (row(i, r) < M)
              static_cast<float*>(out.a.C)[(size_t)row(i, r) * N + nb + 32 * j + col] = St_::rnd(acc[i][j][r]);
      break;
    default: {  // CrossKV: column n = (layer*2 + kv)*HD + h*64 + d, row m = b*S + s
      size_t cbase[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int n = nb + 32 * j + col, lk = n / out.a.HD, nn = n - lk * out.a.HD;
        cbase[j] = (((size_t)lk * out.a.nb) * out.a.H + (nn >> 6)) * out.a.S * 64 + (nn & 63);
      }
      const size_t bstride = (size_t)out.a.H * out.a.S * 64;
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = row(i, r);
          if (m < M) {
            const int b = m / out.a.S, sp = m - b * out.a.S;
            const size_t ro = (size_t)b * bstride + (size_t)sp * 64;
#pragma unroll
            for (int j = 0; j < NJ; ++j) C[cbase[j] + ro] = St_::st(acc[i][j][r]);
          }
        }
    }
  }
}

// C = A B^T (A (M, K), B (N, K) 16-bit, fp32 accumulation) with the GemmOut
// epilogue.  Tile BM x BN x 64, 4 waves in a 2x2 grid (wave tile BM/2 x BN/2 =
// (BM/64) x (BN/64) MFMA 32x32x16 tiles).  Tiles stream global -> LDS with direct
// 16-byte loads (global_load_lds) through an S-deep ring: tile j + S - 1 is
// requested while tile j is multiplied, and a wave waits only for its own
// loads of tile j (vmcnt counts in order) before the barrier.  Where the grid
// fills every CU twice, two stages (64 / 48 KB of LDS) leave room for 2-3
// blocks per CU, which hides more latency than a deeper ring in one block
// (measured); a grid of at most one tile per CU instead takes a deep ring in
// its one block.  Rows past M read row M - 1 (their results are not stored).
// Operand fragments of v_mfma_f32_32x32x16_{bf16,f16}: lane l holds row (l % 32)
// and k = 8*(l / 32) .. +7 of both A (32x16) and B^T (32x16); the 16
// accumulators of lane l hold column l % 32, rows 8*(r/4) + 4*(l/32) + r%4.
// Blocks per CU the register budget is sized for: two wherever the LDS ring
// leaves room for two (at most 80 KB), else one.
constexpr int gemm_min_blocks(int BM, int S, int BN) { return S * (BM + BN) * 128 <= 80 * 1024 ? 2 : 1; }

// Tile of block L of a 1-D grid in the XCD-grouped order: blocks are dealt to
// the 8 XCDs in turn (L % 8), each XCD takes a contiguous range of tile ids,
// and tile ids run down GM row tiles before the next column tile, so the
// blocks that one XCD runs together share GM A tiles and a few B tiles in its
// L2.  A bijection of [0, tm * tn).
__device__ __forceinline__ void grouped_tile(int L, int tm, int tn, int GM, int& mt, int& nt) {
  const int tiles = tm * tn, x = L & 7, q = tiles >> 3, rem = tiles & 7;
  const int pid = x * q + min(x, rem) + (L >> 3);
  const int g = pid / (GM * tn), first = g * GM, gsz = min(tm - first, GM);
  const int w = pid - g * GM * tn;
  mt = first + w % gsz;
  nt = w / gsz;
}

// GM = 0: block (x, y) of a 2-D grid computes tile (y, x); GM > 0: a 1-D grid
// in the grouped_tile order.
template <typename T, int BM, int S, int BN, int GM>
__global__ __launch_bounds__(256, gemm_min_blocks(BM, S, BN)) void k_gemm_mfma(const T* __restrict__ A,
                                                                               const T* __restrict__ B,
                                                   int M, int N, int K, GemmOut<T> out) {
  typedef typename Mfma<T>::v8 v8;
  constexpr int MI = BM / 64;                        // MFMA tiles per wave in M
  constexpr int NJ = BN / 64;                        // MFMA tiles per wave in N
  constexpr int kStageBytes = (BM + BN) * 128;       // A rows then B rows, 128 bytes each
  constexpr int LA = BM / 32 + BN / 32;              // load instructions per wave per tile
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  int mt = blockIdx.y, nt = blockIdx.x;
  if constexpr (GM > 0) grouped_tile(blockIdx.x, (M + BM - 1) / BM, N / BN, GM, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int nk = K / kBK;

  // tile kt -> stage kt % S; wave w loads rows [w*BM/4, +BM/4) of A and
  // [w*32, +32) of B, 8 rows (1 KB) per instruction
  auto issue = [&](int kt) {
    const int ktc = min(kt, nk - 1);  // past the end: reload the last tile into a free stage
    unsigned char* st = lds + (kt % S) * kStageBytes;
    const int r8 = lane >> 3, p = lane & 7;
#pragma unroll
    for (int q = 0; q < BM / 32; ++q) {
      const int r = wid * (BM / 4) + q * 8 + r8;
      const int gm = min(m0 + r, M - 1);
      const T* src = A + (size_t)gm * K + ktc * kBK + ((p ^ swz(r)) << 3);
      __builtin_amdgcn_global_load_lds((const MRT_GLOBAL void*)src,
                                       (MRT_LDS void*)(st + (wid * (BM / 4) + q * 8) * 128), 16, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < BN / 32; ++q) {
      const int r = wid * (BN / 4) + q * 8 + r8;
      const T* src = B + (size_t)(n0 + r) * K + ktc * kBK + ((p ^ swz(r)) << 3);
      __builtin_amdgcn_global_load_lds((const MRT_GLOBAL void*)src,
                                       (MRT_LDS void*)(st + BM * 128 + (wid * (BN / 4) + q * 8) * 128), 16, 0, 0);
    }
  };

  f32x16_t acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

#pragma unroll
  for (int kt = 0; kt < S - 1; ++kt) issue(kt);
  const int lr = lane & 31, lh = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    __builtin_amdgcn_s_waitcnt(vm_wait_imm((S - 2) * LA));  // this wave's loads of tile kt have landed
    ring_barrier();  // every wave's loads of tile kt; every wave is done with tile kt - 1
    issue(kt + S - 1);
    const unsigned char* st = lds + (kt % S) * kStageBytes;
    // every fragment of the tile is read before the first product, so the
    // LDS latency is paid once per tile, not once per 16-deep step
    v8 a[kBK / 16][MI], b[kBK / 16][NJ];
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int c = 2 * ks + lh;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int r = wm * (BM / 2) + i * 32 + lr;
        a[ks][i] = *reinterpret_cast<const v8*>(st + r * 128 + ((c ^ swz(r)) << 4));
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int r = wn * (BN / 2) + j * 32 + lr;
        b[ks][j] = *reinterpret_cast<const v8*>(st + BM * 128 + r * 128 + ((c ^ swz(r)) << 4));
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the products
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks)
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = Mfma<T>::mma(a[ks][i], b[ks][j], acc[i][j]);
  }
  __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));  // no copy into LDS outlives the block

  mfma_epilogue<T, MI, NJ>(out, acc, M, m0 + wm * (BM / 2), n0 + wn * (BN / 2));
}

// Dynamic LDS above 64 KB needs an explicit allowance, once per kernel and device.
void allow_dynamic_lds(const void* fn, size_t bytes) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  int dev = 0;
  MRT_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> g(mu);
  if (done.count({fn, dev})) return;
  MRT_HIP_CHECK(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)));
  done.insert({fn, dev});
}

// Compute units of the current device (cached per device).
int device_cus() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cache[kMaxDev] = {};
  int dev = 0;
  MRT_HIP_CHECK(hipGetDevice(&dev));
  int v = (dev >= 0 && dev < kMaxDev) ? cache[dev].load(std::memory_order_relaxed) : 0;
  if (v == 0) {
    MRT_HIP_CHECK(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev));
    if (dev >= 0 && dev < kMaxDev) cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

template <typename T, int BM, int S = kStages, int BN = kBN, int GM = 0>
void launch_gemm_mfma(const T* A, const T* B, int M, int N, int K, const GemmOut<T>& out, hipStream_t s) {
  static_assert((S - 2) * (BM / 32 + BN / 32) < 64, "vmcnt holds at most 63 outstanding loads");
  static_assert(BM % 64 == 0 && BN % 64 == 0, "wave tiles are whole 32x32 MFMA tiles");
  constexpr size_t lds = (size_t)S * (BM + BN) * 128;
  static_assert(lds <= 160 * 1024, "LDS of one CU");
  MRT_REQUIRE(N % BN == 0, "gemm: N is not a multiple of the tile width");
  allow_dynamic_lds(reinterpret_cast<const void*>(&k_gemm_mfma<T, BM, S, BN, GM>), lds);
  const long tm = (M + BM - 1) / BM, tn = N / BN;
  MRT_REQUIRE(GM == 0 || tm * tn <= 0x7fffffffL, "gemm: too many tiles");
  const dim3 grid = GM > 0 ? dim3(static_cast<unsigned>(tm * tn)) : dim3(tn, tm);
  hipLaunchKernelGGL((k_gemm_mfma<T, BM, S, BN, GM>), grid, dim3(256), lds, s, A, B, M, N, K, out);
}

// Large-M GEMM (the encoder of several streams): 256 x 256 x 64 tiles, 16
// waves in a 4 x 4 grid (wave tile 64 x 64 = 2 x 2 MFMA 32x32x16 tiles, the
// accumulators of k_gemm_mfma's waves), the same swizzled two-stage global ->
// LDS ring.  Against 128 x 128 tiles it halves the operand bytes read from L2
// per FLOP, which is what bounds the smaller tiles at these sizes.  Rows past
// M read row M - 1 (not stored); N % 256 == 0.
constexpr int kGB = 256;                 // block tile, M and N
constexpr int kGBWaves = 16;
constexpr int kGBStage = 2 * kGB * 128;  // A rows then B rows, 128 bytes (64 elements) each

template <typename T>
__global__ __launch_bounds__(64 * kGBWaves) void k_gemm_big(const T* __restrict__ A, const T* __restrict__ B,
                                                            int M, int N, int K, GemmOut<T> out) {
  typedef typename Mfma<T>::v8 v8;
  constexpr int RW = kGB / kGBWaves;  // rows of A (and of B) each wave loads per stage
  constexpr int LA = 2 * RW / 8;      // load instructions per wave per stage (8 rows each)
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 2, wn = wid & 3;
  const int m0 = blockIdx.y * kGB, n0 = blockIdx.x * kGB;
  const int nk = K / kBK;

  auto issue = [&](int kt) {
    const int ktc = min(kt, nk - 1);
    unsigned char* st = lds + (kt % kStages) * kGBStage;
    const int r8 = lane >> 3, p = lane & 7;
#pragma unroll
    for (int q = 0; q < RW / 8; ++q) {
      const int r = wid * RW + q * 8 + r8;
      const int gm = min(m0 + r, M - 1);
      const T* src = A + (size_t)gm * K + ktc * kBK + ((p ^ swz(r)) << 3);
      __builtin_amdgcn_global_load_lds((const MRT_GLOBAL void*)src, (MRT_LDS void*)(st + (wid * RW + q * 8) * 128),
                                       16, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < RW / 8; ++q) {
      const int r = wid * RW + q * 8 + r8;
      const T* src = B + (size_t)(n0 + r) * K + ktc * kBK + ((p ^ swz(r)) << 3);
      __builtin_amdgcn_global_load_lds((const MRT_GLOBAL void*)src,
                                       (MRT_LDS void*)(st + kGB * 128 + (wid * RW + q * 8) * 128), 16, 0, 0);
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

#pragma unroll
  for (int kt = 0; kt < kStages - 1; ++kt) issue(kt);
  const int lr = lane & 31, lh = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    __builtin_amdgcn_s_waitcnt(vm_wait_imm((kStages - 2) * LA));  // this wave's loads of tile kt have landed
    ring_barrier();  // every wave's loads of tile kt; every wave is done with tile kt - 1
    issue(kt + kStages - 1);
    const unsigned char* st = lds + (kt % kStages) * kGBStage;
    // one 16-deep step at a time: 16 waves leave 128 registers a lane, and
    // reading further ahead spills
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int c = 2 * ks + lh;
      v8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = wm * 64 + i * 32 + lr;
        a[i] = *reinterpret_cast<const v8*>(st + r * 128 + ((c ^ swz(r)) << 4));
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = wn * 64 + j * 32 + lr;
        b[j] = *reinterpret_cast<const v8*>(st + kGB * 128 + r * 128 + ((c ^ swz(r)) << 4));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = Mfma<T>::mma(a[i], b[j], acc[i][j]);
    }
  }
  __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));  // no copy into LDS outlives the block

  mfma_epilogue<T, 2>(out, acc, M, m0 + wm * 64, n0 + wn * 64);
}

template <typename T>
void launch_gemm_big(const T* A, const T* B, int M, int N, int K, const GemmOut<T>& out, hipStream_t s) {
  constexpr size_t lds = (size_t)kStages * kGBStage;
  allow_dynamic_lds(reinterpret_cast<const void*>(&k_gemm_big<T>), lds);
  hipLaunchKernelGGL(k_gemm_big<T>, dim3(N / kGB, (M + kGB - 1) / kGB), dim3(64 * kGBWaves), lds, s, A, B, M, N, K, out);
}

// ---- encoder self-attention (bidirectional, no mask, no bias, scale 1.0) -------------
// One lane per query row, 64 rows per block; K/V tiles of 64 keys staged in
// LDS; online softmax per 64-key tile.
template <typename T>
__global__ __launch_bounds__(64) void k_enc_attn(const T* __restrict__ qkv, int S, int H,
                                                 T* __restrict__ out) {
  using St_ = St<T>;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H, lane = threadIdx.x;
  const int HD = H * 64, ld = 3 * HD;
  const int qi = blockIdx.x * 64 + lane;
  __shared__ float Ks[64][64 + 1];
  __shared__ float Vs[64][64];
  float q[64], o[64];
  const T* qrow = qkv + ((size_t)b * S + (qi < S ? qi : 0)) * ld + h * 64;
#pragma unroll
  for (int d = 0; d < 64; ++d) {
    q[d] = St_::ld(qrow[d]);
    o[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  for (int j0 = 0; j0 < S; j0 += 64) {
    const int nk = min(64, S - j0);
    for (int r = 0; r < nk; ++r) {
      const T* row = qkv + ((size_t)b * S + j0 + r) * ld + h * 64;
      Ks[r][lane] = St_::ld(row[HD + lane]);
      Vs[r][lane] = St_::ld(row[2 * HD + lane]);
    }
    __syncthreads();
    float sc[64];
    float mt = -INFINITY;
#pragma unroll
    for (int r = 0; r < 64; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < 64; ++d) acc = fmaf(q[d], Ks[r][d], acc);
      sc[r] = r < nk ? acc : -INFINITY;
      mt = fmaxf(mt, sc[r]);
    }
    const float mn = fmaxf(m, mt);
    const float corr = expf(m - mn);
    l *= corr;
#pragma unroll
    for (int d = 0; d < 64; ++d) o[d] *= corr;
#pragma unroll
    for (int r = 0; r < 64; ++r) {
      const float p = r < nk ? expf(sc[r] - mn) : 0.f;
      l += p;
#pragma unroll
      for (int d = 0; d < 64; ++d) o[d] = fmaf(p, Vs[r][d], o[d]);
    }
    m = mn;
    __syncthreads();
  }
  if (qi < S) {
    T* orow = out + ((size_t)b * S + qi) * HD + h * 64;
    const float inv = 1.0f / l;
#pragma unroll
    for (int d = 0; d < 64; ++d) orow[d] = St_::st(o[d] * inv);
  }
}

// ---- 16-bit encoder self-attention on MFMA ------------------------------------------
// Flash attention for one (row, head) and 128 queries per workgroup (32 per
// wave), keys in tiles of 64 staged in LDS.  Scores are computed transposed,
// S^T = K Q^T (v_mfma_f32_32x32x16_{bf16,f16}), so lane l owns query l % 32 and
// the online-softmax rescale is per lane.  The output is also accumulated
// transposed, O^T += V^T P^T, with P^T taken straight from the score
// accumulators: lane l's accumulators of a 16-key step hold keys
// {4h..4h+3, 8+4h..8+4h+3} (h = l / 32), so V^T is staged with the key order
// inside every 16-key block permuted the same way (swap of key bits 2 and 3).
// Scores and the softmax are fp32, the exponentials taken as
// 2^(s log2 e - m log2 e) with one fma and v_exp_f32 (as fused attention
// kernels do), keys past S masked only in the last tile; P enters the second
// product as the sum of two parts in the storage type (hi + lo: ~16
// significant bits for bf16, ~22 for fp16), as close to the fp32
// probabilities of the reference's fused attention as 16-bit MFMA allows (P
// rounded once to bf16 measured 2.02e-2 on a level slice of the bf16
// two-frame decode against the oracle's 2e-2 bound).
constexpr int kAQ = 128, kAK = 64, kALD = 64 + 8;  // queries, keys per tile, padded LDS row
constexpr float kLog2e = 1.4426950408889634f;

// Element offset of 8-key chunk `ch` in row `dim` of the staged V^T: chunks are
// XOR-swizzled by dim / 8, so the transposed 2-byte stores of 8 dims 8 apart
// fall in different banks (2-way instead of 8-way), while the padded rows keep
// the 16-byte fragment reads of 8 consecutive dims conflict-free.
__device__ __forceinline__ int vt_chunk(int ch, int dim) { return (ch ^ ((dim >> 3) & 7)) << 3; }

// Scores of one 64-key tile from the staged K rows: sc[t] holds S^T for keys
// 32 t + 8 (r / 4) + 4 hf + r % 4 of the tile, query lq.
template <typename T>
__device__ __forceinline__ void attn_scores(const T* Ks, const typename Mfma<T>::v8 (&qf)[4], int lq, int hf,
                                            f32x16_t (&sc)[2]) {
  typedef typename Mfma<T>::v8 v8;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[t][r] = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const v8 a = *reinterpret_cast<const v8*>(&Ks[(32 * t + lq) * kALD + 16 * s + 8 * hf]);
      sc[t] = Mfma<T>::mma(a, qf[s], sc[t]);
    }
  }
}

// Online-softmax step of one tile (keys kb ..): running max m, sum lsum and
// output accumulators acc, with the tile's V^T staged in Vt.
template <typename T>
__device__ __forceinline__ void attn_update(f32x16_t (&sc)[2], int kb, int S, int lq, int hf, const T* Vt, float& m,
                                            float& lsum, f32x16_t (&acc)[2]) {
  typedef typename Mfma<T>::v8 v8;
  float mt = -INFINITY;
  if (kb + kAK <= S) {  // a full tile (wave-uniform): no key to mask
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sc[t][r]);
  } else {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + 32 * t + 8 * (r >> 2) + 4 * hf + (r & 3);
        sc[t][r] = key < S ? sc[t][r] : -INFINITY;
        mt = fmaxf(mt, sc[t][r]);
      }
  }
  mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
  const float mn = fmaxf(m, mt);  // raw-score running max (key 0 is never masked)
  const float mns = mn * kLog2e;
  const float corr = __builtin_amdgcn_exp2f(fmaf(m, kLog2e, -mns));
  float ps = 0.f;
  v8 pb[4], pl[4];  // P^T = hi + lo (storage type each) for the four 16-key steps
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    f32x8_t pv;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pv[i] = __builtin_amdgcn_exp2f(fmaf(sc[g >> 1][8 * (g & 1) + i], kLog2e, -mns));
      ps += pv[i];
    }
    pb[g] = __builtin_convertvector(pv, v8);  // round-to-nearest-even conversions
    pl[g] = __builtin_convertvector(pv - __builtin_convertvector(pb[g], f32x8_t), v8);
  }
  ps += __shfl_xor(ps, 32, 64);
  lsum = lsum * corr + ps;
  m = mn;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] *= corr;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const v8 a = *reinterpret_cast<const v8*>(&Vt[(32 * t + lq) * kALD + vt_chunk(2 * s + hf, 32 * t + lq)]);
      acc[t] = Mfma<T>::mma(a, pb[s], acc[t]);
      acc[t] = Mfma<T>::mma(a, pl[s], acc[t]);
    }
}

// Tile j + 1's K and V are loaded (K rows first, then V rows) while tile j is
// processed.  Sized for three blocks per CU (3 waves per SIMD: the register
// budget is 170), which measured faster than the compiler's 196 registers at
// two.  Every query runs attn_scores / attn_update over the tiles in order,
// the same arithmetic whatever the grid, so a stream's rows do not depend on
// the batch it is encoded in.
template <typename T>
__global__ __launch_bounds__(256, 3) void k_enc_attn_mfma(const T* __restrict__ qkv, int S, int H,
                                                       T* __restrict__ out) {
  typedef typename Mfma<T>::v8 v8;
  __shared__ __attribute__((aligned(16))) T Ks[2][kAK * kALD];
  __shared__ __attribute__((aligned(16))) T Vt[2][64 * kALD];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int HD = H * 64, ld = 3 * HD;
  const T* base = qkv + (size_t)b * S * ld + h * 64;
  const int lq = lane & 31, hf = lane >> 5;
  const int q = blockIdx.x * kAQ + wid * 32 + lq;

  // Q^T fragments (B operand): lane l holds Q[q][16 s + 8 hf .. +7].
  v8 qf[4];
  {
    const T* qr = base + (size_t)min(q, S - 1) * ld;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = *reinterpret_cast<const v8*>(qr + 16 * s + 8 * hf);
  }
  // Tile staging: thread t moves 16 bytes of K (part 1 of the q/k/v row) or V
  // (part 2) for keys t/8 and 32 + t/8, dims 8 (t % 8) .. +7; keys past S are
  // zero.  (Clamping those keys to S - 1 instead, with no conditional load,
  // made the compiler keep the Q fragments in scratch memory.)
  uint4 rk[2], rv[2];
  auto gload = [&](uint4 (&r)[2], int kb, int part) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = kb + (tid >> 3) + 32 * i, c = (tid & 7) * 8;
      r[i] = key < S ? *reinterpret_cast<const uint4*>(base + (size_t)key * ld + part * HD + c)
                     : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto kstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = (tid >> 3) + 32 * i, c = (tid & 7) * 8;
      *reinterpret_cast<uint4*>(&Ks[buf][key * kALD + c]) = rk[i];
    }
  };
  auto vstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = (tid >> 3) + 32 * i, c = (tid & 7) * 8;
      const int slot = (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
      const T* v = reinterpret_cast<const T*>(&rv[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) Vt[buf][(c + e) * kALD + vt_chunk(slot >> 3, c + e) + (slot & 7)] = v[e];
    }
  };

  f32x16_t acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
  float m = -INFINITY, lsum = 0.f;
  const int ntiles = (S + kAK - 1) / kAK;

  gload(rk, 0, 1);
  gload(rv, 0, 2);
  kstore(0);
  vstore(0);
  __syncthreads();
  for (int j = 0; j < ntiles; ++j) {
    const int cur = j & 1, kb = j * kAK;
    if (j + 1 < ntiles) {
      gload(rk, kb + kAK, 1);
      gload(rv, kb + kAK, 2);
    }
    f32x16_t sc[2];
    attn_scores<T>(Ks[cur], qf, lq, hf, sc);
    attn_update<T>(sc, kb, S, lq, hf, Vt[cur], m, lsum, acc);
    if (j + 1 < ntiles) {
      kstore(cur ^ 1);
      vstore(cur ^ 1);
    }
    __syncthreads();
  }
  if (q < S) {
    T* orow = out + ((size_t)b * S + q) * HD + h * 64;
    const float inv = 1.0f / lsum;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * t + 8 * g + 4 * hf;
        uint2 w;
        w.x = St<T>::bits(acc[t][4 * g] * inv) | (St<T>::bits(acc[t][4 * g + 1] * inv) << 16);
        w.y = St<T>::bits(acc[t][4 * g + 2] * inv) | (St<T>::bits(acc[t][4 * g + 3] * inv) << 16);
        *reinterpret_cast<uint2*>(orow + d) = w;
      }
  }
}

}  // namespace

void encoder_embed(DType dt, const void* emb, const void* pe, const int* tok, int M, int S, int D,
                   void* x, hipStream_t s) {
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_encoder_embed<T>, dim3(M), dim3(256), 0, s, (const T*)emb,
                                            (const T*)pe, tok, S, D, (T*)x));
  MRT_HIP_CHECK(hipGetLastError());
}

namespace {

// The wave-per-row norm for rows of 64 V NV elements (NV <= 4) on 16-byte
// aligned pointers; false when the shape or alignment does not fit.
template <typename T>
bool rmsnorm_rows_wave(const T* x, const T* g, float eps, int M, int D, T* y, hipStream_t s) {
  constexpr int W = 64 * St<T>::kVec;
  const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(g) |
                         reinterpret_cast<uintptr_t>(y)) & 15) == 0;
  if (!aligned || D % W != 0 || D / W < 1 || D / W > 4) return false;
  const dim3 grid((M + 3) / 4), block(256);
  switch (D / W) {
    case 1: hipLaunchKernelGGL((k_rmsnorm_rows_wave<T, 1>), grid, block, 0, s, x, g, eps, M, D, y); break;
    case 2: hipLaunchKernelGGL((k_rmsnorm_rows_wave<T, 2>), grid, block, 0, s, x, g, eps, M, D, y); break;
    case 3: hipLaunchKernelGGL((k_rmsnorm_rows_wave<T, 3>), grid, block, 0, s, x, g, eps, M, D, y); break;
    default: hipLaunchKernelGGL((k_rmsnorm_rows_wave<T, 4>), grid, block, 0, s, x, g, eps, M, D, y); break;
  }
  return true;
}

}  // namespace

void rmsnorm_rows(DType dt, const void* x, const void* g, float eps, int M, int D, void* y,
                  hipStream_t s) {
  bool done = false;
  MRT_DTYPE_DISPATCH(dt, done = rmsnorm_rows_wave<T>(static_cast<const T*>(x), static_cast<const T*>(g), eps, M, D,
                                                      static_cast<T*>(y), s));
  if (done) {
    MRT_HIP_CHECK(hipGetLastError());
    return;
  }
  const bool reg = D <= 256 * kNormPer;
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(reg ? k_rmsnorm_rows_reg<T> : k_rmsnorm_rows<T>, dim3(M), dim3(256), 0,
                                            s, (const T*)x, (const T*)g, eps, D, (T*)y));
  MRT_HIP_CHECK(hipGetLastError());
}

namespace {

template <typename T>
void gemm_t(const T* A, const T* B, int M, int N, int K, const GemmEpiArgs& e, hipStream_t s, bool allow_mfma) {
  GemmOut<T> out{e, N};
  if constexpr (sizeof(T) == 2) {
    if (allow_mfma && N % kBN == 0 && K % kBK == 0) {
      // Measured on MI355X (256 CUs) at 2 x 1006 x {1, 8, 32} rows: 256 x 256
      // tiles of 16 waves for outputs up to 4096 wide once they give about
      // one tile per CU (slower for the 5632- and 40960-wide outputs, where
      // 2-3 smaller blocks per CU hide more latency); for the wider outputs
      // other than the gated-GELU pairs (the 40960-wide cross K/V projection)
      // 256 x 256 tiles of 4 waves with 128 x 128 wave tiles (half the LDS
      // fragment reads per product) in the XCD-grouped order: 280 -> 234 us
      // at one stream, 7.35 -> 6.41 ms at 32 (the gated-GELU output measured
      // slower with them).  The XCD-grouped order also serves the 64-row
      // tiles of one stream (O 12.6 -> 11.5 us, FFN down 25.3 -> 23.6 us),
      // the 1024-wide output of K <= 1024 at 32 streams on 192-row tiles
      // (the attention output projection: 249 -> 210 us against k_gemm_big;
      // the FFN down projection, K = 2816, is as fast on k_gemm_big) and the
      // gated-GELU output past two 192-row blocks per CU (1077 -> 998 us at
      // 32 streams).  Below that every block streams
      // its operands at the latency of the last-level cache, so the tile is
      // chosen for the bytes it keeps in flight: a grid of at most one 64-row
      // tile per CU takes a 4-deep ring (96 KB of LDS; 6 deep measured
      // slower); a 128 x 192 tile with
      // a 3-deep ring where that grid fits the CUs once (not for the
      // gated-GELU pairs, which need wave tiles of whole 64-column groups);
      // 192-row tiles where two blocks per CU (80 KB each) cover the grid
      // once; else 128-row tiles when those give >= 1.5 tiles per CU, else
      // 64-row tiles.
      const long cus = device_cus();
      const long t256 = (long)((M + kGB - 1) / kGB) * (N / kGB), t64 = (long)((M + 63) / 64) * (N / kBN);
      const long t128x192 = N % 192 == 0 ? (long)((M + 127) / 128) * (N / 192) : 0;
      const long t192 = (long)((M + 191) / 192) * (N / kBN);
      if (N % kGB == 0 && N <= 4096 && t256 >= cus - cus / 8) {
        if (N == 1024 && K <= 1024)
          launch_gemm_mfma<T, 192, 2, 128, 2>(A, B, M, N, K, out, s);
        else
          launch_gemm_big<T>(A, B, M, N, K, out, s);
      } else if (e.kind != GemmEpi::Geglu && N % 256 == 0 && N > 4096 && t256 >= cus)
        launch_gemm_mfma<T, 256, 2, 256, 4>(A, B, M, N, K, out, s);
      else if (t64 <= cus)
        launch_gemm_mfma<T, 64, 4, 128, 4>(A, B, M, N, K, out, s);
      else if (e.kind != GemmEpi::Geglu && t128x192 > 0 && t128x192 <= cus)
        launch_gemm_mfma<T, 128, 3, 192>(A, B, M, N, K, out, s);
      else if (t192 <= 2 * cus)
        launch_gemm_mfma<T, 192, 2>(A, B, M, N, K, out, s);
      else if (e.kind == GemmEpi::Geglu)
        launch_gemm_mfma<T, 192, 2, 128, 4>(A, B, M, N, K, out, s);
      else if ((long)((M + 127) / 128) * (N / kBN) >= 3 * cus / 2)
        launch_gemm_mfma<T, 128>(A, B, M, N, K, out, s);
      else
        launch_gemm_mfma<T, 64>(A, B, M, N, K, out, s);
      return;
    }
  }
  hipLaunchKernelGGL(k_gemm_valu<T>, dim3((N + 63) / 64, (M + 63) / 64), dim3(256), 0, s, A, B, M, N, K, out);
}

}  // namespace

void gemm(DType dt, const void* A, const void* B, int M, int N, int K, const GemmEpiArgs& e,
          hipStream_t s, bool allow_mfma) {
  MRT_REQUIRE(M >= 1 && N >= 1 && K >= 1, "gemm: empty problem");
  if (e.kind == GemmEpi::Geglu) MRT_REQUIRE(N % 64 == 0, "gemm: gated-GELU needs N % 64 == 0");
  if (e.kind == GemmEpi::CrossKV)
    MRT_REQUIRE(e.HD == e.H * 64 && N % e.HD == 0 && M == e.nb * e.S, "gemm: bad cross-KV shape");
  MRT_DTYPE_DISPATCH(dt, gemm_t<T>(static_cast<const T*>(A), static_cast<const T*>(B), M, N, K, e, s, allow_mfma));
  MRT_HIP_CHECK(hipGetLastError());
}

namespace {

template <typename T>
void encoder_attn_t(const T* qkv, int nb, int S, int H, T* out, hipStream_t s, bool allow_mfma) {
  if constexpr (sizeof(T) == 2) {
    if (allow_mfma) {
      hipLaunchKernelGGL(k_enc_attn_mfma<T>, dim3((S + kAQ - 1) / kAQ, nb * H), dim3(256), 0, s, qkv, S, H, out);
      return;
    }
  }
  hipLaunchKernelGGL(k_enc_attn<T>, dim3((S + 63) / 64, nb * H), dim3(64), 0, s, qkv, S, H, out);
}

}  // namespace

void encoder_attn(DType dt, const void* qkv, int nb, int S, int H, void* out, hipStream_t s, bool allow_mfma) {
  MRT_DTYPE_DISPATCH(dt, encoder_attn_t<T>(static_cast<const T*>(qkv), nb, S, H, static_cast<T*>(out), s, allow_mfma));
  MRT_HIP_CHECK(hipGetLastError());
}

}  // namespace mrt
