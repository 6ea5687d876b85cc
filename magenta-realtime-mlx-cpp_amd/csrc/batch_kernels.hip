// Batched-stream decode kernels for gfx950: B independent streams decoded
// together, R = 2B activation rows (both CFG rows of every stream), R <= 64.
//
// At R = 64 every weight row meets 64 activation rows, so the projections are
// skinny GEMMs and run on the matrix cores: v_mfma_f32_16x16x32_bf16, one
// block per 16 output columns, the 4 waves of a block splitting K and summing
// their partial tiles through LDS in a fixed order (deterministic).  The
// activations (R x K, at most 360 KB) are read by every block from L2; the
// weights stream from HBM/MALL once per step.
#include "batch.hpp"
#include "device_utils.hpp"
#include "kernels.hpp"

namespace mrt {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBgCols = 16;  // output columns per block
constexpr int kBgChunk = 8;  // k-steps (of 32) whose loads a wave keeps in flight

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

struct BResid {
  bf16* r;
  int ldr;
  __device__ void operator()(int m, int n, const float (&v)[1]) const {
    bf16* p = r + (size_t)m * ldr + n;
    *p = St<bf16>::st(St<bf16>::ld(*p) + St<bf16>::rnd(v[0]));
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
// Wave w takes k-steps w, w + 4, ...; rows past M are zero, columns past nout
// re-read the last row and are not stored.
template <int P, class Epi>
__global__ __launch_bounds__(256) void k_bgemm(const bf16* __restrict__ X, int M, int K, const bf16* __restrict__ W,
                                               int nout, Epi epi) {
  __shared__ float part[4][P][kBatchRows][kBgCols + 1];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int j0 = blockIdx.x * kBgCols;
  const int c16 = lane & 15, kg = lane >> 4;
  const bf16* wrow[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int j = min(j0 + c16, nout - 1);
    wrow[p] = W + (size_t)(P == 1 ? j : bg_geglu_row(j, p)) * K + kg * 8;
  }
  const bf16* xrow[4];
  bool xin[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int m = 16 * t + c16;
    xin[t] = m < M;
    xrow[t] = X + (size_t)min(m, M - 1) * K + kg * 8;
  }
  f32x4_t acc[P][4];
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[p][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nks = K / 32;
  for (int s0 = wid; s0 < nks; s0 += 4 * kBgChunk) {
    uint4 b[kBgChunk][P], a[kBgChunk][4];
#pragma unroll
    for (int c = 0; c < kBgChunk; ++c) {
      const int ks = s0 + 4 * c;
      if (ks < nks) {
#pragma unroll
        for (int p = 0; p < P; ++p) b[c][p] = ld_g16(wrow[p] + ks * 32);
#pragma unroll
        for (int t = 0; t < 4; ++t) a[c][t] = xin[t] ? ld_g16(xrow[t] + ks * 32) : make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int c = 0; c < kBgChunk; ++c) {
      if (s0 + 4 * c < nks) {
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int t = 0; t < 4; ++t)
            acc[p][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[c][t]),
                                                                __builtin_bit_cast(bf16x8_t, b[c][p]), acc[p][t], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[wid][p][16 * t + 4 * kg + i][c16] = acc[p][t][i];
  __syncthreads();
  for (int idx = tid; idx < kBatchRows * kBgCols; idx += 256) {
    const int m = idx / kBgCols, n = idx % kBgCols;
    if (m >= M || j0 + n >= nout) continue;
    float v[P];
#pragma unroll
    for (int p = 0; p < P; ++p) v[p] = ((part[0][p][m][n] + part[1][p][m][n]) + part[2][p][m][n]) + part[3][p][m][n];
    epi(m, j0 + n, v);
  }
}

template <int P, class Epi>
void launch_bgemm(const bf16* X, int M, int K, const bf16* W, int nout, const Epi& epi, hipStream_t s) {
  MRT_REQUIRE(M >= 1 && M <= kBatchRows, "batched GEMM: rows must be in [1, 64]");
  MRT_REQUIRE(K % 32 == 0 && K >= 32, "batched GEMM: K must be a multiple of 32");
  MRT_REQUIRE(nout >= 1, "batched GEMM: no outputs");
  hipLaunchKernelGGL((k_bgemm<P, Epi>), dim3((nout + kBgCols - 1) / kBgCols), dim3(256), 0, s, X, M, K, W, nout, epi);
  MRT_HIP_CHECK(hipGetLastError());
}

__global__ void k_set_counter(int* p, int v) { *p = v; }
__global__ void k_advance_counter(int* p) { *p = *p + 1; }

}  // namespace

void set_counter(int* p, int v, hipStream_t s) {
  hipLaunchKernelGGL(k_set_counter, dim3(1), dim3(1), 0, s, p, v);
  MRT_HIP_CHECK(hipGetLastError());
}

void advance_counter(int* p, hipStream_t s) {
  hipLaunchKernelGGL(k_advance_counter, dim3(1), dim3(1), 0, s, p);
  MRT_HIP_CHECK(hipGetLastError());
}

void bgemm_store(const void* X, int M, int K, const void* W, int N, void* Y, int ldy, hipStream_t s) {
  launch_bgemm<1>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W), N, BStore{static_cast<bf16*>(Y), ldy},
                  s);
}

void bgemm_f32(const void* X, int M, int K, const void* W, int N, float* Y, int ldy, hipStream_t s) {
  launch_bgemm<1>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W), N, BF32{Y, ldy}, s);
}

void bgemm_resid(const void* X, int M, int K, const void* W, int N, void* R, int ldr, hipStream_t s) {
  launch_bgemm<1>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W), N, BResid{static_cast<bf16*>(R), ldr},
                  s);
}

void bgemm_qkv(const void* X, int M, int K, const void* W, int HD, void* Q, void* Kc, void* Vc, int H, int Lmax, int pos,
               const int* pos_ptr, hipStream_t s) {
  BQKV e{static_cast<bf16*>(Q), static_cast<bf16*>(Kc), static_cast<bf16*>(Vc), HD, H, Lmax, pos, pos_ptr};
  launch_bgemm<1>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W), 3 * HD, e, s);
}

void bgemm_geglu(const void* X, int M, int K, const void* W01, int F, void* Hout, int ldh, hipStream_t s) {
  MRT_REQUIRE(F % 32 == 0, "batched GEMM: d_ff must be a multiple of 32 (packed gate/up groups)");
  launch_bgemm<2>(static_cast<const bf16*>(X), M, K, static_cast<const bf16*>(W01), F,
                  BGeglu{static_cast<bf16*>(Hout), ldh}, s);
}

}  // namespace mrt
