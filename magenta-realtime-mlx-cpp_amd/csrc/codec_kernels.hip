// Codec decode kernels (fp32): the implicit-GEMM convolution on the matrix
// cores, RVQ dequantisation and the iSTFT overlap-add.
//
// k_conv<BM, BN, KC>: a BM x BN output tile (pixels x channels) per
// 256-thread workgroup (64 x 64: larger tiles measured slower, fewer
// workgroups per CU hide less load latency), 4 waves in a 2 x 2 grid, each
// wave BM/32 x BN/32 tiles of v_mfma_f32_16x16x4_f32.  The K loop runs over (tap, KC-channel chunk);
// each chunk's A rows (the tap's input pixel for every output pixel of the
// tile, zero outside the input, ELU applied on load when asked) and B rows
// (packed weights) are staged through a double-buffered LDS with one barrier
// per chunk; the global loads run two chunks ahead of the multiplies (two
// register sets).  LDS strides: A rows KC + 4 floats (the 16 rows x 4 k lanes of
// an A fragment hit 64 distinct banks), B rows 80 floats (the same for B).
#include "codec.hpp"

#include <type_traits>

namespace mrt {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float elu1(float v) { return v > 0.f ? v : expf(v) - 1.f; }

// The epilogue of output (sub-local row m, channel o): bias, residual (at the
// output pixel divided by the repeat factors), ELU, store (with the stereo
// split of the output channels).
__device__ __forceinline__ void conv_store(const ConvLaunch& a, const ConvSub* sub, int m, int o, float val) {
  const int gy = sub->gy, gx = sub->gx;
  const int img = m / (gy * gx), r = m - img * gy * gx;
  const int yy = r / gx, xx = r - (r / gx) * gx;
  const int oy = yy * sub->oys + sub->oyo, ox = xx * sub->oxs + sub->oxo;
  if (a.bias) val += a.bias[o];
  if (a.res) val += a.res[((size_t)(img * a.res_h + oy / a.rh) * a.res_w + ox / a.rw) * a.cout + o];
  if (a.act_out == kActElu) val = elu1(val);
  else if (a.act_out == kActGelu) val = val * 0.5f * (1.0f + erff(val * 0.7071067811865475f));
  const int oi = (o / a.split) * a.n + img, oc = o - (o / a.split) * a.split;
  const size_t idx = ((size_t)(oi * a.hout + oy) * a.wout + ox) * a.split + oc;
  a.y[idx] = val;
  if (a.y_elu) a.y_elu[idx] = elu1(val);
}

template <int BM, int BN, int KC>
__global__ __launch_bounds__(kThreads) void k_conv(ConvLaunch a) {
  constexpr int AS = KC + 4;  // the 16 rows x 4 k lanes of an A fragment hit 64 distinct banks
  constexpr int BS = BN + 16;  // the 4 k rows x 16 columns of a B fragment hit 64 distinct banks
  constexpr int CPR = KC / 4;             // float4 chunks per A row
  constexpr int RPP = kThreads / CPR;     // A rows per load pass
  constexpr int APASS = BM / RPP;         // A loads per thread
  constexpr int BCPR = BN / 4, BRPP = kThreads / BCPR, BPASS = KC / BRPP;  // B loads per thread
  constexpr int TM = BM / 32, TN = BN / 32;  // 16 x 16 tiles per wave (2 x 2 waves)
  static_assert(BM % RPP == 0 && KC % BRPP == 0 && BPASS >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) float As[2][BM * AS];
  __shared__ __attribute__((aligned(16))) float Bs[2][KC * BS];

  int si = 0;
  while (si + 1 < a.nsub && (int)blockIdx.x >= a.subs[si + 1].tile0) ++si;
  const ConvSub* sub = a.subs + si;
  const int gy = sub->gy, gx = sub->gx, ntaps = sub->ntaps;
  const int M = a.n * gy * gx;
  const int m0 = ((int)blockIdx.x - sub->tile0) * BM;
  const int n0 = (int)blockIdx.y * BN;
  const float* __restrict__ W = sub->w;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  // this thread's A rows: image offset and grid coordinates
  int a_img[APASS], a_y[APASS], a_x[APASS];
  const int a_chunk = tid % CPR;
#pragma unroll
  for (int p = 0; p < APASS; ++p) {
    const int m = min(m0 + tid / CPR + p * RPP, M - 1);
    const int img = m / (gy * gx), r = m - img * gy * gx;
    a_img[p] = img * a.hin;
    a_y[p] = r / gx;
    a_x[p] = r - (r / gx) * gx;
  }
  const int b_col = (tid % BCPR) * 4;
  const int b_row = tid / BCPR;

  const int cpt = a.cin / KC;
  const int nk_all = ntaps * cpt;
  const int kb = (int)blockIdx.z * nk_all / a.ksplit, ke = ((int)blockIdx.z + 1) * nk_all / a.ksplit;
  const int nk = ke - kb;
  // two register sets: chunk kc + 2 is loaded while chunk kc is multiplied
  // and chunk kc + 1 (loaded a whole chunk earlier) goes to the LDS
  float ra[2][APASS][4], rb[2][BPASS][4];
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  // the A rows' input pixels depend on the tap only: recomputed when it changes
  int cur_t = -1;
  bool a_ok[APASS];
  const float* a_src[APASS];
  auto load = [&](int kc, auto S) {
    constexpr int q = decltype(S)::value;
    kc += kb;
    const int t = kc / cpt, c0 = (kc - t * cpt) * KC + a_chunk * 4;
    if (t != cur_t) {
      cur_t = t;
      const int dy = sub->dy[t], dx = sub->dx[t];
#pragma unroll
      for (int p = 0; p < APASS; ++p) {
        const int iy = a_y[p] + dy, ix = a_x[p] + dx;
        a_ok[p] = iy >= 0 && iy < a.hin && ix >= 0 && ix < a.win;
        a_src[p] = a.x + ((size_t)(a_img[p] + (a_ok[p] ? iy : 0)) * a.win + (a_ok[p] ? ix : 0)) * a.cin;
      }
    }
#pragma unroll
    for (int p = 0; p < APASS; ++p) {
      const bool ok = a_ok[p];
      const float4 v = *reinterpret_cast<const float4*>(a_src[p] + c0);
      ra[q][p][0] = ok ? v.x : 0.f;
      ra[q][p][1] = ok ? v.y : 0.f;
      ra[q][p][2] = ok ? v.z : 0.f;
      ra[q][p][3] = ok ? v.w : 0.f;
    }
    const float* wb = W + ((size_t)t * a.cin + (kc - t * cpt) * KC) * a.cout_pad + n0 + b_col;
#pragma unroll
    for (int p = 0; p < BPASS; ++p) {
      const float4 v = *reinterpret_cast<const float4*>(wb + (size_t)(b_row + p * BRPP) * a.cout_pad);
      rb[q][p][0] = v.x;
      rb[q][p][1] = v.y;
      rb[q][p][2] = v.z;
      rb[q][p][3] = v.w;
    }
  };
  auto store = [&](auto S) {  // register set q -> LDS buffer q
    constexpr int q = decltype(S)::value;
#pragma unroll
    for (int p = 0; p < APASS; ++p) {
      float4 v = make_float4(ra[q][p][0], ra[q][p][1], ra[q][p][2], ra[q][p][3]);
      if (a.elu_in) {  // zero padding stays 0 (elu(0) = 0)
        v.x = elu1(v.x);
        v.y = elu1(v.y);
        v.z = elu1(v.z);
        v.w = elu1(v.w);
      }
      *reinterpret_cast<float4*>(&As[q][(tid / CPR + p * RPP) * AS + a_chunk * 4]) = v;
    }
#pragma unroll
    for (int p = 0; p < BPASS; ++p)
      *reinterpret_cast<float4*>(&Bs[q][(b_row + p * BRPP) * BS + b_col]) =
          make_float4(rb[q][p][0], rb[q][p][1], rb[q][p][2], rb[q][p][3]);
  };

  typedef float f4 __attribute__((ext_vector_type(4)));
  f4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, lk = lane >> 4;
  auto step = [&](int kc, auto S) {  // chunk kc, held in LDS buffer q = kc & 1
    constexpr int q = decltype(S)::value;
    if (kc + 2 < nk) load(kc + 2, S);
    const float* Ab = As[q] + (wm * (BM / 2) + lr) * AS + lk;
    const float* Bb = Bs[q] + lk * BS + wn * (BN / 2) + lr;
#pragma unroll
    for (int ks = 0; ks < KC / 4; ++ks) {
      float av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) av[i] = Ab[i * 16 * AS + ks * 4];
#pragma unroll
      for (int j = 0; j < TN; ++j) bv[j] = Bb[ks * 4 * BS + j * 16];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (kc + 1 < nk) store(std::integral_constant<int, 1 - q>{});
    __syncthreads();
  };
  if (nk > 0) {
    load(0, I0{});
    if (nk > 1) load(1, I1{});
    store(I0{});
  }
  __syncthreads();
  for (int kc = 0; kc < nk; kc += 2) {
    step(kc, I0{});
    if (kc + 1 < nk) step(kc + 1, I1{});
  }

  // epilogue: lane holds rows 4 * (lane / 16) + v, column lane % 16 of each tile
  if (a.ksplit > 1) {
    float* part = a.partial + ((size_t)blockIdx.z * a.rows + (size_t)blockIdx.x * BM) * a.cout_pad;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          part[(size_t)(wm * (BM / 2) + i * 16 + 4 * lk + v) * a.cout_pad + n0 + wn * (BN / 2) + j * 16 + lr] =
              acc[i][j][v];
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = m0 + wm * (BM / 2) + i * 16 + 4 * lk + v;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int o = n0 + wn * (BN / 2) + j * 16 + lr;
        if (o < a.cout) conv_store(a, sub, m, o, acc[i][j][v]);
      }
    }
  }
}

// Split-K finish: thread (tile row, channel) sums the slices in order, then
// the epilogue.
__global__ __launch_bounds__(256) void k_conv_finish(ConvLaunch a) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)a.rows * a.cout) return;
  const int row = (int)(i / a.cout), o = (int)(i - (size_t)row * a.cout);
  const int tile = row / 64;
  int si = 0;
  while (si + 1 < a.nsub && tile >= a.subs[si + 1].tile0) ++si;
  const ConvSub* sub = a.subs + si;
  const int m = (tile - sub->tile0) * 64 + (row - tile * 64);
  if (m >= a.n * sub->gy * sub->gx) return;
  float v = 0.f;
  for (int z = 0; z < a.ksplit; ++z) v += a.partial[((size_t)z * a.rows + row) * a.cout_pad + o];
  conv_store(a, sub, m, o, v);
}

// The output convolution (Cout = 2, a 7 x 7 kernel, causal padding, the
// first `crop` rows dropped; spectrostream.cpp:420-427) on the vector ALUs:
// a matrix-core tile would be 2 of 16 columns.  Workgroup: 4 output rows x
// 128 columns of one image and 256 threads, two halves over the input
// channels (waves 0-1 and 2-3, so the weights a wave needs are uniform and
// come through scalar loads); a thread owns a 4-pixel strip x 2 outputs.
// The input halo (4 + 6 rows x 128 + 6 columns) is staged through LDS 8
// channels at a time (4 per half) with the ELU applied; the halves' sums
// meet in LDS at the end.
constexpr int kOcRows = 4, kOcCols = 128, kOcStrip = 4, kOcThreads = 256;
constexpr int kOcCh = 8, kOcK = 7;
constexpr int kOcHaloR = kOcRows + kOcK - 1, kOcHaloC = kOcCols + kOcK - 1;
constexpr int kOcPlane = kOcHaloR * kOcHaloC;

__global__ __launch_bounds__(kOcThreads) void k_out_conv(const float* __restrict__ x, int H, int W, int cin, int crop,
                                                         int elu_in, const float* __restrict__ w,
                                                         const float* __restrict__ bias, float* __restrict__ out,
                                                         int Hs) {
  __shared__ float hl[kOcCh * kOcPlane];  // (channel, halo row, halo column)
  const int tid = threadIdx.x;
  const int img = blockIdx.z;
  const int y0 = blockIdx.y * kOcRows, x0 = blockIdx.x * kOcCols;
  const int half = __builtin_amdgcn_readfirstlane(tid >> 7);  // wave-uniform
  const int st = tid & 127;
  const int ty = st / (kOcCols / kOcStrip), tx = (st % (kOcCols / kOcStrip)) * kOcStrip;
  float acc[kOcStrip][2];
#pragma unroll
  for (int p = 0; p < kOcStrip; ++p) acc[p][0] = acc[p][1] = 0.f;
  // input row of halo row r: y0 + crop + r - (k - 1); column of halo column q: x0 + q - (k - 1) / 2
  const int iy0 = y0 + crop - (kOcK - 1), ix0 = x0 - (kOcK - 1) / 2;
  for (int c0 = 0; c0 < cin; c0 += kOcCh) {
    __syncthreads();  // the previous chunk's reads are done
    for (int i = tid; i < kOcPlane * 2; i += kOcThreads) {
      const int hh = i & 1, pix = i >> 1;
      const int r = pix / kOcHaloC, q = pix - r * kOcHaloC;
      const int iy = iy0 + r, ix = ix0 + q;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (iy >= 0 && iy < H && ix >= 0 && ix < W) {
        v = *reinterpret_cast<const float4*>(x + ((size_t)(img * H + iy) * W + ix) * cin + c0 + hh * 4);
        if (elu_in) {
          v.x = elu1(v.x);
          v.y = elu1(v.y);
          v.z = elu1(v.z);
          v.w = elu1(v.w);
        }
      }
      float* d = hl + (hh * 4) * kOcPlane + pix;
      d[0] = v.x;
      d[kOcPlane] = v.y;
      d[2 * kOcPlane] = v.z;
      d[3 * kOcPlane] = v.w;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int ch = c0 + half * 4 + c;
      const float* hc = hl + (half * 4 + c) * kOcPlane;
#pragma unroll
      for (int kh = 0; kh < kOcK; ++kh) {
        float in[kOcStrip + kOcK - 1];
#pragma unroll
        for (int q = 0; q < kOcStrip + kOcK - 1; ++q) in[q] = hc[(ty + kh) * kOcHaloC + tx + q];
#pragma unroll
        for (int kw = 0; kw < kOcK; ++kw) {
          const float* wk = w + ((size_t)(kh * kOcK + kw) * cin + ch) * 2;
          const float w0 = wk[0], w1 = wk[1];
#pragma unroll
          for (int p = 0; p < kOcStrip; ++p) {
            acc[p][0] = fmaf(in[p + kw], w0, acc[p][0]);
            acc[p][1] = fmaf(in[p + kw], w1, acc[p][1]);
          }
        }
      }
    }
  }
  // the upper half's sums join the lower half's through LDS
  __syncthreads();
  float* red = hl;
  if (half == 1) {
#pragma unroll
    for (int p = 0; p < kOcStrip; ++p) {
      red[(p * 2) * 128 + st] = acc[p][0];
      red[(p * 2 + 1) * 128 + st] = acc[p][1];
    }
  }
  __syncthreads();
  if (half == 1) return;
  const int oy = y0 + ty;
  if (oy >= Hs) return;
#pragma unroll
  for (int p = 0; p < kOcStrip; ++p) {
    const int ox = x0 + tx + p;
    if (ox >= W) continue;
    float* o = out + ((size_t)(img * Hs + oy) * W + ox) * 2;
    o[0] = acc[p][0] + red[(p * 2) * 128 + st] + bias[0];
    o[1] = acc[p][1] + red[(p * 2 + 1) * 128 + st] + bias[1];
  }
}

__global__ void k_rvq_dequant(const int* __restrict__ tokens, int frames, int levels,
                              const float* __restrict__ cb, int codebook, int dim, float* __restrict__ emb) {
  const int f = blockIdx.x;
  for (int d = threadIdx.x; d < dim; d += blockDim.x) {
    float s = 0.f;
    if (f < frames) {
      for (int k = 0; k < levels; ++k) {
        int id = tokens[f * levels + k];
        if (id < 0 || id >= codebook) id = 0;
        s = s + cb[((size_t)k * codebook + id) * dim + d];
      }
    }
    emb[(size_t)f * dim + d] = s;
  }
}

__global__ void k_overlap_add(const float* __restrict__ wf, int H, int n_fft, int T, float* __restrict__ audio) {
  const int hop = n_fft / 2;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 2 * T) return;
  const int t = i >> 1, s = i & 1;
  const int f = t / hop, j = t - f * hop;
  float v = 0.f;
  if (f < H) v = wf[(size_t)(s * H + f) * n_fft + j];
  if (f >= 1 && f - 1 < H) v += wf[(size_t)(s * H + f - 1) * n_fft + hop + j];
  audio[i] = v;
}

}  // namespace

void conv_launch(const ConvLaunch& a, int tiles_m, int tiles_n, hipStream_t s) {
  const dim3 grid(tiles_m, tiles_n, a.ksplit);
  if (a.cin % 32 == 0)
    hipLaunchKernelGGL((k_conv<64, 64, 32>), grid, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((k_conv<64, 64, 16>), grid, dim3(kThreads), 0, s, a);
  MRT_HIP_CHECK(hipGetLastError());
  if (a.ksplit > 1) {
    const size_t n = static_cast<size_t>(a.rows) * a.cout;
    hipLaunchKernelGGL(k_conv_finish, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, a);
    MRT_HIP_CHECK(hipGetLastError());
  }
}

void out_conv(const float* x, int n, int H, int W, int cin, int crop, bool elu_in, const float* w, const float* bias,
              float* out, int Hs, hipStream_t s) {
  MRT_REQUIRE(cin % kOcCh == 0, "codec: output conv input channels must be a multiple of 8");
  const dim3 grid((W + kOcCols - 1) / kOcCols, (Hs + kOcRows - 1) / kOcRows, n);
  hipLaunchKernelGGL(k_out_conv, grid, dim3(kOcThreads), 0, s, x, H, W, cin, crop, elu_in ? 1 : 0, w, bias, out, Hs);
  MRT_HIP_CHECK(hipGetLastError());
}

void rvq_dequant(const int* tokens, int frames, int levels, const float* codebooks, int codebook, int dim, int pad,
                 float* emb, hipStream_t s) {
  hipLaunchKernelGGL(k_rvq_dequant, dim3(frames + pad), dim3(256), 0, s, tokens, frames, levels, codebooks, codebook,
                     dim, emb);
  MRT_HIP_CHECK(hipGetLastError());
}

void overlap_add(const float* wf, int H, int n_fft, int T, float* audio, hipStream_t s) {
  const int n = 2 * T;
  hipLaunchKernelGGL(k_overlap_add, dim3((n + 255) / 256), dim3(256), 0, s, wf, H, n_fft, T, audio);
  MRT_HIP_CHECK(hipGetLastError());
}

}  // namespace mrt
