// MusicCoCa text-path kernels (fp32): embedding, LayerNorm, the attention
// core and RVQ quantisation.  The projections run on the codec's matrix-core
// GEMM (codec_kernels.hip).
#include "coca.hpp"

namespace mrt {
namespace {

constexpr int kT = 256;

__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += red[i];
  return s;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float s = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) s = fmaxf(s, red[i]);
  return s;
}

// musiccoca.cpp:272-277: x = table[id] * sqrt(d_model).
__global__ void k_coca_embed(const int* __restrict__ ids, const float* __restrict__ table, int vocab, int D, float scale,
                             float* __restrict__ x) {
  int id = ids[blockIdx.x];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  for (int d = threadIdx.x; d < D; d += blockDim.x) x[(size_t)blockIdx.x * D + d] = table[(size_t)id * D + d] * scale;
}

// musiccoca.cpp:71-79: mean, centred, variance of the centred values, then
// centred * rsqrt(var + eps) * w + b.  One workgroup per row.
__global__ __launch_bounds__(kT) void k_layer_norm(const float* __restrict__ x, int D, const float* __restrict__ w,
                                                   const float* __restrict__ b, float eps, float* __restrict__ y) {
  __shared__ float red[kT / 64];
  const float* xr = x + (size_t)blockIdx.x * D;
  float s = 0.f;
  for (int d = threadIdx.x; d < D; d += kT) s += xr[d];
  const float mean = block_sum(s, red) / (float)D;
  float v = 0.f;
  for (int d = threadIdx.x; d < D; d += kT) {
    const float c = xr[d] - mean;
    v += c * c;
  }
  const float var = block_sum(v, red) / (float)D;
  const float inv = rsqrtf(var + eps);
  for (int d = threadIdx.x; d < D; d += kT) y[(size_t)blockIdx.x * D + d] = (xr[d] - mean) * inv * w[d] + b[d];
}

// One workgroup per (query, head): thread j < Sk scores key j, the softmax
// runs over the workgroup, then threads split the head's D outputs.
__global__ __launch_bounds__(kT) void k_coca_attention(const float* __restrict__ q, int ldq,
                                                       const float* __restrict__ k, int ldk,
                                                       const float* __restrict__ v, int ldv, int Sk, int D,
                                                       const float* __restrict__ qscale, float cap,
                                                       const float* __restrict__ mask, float* __restrict__ out,
                                                       int ldo) {
  __shared__ float qs[256];
  __shared__ float p[256];
  __shared__ float red[kT / 64];
  const int i = blockIdx.x, h = blockIdx.y;
  for (int d = threadIdx.x; d < D; d += kT) {
    const float qv = q[(size_t)i * ldq + h * D + d];
    qs[d] = qscale ? qv * qscale[d] : qv;
  }
  __syncthreads();
  const int j = threadIdx.x;
  float s = -INFINITY;
  if (j < Sk) {
    const float* kr = k + (size_t)j * ldk + h * D;
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc += qs[d] * kr[d];
    s = acc * (1.0f / sqrtf((float)D));
    if (cap > 0.f) s = cap * tanhf(s / cap);
    if (mask) s += mask[j];
  }
  const float m = block_max(s, red);
  const float e = j < Sk ? expf(s - m) : 0.f;
  const float sum = block_sum(e, red);
  p[j] = e / sum;
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += kT) {
    float acc = 0.f;
    for (int t = 0; t < Sk; ++t) acc += p[t] * v[(size_t)t * ldv + h * D + d];
    out[(size_t)i * ldo + h * D + d] = acc;
  }
}

// The same attention for a block of 4 queries of one head (self-attention of
// the text layers: Sk <= 128, D <= 64, D % 4 == 0): the head's K and V rows
// are staged in LDS (16-byte global loads) once per block instead of being
// read from global memory per query.  Wave r owns query row r: its lanes
// score keys l and l + 64 (rows padded to D + 1 floats: a half-wave's keys sit
// in distinct banks), the softmax runs in registers, and lane l < D then sums
// output column l.
constexpr int kAttQ = 4, kAttSk = 128, kAttD = 64;
__global__ __launch_bounds__(kT) void k_coca_attention_tile(const float* __restrict__ q, int ldq,
                                                            const float* __restrict__ k, int ldk,
                                                            const float* __restrict__ v, int ldv, int Sq, int Sk,
                                                            int D, float cap, const float* __restrict__ mask,
                                                            float* __restrict__ out, int ldo) {
  __shared__ float ks[kAttSk][kAttD + 1];
  __shared__ float vs[kAttSk][kAttD + 1];
  __shared__ float qs[kAttQ][kAttD];
  __shared__ float ps[kAttQ][kAttSk];
  const int q0 = blockIdx.x * kAttQ, h = blockIdx.y, t = threadIdx.x;
  const int nq = min(kAttQ, Sq - q0), D4 = D >> 2;
  for (int i = t; i < Sk * D4; i += kT) {
    const int j = i / D4, c = 4 * (i - j * D4);
    const float4 kv = *reinterpret_cast<const float4*>(k + (size_t)j * ldk + h * D + c);
    const float4 vv = *reinterpret_cast<const float4*>(v + (size_t)j * ldv + h * D + c);
    ks[j][c] = kv.x;
    ks[j][c + 1] = kv.y;
    ks[j][c + 2] = kv.z;
    ks[j][c + 3] = kv.w;
    vs[j][c] = vv.x;
    vs[j][c + 1] = vv.y;
    vs[j][c + 2] = vv.z;
    vs[j][c + 3] = vv.w;
  }
  for (int i = t; i < nq * D; i += kT) {
    const int r = i / D, d = i - r * D;
    qs[r][d] = q[(size_t)(q0 + r) * ldq + h * D + d];
  }
  __syncthreads();
  const int r = t >> 6, l = t & 63;
  if (r >= nq) return;  // no barrier follows
  const float scale = 1.0f / sqrtf((float)D);
  float sc[kAttSk / 64];
#pragma unroll
  for (int m = 0; m < kAttSk / 64; ++m) {
    const int j = l + 64 * m;
    float s = -INFINITY;
    if (j < Sk) {
      float acc = 0.f;
      for (int d = 0; d < D; ++d) acc += qs[r][d] * ks[j][d];
      s = acc * scale;
      if (cap > 0.f) s = cap * tanhf(s / cap);
      if (mask) s += mask[j];
    }
    sc[m] = s;
  }
  float mx = sc[0];
#pragma unroll
  for (int m = 1; m < kAttSk / 64; ++m) mx = fmaxf(mx, sc[m]);
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  float sum = 0.f;
#pragma unroll
  for (int m = 0; m < kAttSk / 64; ++m) {
    sc[m] = l + 64 * m < Sk ? expf(sc[m] - mx) : 0.f;
    sum += sc[m];
  }
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
#pragma unroll
  for (int m = 0; m < kAttSk / 64; ++m)
    if (l + 64 * m < Sk) ps[r][l + 64 * m] = sc[m] / sum;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the row's probabilities are in LDS
  if (l < D) {
    float acc = 0.f;
    for (int j = 0; j < Sk; ++j) acc += ps[r][j] * vs[j][l];
    out[(size_t)(q0 + r) * ldo + h * D + l] = acc;
  }
}

// rvq.cpp:24-62, one vector: per level, every code's distance (|r|^2 - 2
// r.c) + |c|^2 (one thread per code), the first minimum, then residual -=
// the chosen row.  One workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void k_rvq_quantize(const float* __restrict__ vec, const float* __restrict__ cb,
                                                       int K, int C, int D, float* __restrict__ res,
                                                       int* __restrict__ tokens) {
  __shared__ float r[4096];
  __shared__ float red[16];
  __shared__ float bestv[16];
  __shared__ int besti[16];
  __shared__ int tok_s;
  const int t = threadIdx.x;
  for (int d = t; d < D; d += 1024) r[d] = vec[d];
  __syncthreads();
  for (int k = 0; k < K; ++k) {
    float part = 0.f;
    for (int d = t; d < D; d += 1024) part += r[d] * r[d];
    const float r2 = block_sum(part, red);
    float dist = INFINITY;
    if (t < C) {
      const float* row = cb + ((size_t)k * C + t) * D;
      float cross = 0.f, c2 = 0.f;
      for (int d = 0; d < D; ++d) {
        const float c = row[d];
        cross += r[d] * c;
        c2 += c * c;
      }
      dist = (r2 - 2.0f * cross) + c2;
    }
    // first minimum: (value, index) with the lower index on ties
    int idx = t;
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(dist, o);
      const int oi = __shfl_xor(idx, o);
      if (ov < dist || (ov == dist && oi < idx)) {
        dist = ov;
        idx = oi;
      }
    }
    if ((t & 63) == 0) {
      bestv[t >> 6] = dist;
      besti[t >> 6] = idx;
    }
    __syncthreads();
    if (t == 0) {
      float bv = bestv[0];
      int bi = besti[0];
      for (int w = 1; w < 16; ++w)
        if (bestv[w] < bv || (bestv[w] == bv && besti[w] < bi)) {
          bv = bestv[w];
          bi = besti[w];
        }
      tok_s = bi < C ? bi : 0;
      tokens[k] = tok_s;
    }
    __syncthreads();
    const float* chosen = cb + ((size_t)k * C + tok_s) * D;
    for (int d = t; d < D; d += 1024) r[d] = r[d] - chosen[d];
    __syncthreads();
  }
  for (int d = t; d < D; d += 1024) res[d] = r[d];
}

}  // namespace

void coca_embed(const int* ids, int rows, const float* table, int vocab, int D, float scale, float* x,
                hipStream_t s) {
  hipLaunchKernelGGL(k_coca_embed, dim3(rows), dim3(kT), 0, s, ids, table, vocab, D, scale, x);
  MRT_HIP_CHECK(hipGetLastError());
}

void layer_norm_rows(const float* x, int rows, int D, const float* w, const float* b, float eps, float* y,
                     hipStream_t s) {
  hipLaunchKernelGGL(k_layer_norm, dim3(rows), dim3(kT), 0, s, x, D, w, b, eps, y);
  MRT_HIP_CHECK(hipGetLastError());
}

void coca_attention(const float* q, int ldq, const float* k, int ldk, const float* v, int ldv, int Sq, int Sk, int H,
                    int D, const float* qscale, float cap, const float* mask, float* out, hipStream_t s) {
  MRT_REQUIRE(Sk >= 1 && Sk <= kT && D >= 1 && D <= 256, "coca attention: Sk <= 256 and d_head <= 256");
  if (!qscale && Sk <= kAttSk && D <= kAttD && D % 4 == 0 && ldk % 4 == 0 && ldv % 4 == 0 &&
      reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0) {
    // query blocks with the head's K / V in LDS
    hipLaunchKernelGGL(k_coca_attention_tile, dim3((Sq + kAttQ - 1) / kAttQ, H), dim3(kT), 0, s, q, ldq, k, ldk, v,
                       ldv, Sq, Sk, D, cap, mask, out, H * D);
  } else {
    hipLaunchKernelGGL(k_coca_attention, dim3(Sq, H), dim3(kT), 0, s, q, ldq, k, ldk, v, ldv, Sk, D, qscale, cap,
                       mask, out, H * D);
  }
  MRT_HIP_CHECK(hipGetLastError());
}

void rvq_quantize(const float* vec, const float* codebooks, int K, int C, int D, float* residual, int* tokens,
                  hipStream_t s) {
  MRT_REQUIRE(C >= 1 && C <= 1024 && D >= 1 && D <= 4096, "rvq_quantize: codebook <= 1024, dim <= 4096");
  hipLaunchKernelGGL(k_rvq_quantize, dim3(1), dim3(1024), 0, s, vec, codebooks, K, C, D, residual, tokens);
  MRT_HIP_CHECK(hipGetLastError());
}

}  // namespace mrt
