// Token plumbing between chunks of a stream, on the device (the LLM half of
// System::generate_chunk around the decode): the next chunk's encoder inputs
// from the RVQ context (system.cpp:62-95), and the decoded LLM ids turned into
// RVQ codes (rvq.cpp:112-132, safe mode) that roll into the context
// (system.cpp:320-333).  Integer work, bit-exact with the reference.
#include "stream.hpp"

#include "device_utils.hpp"

namespace mrt {
namespace {

// out (2, frames * e + s): row 0 = codec ids of levels 0..e-1 of every frame
// (offset + C * level + code, MASK for an empty code), then the style ids (or
// MASK); row 1 = the same codec ids, every style slot MASK (system.cpp:62-95).
__global__ void k_encoder_inputs(const int* __restrict__ ctx, int frames, int levels, int e, const int* __restrict__ style,
                                 int s, int C, int offset, int mask, int* __restrict__ out) {
  const int n = frames * e + s;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    int id0, id1;
    if (i < frames * e) {
      const int f = i / e, d = i - f * e;
      const int v = ctx[f * levels + d];
      id0 = id1 = v >= 0 ? offset + C * d + v : mask;
    } else {
      id0 = style ? style[i - frames * e] : mask;
      id1 = mask;
    }
    out[i] = id0;
    out[n + i] = id1;
  }
}

// One workgroup: every thread reads its (up to kRollPer) elements of the
// rolled context into registers, then all write after a barrier, so the roll
// is in place.  Row r < frames - n takes context row r + n; row frames - n + j
// takes the RVQ codes of chunk frame j: code = (t - offset) mod C (floor), and
// (t - offset) - code must equal C * level.  One id at the wrong level leaves
// the context untouched and sets *err = 1 (the reference's safe mode raises
// before the context is replaced).
constexpr int kRollThreads = 256, kRollPer = 32;

__global__ __launch_bounds__(kRollThreads) void k_llm_to_rvq_roll(const int* __restrict__ llm, int n, int levels, int C,
                                                                  int offset, int* ctx, int frames, int* err) {
  const int total = frames * levels;
  int val[kRollPer];
  bool bad = false;
#pragma unroll
  for (int u = 0; u < kRollPer; ++u) {
    const int i = threadIdx.x + u * kRollThreads;
    val[u] = 0;
    if (i < total) {
      const int r = i / levels, l = i - r * levels;
      if (r < frames - n) {
        val[u] = ctx[(r + n) * levels + l];
      } else {
        const int shifted = llm[(r - (frames - n)) * levels + l] - offset;
        const int code = ((shifted % C) + C) % C;
        bad = bad || shifted - code != C * l;
        val[u] = code;
      }
    }
  }
  __shared__ int any_bad;
  if (threadIdx.x == 0) any_bad = 0;
  __syncthreads();  // also orders every read of ctx before the first write
  if (bad) any_bad = 1;
  __syncthreads();
  if (any_bad) {
    if (threadIdx.x == 0) *err = 1;
    return;
  }
#pragma unroll
  for (int u = 0; u < kRollPer; ++u) {
    const int i = threadIdx.x + u * kRollThreads;
    if (i < total) ctx[i] = val[u];
  }
}

// The codec input of a chunk (system.cpp:294-313) from the rolled context
// (frames, levels): xf rows = the context's rows before the chunk's (the last
// rows before the roll), negative ids clamped to 0, zeros on the first chunk;
// then the chunk's n rows.
__global__ void k_codec_frames(const int* __restrict__ ctx, int frames, int levels, int n, int xf, int first,
                               int* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (n + xf) * levels) return;
  const int f = i / levels;
  const int v = ctx[(size_t)(frames - n - xf) * levels + i];
  out[i] = f < xf ? (first ? 0 : max(v, 0)) : v;
}

// system.cpp:410-437: out = audio[0, T - xf) with its first xf samples ramped
// in (sin(t pi/2)) against the previous tail ramped out (sin((1 - t) pi/2)),
// t = i / (xf - 1), unless `fade` is 0; the tail becomes audio[T - xf, T).
// Thread i reads tail[i] before it writes it (i < 2 xf), so the update is
// race-free.
__global__ void k_crossfade(const float* __restrict__ audio, int T, int xf, int fade, float* __restrict__ tail,
                            float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 2 * T) return;
  const int j = i >> 1;
  if (j < T - xf) {
    float v = audio[i];
    if (fade && j < xf) {
      const float t = (float)j / (float)(xf - 1 == 0 ? 1 : xf - 1);
      const float fin = sinf(t * 1.5707963267948966f);
      const float fout = sinf((1.0f - t) * 1.5707963267948966f);
      v = v * fin + tail[i] * fout;
    }
    out[i] = v;
  }
  if (i < 2 * xf) tail[i] = audio[2 * (T - xf) + i];
}

}  // namespace

void encoder_inputs(const int* ctx, int frames, int levels, int e, const int* style, int s, int C, int offset,
                    int mask, int* out, hipStream_t st) {
  const int n = frames * e + s;
  hipLaunchKernelGGL(k_encoder_inputs, dim3((n + 255) / 256), dim3(256), 0, st, ctx, frames, levels, e, style, s, C,
                     offset, mask, out);
  MRT_HIP_CHECK(hipGetLastError());
}

bool llm_to_rvq_roll_fits(int frames, int levels) { return frames * levels <= kRollThreads * kRollPer; }

void llm_to_rvq_roll(const int* llm, int n, int levels, int C, int offset, int* ctx, int frames, int* err,
                     hipStream_t st) {
  hipLaunchKernelGGL(k_llm_to_rvq_roll, dim3(1), dim3(kRollThreads), 0, st, llm, n, levels, C, offset, ctx, frames,
                     err);
  MRT_HIP_CHECK(hipGetLastError());
}

void codec_frames(const int* ctx, int frames, int levels, int n, int xf, bool first, int* out, hipStream_t st) {
  const int m = (n + xf) * levels;
  hipLaunchKernelGGL(k_codec_frames, dim3((m + 255) / 256), dim3(256), 0, st, ctx, frames, levels, n, xf, first ? 1 : 0,
                     out);
  MRT_HIP_CHECK(hipGetLastError());
}

void crossfade(const float* audio, int T, int xf, bool fade, float* tail, float* out, hipStream_t st) {
  hipLaunchKernelGGL(k_crossfade, dim3((2 * T + 255) / 256), dim3(256), 0, st, audio, T, xf, fade ? 1 : 0, tail, out);
  MRT_HIP_CHECK(hipGetLastError());
}

}  // namespace mrt
