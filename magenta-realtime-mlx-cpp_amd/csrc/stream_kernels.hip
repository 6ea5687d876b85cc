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

}  // namespace mrt
