// Speculative depth decoding (decode.cpp:150-237, 380-446): the token
// plumbing around the verification pass.  The drafts of frame f are the
// previous chunk's tokens of frame f (build_depth_draft, decode.cpp:150-166);
// one causal pass over [temporal_out, emb(draft 0..L-2)] gives every level's
// logits (depth_forward_full, model.cpp:243-268); every level is drawn with
// its own noise, the drafts are accepted up to the first disagreement, whose
// draw is the model's token, and the remaining levels run as ordinary depth
// steps.  Tokens come out as generate_tokens would produce them from the same
// logits.
#include "device_utils.hpp"
#include "kernels.hpp"
#include "spec.hpp"

namespace mrt {
namespace {

// out rows m = 2i + r: i = 0 -> the temporal output row r; i >= 1 ->
// emb(draft[i - 1]) (both CFG rows take the same token, decode.cpp:184-197).
template <typename T>
__global__ void k_spec_inputs(const T* __restrict__ t_out, const T* __restrict__ emb, const int* __restrict__ draft,
                              int D, T* __restrict__ out) {
  const int m = blockIdx.x, i = m >> 1, r = m & 1;
  const T* src = i == 0 ? t_out + (size_t)r * D : emb + (size_t)draft[i - 1] * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) out[(size_t)m * D + d] = src[d];
}

// decode.cpp:225-236: the first level whose draw differs from its draft ends
// the accepted run and takes the draw; tokens[0..n] = drawn[0..n], *decided =
// n (L when every draft was accepted).  Level 0's token is always decided:
// both rows of next_in = emb(drawn[0]), the input of depth step 1.
template <typename T>
__global__ void k_spec_accept(const int* __restrict__ drawn, const int* __restrict__ draft, int L,
                              int* __restrict__ tokens, int* __restrict__ decided, const T* __restrict__ emb, int D,
                              T* __restrict__ next_in) {
  if (threadIdx.x == 0) {
    int n = L;
    for (int i = 0; i < L; ++i)
      if (drawn[i] != draft[i]) {
        n = i;
        break;
      }
    for (int i = 0; i <= n && i < L; ++i) tokens[i] = drawn[i];
    *decided = n;
  }
  const T* src = emb + (size_t)drawn[0] * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    next_in[d] = src[d];
    next_in[D + d] = src[d];
  }
}

// The frame mean of the L fed tokens (decode.cpp:476-484): sum in the model
// dtype, rounded after every level, divided by L in the model dtype; both rows.
template <typename T>
__global__ void k_frame_mean_tokens(const int* __restrict__ tokens, int L, const T* __restrict__ emb, int D,
                                    T* __restrict__ out) {
  using S = St<T>;
  const float Lf = S::rnd((float)L);
  for (int d = blockIdx.x * blockDim.x + threadIdx.x; d < D; d += gridDim.x * blockDim.x) {
    float fs = S::ld(emb[(size_t)tokens[0] * D + d]);
    for (int l = 1; l < L; ++l) fs = S::rnd(fs + S::ld(emb[(size_t)tokens[l] * D + d]));
    const T m = S::st(fs / Lf);
    out[d] = m;
    out[D + d] = m;
  }
}

// The logits level l was drawn from: the verification pass's rows (2l, 2l+1)
// when l <= *decided, else the depth step's slice (nullptr: left alone, the
// level's step records its own).
__global__ void k_spec_record(const float* __restrict__ all, const float* __restrict__ slice,
                              const int* __restrict__ decided, int l, int C, float* __restrict__ dst) {
  const float* src = l <= *decided ? all + (size_t)2 * l * C : slice;
  if (src == nullptr) return;
  for (int i = threadIdx.x; i < 2 * C; i += blockDim.x) dst[i] = src[i];
}

}  // namespace

void spec_inputs(DType dt, const void* t_out, const void* emb, const int* draft, int L, int D, void* out,
                 hipStream_t s) {
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_spec_inputs<T>, dim3(2 * L), dim3(256), 0, s, (const T*)t_out,
                                            (const T*)emb, draft, D, (T*)out));
  MRT_HIP_CHECK(hipGetLastError());
}

void spec_accept(DType dt, const int* drawn, const int* draft, int L, int* tokens, int* decided, const void* emb,
                 int D, void* next_in, hipStream_t s) {
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_spec_accept<T>, dim3(1), dim3(256), 0, s, drawn, draft, L, tokens,
                                            decided, (const T*)emb, D, (T*)next_in));
  MRT_HIP_CHECK(hipGetLastError());
}

void frame_mean_tokens(DType dt, const int* tokens, int L, const void* emb, int D, void* out, hipStream_t s) {
  const dim3 grid((D + 255) / 256);
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_frame_mean_tokens<T>, grid, dim3(256), 0, s, tokens, L, (const T*)emb, D,
                                            (T*)out));
  MRT_HIP_CHECK(hipGetLastError());
}

void spec_record(const float* all, const float* slice, const int* decided, int l, int C, float* dst, hipStream_t s) {
  hipLaunchKernelGGL(k_spec_record, dim3(1), dim3(256), 0, s, all, slice, decided, l, C, dst);
  MRT_HIP_CHECK(hipGetLastError());
}

}  // namespace mrt
