// On-device CFG + level-masked top-k temperature sampling and token feedback
// for one RVQ level (decode.cpp:71-148, 458-484).
//
// One 256-thread workgroup per stream (or per level, for the speculative
// verification pass) runs the block draw of draw_block.hpp, the frame
// kernel's: Gumbel-max over the kept entries with Philox-4x32-10 noise; when
// the winner over every candidate is itself in the top-k set it is the
// answer; else up to 3 winners over {v > v_previous winner} are tried the
// same way; otherwise the top-k threshold (the k-th largest value, counting
// ties, i.e. min(topk(x, k)) of decode.cpp:119-120) comes from a byte-wise
// radix select over order-preserving float keys.
#include <cmath>
#include <mutex>

#include "device_utils.hpp"
#include "kernels.hpp"
#include "draw_block.hpp"

namespace mrt {
namespace {

constexpr int kFeedPer = 8;      // d_model elements per thread in the feedback (d_model <= 2048)
constexpr int kQkvPer = 8;       // q (k, v) table elements per thread (heads x 64 <= 2048)

// Stages a draw: the level slice's two logit rows (l0, l0 + C; C <= 1024)
// into LDS `lg`, the noise of this thread's candidates into pf (the
// tabulated row nz, or computed from the seed), the radix buffers 0 / 1 of
// `hist` cleared.  Every load is issued before the first LDS store.  The
// caller sets pf.teacher_id and orders the draw after a barrier.
__device__ __forceinline__ void stage_draw(const float* __restrict__ l0, int C, const float* __restrict__ nz,
                                           uint64_t seed, int frame, int level, float temperature, float* lg,
                                           DrawPrefetch& pf, unsigned* hist) {
  constexpr int kRowsPer = 2 * 1024 / kDrawThreads;  // logit-row elements per thread
  const int tid = threadIdx.x;
  float lv[kRowsPer];
#pragma unroll
  for (int i = 0; i < kRowsPer; ++i) lv[i] = l0[min(tid + kDrawThreads * i, 2 * C - 1)];
#pragma unroll
  for (int t = 0; t < kDrawPer; ++t) {
    const int c = tid + kDrawThreads * t;
    pf.gn[t] = (c < C && temperature != 0.0f) ? (nz != nullptr ? nz[c] : gumbel(seed, frame, level, c)) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < kRowsPer; ++i)
    if (tid + kDrawThreads * i < 2 * C) lg[tid + kDrawThreads * i] = lv[i];
  draw_clear(hist);
}

// Every level of one frame drawn at once (block l draws level l from logit
// rows 2l, 2l + 1 with the block draw; the speculative verification pass):
// drawn[l] = the LLM id.
__global__ __launch_bounds__(kDrawThreads) void k_draw_levels(const float* __restrict__ logits, SampleParams p,
                                                              int frame, int* __restrict__ drawn) {
  __shared__ float lg[2 * 1024];
  __shared__ __align__(16) unsigned hist[kDrawHistWords];
  __shared__ int wres[16];
  const int l = blockIdx.x, C = p.codebook, tid = threadIdx.x;
  const float* nz = p.noise != nullptr ? p.noise + ((size_t)frame * p.rvq_depth + l) * C : nullptr;
  DrawPrefetch pf;
  stage_draw(logits + (size_t)(2 * l) * C, C, nz, p.seed != nullptr ? p.seed[0] : p.seed_value, frame, l,
             p.temperature, lg, pf, hist);
  pf.teacher_id = 0;
  __syncthreads();
  const int bi = block_draw(p, pf, lg, hist, wres, [](int) {});
  if (tid == 0) drawn[l] = p.codec_offset + l * C + bi;
}

// Block b draws for stream b: logits rows (2b, 2b + 1), seed p.seed[b], token
// slots slot + b * tstride; a non-null frame_ptr supplies the frame index.
// The whole block draws (block_draw, the frame kernel's draw) from the two
// logit rows staged in LDS, then writes the token's embedding to both rows of
// next_in and updates the frame sum (whose rows it loads before the draw).
template <typename T>
__global__ __launch_bounds__(kDrawThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_sample(
    const float* __restrict__ logits, SampleParams p, int frame, const int* __restrict__ frame_ptr, int level,
    int slot, int tstride, const int* __restrict__ teacher, int* __restrict__ tokens, int* __restrict__ drawn,
    const T* __restrict__ emb, int D, T* __restrict__ next_in, T* __restrict__ fsum, T* __restrict__ fmean,
    QkvFeed feed) {
  using S = St<T>;
  __shared__ float lg[2 * 1024];
  __shared__ __align__(16) unsigned hist[kDrawHistWords];
  __shared__ int wres[16];
  const int tid = threadIdx.x;
  const int stream = blockIdx.x;
  const int C = p.codebook, L = p.rvq_depth;
  if (frame_ptr != nullptr) {
    frame = *frame_ptr;
    slot += frame * L;
  }
  slot += stream * tstride;
  T* ni = next_in + (size_t)(2 * stream) * D;
  if (p.decided != nullptr && *p.decided >= level) {
    // the level's token is already known: only feed it to the next depth step
    // (the frame sum is not kept on this path)
    const T* e = emb + (size_t)tokens[slot] * D;
    for (int d = tid; d < D; d += kDrawThreads) {
      ni[d] = e[d];
      ni[D + d] = e[d];
    }
    return;
  }
  T* fs = fsum + (size_t)(2 * stream) * D;
  T* fm = fmean + (size_t)(2 * stream) * D;
  // Every load that does not depend on the token, issued before the first
  // store: the frame sum rows, the level slice's two logit rows, the draw's
  // noise (tabulated, or computed from the seed) and the teacher id.
  T fv[kFeedPer];
#pragma unroll
  for (int i = 0; i < kFeedPer; ++i) fv[i] = fs[min(tid + kDrawThreads * i, D - 1)];  // unused at level 0
  const float* nz = p.noise != nullptr
                        ? p.noise + (((size_t)stream * p.noise_frames + frame) * p.rvq_depth + level) * C
                        : nullptr;
  DrawPrefetch pf;
  pf.teacher_id = teacher ? teacher[slot] : 0;
  stage_draw(logits + (size_t)(2 * stream) * C, C, nz, p.seed != nullptr ? p.seed[stream] : p.seed_value, frame,
             level, p.temperature, lg, pf, hist);
  __syncthreads();
  const int bi = block_draw(p, pf, lg, hist, wres, [](int) {});
  const int drawn_id = p.codec_offset + level * C + bi;
  const int fed = teacher ? pf.teacher_id : drawn_id;
  if (tid == 0) {
    tokens[slot] = fed;
    if (drawn) drawn[slot] = drawn_id;
  }
  // Token feedback (decode.cpp:476-484): both CFG rows take emb(fed); the
  // frame sum accumulates in the model dtype; at the last level the mean is
  // the sum divided by L in the model dtype.  With a q/k/v feed, the fed
  // token's table row (the next level's depth layer-0 q | k | v) is written
  // for both rows too.  Every load of the token's rows is issued before the
  // first store: the stores could alias them as far as the compiler knows, so
  // interleaved they would serialise the round trips.
  const T* e = emb + (size_t)fed * D;
  const float Lf = S::rnd((float)L);
  T ev[kFeedPer];
#pragma unroll
  for (int i = 0; i < kFeedPer; ++i) ev[i] = e[min(tid + 256 * i, D - 1)];
  const int row = fed - feed.offset;
  const bool fed_qkv = feed.table != nullptr && level + 1 < L && row >= 0 && row < feed.rows;
  const int HD = feed.HD;
  T qv[3][kQkvPer];  // q, k, v: elements tid + 256 i of each
  if (fed_qkv) {
    const T* src = static_cast<const T*>(feed.table) + (size_t)row * 3 * HD;
#pragma unroll
    for (int w = 0; w < 3; ++w)
#pragma unroll
      for (int i = 0; i < kQkvPer; ++i)
        if (tid + 256 * i < HD) qv[w][i] = src[w * HD + tid + 256 * i];
  }
#pragma unroll
  for (int i = 0; i < kFeedPer; ++i) {
    const int d = tid + 256 * i;
    if (d >= D) continue;
    const float sum = (level == 0) ? S::ld(ev[i]) : S::rnd(S::ld(fv[i]) + S::ld(ev[i]));
    ni[d] = ev[i];
    ni[D + d] = ev[i];
    fs[d] = S::st(sum);
    fs[D + d] = S::st(sum);
    if (level == L - 1) {
      const T m = S::st(sum / Lf);
      fm[d] = m;
      fm[D + d] = m;
    }
  }
  if (fed_qkv) {
    T* q = static_cast<T*>(feed.q);
    T* kc = static_cast<T*>(feed.kc);
    T* vc = static_cast<T*>(feed.vc);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const size_t m = 2 * stream + b;
#pragma unroll
      for (int i = 0; i < kQkvPer; ++i) {
        const int nn = tid + 256 * i;
        if (nn >= HD) continue;
        const size_t slot = ((m * feed.H + (nn >> 6)) * feed.Lmax + level + 1) * 64 + (nn & 63);
        q[m * HD + nn] = qv[0][i];
        kc[slot] = qv[1][i];
        vc[slot] = qv[2][i];
      }
    }
  }
}

}  // namespace

void sample_level(DType dt, const float* logits, const SampleParams& p, int frame, int level, int slot,
                  const int* teacher, int* tokens, int* drawn, const void* emb, int D,
                  void* next_in, void* fsum, void* frame_mean, hipStream_t s) {
  sample_levels(dt, 1, logits, p, frame, nullptr, level, slot, 0, teacher, tokens, drawn, emb, D, next_in, fsum,
                frame_mean, s);
}

void draw_levels(const float* logits, const SampleParams& p, int frame, int levels, int* drawn, hipStream_t s) {
  MRT_REQUIRE(p.codebook >= 1 && p.codebook <= kDrawThreads * kDrawPer, "draw: codebook must be <= 1024");
  hipLaunchKernelGGL(k_draw_levels, dim3(levels), dim3(kDrawThreads), 0, s, logits, p, frame, drawn);
  MRT_HIP_CHECK(hipGetLastError());
}

void sample_levels(DType dt, int streams, const float* logits, const SampleParams& p, int frame,
                   const int* frame_ptr, int level, int slot, int tstride, const int* teacher, int* tokens,
                   int* drawn, const void* emb, int D, void* next_in, void* fsum, void* frame_mean, hipStream_t s,
                   const QkvFeed* feed) {
  MRT_REQUIRE(p.codebook >= 1 && p.codebook <= kDrawThreads * kDrawPer, "sample: codebook must be <= 1024");
  MRT_REQUIRE(streams >= 1, "sample: no streams");
  MRT_REQUIRE(D >= 1 && D <= 256 * kFeedPer, "sample: d_model must be in [1, 2048]");
  const QkvFeed fd = feed != nullptr ? *feed : QkvFeed{};
  if (fd.table != nullptr)
    MRT_REQUIRE(fd.q && fd.kc && fd.vc && fd.HD == fd.H * 64 && fd.HD <= 256 * kQkvPer &&
                    fd.Lmax >= p.rvq_depth && fd.rows >= 0,
                "sample: bad q/k/v feed");
  MRT_DTYPE_DISPATCH(dt, hipLaunchKernelGGL(k_sample<T>, dim3(streams), dim3(kDrawThreads), 0, s, logits, p, frame, frame_ptr,
                                            level, slot, tstride, teacher, tokens, drawn, (const T*)emb, D,
                                            (T*)next_in, (T*)fsum, (T*)frame_mean, fd));
  MRT_HIP_CHECK(hipGetLastError());
}

// ---- the draw without library allocations ---------------------------------------------
namespace {

// Scratch of sample_level_noalloc on each device: the three feedback row
// pairs k_sample writes (next depth input, frame sum, frame mean: 2 x d_model
// elements each, model dtype) from offset 256 (the first 256 bytes are
// unused).  The caller discards them; the seed travels by value in the
// kernel arguments, so calls that overlap on one device still draw their own
// tokens.  Every call on a device shares its copy, which keeps the last
// call's contents.
constexpr size_t kNoAllocBytes = 32 * 1024;
constexpr size_t kNoAllocRows = 256;
__device__ __align__(256) unsigned char scratch[kNoAllocBytes];

constexpr int kMaxNoAllocDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kMaxNoAllocDevices];  // device address of `scratch`, per device

}  // namespace

size_t noalloc_scratch_bytes() { return kNoAllocBytes; }

// The device address of `scratch` on `device` (the current device), looked up
// once per device.  The host-side name of a __device__ array is not its device
// address, so kernels only ever receive this pointer.
static unsigned char* scratch_on(int device) {
  MRT_REQUIRE(device >= 0 && device < kMaxNoAllocDevices, "sample_noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    MRT_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    g_scratch_ptr[device] = static_cast<unsigned char*>(ptr);
  }
  return g_scratch_ptr[device];
}

void sample_level_noalloc(DType dt, int device, const void* emb, int D, const float* logits, const SampleParams& p,
                          uint64_t seed, int frame, int level, int* token, hipStream_t s) {
  const size_t esz = dtype_size(dt);
  const size_t need = kNoAllocRows + 3 * 2 * static_cast<size_t>(D) * esz;
  if (need > kNoAllocBytes)
    throw Error(1, "sample_noalloc: d_model " + std::to_string(D) + " needs " + std::to_string(need) +
                       " bytes of scratch, more than the fixed " + std::to_string(kNoAllocBytes));
  unsigned char* base = scratch_on(device);
  unsigned char* rows = base + kNoAllocRows;
  const size_t row_pair = 2 * static_cast<size_t>(D) * esz;
  SampleParams sp = p;
  sp.seed = nullptr;
  sp.seed_value = seed;
  sp.noise = nullptr;
  sp.decided = nullptr;
  sample_level(dt, logits, sp, frame, level, 0, nullptr, token, nullptr, emb, D, rows, rows + row_pair,
               rows + 2 * row_pair, s);
}

}  // namespace mrt
