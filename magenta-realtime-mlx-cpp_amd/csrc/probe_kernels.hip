// Probes of the device for the roofline figures of the benchmark.
//
// Read bandwidth of the memory hierarchy: a buffer of `bytes` is read `passes` times by a
// grid of 8 workgroups per CU.  Each workgroup reads contiguous 32 KiB tiles
// (8 16-byte loads per thread, all issued before any is consumed), so every
// buffer size keeps the same number of loads in flight.  A buffer that the
// 256 MB last-level cache (MALL) of MI355X retains is served from it after
// the first pass; a buffer of several GB streams from HBM on every pass.  The
// loaded words are folded into one value that is stored only if it equals a
// constant, so no load is dropped.
#include "common.hpp"
#include "device_utils.hpp"
#include "kernels.hpp"
#include "persist.hpp"

namespace mrt {
namespace {

constexpr int kSweepUnroll = 8;

__global__ __launch_bounds__(256) void k_read_sweep(const uint4* __restrict__ p, size_t n16, int passes,
                                                    unsigned* __restrict__ sink) {
  const size_t tile = (size_t)blockDim.x * kSweepUnroll;
  const size_t step = (size_t)gridDim.x * tile;
  uint32_t acc = 0;
  for (int r = 0; r < passes; ++r) {
    for (size_t base = (size_t)blockIdx.x * tile + threadIdx.x; base < n16; base += step) {
      uint4 v[kSweepUnroll];
      // clamped indices keep every load in bounds and unconditional; the
      // values of clamped lanes are discarded below
#pragma unroll
      for (int u = 0; u < kSweepUnroll; ++u) v[u] = p[min(base + (size_t)u * blockDim.x, n16 - 1)];
#pragma unroll
      for (int u = 0; u < kSweepUnroll; ++u) {
        // every word of every load is used, so no load is narrowed
        const uint32_t f = (v[u].x ^ v[u].y) + (v[u].z ^ v[u].w);
        acc ^= base + (size_t)u * blockDim.x < n16 ? f : 0u;
      }
    }
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

// Hand-off latency of the persistent kernels' phases.  k_handoff runs rounds of
// an all-gather of tagged 64-bit words among the grid's workgroups: in round r
// each workgroup stores its words / G words {r, index} with agent-scope
// atomic stores, then polls all `words` words with agent-scope atomic loads
// until each carries round r or later -- one phase hand-off of the step
// kernels.  `delay` rounds of s_sleep(1) precede each round's first poll.  k_pingpong bounces one word between workgroup 0 and workgroup
// `peer` (one thread each).  Every poll gives up after kSpinLimit rounds and
// flags an error, so both kernels always end.
__device__ __forceinline__ uint64_t probe_aload(const uint64_t* p) {
  return __hip_atomic_load((const MRT_GLOBAL uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void probe_astore(uint64_t* p, uint64_t v) {
  __hip_atomic_store((MRT_GLOBAL uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(256) void k_handoff(uint64_t* __restrict__ w, int words, int rounds, int delay,
                                                 uint64_t* __restrict__ clk, int* __restrict__ err) {
  const int G = gridDim.x, b = blockIdx.x, t = threadIdx.x;
  const int per = words / G;
  const uint64_t t0 = wall_clock64();
  for (int r = 1; r <= rounds; ++r) {
    if (t < per) probe_astore(w + b * per + t, ((uint64_t)r << 32) | (uint32_t)(b * per + t));
    uint32_t pend = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (t + 256 * i < words) pend |= 1u << i;
    uint32_t spins = 0;
    for (int i = 0; i < delay; ++i) __builtin_amdgcn_s_sleep(1);  // 64 clocks each, before the first poll
    while (pend != 0) {
      uint64_t v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if ((pend >> i) & 1u) v[i] = probe_aload(w + t + 256 * i);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (((pend >> i) & 1u) && (v[i] >> 32) >= (uint64_t)r) pend &= ~(1u << i);
      if (pend != 0 && ++spins > kSpinLimit) {
        __hip_atomic_store((MRT_GLOBAL int*)err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    __syncthreads();
    if (__hip_atomic_load((const MRT_GLOBAL int*)err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
  }
  if (b == 0 && t == 0) clk[0] = wall_clock64() - t0;
}

__global__ void k_pingpong(uint64_t* __restrict__ w, int rounds, int peer, uint64_t* __restrict__ clk,
                           int* __restrict__ err) {
  if (threadIdx.x != 0 || (blockIdx.x != 0 && (int)blockIdx.x != peer)) return;
  const bool first = blockIdx.x == 0;
  uint64_t* mine = w + (first ? 0 : 16);  // separate 128-byte lines
  const uint64_t* theirs = w + (first ? 16 : 0);
  const uint64_t t0 = wall_clock64();
  for (int i = 1; i <= rounds; ++i) {
    if (first) probe_astore(mine, (uint64_t)i);
    uint32_t spins = 0;
    while (probe_aload(theirs) < (uint64_t)i) {
      if (++spins > kSpinLimit) {
        __hip_atomic_store((MRT_GLOBAL int*)err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
    }
    if (!first) probe_astore(mine, (uint64_t)i);
  }
  if (first) clk[0] = wall_clock64() - t0;
}

}  // namespace

float probe_read_bandwidth(int device, size_t bytes, int passes) {
  MRT_REQUIRE(bytes >= (1u << 20) && bytes % 16 == 0, "probe: bytes must be a multiple of 16, at least 1 MiB");
  MRT_REQUIRE(passes >= 1 && passes <= 1000, "probe: passes must be in [1, 1000]");
  MRT_HIP_CHECK(hipSetDevice(device));
  int num_cu = 0;
  MRT_HIP_CHECK(hipDeviceGetAttribute(&num_cu, hipDeviceAttributeMultiprocessorCount, device));
  void* buf = nullptr;
  unsigned* sink = nullptr;
  hipStream_t s = nullptr;
  hipEvent_t ev[2] = {nullptr, nullptr};
  float ms = 0.f;
  auto release = [&]() {
    if (ev[0]) (void)hipEventDestroy(ev[0]);
    if (ev[1]) (void)hipEventDestroy(ev[1]);
    if (s) (void)hipStreamDestroy(s);
    if (buf) (void)hipFree(buf);
    if (sink) (void)hipFree(sink);
  };
  try {
    MRT_HIP_CHECK(hipMalloc(&buf, bytes));
    MRT_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&sink), 64));
    MRT_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    MRT_HIP_CHECK(hipEventCreate(&ev[0]));
    MRT_HIP_CHECK(hipEventCreate(&ev[1]));
    MRT_HIP_CHECK(hipMemsetAsync(buf, 0x5a, bytes, s));
    const size_t n16 = bytes / 16;
    const dim3 grid(8 * num_cu);
    // warm pass: brings a cache-sized buffer into the MALL
    hipLaunchKernelGGL(k_read_sweep, grid, dim3(256), 0, s, static_cast<const uint4*>(buf), n16, 1, sink);
    MRT_HIP_CHECK(hipGetLastError());
    MRT_HIP_CHECK(hipEventRecord(ev[0], s));
    hipLaunchKernelGGL(k_read_sweep, grid, dim3(256), 0, s, static_cast<const uint4*>(buf), n16, passes, sink);
    MRT_HIP_CHECK(hipGetLastError());
    MRT_HIP_CHECK(hipEventRecord(ev[1], s));
    MRT_HIP_CHECK(hipEventSynchronize(ev[1]));
    MRT_HIP_CHECK(hipEventElapsedTime(&ms, ev[0], ev[1]));
  } catch (...) {
    release();
    throw;
  }
  release();
  return static_cast<float>(static_cast<double>(bytes) * passes / (ms * 1e-3) / 1e9);
}

namespace {

// Runs one probe launch on a fresh zeroed 16 KiB word buffer and returns the
// time its workgroup 0 measured on the device's wall clock, in microseconds.
template <class Launch>
double probe_ticks_us(int device, Launch launch) {
  MRT_HIP_CHECK(hipSetDevice(device));
  int khz = 0;
  MRT_HIP_CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device));
  MRT_REQUIRE(khz > 0, "probe: the device reports no wall-clock rate");
  uint64_t* w = nullptr;
  uint64_t* clk = nullptr;
  int* err = nullptr;
  hipStream_t s = nullptr;
  auto release = [&]() {
    if (s) (void)hipStreamDestroy(s);
    if (w) (void)hipFree(w);
    if (clk) (void)hipFree(clk);
    if (err) (void)hipFree(err);
  };
  uint64_t ticks = 0;
  int e = 0;
  try {
    MRT_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&w), 16384));
    MRT_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&clk), 64));
    MRT_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&err), 64));
    MRT_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    MRT_HIP_CHECK(hipMemsetAsync(w, 0, 16384, s));
    MRT_HIP_CHECK(hipMemsetAsync(clk, 0, 64, s));
    MRT_HIP_CHECK(hipMemsetAsync(err, 0, 64, s));
    launch(w, clk, err, s);
    MRT_HIP_CHECK(hipGetLastError());
    MRT_HIP_CHECK(hipMemcpyAsync(&ticks, clk, sizeof ticks, hipMemcpyDeviceToHost, s));
    MRT_HIP_CHECK(hipMemcpyAsync(&e, err, sizeof e, hipMemcpyDeviceToHost, s));
    MRT_HIP_CHECK(hipStreamSynchronize(s));
  } catch (...) {
    release();
    throw;
  }
  release();
  if (e != 0) throw Error(3, "probe: a poll reached its spin limit (the workgroups were not all resident)");
  return static_cast<double>(ticks) * 1000.0 / khz;  // microseconds
}

}  // namespace

float probe_handoff(int device, int workgroups, int words, int rounds, int delay) {
  MRT_HIP_CHECK(hipSetDevice(device));
  int num_cu = 0;
  MRT_HIP_CHECK(hipDeviceGetAttribute(&num_cu, hipDeviceAttributeMultiprocessorCount, device));
  MRT_REQUIRE(workgroups >= 1 && workgroups <= num_cu, "probe: workgroups must be in [1, CU count]");
  MRT_REQUIRE(words >= workgroups && words <= 1024 && words % workgroups == 0,
              "probe: words must be a multiple of workgroups, at most 1024");
  MRT_REQUIRE(words / workgroups <= 256, "probe: at most 256 words per workgroup (one per thread)");
  MRT_REQUIRE(rounds >= 1 && rounds <= 100000, "probe: rounds must be in [1, 100000]");
  MRT_REQUIRE(delay >= 0 && delay <= 256, "probe: delay must be in [0, 256]");
  const double us = probe_ticks_us(device, [&](uint64_t* w, uint64_t* clk, int* err, hipStream_t s) {
    // its workgroups poll each other, like a persistent grid's: never beside one
    PersistSection gate(device, s);
    hipLaunchKernelGGL(k_handoff, dim3(workgroups), dim3(256), 0, s, w, words, rounds, delay, clk, err);
  });
  return static_cast<float>(us / rounds);
}

float probe_pingpong(int device, int peer, int rounds) {
  MRT_HIP_CHECK(hipSetDevice(device));
  int num_cu = 0;
  MRT_HIP_CHECK(hipDeviceGetAttribute(&num_cu, hipDeviceAttributeMultiprocessorCount, device));
  MRT_REQUIRE(peer >= 1 && peer < num_cu, "probe: peer must be in [1, CU count)");
  MRT_REQUIRE(rounds >= 1 && rounds <= 100000, "probe: rounds must be in [1, 100000]");
  const double us = probe_ticks_us(device, [&](uint64_t* w, uint64_t* clk, int* err, hipStream_t s) {
    PersistSection gate(device, s);
    hipLaunchKernelGGL(k_pingpong, dim3(peer + 1), dim3(64), 0, s, w, rounds, peer, clk, err);
  });
  return static_cast<float>(us / (2.0 * rounds));
}

}  // namespace mrt
