// Read-bandwidth probe of the device's memory hierarchy, for the roofline
// figures of the benchmark: a buffer of `bytes` is read `passes` times by a
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

}  // namespace mrt
