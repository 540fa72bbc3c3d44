// probe.hip -- streaming-read probe: the rate at which this GPU reads a buffer of
// a given size from HBM with nothing else to do.  A measurement aid with no
// counterpart in the reference: the benchmark times it over the same weight
// buffers as each decode Linear, so a Linear's time can be set against a pure
// read of the same bytes (launch cost, ramp-up and drain included) and not
// only against the HBM peak.
//
// 4096 workgroups of 256 threads (the best of 1024 / 2048 / 4096 for 18-290 MB
// on MI355X) walk the buffer in a grid stride of 16-byte non-temporal loads,
// four in flight per thread, and fold them into one word that is stored only if
// it equals a constant (so the loads are kept and nothing is written in
// practice).
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

constexpr int kProbeGrid = 4096;
constexpr int kProbeThreads = 256;
constexpr uint32_t kProbeMagic = 0x9e3779b9u;

__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u32x4* __restrict__ src,
                                                                    uint64_t n16,
                                                                    uint32_t* __restrict__ sink) {
  const uint64_t stride = (uint64_t)gridDim.x * kProbeThreads;
  uint64_t i = (uint64_t)blockIdx.x * kProbeThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(src + i);
    const u32x4 b = __builtin_nontemporal_load(src + i + stride);
    const u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(src + i + 3 * stride);
    acc ^= a.x ^ b.y ^ c.z ^ d.w;
  }
  for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(src + i).x;
  if (acc == kProbeMagic) sink[0] = acc;
}

}  // namespace

hipError_t launch_stream_read(const void* src, int64_t bytes, uint32_t* sink,
                              hipStream_t stream) {
  if (src == nullptr || sink == nullptr || bytes < 0 || bytes % 16 != 0)
    return hipErrorInvalidValue;
  if (bytes == 0) return hipSuccess;
  hipLaunchKernelGGL(stream_read_kernel, dim3(kProbeGrid), dim3(kProbeThreads), 0, stream,
                     static_cast<const u32x4*>(src), (uint64_t)bytes / 16, sink);
  return hipGetLastError();
}

}  // namespace mle
