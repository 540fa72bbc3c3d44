// elementwise.hip -- the unfused SwiGLU op of the HIP backend, and a uint32
// fill used to clear workspace counters.
//
// y[i] = silu(gate[i]) * up[i] = (g / (1 + exp(-g))) * u, the reference's
// operation order (src/runtime/kernels/cpu_kernels.cpp:848-858; device twin
// cuda_kernels.cu:245-248).  Used for graphs whose gate / up values are not two
// Q8_0 Linears of one input (those run as one fused Linear launch instead).
// Memory-bound: 12 bytes per element; 4 elements per thread as 16-byte accesses
// when the buffers allow.
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

__global__ __launch_bounds__(256) void swiglu_f32_kernel(const float* __restrict__ g,
                                                         const float* __restrict__ u,
                                                         float* __restrict__ y, int64_t n,
                                                         int vec) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  if (vec && i + 4 <= n) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(g + i);
    const f32x4 b = *reinterpret_cast<const f32x4*>(u + i);
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (a[e] / (1.0f + expf(-a[e]))) * b[e];
    *reinterpret_cast<f32x4*>(y + i) = r;
    return;
  }
  for (int64_t j = i; j < n && j < i + 4; ++j) y[j] = (g[j] / (1.0f + expf(-g[j]))) * u[j];
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n,
                                                      uint32_t v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

hipError_t launch_fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p, (int64_t)n,
                     v);
  return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, float* y, int64_t n,
                         hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int vec = (((uintptr_t)g | (uintptr_t)u | (uintptr_t)y) & 15) == 0;
  const int64_t blocks = (n + 1023) / 1024;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(swiglu_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, g, u, y,
                     n, vec);
  return hipGetLastError();
}

}  // namespace mle
