// argmax.hip -- greedy-decode argmax of lm_head logits on the device.
//
// idx[r] = the first index of the largest value of logits[r, 0:n] (ties go to
// the lower index, as the reference's greedy pick does: it scans candidates in
// index order and replaces the best only on a strictly larger value,
// src/runtime/sampler.cpp:108-118; -0 and +0 compare equal).  NaN entries are
// ignored; a row of NaN only gives index 0 and value NaN.  Replaces the
// per-token device-to-host copy of the whole logits row that the reference's
// CUDA generator makes before sampling on the host
// (examples/generate_cuda.cpp:81-94, 305-314).
//
// Two launches: pass 1 (grid chunks x rows) reduces a contiguous chunk of a row
// per workgroup to one 64-bit key; pass 2 reduces a row's chunk keys and
// decodes the winner.  key = (order(v) << 32) | ~index, where order() maps float
// bits to unsigned integers in value order, so the largest key is the largest
// value with the smallest index.  Deterministic; no atomics.
#include "../launch.hpp"

namespace mle {
namespace {

constexpr int kArgThreads = 256;

__device__ __forceinline__ uint64_t arg_key(float v, uint32_t i) {
  if (v != v) return 0;  // NaN: never selected
  if (v == 0.0f) v = 0.0f;  // -0 -> +0
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)~i;
}

__device__ __forceinline__ uint64_t wave_max(uint64_t k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)k, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(k >> 32), off, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    k = o > k ? o : k;
  }
  return k;
}

__device__ __forceinline__ uint64_t block_max(uint64_t k) {
  __shared__ uint64_t part[kArgThreads / 64];
  k = wave_max(k);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) part[wave] = k;
  __syncthreads();
  uint64_t r = part[0];
#pragma unroll
  for (int i = 1; i < kArgThreads / 64; ++i) r = part[i] > r ? part[i] : r;
  return r;
}

// Pass 1: workgroup (c, r) reduces logits[r, c*chunk : (c+1)*chunk).
__global__ __launch_bounds__(kArgThreads) void argmax_chunks_kernel(const float* __restrict__ x,
                                                                   int64_t n, int64_t chunk,
                                                                   uint64_t* __restrict__ keys) {
  const int64_t r = blockIdx.y;
  const int64_t b = (int64_t)blockIdx.x * chunk;
  const int64_t e = b + chunk < n ? b + chunk : n;
  const float* row = x + r * n;
  uint64_t k = 0;
  for (int64_t i = b + threadIdx.x; i < e; i += kArgThreads) {
    const uint64_t c = arg_key(row[i], (uint32_t)i);
    k = c > k ? c : k;
  }
  k = block_max(k);
  if (threadIdx.x == 0) keys[r * gridDim.x + blockIdx.x] = k;
}

// Pass 2: one workgroup per row over its `chunks` keys.
__global__ __launch_bounds__(kArgThreads) void argmax_final_kernel(
    const uint64_t* __restrict__ keys, int chunks, int32_t* __restrict__ idx,
    float* __restrict__ val) {
  const int64_t r = blockIdx.x;
  uint64_t k = 0;
  for (int i = threadIdx.x; i < chunks; i += kArgThreads) {
    const uint64_t c = keys[r * chunks + i];
    k = c > k ? c : k;
  }
  k = block_max(k);
  if (threadIdx.x != 0) return;
  if (k == 0) {  // NaN only
    idx[r] = 0;
    if (val) val[r] = __builtin_nanf("");
    return;
  }
  idx[r] = (int32_t)~(uint32_t)k;
  if (val) {
    uint32_t u = (uint32_t)(k >> 32);
    u = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
    val[r] = __builtin_bit_cast(float, u);
  }
}

}  // namespace

int argmax_chunks(int64_t n) {
  // Chunks of at least 2048 values, at most 256 per row.
  const int64_t c = (n + 2047) / 2048;
  return (int)(c < 1 ? 1 : c > 256 ? 256 : c);
}

hipError_t launch_argmax(const float* x, int rows, int64_t n, int32_t* idx, float* val,
                         uint64_t* keys, hipStream_t stream) {
  if (rows <= 0 || n <= 0 || n > 0x7fffffff || rows > 65535) return hipErrorInvalidValue;
  const int chunks = argmax_chunks(n);
  const int64_t chunk = (n + chunks - 1) / chunks;
  hipLaunchKernelGGL(argmax_chunks_kernel, dim3((unsigned)chunks, (unsigned)rows),
                     dim3(kArgThreads), 0, stream, x, n, chunk, keys);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)rows), dim3(kArgThreads), 0, stream,
                     keys, chunks, idx, val);
  return hipGetLastError();
}

}  // namespace mle
