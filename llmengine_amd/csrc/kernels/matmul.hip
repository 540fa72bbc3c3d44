// matmul.hip -- Q8_0 MatMul C[M,N] = A[M,K] . B[K,N] for gfx950.
//
// B is one Q8_0 stream in row-major [K, N] order, so element (k, n) is flat
// index k*N + n and blocks run along N (reference
// src/runtime/kernels/cpu_kernels.cpp:116-130, cuda_kernels.cu:296-331).
//
// One thread owns 4 consecutive output columns of one token row and walks k
// in ascending order with acc = fma(a[k], d*q, acc) starting from +0.0f: the
// reference CPU kernel's exact rounding sequence, so results are bit-identical
// to it.  Per k the 8 threads of a block read its scale and 32 quants (34
// contiguous bytes) through L1 with 2-byte loads; consecutive lanes cover
// consecutive blocks of the same B row, so a wavefront reads 8 blocks
// (272 contiguous bytes) per k.
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

__global__ __launch_bounds__(256) void matmul_q8_0_kernel(
    const float* __restrict__ a, const uint8_t* __restrict__ b, float* __restrict__ c,
    int M, int N, int K) {
  const int quads = N / 4;
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (int64_t)M * quads) return;
  const int m = (int)(g / quads);
  const int n = (int)(g - (int64_t)m * quads) * 4;
  const int NB = N / kBlockElems;
  const int nb = n / kBlockElems;
  const int o = (n % kBlockElems) / 2;  // u16 index of the quant pair, past the scale
  const float* arow = a + (int64_t)m * K;
  float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
#pragma unroll 4
  for (int k = 0; k < K; ++k) {
    const uint16_t* hp =
        reinterpret_cast<const uint16_t*>(b + ((int64_t)k * NB + nb) * kBlockBytes);
    const float d = scale_to_f32(hp[0]);
    const uint32_t q = (uint32_t)hp[1 + o] | ((uint32_t)hp[2 + o] << 16);
    const float av = arow[k];
    acc0 = __builtin_fmaf(av, d * q_at(q, 0), acc0);
    acc1 = __builtin_fmaf(av, d * q_at(q, 1), acc1);
    acc2 = __builtin_fmaf(av, d * q_at(q, 2), acc2);
    acc3 = __builtin_fmaf(av, d * q_at(q, 3), acc3);
  }
  *reinterpret_cast<f32x4*>(c + (int64_t)m * N + n) = f32x4{acc0, acc1, acc2, acc3};
}

}  // namespace

hipError_t launch_matmul(const float* a, const uint8_t* b, float* c, int M, int N,
                         int K, hipStream_t stream) {
  const int64_t total = (int64_t)M * (N / 4);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(matmul_q8_0_kernel, dim3((unsigned)((total + 255) / 256)),
                     dim3(256), 0, stream, a, b, c, M, N, K);
  return hipGetLastError();
}

}  // namespace mle
