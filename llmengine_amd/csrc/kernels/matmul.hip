// matmul.hip -- Q8_0 MatMul C[M,N] = A[M,K] . B[K,N] for gfx950.
//
// B is one Q8_0 stream in row-major [K, N] order, so element (k, n) is flat
// index k*N + n and blocks run along N (reference
// src/runtime/kernels/cpu_kernels.cpp:116-130, cuda_kernels.cu:296-331).
//
// One thread owns 4 consecutive output columns of MR token rows (MR = 4 when
// M >= 4, else 1) and walks k in ascending order with acc = fma(a[k], d*q, acc)
// starting from +0.0f for each of its outputs: the reference CPU kernel's exact
// rounding sequence, so results are bit-identical to it.  The MR rows share each
// decoded B value (v = d*q formed once per k and column), so B is read M/MR
// times instead of M times; the activations come four k at a time as one 16-byte
// load per row when K % 4 == 0.  Per k the 8 threads of a block read its scale
// and 32 quants (34 contiguous bytes) through L1 with 2-byte loads; consecutive
// lanes cover consecutive blocks of the same B row, so a wavefront reads 8
// blocks (272 contiguous bytes) per k.
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

template <int MR>
__global__ __launch_bounds__(256) void matmul_q8_0_kernel(
    const float* __restrict__ a, const uint8_t* __restrict__ b, float* __restrict__ c,
    int M, int N, int K) {
  const int quads = N / 4;
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row_tiles = ((int64_t)M + MR - 1) / MR;
  if (g >= row_tiles * quads) return;
  const int m0 = (int)(g / quads) * MR;
  const int n = (int)(g % quads) * 4;
  const int rows = min(MR, M - m0);
  const int NB = N / kBlockElems;
  const int nb = n / kBlockElems;
  const int o = (n % kBlockElems) / 2;  // u16 index of the quant pair, past the scale
  const float* arow[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) arow[r] = a + (int64_t)(m0 + min(r, rows - 1)) * K;
  float acc[MR][4];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[r][j] = 0.0f;
  auto step = [&](int k, const float (&av)[MR]) {
    const uint16_t* hp =
        reinterpret_cast<const uint16_t*>(b + ((int64_t)k * NB + nb) * kBlockBytes);
    const float d = scale_to_f32(hp[0]);
    const uint32_t q = (uint32_t)hp[1 + o] | ((uint32_t)hp[2 + o] << 16);
    const float v[4] = {d * q_at(q, 0), d * q_at(q, 1), d * q_at(q, 2), d * q_at(q, 3)};
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[r][j] = __builtin_fmaf(av[r], v[j], acc[r][j]);
  };
  int k = 0;
  if ((K & 3) == 0) {
    for (; k < K; k += 4) {
      f32x4 a4[MR];
#pragma unroll
      for (int r = 0; r < MR; ++r) a4[r] = *reinterpret_cast<const f32x4*>(arow[r] + k);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        float av[MR];
#pragma unroll
        for (int r = 0; r < MR; ++r) av[r] = a4[r][kk];
        step(k + kk, av);
      }
    }
  }
  for (; k < K; ++k) {
    float av[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) av[r] = arow[r][k];
    step(k, av);
  }
#pragma unroll
  for (int r = 0; r < MR; ++r)
    if (r < rows)
      *reinterpret_cast<f32x4*>(c + (int64_t)(m0 + r) * N + n) =
          f32x4{acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
}

}  // namespace

hipError_t launch_matmul(const float* a, const uint8_t* b, float* c, int M, int N,
                         int K, hipStream_t stream) {
  if ((int64_t)M * (N / 4) == 0) return hipSuccess;
  const int mr = M >= 4 ? 4 : 1;
  const int64_t total = ((int64_t)M + mr - 1) / mr * (N / 4);
  const dim3 grid((unsigned)((total + 255) / 256));
  if (mr == 4)
    hipLaunchKernelGGL(matmul_q8_0_kernel<4>, grid, dim3(256), 0, stream, a, b, c, M, N, K);
  else
    hipLaunchKernelGGL(matmul_q8_0_kernel<1>, grid, dim3(256), 0, stream, a, b, c, M, N, K);
  return hipGetLastError();
}

}  // namespace mle
