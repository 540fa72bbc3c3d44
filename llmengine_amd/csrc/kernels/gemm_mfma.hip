// gemm_mfma.hip -- Q8_0 Linear prefill GEMM on bf16 MFMA for gfx950.
//
// Y[M, N] = X[M, K] . W^T (+ bias), W in Q8_0 blocks along K.
// Same contract as cpu::sgemm_nt(const float*, const uint8_t*, ...)
// (src/runtime/kernels/cpu_kernels.cpp:208-218); used for M >= 64.
//
// Workgroup tile BM x BN = 128 x 128, K step BK = 64 (two Q8_0 blocks per
// output row), 256 threads = 4 wavefronts, each owning a 64 x 64 sub-tile as
// 2 x 2 v_mfma_f32_32x32x16_bf16 accumulators.
//
// Staging into LDS (bf16, rows padded by 16 bytes against bank conflicts):
//   * X tile: fp32 loads, one rounding to bf16;
//   * W tile: each thread loads one 34-byte block, forms v = d * q in fp32
//     (exactly the reference's element value) and rounds it once to bf16.
// The per-block scale is thus folded into the B operand before the MFMA
// instead of being applied to the accumulator after every 32-wide K block:
// the latter costs one VALU FMA per output per block, i.e. one VALU op per 64
// MFMA flops, which on CDNA4 equals the whole non-packed VALU rate and would cap
// the MFMA pipe at about half its peak.  Error vs the fp32 reference is then
// the bf16 rounding of both operands (relative L2 ~1.6e-3), inside the 1e-2
// bound stated for this path.
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (144 bytes)

__global__ __launch_bounds__(256) void gemm_q8_0_mfma_kernel(
    const float* __restrict__ x, const uint8_t* __restrict__ w,
    const float* __restrict__ bias, float* __restrict__ y, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDS_STRIDE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  const int KB = K / kBlockElems;
  const int64_t row_bytes = (int64_t)KB * kBlockBytes;

  const int wm = (wave >> 1) * 64;
  const int wn = (wave & 1) * 64;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  for (int k0 = 0; k0 < K; k0 += BK) {
    // ---- stage X tile: 128 rows x 64 k (fp32 -> bf16) ----
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f = tid + 256 * i;  // float4 index in the tile
      const int r = f >> 4;
      const int c4 = (f & 15) * 4;
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      if (m0 + r < M && k0 + c4 < K)
        v = *reinterpret_cast<const f32x4*>(x + (m0 + r) * K + k0 + c4);
      uint32_t* dst = reinterpret_cast<uint32_t*>(As + r * LDS_STRIDE + c4);
      dst[0] = pack_bf16x2(v.x, v.y);
      dst[1] = pack_bf16x2(v.z, v.w);
    }
    // ---- stage W tile: 128 rows x 2 blocks, v = d*q -> bf16 ----
    {
      const int r = tid >> 1;
      const int hb = tid & 1;
      const int kb = k0 / kBlockElems + hb;
      u32x4 out[4];
      if (n0 + r < N && kb < KB) {
        const Block b = load_block(w + (n0 + r) * row_bytes + (int64_t)kb * kBlockBytes);
        const float d = scale_to_f32_fast(b.scale_bits);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t q0 = b.q[2 * i], q1 = b.q[2 * i + 1];
          out[i].x = pack_bf16x2(d * q_at(q0, 0), d * q_at(q0, 1));
          out[i].y = pack_bf16x2(d * q_at(q0, 2), d * q_at(q0, 3));
          out[i].z = pack_bf16x2(d * q_at(q1, 0), d * q_at(q1, 1));
          out[i].w = pack_bf16x2(d * q_at(q1, 2), d * q_at(q1, 3));
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = u32x4{0u, 0u, 0u, 0u};
      }
      u32x4* dst = reinterpret_cast<u32x4*>(Bs + r * LDS_STRIDE + hb * 32);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = out[i];
    }
    __syncthreads();

    // ---- MFMA over the 64-wide K step: 4 sub-steps of 16 ----
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
      const int kk = ks + 8 * (lane >> 5);
      bf16x8 a[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = wm + 32 * i + (lane & 31);
        a[i] = *reinterpret_cast<const bf16x8*>(As + r * LDS_STRIDE + kk);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = wn + 32 * j + (lane & 31);
        bfr[j] = *reinterpret_cast<const bf16x8*>(Bs + r * LDS_STRIDE + kk);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // ---- epilogue: D[i][j] of lane l is row 4*(l/32) + (v%4) + 8*(v/4), col l%32 ----
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = n0 + wn + 32 * j + (lane & 31);
    if (n >= N) continue;
    const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm + 32 * i + 4 * (lane >> 5) + (v & 3) + 8 * (v >> 2);
        if (m < M) y[m * N + n] = acc[i][j][v] + bv;
      }
    }
  }
}

}  // namespace

hipError_t launch_gemm_mfma(const float* x, const uint8_t* w, const float* bias,
                            float* y, int M, int N, int K, hipStream_t stream) {
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  hipLaunchKernelGGL(gemm_q8_0_mfma_kernel, grid, dim3(256), 0, stream, x, w, bias, y,
                     M, N, K);
  return hipGetLastError();
}

}  // namespace mle
