// matmul.hip -- Q8_0 MatMul C[M,N] = A[M,K] . B[K,N] for gfx950.
//
// B is one Q8_0 stream in row-major [K, N] order, so element (k, n) is flat
// index k*N + n and blocks run along N (reference
// src/runtime/kernels/cpu_kernels.cpp:116-130, cuda_kernels.cu:296-331).  Each
// element is formed as the reference forms it, v = d * q in fp32, and the K sum
// is an fp32 FMA chain split into fixed pieces added in a fixed order, so the
// result is deterministic and within fp32 rounding of the reference's
// sequential sum (relative L2 ~1e-7), as the reference's own device kernel is
// (it splits K over 8 warps and adds their partials).
//
// Work split.  A workgroup owns a tile of 256 output columns (8 blocks of a B
// row: lane l of every wave takes columns 4l .. 4l+3) for MR token rows, and a
// run of 256-row K slices.  Its 16 waves take 16 consecutive rows of each slice
// each, issue all 16 rows' loads (the block scale and the lane's 4 quants, as
// 2-byte loads: blocks are 34 bytes, so only 2-byte alignment holds) before
// using any, and fold them into fp32 accumulators in row order; the
// activations of a row are wave-uniform (scalar loads).  The 16 waves' sums
// are then added in LDS in wave order.  When the column and token tiles alone
// leave the GPU's 256 CUs short of work, the K slices are spread over S
// workgroups per tile: each writes its partial tile to a workspace
// [S][M][N], and a second launch adds the S partials of every output in slice
// order.  B is read once per MR token rows (MR = 8 at most).
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

constexpr int kMmCols = 256;                 // output columns per workgroup
constexpr int kMmWaves = 16;                 // waves per workgroup
constexpr int kMmRun = 16;                   // B rows per wave per slice
constexpr int kMmSlice = kMmWaves * kMmRun;  // B rows per slice
constexpr int kMmTargetGroups = 512;         // workgroups wanted per launch (2 per CU)

struct MmGrid {
  unsigned col_tiles, row_tiles, splits;
  int slices_per_split;
};

MmGrid mm_grid(int M, int N, int K, int mr) {
  MmGrid g;
  g.col_tiles = (unsigned)((N + kMmCols - 1) / kMmCols);
  g.row_tiles = (unsigned)((M + mr - 1) / mr);
  const int slices = (K + kMmSlice - 1) / kMmSlice;
  const int64_t tiles = (int64_t)g.col_tiles * g.row_tiles;
  int s = (int)((kMmTargetGroups + tiles - 1) / tiles);
  if (s > slices) s = slices;
  if (s < 1) s = 1;
  g.slices_per_split = (slices + s - 1) / s;
  g.splits = (unsigned)((slices + g.slices_per_split - 1) / g.slices_per_split);
  return g;
}

int mm_rows_per_tile(int M) { return M >= 8 ? 8 : M >= 4 ? 4 : M >= 2 ? 2 : 1; }

template <int MR>
__global__ __launch_bounds__(64 * kMmWaves) void matmul_q8_0_kernel(
    const float* __restrict__ a, const uint8_t* __restrict__ b, float* __restrict__ out,
    int M, int N, int K, int slices_per_split) {
  __shared__ float red[kMmWaves][MR][kMmCols];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * kMmCols;
  const int n = n0 + 4 * lane;  // this lane's 4 columns
  const bool live_n = n < N;    // N % 32 == 0: the 4 columns are all inside or all outside
  const int m0 = blockIdx.z * MR;
  const int64_t NB = N / kBlockElems;
  const int blk = n / kBlockElems, o = n % kBlockElems;  // o: 0, 4, .., 28
  const int s_begin = blockIdx.y * slices_per_split;
  const int nslices = (K + kMmSlice - 1) / kMmSlice;
  const int s_end = min(s_begin + slices_per_split, nslices);
  // Activation rows of the tile (rows past M read row M - 1 and are never stored).
  const float* arow[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) arow[r] = a + (int64_t)min(m0 + r, M - 1) * K;

  float acc[MR][4];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[r][j] = 0.0f;
  for (int sl = s_begin; sl < s_end; ++sl) {
    const int k0 = sl * kMmSlice + wave * kMmRun;  // this wave's rows k0 .. k0 + 15
    uint16_t sc[kMmRun], q01[kMmRun], q23[kMmRun];
#pragma unroll
    for (int j = 0; j < kMmRun; ++j) {
      const int k = k0 + j;
      if (live_n && k < K) {
        const uint16_t* hp =
            reinterpret_cast<const uint16_t*>(b + ((int64_t)k * NB + blk) * kBlockBytes);
        sc[j] = hp[0];
        q01[j] = hp[1 + o / 2];
        q23[j] = hp[2 + o / 2];
      } else {
        sc[j] = 0;  // scale +0: the row adds nothing
        q01[j] = q23[j] = 0;
      }
    }
#pragma unroll
    for (int j = 0; j < kMmRun; ++j) {
      const int k = k0 + j;
      const float d = scale_to_f32(sc[j]);
      const uint32_t q = (uint32_t)q01[j] | ((uint32_t)q23[j] << 16);
      const float v[4] = {d * q_at(q, 0), d * q_at(q, 1), d * q_at(q, 2), d * q_at(q, 3)};
#pragma unroll
      for (int r = 0; r < MR; ++r) {
        const float av = k < K ? arow[r][k] : 0.0f;  // wave-uniform
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][i] = __builtin_fmaf(av, v[i], acc[r][i]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < MR; ++r)
    *reinterpret_cast<f32x4*>(&red[wave][r][4 * lane]) =
        f32x4{acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
  __syncthreads();
  // The 16 waves' sums of each output, in wave order; outputs (r, column).
  for (int idx = tid; idx < MR * kMmCols; idx += 64 * kMmWaves) {
    const int r = idx / kMmCols, col = idx % kMmCols;
    float s = red[0][r][col];
#pragma unroll
    for (int w = 1; w < kMmWaves; ++w) s += red[w][r][col];
    const int m = m0 + r, nn = n0 + col;
    if (m < M && nn < N) out[((int64_t)blockIdx.y * M + m) * N + nn] = s;
  }
}

// out[m, n] = sum over s of part[s][m][n], in s order (four columns a thread).
__global__ __launch_bounds__(256) void matmul_splits_kernel(const float* __restrict__ part,
                                                           float* __restrict__ c, int64_t mn4,
                                                           int splits) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= mn4) return;
  const f32x4* p = reinterpret_cast<const f32x4*>(part);
  f32x4 s = p[i];
  for (int sp = 1; sp < splits; ++sp) s += p[(int64_t)sp * mn4 + i];
  reinterpret_cast<f32x4*>(c)[i] = s;
}

template <int MR>
void launch_mm(const MmGrid& g, const float* a, const uint8_t* b, float* dst, int M, int N,
               int K, hipStream_t stream) {
  hipLaunchKernelGGL(matmul_q8_0_kernel<MR>, dim3(g.col_tiles, g.splits, g.row_tiles),
                     dim3(64 * kMmWaves), 0, stream, a, b, dst, M, N, K, g.slices_per_split);
}

}  // namespace

size_t matmul_workspace_floats(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const MmGrid g = mm_grid(M, N, K, mm_rows_per_tile(M));
  return g.splits > 1 ? (size_t)g.splits * M * N : 0;
}

hipError_t launch_matmul(const float* a, const uint8_t* b, float* c, int M, int N, int K,
                         float* partials, hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) return hipSuccess;
  if (N % kBlockElems != 0 || K % kBlockElems != 0) return hipErrorInvalidValue;
  const int mr = mm_rows_per_tile(M);
  const MmGrid g = mm_grid(M, N, K, mr);
  if (g.row_tiles > 65535 || g.splits > 65535) return hipErrorInvalidValue;
  if (g.splits > 1 && partials == nullptr) return hipErrorInvalidValue;
  float* dst = g.splits > 1 ? partials : c;
  switch (mr) {
    case 1: launch_mm<1>(g, a, b, dst, M, N, K, stream); break;
    case 2: launch_mm<2>(g, a, b, dst, M, N, K, stream); break;
    case 4: launch_mm<4>(g, a, b, dst, M, N, K, stream); break;
    default: launch_mm<8>(g, a, b, dst, M, N, K, stream); break;
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || g.splits == 1) return err;
  const int64_t mn4 = (int64_t)M * N / 4;
  hipLaunchKernelGGL(matmul_splits_kernel, dim3((unsigned)((mn4 + 255) / 256)), dim3(256), 0,
                     stream, partials, c, mn4, (int)g.splits);
  return hipGetLastError();
}

}  // namespace mle
