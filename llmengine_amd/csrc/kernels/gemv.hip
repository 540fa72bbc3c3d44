// gemv.hip -- Q8_0 Linear decode GEMV (M <= 8 tokens) for gfx950.
//
// y[m, n] = sum_k x[m, k] * d[n, k/32] * q[n, k]  (+ bias[n])
//
// Replaces the reference's sgemm_nt_q8_0_warp_kernel
// (src/runtime/kernels/cuda_kernels.cu:333-358) and computes what
// cpu::sgemm_nt(const float*, const uint8_t*, ...) computes
// (src/runtime/kernels/cpu_kernels.cpp:208-218).
//
// HBM-bound: every weight byte is read once.  Work split:
//   * a lane group of LPR lanes owns RW consecutive output rows;
//   * lane l of the group walks the Q8_0 blocks b = l, l+LPR, l+2*LPR, ... of
//     those rows, so the group's lanes read LPR consecutive 34-byte blocks of a
//     row per step (one contiguous span of LPR*34 bytes per row);
//   * the 32 activations of block b are loaded once per lane and reused for all
//     RW rows (activation traffic = 4*MT*32 / (34*RW) bytes per weight byte);
//   * each block is dequantised in registers: s = sum_j x_j * q_j in fp32 FMAs,
//     then acc = fma(d, s, acc), i.e. the fp16 scale is applied once per block;
//   * the LPR partial sums of a row are reduced with cross-lane shuffles.
// Accumulation order differs from the reference's sequential chain, so results
// agree to fp32 rounding (relative L2 ~1e-7), not bit for bit.
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

template <int MT, int LPR, int RW>
__global__ __launch_bounds__(256) void gemv_q8_0_kernel(
    const float* __restrict__ x, const uint8_t* __restrict__ w,
    const float* __restrict__ bias, float* __restrict__ y, int M, int N, int K) {
  constexpr int G = 256 / LPR;  // lane groups per workgroup
  const int li = threadIdx.x % LPR;
  const int grp = threadIdx.x / LPR;
  const int64_t row0 = ((int64_t)blockIdx.x * G + grp) * RW;
  const int KB = K / kBlockElems;
  const int64_t row_bytes = (int64_t)KB * kBlockBytes;

  float acc[MT][RW];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[m][r] = 0.0f;

  bool row_ok[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) row_ok[r] = (row0 + r) < N;

  for (int b = li; b < KB; b += LPR) {
    Block blk[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      if (row_ok[r]) {
        blk[r] = load_block(w + (row0 + r) * row_bytes + (int64_t)b * kBlockBytes);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) blk[r].q[i] = 0u;
        blk[r].scale_bits = 0u;
      }
    }
    float part[MT][RW];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < RW; ++r) part[m][r] = 0.0f;

    // Activations in quarters of a block (8 values per token) to bound VGPRs.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      f32x4 xv[MT][2];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m < M) {
          const f32x4* xp = reinterpret_cast<const f32x4*>(
              x + (int64_t)m * K + (int64_t)b * kBlockElems + 8 * c);
          xv[m][0] = xp[0];
          xv[m][1] = xp[1];
        } else {
          xv[m][0] = f32x4{0.f, 0.f, 0.f, 0.f};
          xv[m][1] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const uint32_t q0 = blk[r].q[2 * c];
        const uint32_t q1 = blk[r].q[2 * c + 1];
        float qf[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          qf[j] = q_at(q0, j);
          qf[4 + j] = q_at(q1, j);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          float s = part[m][r];
          s = __builtin_fmaf(xv[m][0].x, qf[0], s);
          s = __builtin_fmaf(xv[m][0].y, qf[1], s);
          s = __builtin_fmaf(xv[m][0].z, qf[2], s);
          s = __builtin_fmaf(xv[m][0].w, qf[3], s);
          s = __builtin_fmaf(xv[m][1].x, qf[4], s);
          s = __builtin_fmaf(xv[m][1].y, qf[5], s);
          s = __builtin_fmaf(xv[m][1].z, qf[6], s);
          s = __builtin_fmaf(xv[m][1].w, qf[7], s);
          part[m][r] = s;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const float d = scale_to_f32_fast(blk[r].scale_bits);
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[m][r] = __builtin_fmaf(d, part[m][r], acc[m][r]);
    }
  }

  // Reduce the LPR partial sums of every (token, row) pair within the group.
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < RW; ++r) acc[m][r] += __shfl_xor(acc[m][r], off, LPR);
  }

  if (li == 0) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      if (!row_ok[r]) continue;
      const float bv = bias ? bias[row0 + r] : 0.0f;
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (m < M) y[(int64_t)m * N + row0 + r] = acc[m][r] + bv;
    }
  }
}

template <int MT, int LPR, int RW>
hipError_t launch_one(const float* x, const uint8_t* w, const float* bias, float* y,
                      int M, int N, int K, hipStream_t stream) {
  constexpr int rows_per_wg = (256 / LPR) * RW;
  const int64_t grid = ((int64_t)N + rows_per_wg - 1) / rows_per_wg;
  hipLaunchKernelGGL((gemv_q8_0_kernel<MT, LPR, RW>), dim3((unsigned)grid), dim3(256),
                     0, stream, x, w, bias, y, M, N, K);
  return hipGetLastError();
}

template <int MT, int LPR>
hipError_t dispatch_rw(int rw, const float* x, const uint8_t* w, const float* bias,
                       float* y, int M, int N, int K, hipStream_t stream) {
  switch (rw) {
    case 1: return launch_one<MT, LPR, 1>(x, w, bias, y, M, N, K, stream);
    case 2: return launch_one<MT, LPR, 2>(x, w, bias, y, M, N, K, stream);
    case 4: return launch_one<MT, LPR, 4>(x, w, bias, y, M, N, K, stream);
    case 8: return launch_one<MT, LPR, 8>(x, w, bias, y, M, N, K, stream);
  }
  return hipErrorInvalidValue;
}

template <int MT>
hipError_t dispatch_lpr(int lpr, int rw, const float* x, const uint8_t* w,
                        const float* bias, float* y, int M, int N, int K,
                        hipStream_t stream) {
  switch (lpr) {
    case 16: return dispatch_rw<MT, 16>(rw, x, w, bias, y, M, N, K, stream);
    case 32: return dispatch_rw<MT, 32>(rw, x, w, bias, y, M, N, K, stream);
    case 64: return dispatch_rw<MT, 64>(rw, x, w, bias, y, M, N, K, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace

bool gemv_config_valid(const GemvConfig& c) {
  const bool mt = c.mt == 1 || c.mt == 2 || c.mt == 4 || c.mt == 8;
  const bool lpr = c.lpr == 16 || c.lpr == 32 || c.lpr == 64;
  const bool rw = c.rw == 1 || c.rw == 2 || c.rw == 4 || c.rw == 8;
  return mt && lpr && rw;
}

GemvConfig gemv_pick_config(int M, int N, int K) {
  GemvConfig c;
  c.mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const int kb = K / kBlockElems;
  // Lanes per row: the width that leaves the fewest idle lanes on the last
  // block step, preferring wider groups on ties.
  int best = 64;
  int64_t best_waste = -1;
  for (int lpr : {64, 32, 16}) {
    const int64_t steps = (kb + lpr - 1) / lpr;
    const int64_t waste = steps * lpr - kb;
    if (best_waste < 0 || waste < best_waste) {
      best = lpr;
      best_waste = waste;
    }
  }
  c.lpr = best;
  // Rows per group: reuse activations across rows, but keep >= 1024
  // workgroups in flight when the matrix is large enough.
  c.rw = c.mt >= 4 ? 2 : 4;
  while (c.rw > 1) {
    const int64_t rows_per_wg = (int64_t)(256 / c.lpr) * c.rw;
    if ((N + rows_per_wg - 1) / rows_per_wg >= 1024) break;
    c.rw /= 2;
  }
  return c;
}

hipError_t launch_gemv(const GemvConfig& cfg, const float* x, const uint8_t* w,
                       const float* bias, float* y, int M, int N, int K,
                       hipStream_t stream) {
  switch (cfg.mt) {
    case 1: return dispatch_lpr<1>(cfg.lpr, cfg.rw, x, w, bias, y, M, N, K, stream);
    case 2: return dispatch_lpr<2>(cfg.lpr, cfg.rw, x, w, bias, y, M, N, K, stream);
    case 4: return dispatch_lpr<4>(cfg.lpr, cfg.rw, x, w, bias, y, M, N, K, stream);
    case 8: return dispatch_lpr<8>(cfg.lpr, cfg.rw, x, w, bias, y, M, N, K, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace mle
