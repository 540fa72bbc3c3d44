// gemv_tiled.hip -- Q8_0 Linear decode GEMV (M <= 4 tokens) on 16-row tiled
// weights (WeightLayout::kTiled), FP32 arithmetic, for gfx950.
//
// y[m, n] = sum_k x[m, k] * d[n, k/32] * q[n, k]  (+ bias[n]), as
// cpu::sgemm_nt(const float*, const uint8_t*, ...) computes it
// (src/runtime/kernels/cpu_kernels.cpp:208-218), for the few-token case that
// the reference's sgemm_nt_q8_0_warp_kernel covers (cuda_kernels.cu:333-358).
//
// Work split: a workgroup owns one 16-row group of a weight (SwiGLU: the same
// group of the gate and the up weight, half the waves each) and its waves split
// K in chunks of PPW block pairs (chunk c -> wave c % waves).  Per chunk a wave
// issues PPW contiguous 1 KB quant loads (lane l: row l % 16, quants
// 8 (l/16) .. +7 of both blocks of the pair) and PPW 4-byte scale loads (the
// row's two scales), copies the chunk's activations into its own LDS area and
// reads back the 16 it needs per pair (16 lanes share each address).  Per block
// a lane forms s = sum_j x_j q_j over its 8 quants in fp32 FMAs and applies the
// scale once, acc = fma(d, s, acc); the four lanes of a row are summed with
// cross-lane shuffles and the waves' partial sums in LDS, in wave order, so
// the result is deterministic.  There is no split-K hand-off through memory:
// the reduction never leaves the workgroup.
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Orders this wave's LDS accesses on either side (other lanes' values are read).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// silu(g) * u with the reference's operation order (cpu_kernels.cpp:848-858).
__device__ __forceinline__ float silu_mul_t(float g, float u) {
  return (g / (1.0f + expf(-g))) * u;
}

struct TiledGemvArgs {
  LinearSeg seg[3];
  unsigned grp_end[3];  // segment i owns row groups [grp_end[i-1], grp_end[i])
  int count;
};

// One pair of blocks: 8 quants of each (q0: block 2p, q1: block 2p+1) against
// the lane's activations; scale applied once per block.
__device__ __forceinline__ float dot8(uint32_t qa, uint32_t qb, const f32x4 xa, const f32x4 xb) {
  float s = 0.0f;
  s = __builtin_fmaf(xa.x, q_at(qa, 0), s);
  s = __builtin_fmaf(xa.y, q_at(qa, 1), s);
  s = __builtin_fmaf(xa.z, q_at(qa, 2), s);
  s = __builtin_fmaf(xa.w, q_at(qa, 3), s);
  s = __builtin_fmaf(xb.x, q_at(qb, 0), s);
  s = __builtin_fmaf(xb.y, q_at(qb, 1), s);
  s = __builtin_fmaf(xb.z, q_at(qb, 2), s);
  s = __builtin_fmaf(xb.w, q_at(qb, 3), s);
  return s;
}

template <int MT, int PPW, int MODE>
__global__ __launch_bounds__(1024) void gemv_tiled_kernel(const float* __restrict__ x,
                                                          const TiledGemvArgs args, int M,
                                                          int K, int wpg) {
  constexpr bool kSwi = MODE == 1;
  constexpr int XCH = PPW * 64;  // activations per token per chunk
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int half = kSwi && wave >= wpg ? 1 : 0;  // SwiGLU: 0 gate, 1 up
  const int wv = wave - half * wpg;              // wave within its weight
  const int sub = lane >> 4, r = lane & 15;
  const int KB = K / kBlockElems;
  const int KP = (KB + 1) >> 1;

  const unsigned grp = blockIdx.x;
  const int si = (!kSwi && args.count > 1 && grp >= args.grp_end[0])
                     ? ((args.count > 2 && grp >= args.grp_end[1]) ? 2 : 1)
                     : 0;
  const unsigned grp0 = si == 0 ? 0u : si == 1 ? args.grp_end[0] : args.grp_end[1];
  const uint8_t* w = si == 0 ? args.seg[0].w : si == 1 ? args.seg[1].w : args.seg[2].w;
  const void* bias = si == 0 ? args.seg[0].bias : si == 1 ? args.seg[1].bias : args.seg[2].bias;
  const int bias_bf16 =
      si == 0 ? args.seg[0].bias_bf16 : si == 1 ? args.seg[1].bias_bf16 : args.seg[2].bias_bf16;
  float* y = si == 0 ? args.seg[0].y : si == 1 ? args.seg[1].y : args.seg[2].y;
  const int N = si == 0 ? args.seg[0].N : si == 1 ? args.seg[1].N : args.seg[2].N;
  if (half) w = args.seg[1].w;
  const int64_t g = grp - grp0;
  const int64_t G = ((int64_t)N + kTileRows - 1) / kTileRows;
  const __amdgpu_buffer_rsrc_t qrs =
      rsrc_of(w + g * KP * kTilePieceBytes, (uint32_t)KP * kTilePieceBytes);
  const __amdgpu_buffer_rsrc_t srs =
      rsrc_of(w + G * KP * kTilePieceBytes + g * KP * kTileScaleBytes,
              (uint32_t)KP * kTileScaleBytes);
  const __amdgpu_buffer_rsrc_t xrs = rsrc_of(x, (uint32_t)((int64_t)M * K * 4));
  float* xs = smem + wave * (MT * XCH);

  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
  for (int c = wv; c * PPW < KP; c += wpg) {
    const int p0 = c * PPW;
    u32x4 q[PPW];
    uint32_t sc[PPW];
#pragma unroll
    for (int j = 0; j < PPW; ++j) {
      const bool live = p0 + j < KP;
      q[j] = __builtin_amdgcn_raw_buffer_load_b128(
          qrs, live ? (uint32_t)(p0 + j) * kTilePieceBytes + (uint32_t)lane * 16 : 0x80000000u,
          0, kNonTemporal);
      sc[j] = __builtin_amdgcn_raw_buffer_load_b32(
          srs, live ? (uint32_t)(p0 + j) * kTileScaleBytes + (uint32_t)r * 4 : 0x80000000u, 0,
          0);
    }
    // Activations of the chunk, k = 64 p0 .. 64 (p0 + PPW), token-major;
    // past K or M: zeros (K is a multiple of 32, so a 4-float piece is whole).
    f32x4 xv[MT][PPW / 4];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int v = 0; v < PPW / 4; ++v) {
        const int idx = (v * 64 + lane) * 4;
        const int k = 64 * p0 + idx;
        xv[m][v] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       xrs, m < M && k < K ? (uint32_t)(m * K + k) * 4 : 0x80000000u, 0, 0));
      }
    wave_lds_sync();  // the previous chunk's reads of xs are done
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int v = 0; v < PPW / 4; ++v)
        *reinterpret_cast<f32x4*>(xs + m * XCH + (v * 64 + lane) * 4) = xv[m][v];
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < PPW; ++j) {
      const float d0 = scale_to_f32_fast(sc[j] & 0xffffu);
      const float d1 = scale_to_f32_fast(sc[j] >> 16);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float* xr = xs + m * XCH + j * 64 + 8 * sub;
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(xr);
        const f32x4 a1 = *reinterpret_cast<const f32x4*>(xr + 4);
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(xr + 32);
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(xr + 36);
        acc[m] = __builtin_fmaf(d0, dot8(q[j].x, q[j].y, a0, a1), acc[m]);
        acc[m] = __builtin_fmaf(d1, dot8(q[j].z, q[j].w, b0, b1), acc[m]);
      }
    }
  }
  // Row sums: the four quarter-block lanes of row r, then the waves in order.
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    acc[m] += __shfl_xor(acc[m], 16);
    acc[m] += __shfl_xor(acc[m], 32);
  }
  float* red = smem + nwaves * (MT * XCH);
  if (lane < 16) {
#pragma unroll
    for (int m = 0; m < MT; ++m) red[(wave * MT + m) * 16 + lane] = acc[m];
  }
  __syncthreads();
  if (wave != 0 || lane >= MT * 16) return;
  const int m = lane >> 4, rr = lane & 15;
  const int64_t n = g * kTileRows + rr;
  if (m >= M || n >= N) return;
  float s = 0.0f;
  for (int wi = 0; wi < wpg; ++wi) s += red[(wi * MT + m) * 16 + rr];
  if constexpr (kSwi) {
    float u = 0.0f;
    for (int wi = 0; wi < wpg; ++wi) u += red[((wpg + wi) * MT + m) * 16 + rr];
    y[(int64_t)m * N + n] = silu_mul_t(s, u);
  } else {
    y[(int64_t)m * N + n] = s + (bias ? bias_at(bias, bias_bf16, n) : 0.0f);
  }
}

template <int MT, int PPW>
hipError_t launch_mt(const TiledGemvArgs& a, unsigned groups, int waves, Epilogue mode,
                     const float* x, int M, int K, int wpg, hipStream_t stream) {
  const size_t lds = (size_t)waves * MT * (PPW * 64 + 16) * sizeof(float);
  if (mode == Epilogue::kSwiGLU)
    hipLaunchKernelGGL((gemv_tiled_kernel<MT, PPW, 1>), dim3(groups), dim3(64 * waves), lds,
                       stream, x, a, M, K, wpg);
  else
    hipLaunchKernelGGL((gemv_tiled_kernel<MT, PPW, 0>), dim3(groups), dim3(64 * waves), lds,
                       stream, x, a, M, K, wpg);
  return hipGetLastError();
}

template <int MT>
hipError_t launch_ppw(const TiledGemvConfig& c, const TiledGemvArgs& a, unsigned groups,
                      int waves, Epilogue mode, const float* x, int M, int K, hipStream_t s) {
  switch (c.ppw) {
    case 4: return launch_mt<MT, 4>(a, groups, waves, mode, x, M, K, c.wpg, s);
    case 8: return launch_mt<MT, 8>(a, groups, waves, mode, x, M, K, c.wpg, s);
    case 16:  // 4 KB of quants per lane set: one token only within 128 registers
      if constexpr (MT == 1) return launch_mt<MT, 16>(a, groups, waves, mode, x, M, K, c.wpg, s);
      break;
  }
  return hipErrorInvalidValue;
}

}  // namespace

size_t gemv_tiled_lds_bytes(const TiledGemvConfig& c, bool swiglu) {
  const int waves = c.wpg * (swiglu ? 2 : 1);
  return (size_t)waves * c.mt * (c.ppw * 64 + 16) * sizeof(float);
}

bool gemv_tiled_config_valid(const TiledGemvConfig& c, bool swiglu) {
  const bool mt = c.mt == 1 || c.mt == 2 || c.mt == 4;
  const bool ppw = c.ppw == 4 || c.ppw == 8 || (c.ppw == 16 && c.mt == 1);
  const bool wpg = c.wpg >= 1 && c.wpg * (swiglu ? 2 : 1) <= 16;
  return mt && ppw && wpg && gemv_tiled_lds_bytes(c, swiglu) <= 64 * 1024;
}

TiledGemvConfig gemv_tiled_pick(int M, int rows, int K, bool swiglu) {
  // Measured on MI355X (Llama-7B and Qwen2.5-0.5B projections, Qwen lm_head,
  // M = 1..4): chunks of 4 block pairs win everywhere; about 2-3 thousand
  // waves in flight do, so waves per 16-row group = 49152 / rows rounded down
  // to a power of two, at least 4 (a vocabulary-sized weight still gains from
  // 4), at most 16 (8 per weight for SwiGLU) and at most the chunks of a row.
  // `rows`: output rows of the launch (all segments; SwiGLU: one weight's).
  TiledGemvConfig c;
  c.mt = M <= 1 ? 1 : M <= 2 ? 2 : 4;
  c.ppw = 4;
  const int KP = (K / kBlockElems + 1) / 2;
  const int chunks = (KP + c.ppw - 1) / c.ppw;
  int w = 4;
  while (w < 16 && (int64_t)(2 * w) * rows <= 49152) w *= 2;
  if (swiglu && w > 8) w = 8;
  c.wpg = w < chunks ? w : chunks;
  while (!gemv_tiled_config_valid(c, swiglu) && c.wpg > 1) --c.wpg;
  return c;
}

bool gemv_tiled_wins(int M, int rows, int K) {
  // Against the MFMA decode on tiled weights (same sweep): one token always;
  // two tokens below vocabulary-sized outputs; up to four on short rows.
  return M == 1 || (M == 2 && rows < 65536) || (M <= 4 && K <= 1024 && rows <= 32768);
}

hipError_t launch_gemv_tiled_segs(const TiledGemvConfig& c, const float* x,
                                  const LinearSegs& s, int M, int K, hipStream_t stream) {
  const bool swi = s.mode == Epilogue::kSwiGLU;
  if (s.layout != WeightLayout::kTiled || !gemv_tiled_config_valid(c, swi) || M < 1 ||
      M > c.mt || s.count < 1 || s.count > 3 || (swi && s.count != 2))
    return hipErrorInvalidValue;
  if ((int64_t)M * K * 4 >= (int64_t(1) << 31) ||
      (int64_t)((K / kBlockElems + 1) / 2) * kTilePieceBytes >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  TiledGemvArgs a{};
  unsigned end = 0;
  const int count = swi ? 1 : s.count;
  for (int i = 0; i < 3; ++i) {
    a.seg[i] = s.seg[i];
    if (i < count) {
      if (s.seg[i].N <= 0 || s.seg[i].w == nullptr) return hipErrorInvalidValue;
      end += (unsigned)((s.seg[i].N + kTileRows - 1) / kTileRows);
    }
    a.grp_end[i] = end;
  }
  if (swi) {
    if (s.seg[1].w == nullptr) return hipErrorInvalidValue;
    a.seg[1].N = s.seg[0].N;
  }
  a.count = count;
  const int waves = c.wpg * (swi ? 2 : 1);
  switch (c.mt) {
    case 1: return launch_ppw<1>(c, a, end, waves, s.mode, x, M, K, stream);
    case 2: return launch_ppw<2>(c, a, end, waves, s.mode, x, M, K, stream);
    case 4: return launch_ppw<4>(c, a, end, waves, s.mode, x, M, K, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace mle
