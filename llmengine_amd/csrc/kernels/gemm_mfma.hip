// gemm_mfma.hip -- Q8_0 Linear prefill GEMM on bf16 MFMA for gfx950.
//
// Y[M, N] = X[M, K] . W^T (+ bias), W in Q8_0 blocks along K.
// Same contract as cpu::sgemm_nt(const float*, const uint8_t*, ...)
// (src/runtime/kernels/cpu_kernels.cpp:208-218); used for M >= 64.
//
// Workgroup tile BM x BN = 128 x 128, K step BK = 64 (two Q8_0 blocks per
// output row), 256 threads = 4 wavefronts in a 2 x 2 grid, each owning a 64 x 64
// sub-tile as 2 x 2 v_mfma_f32_32x32x16_bf16 accumulators.
//
// Operands are staged in LDS as bf16 (rows padded by 16 bytes against bank
// conflicts):
//   * X tile: fp32 -> bf16 (v_cvt_pk_bf16_f32, round to nearest even);
//   * W tile: each thread takes one 34-byte block, forms v = d * q in fp32
//     (exactly the reference's element value) and rounds it once to bf16.
// The per-block scale is thus folded into the B operand before the MFMA
// instead of being applied to the accumulator after every 32-wide K block:
// the latter costs one VALU FMA per output per block, i.e. one VALU op per 64
// MFMA flops, which on CDNA4 equals the whole non-packed VALU rate and would cap
// the MFMA pipe at about half its peak.  Error vs the fp32 reference is then
// the bf16 rounding of both operands (relative L2 ~2e-3), inside the 1e-2 bound
// stated for this path.
//
// Software pipeline: while the MFMAs consume K step t from one LDS buffer, the
// global loads of steps t+1 and t+2 (buffer loads, every one unconditional:
// rows and steps past the end read as zero) are in flight into registers; step
// t+1 is then converted into the other LDS buffer.  One barrier per K step.
//
// Split K (gridDim.z > 1, for shapes with too few tiles to fill the GPU): each
// workgroup stores its 128 x 128 fp32 partial tile with device-scope (sc1)
// stores, waits for their completion and bumps a per-tile counter; the last
// workgroup of the tile adds the partials in split order (deterministic),
// adds the bias, writes Y and resets the counter for the next launch.
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (144 bytes)
constexpr int TILE_ELEMS = BM * BN;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t cvt_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Global data of one K step held by one thread.
struct Stage {
  f32x4 x[8];    // X: 8 float4 of the 128 x 64 tile
  RawBlock w;    // W: one 34-byte block of the 128 x 2-block tile
};

__global__ __launch_bounds__(256, 2) void gemm_q8_0_mfma_kernel(
    const float* __restrict__ x, const uint8_t* __restrict__ w,
    const float* __restrict__ bias, float* __restrict__ y, int M, int N, int K,
    int steps_per_split, float* __restrict__ partials, uint32_t* __restrict__ counters) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDS_STRIDE];
  __shared__ uint32_t arrived;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  const int KB = K / kBlockElems;
  const uint32_t row_bytes = (uint32_t)KB * kBlockBytes;
  const int n_steps = (K + BK - 1) / BK;
  const int s_begin = blockIdx.z * steps_per_split;
  const int s_end = min(s_begin + steps_per_split, n_steps);

  // Buffer resources starting at this tile's first row: offsets stay small and
  // rows past M (X) or N (W) read as zero.
  const int64_t xrows = min((int64_t)BM, (int64_t)M - m0);
  const __amdgpu_buffer_rsrc_t xrs = rsrc(x + m0 * K, (uint32_t)(xrows * K * 4));
  const int64_t wrows = min((int64_t)BN, (int64_t)N - n0);
  const uint8_t* wtile = w + n0 * row_bytes;
  const __amdgpu_buffer_rsrc_t wrs = rsrc(wtile, (uint32_t)(wrows * row_bytes));

  // This thread's load slots: X float4 f = tid + 256 i is row f/16, columns
  // 4 (f%16) .. +3 of the step; W block is row tid/2, block tid%2 of the step.
  const int wr_row = tid >> 1, wr_hb = tid & 1;

  auto load = [&](int s, Stage& st) {
    const bool live = s < s_end;
    const int k0 = s * BK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f = tid + 256 * i;
      const int r = f >> 4, c4 = (f & 15) * 4;
      const uint32_t off = live && k0 + c4 < K ? (uint32_t)(r * K + k0 + c4) * 4u : 0x80000000u;
      st.x[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
    }
    const int kb = s * (BK / kBlockElems) + wr_hb;
    const uint32_t boff = (uint32_t)wr_row * row_bytes + (uint32_t)kb * kBlockBytes;
    const uint32_t mis = (uint32_t)(((uintptr_t)wtile + boff) & 2u);
    const bool wlive = live && kb < KB;
    const uint32_t v8 = wlive ? boff + mis : 0x80000000u;
    const uint32_t v2 = wlive ? boff + (mis ? 0u : 32u) : 0x80000000u;
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8, 0, 0);
    const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8 + 16, 0, 0);
    st.w.v0 = u32x4_a4{a.x, a.y, a.z, a.w};
    st.w.v1 = u32x4_a4{b.x, b.y, b.z, b.w};
    st.w.u = __builtin_amdgcn_raw_buffer_load_b16(wrs, v2, 0, 0);
    st.w.mis = mis;
  };

  auto store = [&](const Stage& st, uint16_t* as, uint16_t* bs) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f = tid + 256 * i;
      const int r = f >> 4, c4 = (f & 15) * 4;
      const f32x4 v = st.x[i];
      *reinterpret_cast<uint2*>(as + r * LDS_STRIDE + c4) =
          make_uint2(cvt_bf16x2(v.x, v.y), cvt_bf16x2(v.z, v.w));
    }
    const Block b = finish_block(st.w);
    const float d = scale_to_f32_fast(b.scale_bits);
    u32x4* dst = reinterpret_cast<u32x4*>(bs + wr_row * LDS_STRIDE + wr_hb * kBlockElems);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q0 = b.q[2 * i], q1 = b.q[2 * i + 1];
      dst[i] = u32x4{cvt_bf16x2(d * q_at(q0, 0), d * q_at(q0, 1)),
                     cvt_bf16x2(d * q_at(q0, 2), d * q_at(q0, 3)),
                     cvt_bf16x2(d * q_at(q1, 0), d * q_at(q1, 1)),
                     cvt_bf16x2(d * q_at(q1, 2), d * q_at(q1, 3))};
    }
  };

  const int wm = (wave >> 1) * 64;
  const int wn = (wave & 1) * 64;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  auto mfma_step = [&](const uint16_t* as, const uint16_t* bs) {
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
      const int kk = ks + 8 * (lane >> 5);
      bf16x8 a[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(as + (wm + 32 * i + (lane & 31)) * LDS_STRIDE + kk);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const bf16x8*>(bs + (wn + 32 * j + (lane & 31)) * LDS_STRIDE + kk);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  // Two K steps of global data in flight: step s loads step s+2 into the
  // register stage freed by step s+1's store, so two stages alternate (unroll 2).
  Stage sa, sb;
  load(s_begin, sa);
  load(s_begin + 1, sb);
  store(sa, As[0], Bs[0]);
  __syncthreads();
  auto step = [&](int s, int buf, Stage& next, Stage& far) {
    load(s + 2, far);  // past s_end: zeros
    mfma_step(As[buf], Bs[buf]);
    store(next, As[buf ^ 1], Bs[buf ^ 1]);
    __syncthreads();
  };
  int s = s_begin;
  for (; s + 2 <= s_end; s += 2) {
    step(s, 0, sb, sa);
    step(s + 1, 1, sa, sb);
  }
  if (s < s_end) step(s, 0, sb, sa);

  // D[i][j] of lane l is row 4*(l/32) + (v%4) + 8*(v/4), column l%32.
  if (gridDim.z == 1) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + wn + 32 * j + (lane & 31);
      if (n >= N) continue;
      const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t m = m0 + wm + 32 * i + 4 * (lane >> 5) + (v & 3) + 8 * (v >> 2);
          if (m < M) y[m * N + n] = acc[i][j][v] + bv;
        }
    }
    return;
  }

  // Split K: partial tile [tile][split][16 KB x 4] by device-scope stores; the
  // last workgroup of the tile reduces in split order.  Partials are stored
  // lane-major (slot (i, j, quad) x 256 threads x 16 bytes), so each store
  // instruction writes 4 KB contiguously and the reader finds its own slots.
  constexpr int SC1 = 16;  // cache-policy bit: device scope
  const uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x;
  const __amdgpu_buffer_rsrc_t prs =
      rsrc(partials + (int64_t)tile * gridDim.z * TILE_ELEMS, gridDim.z * TILE_ELEMS * 4u);
  auto slot = [&](int i, int j, int q) {  // byte offset of 4 accumulators
    return (uint32_t)((((i * 2 + j) * 4 + q) * 256 + tid) * 16);
  };
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v = f32x4{acc[i][j][4 * q + 0], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                              acc[i][j][4 * q + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs,
                                               blockIdx.z * TILE_ELEMS * 4u + slot(i, j, q), 0,
                                               SC1);
      }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // every partial has reached the coherence point
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (tid == 0)
    arrived = __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (arrived != gridDim.z - 1) return;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 sum[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) sum[q] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (unsigned sp = 0; sp < gridDim.z; ++sp)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          sum[q] += __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         prs, sp * TILE_ELEMS * 4u + slot(i, j, q), 0, SC1));
      const int64_t n = n0 + wn + 32 * j + (lane & 31);
      if (n >= N) continue;
      const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm + 32 * i + 4 * (lane >> 5) + (v & 3) + 8 * (v >> 2);
        if (m < M) y[m * N + n] = sum[v >> 2][v & 3] + bv;
      }
    }
  if (tid == 0)
    __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct GemmGrid {
  unsigned tn, tm, splits;
  int steps_per_split;
};

GemmGrid gemm_grid(int M, int N, int K, int splits) {
  GemmGrid g;
  g.tn = (unsigned)((N + BN - 1) / BN);
  g.tm = (unsigned)((M + BM - 1) / BM);
  const int n_steps = (K + BK - 1) / BK;
  if (splits < 1) splits = 1;
  if (splits > n_steps) splits = n_steps;
  g.steps_per_split = (n_steps + splits - 1) / splits;
  g.splits = (unsigned)((n_steps + g.steps_per_split - 1) / g.steps_per_split);
  return g;
}

}  // namespace

int gemm_mfma_pick_splits(int M, int N, int K) {
  // Split K until the tiles give every CU (256) about one workgroup.
  const int64_t tiles = (int64_t)((N + BN - 1) / BN) * ((M + BM - 1) / BM);
  int splits = 1;
  while (tiles * splits * 2 <= 256 && splits < 8) splits *= 2;
  return gemm_grid(M, N, K, splits).splits;
}

SplitKNeed gemm_mfma_workspace(int M, int N, int K, int splits) {
  const GemmGrid g = gemm_grid(M, N, K, splits);
  SplitKNeed need;
  need.splits = (int)g.splits;
  const size_t tiles = (size_t)g.tn * g.tm;
  need.partial_floats = g.splits > 1 ? tiles * g.splits * TILE_ELEMS : 0;
  need.counters = g.splits > 1 ? tiles : 0;
  return need;
}

bool gemm_mfma_fits(int M, int N, int K) {
  // 32-bit buffer offsets within one tile's rows of X and of W.
  const int64_t row_bytes = (int64_t)(K / kBlockElems) * kBlockBytes;
  (void)M;
  (void)N;
  return (int64_t)BM * K * 4 < (int64_t(1) << 31) && (int64_t)BN * row_bytes < (int64_t(1) << 31);
}

hipError_t launch_gemm_mfma(const float* x, const uint8_t* w, const float* bias, float* y,
                            int M, int N, int K, int splits, const SplitKWorkspace& ws,
                            hipStream_t stream) {
  if (!gemm_mfma_fits(M, N, K)) return hipErrorInvalidValue;
  const GemmGrid g = gemm_grid(M, N, K, splits);
  hipLaunchKernelGGL(gemm_q8_0_mfma_kernel, dim3(g.tn, g.tm, g.splits), dim3(256), 0, stream,
                     x, w, bias, y, M, N, K, g.steps_per_split, ws.partials, ws.counters);
  return hipGetLastError();
}

}  // namespace mle
