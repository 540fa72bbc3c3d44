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
// Two kernels (from 64 rows of A the MatMul runs the bf16 MFMA GEMM instead):
//   * M <= 8: the half-block kernel below, lanes reading 16-byte pieces of whole
//     blocks along a B row;
//   * 9 <= M < 64: the column-quad kernel.  A workgroup owns a tile of 256 output
//     columns (8 blocks of a B row: lane l of every wave takes columns 4l .. 4l+3)
//     for MR token rows, and a run of 256-row K slices.  Its 16 waves take 16
//     consecutive rows of each slice each, issue all 16 rows' loads (the block
//     scale and the lane's 4 quants, as 2-byte loads) before using any, and fold
//     them into fp32 accumulators in row order; the activations of a row are
//     wave-uniform (scalar loads).  The 16 waves' sums are then added in LDS in
//     wave order.  When the column and token tiles alone leave the GPU's 256 CUs
//     short of work, the K slices are spread over S workgroups per tile: each
//     writes its partial tile to a workspace [S][M][N], and a second launch adds
//     the S partials of every output in fixed runs of slices.  B is read once per
//     MR token rows (MR = 8 at most).
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

// Half-block kernel (M <= 8).  A workgroup owns a tile of 256 output columns (8
// blocks of a B row) for MR token rows and a run of K.  Lane c of a 16-lane group
// takes 16 columns, half h = c % 2 of block c / 2 of the tile, of one B row per
// step, so a group reads the tile's 272 contiguous bytes of a row and a wave four
// rows.  Per row a lane issues one 16-byte load and one 2-byte load, both inside
// its block:
//   h = 0, block 4-aligned: 16 bytes at the block (scale, q0 .. q13), 2 at +16;
//   h = 0, block 2 mod 4:   16 bytes at +2 (q0 .. q15), the scale at +0;
//   h = 1, block 4-aligned: 16 bytes at +16 (q14 .. q29), 2 at +32 (q30, q31);
//   h = 1, block 2 mod 4:   16 bytes at +18 (q16 .. q31), 2 at +16 (not used);
// and the h = 1 lane takes the scale from its h = 0 neighbour.  Loads go through
// buffer resources, so rows of B past K and activations past M or K read as
// zeros.  A lane issues the loads of U rows (a batch) and of their MR activations
// each before using any.  Values are formed as the reference forms them,
// v = d * q in fp32 (exact: an 11-bit by 8-bit significand product), and folded
// into per-token fp32 accumulators, acc = fma(a, v, acc).  The
// workgroup's 32 row phases (8 waves x 4 rows) are then added in LDS in a fixed
// order, one token at a time.  When K is spread over S workgroups per tile, each
// stores its sums to the workspace by device-scope stores, waits for their
// completion and bumps the tile's counter; the last to arrive resets the counter
// and adds the S partials of every output in fixed runs of consecutive splits, the
// runs' sums in run order (deterministic).
constexpr int kLnWaves = 8;                              // waves per workgroup
constexpr int kLnNT = 64 * kLnWaves;
constexpr int kLnLanes = 16;                             // lanes per B row
constexpr int kLnRows = 64 / kLnLanes;                   // B rows per wave step
constexpr int kLnCols = kLnLanes / 2 * kBlockElems;      // 256 columns per tile
constexpr int kLnMaxSplits = 64;

struct LnGrid {
  unsigned col_tiles, row_tiles, splits;
  int batches_per_split, mr, unroll;
};

LnGrid ln_grid(int M, int N, int K) {
  LnGrid g;
  const int NB = N / kBlockElems;
  g.mr = M >= 8 ? 8 : M >= 4 ? 4 : M >= 2 ? 2 : 1;
  g.unroll = g.mr >= 4 ? 4 : 8;  // 16 MR accumulators + 5 U load registers per lane
  g.col_tiles = (unsigned)((NB + kLnLanes / 2 - 1) / (kLnLanes / 2));
  g.row_tiles = (unsigned)((M + g.mr - 1) / g.mr);
  const int batch = g.unroll * kLnWaves * kLnRows;
  const int batches = (K + batch - 1) / batch;
  const int64_t tiles = (int64_t)g.col_tiles * g.row_tiles;
  int s = (int)((512 + tiles - 1) / tiles);  // about two workgroups per CU
  if (s > batches) s = batches;
  if (s > kLnMaxSplits) s = kLnMaxSplits;
  if (s < 1) s = 1;
  g.batches_per_split = (batches + s - 1) / s;
  g.splits = (unsigned)((batches + g.batches_per_split - 1) / g.batches_per_split);
  return g;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t mm_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

template <int MR, int U>
__global__ __launch_bounds__(kLnNT) void matmul_q8_0_half_kernel(
    const float* __restrict__ a, const uint8_t* __restrict__ b, float* __restrict__ c,
    int M, int N, int K, int batches_per_split, float* __restrict__ partials,
    uint32_t* __restrict__ counters) {
  constexpr int BATCH = U * kLnWaves * kLnRows;  // B rows per batch
  constexpr int SC1 = 16;                        // cache-policy bit: device scope
  __shared__ __attribute__((aligned(16))) float red[kLnWaves * 64 * 16];
  __shared__ uint32_t arrived;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane % kLnLanes, rsub = lane / kLnLanes, h = c16 & 1;
  const int NB = N / kBlockElems;
  const uint32_t row_bytes = (uint32_t)NB * kBlockBytes;
  const int jb = blockIdx.x * (kLnLanes / 2) + (c16 >> 1);
  const uint32_t cb = (uint32_t)(jb < NB ? jb : NB - 1) * kBlockBytes;  // columns past N: dead
  // A lane's rows all have the parity of rsub, so its blocks' 4-byte phase is fixed.
  const uint32_t mis =
      (uint32_t)(((uintptr_t)b + cb + ((rsub & 1) ? row_bytes : 0u)) & 2u);
  const uint32_t offx = cb + 16 * h + mis;
  const uint32_t offu = cb + 16 * h + (mis ? 0u : 16u);
  // Buffer resources: B rows past K and A entries past M or K read as zeros.
  const __amdgpu_buffer_rsrc_t brs = mm_rsrc(b, (uint32_t)K * row_bytes);
  const __amdgpu_buffer_rsrc_t ars = mm_rsrc(a, (uint32_t)M * (uint32_t)K * 4u);
  const int m0 = blockIdx.z * MR;
  const int nbatches = (K + BATCH - 1) / BATCH;
  const int bt0 = blockIdx.y * batches_per_split;
  const int bt1 = min(bt0 + batches_per_split, nbatches);

  float acc[MR][16];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[r][i] = 0.0f;

  // One batch: U rows of B per lane (16 + 2 bytes each) and their activations.
  // The 2-byte loads stay 16 bits wide until used, so no instruction placed with
  // the loads waits for them.
  struct Batch {
    u32x4 q4[U];
    uint16_t u2[U];
    float x[U][MR];
  };
  auto load = [&](Batch& t, int bt) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = bt * BATCH + (u * kLnWaves + wave) * kLnRows + rsub;
      const bool kv = k < K;
      const uint32_t ro = kv ? (uint32_t)k * row_bytes : 0x80000000u;
      t.q4[u] = __builtin_amdgcn_raw_buffer_load_b128(brs, ro + offx, 0, 0);
      t.u2[u] = __builtin_amdgcn_raw_buffer_load_b16(brs, ro + offu, 0, 0);
#pragma unroll
      for (int r = 0; r < MR; ++r)
        t.x[u][r] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(
                       ars, kv && m0 + r < M ? ((uint32_t)(m0 + r) * (uint32_t)K + k) * 4u
                                             : 0x80000000u,
                       0, 0));
    }
  };
  auto consume = [&](const Batch& t) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t w[5] = {t.q4[u].x, t.q4[u].y, t.q4[u].z, t.q4[u].w, (uint32_t)t.u2[u]};
      uint32_t q[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) q[i] = mis ? w[i] : __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
      const uint32_t own = mis ? w[4] : (w[0] & 0xffffu);  // the scale, on h = 0 lanes
      const uint32_t other = (uint32_t)__shfl_xor((int)own, 1);
      const float d = scale_to_f32(h ? other : own);
      float v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = d * q_at(q[i >> 2], i & 3);
#pragma unroll
      for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[r][i] = __builtin_fmaf(t.x[u][r], v[i], acc[r][i]);
    }
  };

  // Every load of a batch is issued before the first use of any.  (Issuing the
  // next batch's loads before using the current one, in a second register set,
  // measured no faster: the extra registers halve the workgroups per CU.)
  for (int bt = bt0; bt < bt1; ++bt) {
    Batch t;
    load(t, bt);
    __builtin_amdgcn_sched_barrier(0);
    consume(t);
  }

  // Per token: every lane's 16 sums to LDS, then each column's 32 row-phase sums in
  // (wave, row) order.
  const unsigned tile = blockIdx.z * gridDim.x + blockIdx.x;
  const int n = blockIdx.x * kLnCols + (tid % kLnCols);
  const bool split = gridDim.y > 1;
  const uint32_t region = MR * kLnCols;  // floats of one workgroup's partial sums
  const __amdgpu_buffer_rsrc_t prs =
      mm_rsrc(partials, split ? (uint32_t)((tile + 1) * gridDim.y * region * 4) : 0u);
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    float* mine = red + (wave * 64 + lane) * 16;
#pragma unroll
    for (int i = 0; i < 16; i += 4)
      *reinterpret_cast<f32x4*>(mine + i) = f32x4{acc[r][i], acc[r][i + 1], acc[r][i + 2],
                                                  acc[r][i + 3]};
    __syncthreads();
    if (tid < kLnCols) {
      const int cc = tid / 16, i = tid % 16;  // lane of the group, column within its half
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < kLnWaves; ++w)
#pragma unroll
        for (int p = 0; p < kLnRows; ++p) s += red[(w * 64 + p * kLnLanes + cc) * 16 + i];
      const int m = m0 + r;
      if (!split) {
        if (m < M && n < N) c[(int64_t)m * N + n] = s;
      } else {
        __builtin_amdgcn_raw_buffer_store_b32(
            __builtin_bit_cast(uint32_t, s), prs,
            (uint32_t)(((tile * gridDim.y + blockIdx.y) * region + r * kLnCols + tid) * 4), 0,
            SC1);
      }
    }
    __syncthreads();
  }
  if (!split) return;

  uint32_t* const counter = counters + (size_t)tile * kCounterStride;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // every partial has reached the coherence point
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (tid == 0)
    arrived = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (arrived != gridDim.y - 1) return;
  if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // The last workgroup adds the S partials of every output: the region's 16-byte
  // pieces are split over the threads as (piece, run of consecutive splits); each
  // thread sums its run in split order with the loads of 8 splits issued together,
  // then the runs' sums of a piece are added in run order in LDS.
  constexpr int PIECES = MR * kLnCols / 4;
  constexpr int RUNS = kLnNT / PIECES;  // 8, 4, 2 or 1 for MR = 1, 2, 4, 8
  const unsigned nspl = gridDim.y, per = (nspl + RUNS - 1) / RUNS;
  const int pc = tid % PIECES, run = tid / PIECES;
  f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
  const unsigned s0 = run * per, s1 = min(nspl, s0 + per);
  for (unsigned sp = s0; sp < s1; sp += 8) {
    f32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      v[j] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     prs, sp + j < s1 ? (uint32_t)(((tile * nspl + sp + j) * region + 4 * pc) * 4)
                                      : 0x80000000u,
                     0, SC1));
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (sp + j < s1) sum += v[j];
  }
  f32x4* const runs = reinterpret_cast<f32x4*>(red);  // [RUNS][PIECES]
  runs[run * PIECES + pc] = sum;
  __syncthreads();
  if (run == 0) {
    f32x4 t = runs[pc];
    for (int q = 1; q < RUNS; ++q) t += runs[q * PIECES + pc];
    const int r = (4 * pc) / kLnCols, m = m0 + r;
    const int nn = blockIdx.x * kLnCols + (4 * pc) % kLnCols;  // N % 32 == 0: 4 columns in or out
    if (m < M && nn < N) *reinterpret_cast<f32x4*>(c + (int64_t)m * N + nn) = t;
  }
}

// out[m, n] = sum over s of part[s][m][n], four columns a thread: the splits are
// taken in kSpGroups runs of consecutive splits, each run summed in split order by
// its own thread (their loads in flight together), and the runs' sums added in run
// order, so the grouping is fixed and the result deterministic.
constexpr int kSpGroups = 8;
constexpr int kSpCols = 256 / kSpGroups;  // float4 columns per workgroup

__global__ __launch_bounds__(256) void matmul_splits_kernel(const float* __restrict__ part,
                                                           float* __restrict__ c, int64_t mn4,
                                                           int splits) {
  __shared__ f32x4 run[kSpGroups][kSpCols];
  const int col = threadIdx.x % kSpCols, g = threadIdx.x / kSpCols;
  const int64_t i = (int64_t)blockIdx.x * kSpCols + col;
  const int per = (splits + kSpGroups - 1) / kSpGroups;
  const int s0 = g * per, s1 = min(s0 + per, splits);
  const f32x4* p = reinterpret_cast<const f32x4*>(part);
  f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
  if (i < mn4 && s0 < s1) {
    s = p[(int64_t)s0 * mn4 + i];
#pragma unroll 8
    for (int sp = s0 + 1; sp < s1; ++sp) s += p[(int64_t)sp * mn4 + i];
  }
  run[g][col] = s;
  __syncthreads();
  if (g == 0 && i < mn4) {
    f32x4 t = run[0][col];
    for (int r = 1; r < kSpGroups && r * per < splits; ++r) t += run[r][col];
    reinterpret_cast<f32x4*>(c)[i] = t;
  }
}

template <int MR>
void launch_mm(const MmGrid& g, const float* a, const uint8_t* b, float* dst, int M, int N,
               int K, hipStream_t stream) {
  hipLaunchKernelGGL(matmul_q8_0_kernel<MR>, dim3(g.col_tiles, g.splits, g.row_tiles),
                     dim3(64 * kMmWaves), 0, stream, a, b, dst, M, N, K, g.slices_per_split);
}

template <int MR, int U>
void launch_ln(const LnGrid& g, const float* a, const uint8_t* b, float* c, int M, int N, int K,
               float* partials, uint32_t* counters, hipStream_t stream) {
  hipLaunchKernelGGL((matmul_q8_0_half_kernel<MR, U>), dim3(g.col_tiles, g.splits, g.row_tiles),
                     dim3(kLnNT), 0, stream, a, b, c, M, N, K, g.batches_per_split, partials,
                     counters);
}

// The half-block kernel takes M <= 8 (larger M keeps the column-quad kernel,
// which reads B once per 8 token rows as well) and B below 2 GiB (32-bit buffer
// offsets).
bool use_half(int M, int N, int K) {
  return M <= 8 && (int64_t)K * (N / kBlockElems) * kBlockBytes < (int64_t(1) << 31) &&
         (int64_t)M * K * 4 < (int64_t(1) << 31);
}

}  // namespace

MatmulNeed matmul_workspace(int M, int N, int K) {
  MatmulNeed need;
  if (M <= 0 || N <= 0 || K <= 0) return need;
  if (use_half(M, N, K)) {
    const LnGrid g = ln_grid(M, N, K);
    if (g.splits > 1) {
      const size_t tiles = (size_t)g.col_tiles * g.row_tiles;
      need.partial_floats = tiles * g.splits * g.mr * kLnCols;
      need.counters = tiles * kCounterStride;
    }
    return need;
  }
  const MmGrid g = mm_grid(M, N, K, mm_rows_per_tile(M));
  if (g.splits > 1) need.partial_floats = (size_t)g.splits * M * N;
  return need;
}

hipError_t launch_matmul(const float* a, const uint8_t* b, float* c, int M, int N, int K,
                         float* partials, uint32_t* counters, hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) return hipSuccess;
  if (N % kBlockElems != 0 || K % kBlockElems != 0) return hipErrorInvalidValue;
  if (use_half(M, N, K)) {
    const LnGrid g = ln_grid(M, N, K);
    if (g.row_tiles > 65535 || g.splits > 65535) return hipErrorInvalidValue;
    if (g.splits > 1) {
      const int64_t bytes = (int64_t)g.col_tiles * g.row_tiles * g.splits * g.mr * kLnCols * 4;
      if (partials == nullptr || counters == nullptr || bytes >= (int64_t(1) << 32))
        return hipErrorInvalidValue;
    }
    switch (g.mr) {
      case 1: launch_ln<1, 8>(g, a, b, c, M, N, K, partials, counters, stream); break;
      case 2: launch_ln<2, 8>(g, a, b, c, M, N, K, partials, counters, stream); break;
      case 4: launch_ln<4, 4>(g, a, b, c, M, N, K, partials, counters, stream); break;
      default: launch_ln<8, 4>(g, a, b, c, M, N, K, partials, counters, stream); break;
    }
    return hipGetLastError();
  }
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
  hipLaunchKernelGGL(matmul_splits_kernel, dim3((unsigned)((mn4 + kSpCols - 1) / kSpCols)),
                     dim3(256), 0, stream, partials, c, mn4, (int)g.splits);
  return hipGetLastError();
}

}  // namespace mle
