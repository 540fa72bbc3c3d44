// gemm_mfma.hip -- Q8_0 Linear prefill GEMM on bf16 MFMA for gfx950.
//
// Y[M, N] = X[M, K] . W^T (+ bias), W in Q8_0 blocks along K.
// Same contract as cpu::sgemm_nt(const float*, const uint8_t*, ...)
// (src/runtime/kernels/cpu_kernels.cpp:208-218); used for M >= 64.
//
// Two launches:
//   1. x_to_frag: X (fp32) -> Xf (bf16, round to nearest even) in a workspace,
//      stored in MFMA A-fragment order (rows padded to 32, K to 64, with zeros).
//      X is re-read by every column tile of the GEMM: converting it once halves
//      those re-reads and takes the conversion off the GEMM's vector ALUs, and
//      the fragment order turns each A-fragment load into 1 KB of contiguous
//      memory (loading fragments from a row-major X spreads each load
//      instruction over 32 rows, which halves the L2->CU throughput).
//   2. the GEMM.  Workgroup tile BM x BN (BM = 128 MI, BN = 32 NJ), K step 64
//      (two Q8_0 blocks per W row), waves in two roles:
//        * CW consumer waves stacked along M: wave w owns rows
//          [32 MW w, 32 MW (w+1)) of the tile and all BN columns as MW x NJ
//          v_mfma_f32_32x32x16_bf16 accumulators.  128-row tiles: CW = 4,
//          MW = 1; 256-row tiles: CW = 8, MW = 1 (two consumer waves per SIMD,
//          so one's MFMAs cover the other's waits: 2-6% faster than 4 waves of
//          64 rows);
//        * 4 producer waves that load and dequantise W.
//      Each SIMD runs consumer and producer waves side by side, so the
//      producers' vector ALU work overlaps the consumers' MFMAs.
//
// Operands:
//   * A (X): each consumer wave loads its own rows' bf16 fragments straight from
//     the fragment-ordered copy into registers (no LDS; no row is read by two
//     waves).
//   * B (W): per K step, producer thread t < 2 BN takes one 34-byte block (row
//     t/2, block t%2 of the step), forms v = d * q in fp32 (exactly the
//     reference's element value), rounds it once to bf16 and writes the 32
//     values to an LDS tile that all consumer waves read.  Each W element is
//     thus dequantised once per workgroup, and one dequantised element feeds
//     2 BM flops.
//   The per-block scale is folded into B rather than applied to the accumulator
//   after every 32-wide K block: the latter costs one fp32 FMA per output per
//   block, i.e. one VALU op per 64 MFMA flops, which is the whole non-packed VALU
//   rate and would cap the MFMA pipe at about half its peak.  Error vs the fp32
//   reference is the bf16 rounding of both operands (relative L2 ~2e-3), inside
//   the 1e-2 bound stated for this path.
//
// K order inside a step: MFMA j (0..3) of a step gives lane half h (lanes 32h..)
// the eight K values 32 h + 8 j .. +7, i.e. half h walks block h of the step.  A
// and B use the same order, so the product is unchanged, and each W block is
// dequantised by a single thread into contiguous LDS.
//
// Software pipeline, one barrier per pair of K steps (halving the barriers
// measured 3-5% faster than one per step; four per barrier was slower):
//   * consumers keep X in a ring of three register stages, loading X(t+2)
//     before the MFMAs of step t; the pair (t, t+1) reads its bf16 W from the
//     two halves of LDS buffer p;
//   * producers keep raw W blocks in a ring of eight, and during pair (t, t+1)
//     dequantise W(t+2), W(t+3) into the other buffer while loading W(t+8),
//     W(t+9).
// Every load is unconditional: rows past M or N and blocks past K read as zero
// through the buffer range check, and steps past the end re-read the last step.
//
// MatMul (LAYOUT kKN): the same GEMM with B[K, N] in Q8_0 blocks along N
// (cpu::sgemm, src/runtime/kernels/cpu_kernels.cpp:116-130).  A 34-byte block
// then holds 32 consecutive columns of one K row, so producer item (k pair kp,
// block column c) loads the blocks of rows 2 kp and 2 kp + 1 of the step in
// column block c and writes their 32 columns transposed into the W tile, one
// dword (the bf16 values of both rows) per column.  The consumers, the K order
// and the epilogue are the Linear's.
//
// Split K (gridDim.z > 1, for shapes with too few tiles to fill the GPU): each
// workgroup stores its BM x BN fp32 partial tile with device-scope (sc1)
// stores, waits for their completion and bumps a per-tile counter; the last
// workgroup of the tile adds the partials in split order (deterministic), adds
// the bias, writes Y and resets the counter for the next launch.
#include "../launch.hpp"
#include "../q8_0_device.hpp"

#include <type_traits>

namespace mle {
namespace {

constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row of the W tile (144 bytes)

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t cvt_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

int padded_k(int K) { return (K + BK - 1) / BK * BK; }

// X fp32 [M, K] -> Xf: bf16 (round to nearest even) in MFMA fragment order.
// Piece p (16 bytes = 8 bf16) is lane p % 64 of fragment f = p / 64, with
// f = (R * n_steps + s) * 4 + j: rows 32 R + lane % 32, K values
// 64 s + 32 (lane / 32) + 8 j .. +7.  Rows >= M and K values >= K are zero.  A
// GEMM wave then loads one whole A fragment as 1 KB of contiguous memory.
//
// One workgroup converts one (32-row tile R, K step s): 256 threads read the
// 32 x 64 fp32 tile row by row (8 threads per 256-byte row piece: coalesced),
// round to bf16 into LDS, then each thread writes one 16-byte piece of the four
// 1 KB fragments (coalesced).
__global__ __launch_bounds__(256) void x_to_frag_kernel(const float* __restrict__ x,
                                                        u32x4* __restrict__ xf, int M, int K,
                                                        int n_steps) {
  __shared__ u32x4 tile[32][9];  // [row][8-value chunk], padded against bank conflicts
  const int tid = threadIdx.x;
  const int R = blockIdx.y, s = blockIdx.x;
  {
    const int r = tid >> 3, c8 = tid & 7;
    const int64_t m = (int64_t)R * 32 + r;
    const int k = s * 64 + 8 * c8;
    u32x4 out = {0u, 0u, 0u, 0u};
    if (m < M && k < K) {  // K % 8 == 0: the 8 values are all inside or all outside
      const f32x4 a = *reinterpret_cast<const f32x4*>(x + m * K + k);
      const f32x4 b = *reinterpret_cast<const f32x4*>(x + m * K + k + 4);
      out = u32x4{cvt_bf16x2(a.x, a.y), cvt_bf16x2(a.z, a.w), cvt_bf16x2(b.x, b.y),
                  cvt_bf16x2(b.z, b.w)};
    }
    tile[r][c8] = out;
  }
  __syncthreads();
  const int j = tid >> 6, lane = tid & 63;
  xf[((int64_t)((int64_t)R * n_steps + s) * 4 + j) * 64 + lane] = tile[lane & 31][4 * (lane >> 5) + j];
}

// X fragments of one K step held by one consumer lane.
template <int MI>
struct XStage {
  u32x4 x[MI][4];
};

// Consumer (MFMA) waves: 8 for 256-row tiles (two per SIMD, 32 rows each), else
// 4; plus 4 producer (W) waves.
template <int MI>
struct Roles {
  static constexpr int CW = MI == 2 ? 8 : 4;
  static constexpr int MW = MI * 4 / CW;
  static constexpr int kThreads = 64 * (CW + 4);
};

// Output segments as the kernel sees them: segment i owns the column tiles
// [tile_end[i-1], tile_end[i]) of the grid.
struct GemmArgs {
  LinearSeg seg[3];
  unsigned tile_end[3];
  int count;
};

// silu(g) * u with the reference's operation order (cpu_kernels.cpp:848-858).
__device__ __forceinline__ float silu_mul(float g, float u) {
  return (g / (1.0f + expf(-g))) * u;
}

// MODE 0: plain / multi-output Linear.  MODE 1 (SwiGLU): tile columns
// [0, BN/2) are rows of the gate weight and [BN/2, BN) the same rows of the up
// weight; producer waves 0-1 dequantise the gate rows and 2-3 the up rows, so
// each wave reads one weight; the epilogue writes silu(gate) * up for BN/2
// output columns.
template <int MI, int NJ, int MODE, int LAYOUT>
__global__ __launch_bounds__(Roles<MI>::kThreads, 1) void gemm_q8_0_mfma_kernel(
    const u32x4* __restrict__ xf, uint32_t xf_bytes, const GemmArgs args, int M, int K,
    int steps_per_split, float* __restrict__ partials, uint32_t* __restrict__ counters) {
  constexpr int BM = 128 * MI;
  constexpr int CW = Roles<MI>::CW, MW = Roles<MI>::MW;  // consumer waves, 32-row blocks each
  constexpr int BN = 32 * NJ;
  constexpr bool kSwi = MODE == 1;
  constexpr int BNO = kSwi ? BN / 2 : BN;  // output columns per tile
  // SwiGLU: two producer waves (128 threads) cover each weight's 2 BNO blocks per step.
  static_assert(!kSwi || (BNO <= 64 && BNO % 4 == 0), "SwiGLU tiles need BN <= 128");
  constexpr int NBLK = 2 * BN;  // W blocks per K step (<= 256 producer threads)
  constexpr int TILE_ELEMS = BM * BN;
  constexpr int BUF = BN * LDS_STRIDE;
  // X register stages per consumer lane (32 MW VGPRs each).
  constexpr int XS = 3;
  __shared__ __attribute__((aligned(16))) uint16_t Bs[4 * BUF];  // 2 buffers x 2 steps
  __shared__ uint32_t arrived;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const bool consumer = wave < CW;  // wave-uniform role
  const int cw = wave;              // consumer wave: rows 32 MW cw .. of the tile
  const int pt = tid - 64 * CW;     // producer thread: W block pt of each step
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  // Segment of this column tile (uniform selects: no indexing into the argument).
  const unsigned tile = blockIdx.x;
  const int si = (!kSwi && args.count > 1 && tile >= args.tile_end[0])
                     ? ((args.count > 2 && tile >= args.tile_end[1]) ? 2 : 1)
                     : 0;
  const unsigned tile0 = si == 0 ? 0u : si == 1 ? args.tile_end[0] : args.tile_end[1];
  const uint8_t* w = si == 0 ? args.seg[0].w : si == 1 ? args.seg[1].w : args.seg[2].w;
  const void* bias = si == 0 ? args.seg[0].bias : si == 1 ? args.seg[1].bias : args.seg[2].bias;
  const int bias_bf16 =
      si == 0 ? args.seg[0].bias_bf16 : si == 1 ? args.seg[1].bias_bf16 : args.seg[2].bias_bf16;
  float* y = si == 0 ? args.seg[0].y : si == 1 ? args.seg[1].y : args.seg[2].y;
  const int N = si == 0 ? args.seg[0].N : si == 1 ? args.seg[1].N : args.seg[2].N;
  const int64_t n0 = (int64_t)(tile - tile0) * BNO;
  const int KB = K / kBlockElems;
  const uint32_t row_bytes = (uint32_t)KB * kBlockBytes;
  const int n_steps = (K + BK - 1) / BK;
  const int s_begin = blockIdx.z * steps_per_split;
  const int s_end = min(s_begin + steps_per_split, n_steps);
  const int s_last = s_end - 1;

  // Epilogue (consumer waves store; every wave takes part in the barriers).
  // D[i][jj] of lane l holds rows 4 (l/32) + v%4 + 8 (v/4), column l%32, i.e.
  // four rows of one column per register quad: storing that directly takes one
  // 4-byte store per value.  Instead each consumer wave stages 16-row chunks of
  // its 32 MW x BN tile in its own part of the (now idle) W buffers and writes
  // them back as 16-byte pieces of contiguous rows (bias added on the way), as
  // non-temporal stores: Y is not read again here, and every workgroup writes
  // its tile at the same time at the end, so keeping Y out of L2 leaves it to
  // the other workgroups' W and X lines (2-6% faster on the Llama prefill
  // shapes, MI355X).
  const int wm = cw * 32 * MW;
  constexpr int EP_STRIDE = BN + 4;  // floats per staged row: 16-byte rows, banks spread
  static_assert(CW * 16 * EP_STRIDE * 4 <= 4 * BUF * 2, "epilogue staging exceeds LDS");
  auto store_tile = [&](auto role, const f32x16 (&v)[MW][NJ]) {
    constexpr bool kConsumer = decltype(role)::value;
    float* ep = reinterpret_cast<float*>(Bs) + cw * 16 * EP_STRIDE;
    const bool vec = (N & 3) == 0;
#pragma unroll
    for (int c = 0; c < 2 * MW; ++c) {  // rows 16 c .. 16 c + 15 of this wave's rows
      const int i = c >> 1, h = c & 1;
      __syncthreads();  // the previous reads of this staging area are done
      if constexpr (kConsumer) {
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
          for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              ep[(4 * (lane >> 5) + e + 8 * q) * EP_STRIDE + 32 * jj + (lane & 31)] =
                  v[i][jj][4 * (2 * h + q) + e];
      }
      __syncthreads();
      if constexpr (!kConsumer) continue;
      constexpr int PER_ROW = BNO / 4;
#pragma unroll
      for (int u = 0; u < (16 * PER_ROW + 63) / 64; ++u) {
        const int idx = lane + 64 * u;
        if (16 * PER_ROW % 64 != 0 && idx >= 16 * PER_ROW) continue;
        const int rr = idx / PER_ROW, c4 = idx % PER_ROW;
        f32x4 val = *reinterpret_cast<const f32x4*>(ep + rr * EP_STRIDE + 4 * c4);
        if constexpr (kSwi) {
          const f32x4 up = *reinterpret_cast<const f32x4*>(ep + rr * EP_STRIDE + BNO + 4 * c4);
          val = f32x4{silu_mul(val.x, up.x), silu_mul(val.y, up.y), silu_mul(val.z, up.z),
                      silu_mul(val.w, up.w)};
        }
        const int64_t m = m0 + wm + 16 * c + rr;
        const int64_t n = n0 + 4 * c4;
        if (m >= M) continue;
        if (vec) {
          if (n >= N) continue;
          if (bias)
            val += f32x4{bias_at(bias, bias_bf16, n), bias_at(bias, bias_bf16, n + 1),
                         bias_at(bias, bias_bf16, n + 2), bias_at(bias, bias_bf16, n + 3)};
          __builtin_nontemporal_store(val, reinterpret_cast<f32x4*>(y + m * N + n));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < N) y[m * N + n + e] = val[e] + (bias ? bias_at(bias, bias_bf16, n + e) : 0.0f);
        }
      }
    }
  };
  auto finish = [&](auto role, f32x16 (&acc)[MW][NJ]) {
  constexpr bool kConsumer = decltype(role)::value;
  if (gridDim.z == 1) {
    store_tile(role, acc);
    return;
  }

  // Split K: partial tile [tile][split][TILE_ELEMS] by device-scope stores; the
  // last workgroup of the tile reduces in split order.  Partials are stored
  // lane-major (slot (i, jj, quad) x 256 consumer threads x 16 bytes), so each
  // store instruction writes 4 KB contiguously and the reader finds its own slots.
  constexpr int SC1 = 16;  // cache-policy bit: device scope
  const uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x;
  const __amdgpu_buffer_rsrc_t prs =
      rsrc(partials + (int64_t)tile * gridDim.z * TILE_ELEMS, gridDim.z * TILE_ELEMS * 4u);
  auto slot = [&](int i, int jj, int q) {  // byte offset of 4 accumulators
    return (uint32_t)((((i * NJ + jj) * 4 + q) * (64 * CW) + tid) * 16);
  };
  if constexpr (kConsumer) {
#pragma unroll
    for (int i = 0; i < MW; ++i)
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = f32x4{acc[i][jj][4 * q + 0], acc[i][jj][4 * q + 1],
                                acc[i][jj][4 * q + 2], acc[i][jj][4 * q + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs,
                                                 blockIdx.z * TILE_ELEMS * 4u + slot(i, jj, q),
                                                 0, SC1);
        }
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
  if constexpr (kConsumer) {
#pragma unroll
    for (int i = 0; i < MW; ++i)
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) {
        f32x4 sum[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) sum[q] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (unsigned sp = 0; sp < gridDim.z; ++sp)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            sum[q] += __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           prs, sp * TILE_ELEMS * 4u + slot(i, jj, q), 0, SC1));
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][jj][v] = sum[v >> 2][v & 3];
      }
  }
  if (tid == 0)
    __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  store_tile(role, acc);
  };


  // Both roles run the same number of iterations, each ending in one barrier:
  // iteration t publishes the bf16 W tile of step t+1 (producers) and retires
  // the MFMAs of step t (consumers), which read LDS buffer (t - s_begin) % 2.
  if (consumer) {
    f32x16 acc[MW][NJ];
#pragma unroll
    for (int i = 0; i < MW; ++i)
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][jj][v] = 0.0f;
    // A: fragments of 32-row tile R at step s start at byte ((R n_steps + s) 4
    // + j) KB; tiles past the converted rows read as zero.
    const __amdgpu_buffer_rsrc_t xrs = rsrc(xf, xf_bytes);
    uint32_t xoff[MW];
#pragma unroll
    for (int i = 0; i < MW; ++i)
      xoff[i] = (uint32_t)((m0 / 32 + cw * MW + i) * n_steps) * 4096u + lane * 16u;
    auto load_x = [&](int s, XStage<MW>& st) {
      const uint32_t sx = (uint32_t)min(s, s_last) * 4096u;
#pragma unroll
      for (int i = 0; i < MW; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          st.x[i][j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[i] + 1024 * j, sx, 0);
    };
    // B fragment of lane (c, h) for MFMA j: row 32 jj + c, K values 32 h + 8 j .. +7.
    const int boff_lds = (lane & 31) * LDS_STRIDE + 32 * (lane >> 5);
    auto mfma_step = [&](const uint16_t* bs, const XStage<MW>& st) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16x8 bf[NJ];
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj)
          bf[jj] = *reinterpret_cast<const bf16x8*>(bs + jj * 32 * LDS_STRIDE + boff_lds + 8 * j);
#pragma unroll
        for (int i = 0; i < MW; ++i) {
          const bf16x8 a = __builtin_bit_cast(bf16x8, st.x[i][j]);
#pragma unroll
          for (int jj = 0; jj < NJ; ++jj)
            acc[i][jj] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bf[jj], acc[i][jj], 0, 0, 0);
        }
      }
    };
    // Ring of XS register stages: slot (s - s_begin) % XS holds X of step s,
    // loaded XS - 1 iterations before its MFMAs.
    // One barrier per pair of K steps: buffer p holds the bf16 W of steps
    // (t, t + 1) of the current pair in its halves.
    static_assert(XS == 3, "pair loop unrolls by lcm(2, XS) = 6 steps");
    XStage<MW> st[XS];
#pragma unroll
    for (int u = 0; u < XS - 1; ++u) load_x(s_begin + u, st[u]);
    __syncthreads();  // W of steps s_begin, s_begin + 1 are in buffer 0
    int p = 0;
    auto half = [&](int t, int u, int h) {  // u = (t - s_begin) % XS
      load_x(t + XS - 1, st[(u + XS - 1) % XS]);
      mfma_step(Bs + (2 * p + h) * BUF, st[u]);
    };
    auto pair = [&](int t, int u0) {
      half(t, u0, 0);
      if (t + 1 < s_end) half(t + 1, (u0 + 1) % XS, 1);
      __syncthreads();
      p ^= 1;
    };
    int t = s_begin;
    for (; t + 6 <= s_end; t += 6) {
      pair(t, 0);
      pair(t + 2, 2);
      pair(t + 4, 1);
    }
    if (t < s_end) pair(t, 0);
    if (t + 2 < s_end) pair(t + 2, 2);
    if (t + 4 < s_end) pair(t + 4, 1);
    finish(std::true_type{}, acc);
  } else {
    // B: buffer over this tile's rows of W; rows past N read as zero.  Thread pt
    // loads block (2 s + h) of row n every step s; the block's 2-byte alignment
    // phase is the same for every step (a step advances 68 bytes).
    // Item (row, block) of this thread within its weight.  Plain: items
    // pt < 2 BN.  SwiGLU: producer waves 0-1 take the gate items, 2-3 the up
    // items (tile rows BNO + row), so the weight is uniform per wave.
    const int pwave = __builtin_amdgcn_readfirstlane(wave) - CW;
    const bool up_rows = kSwi && pwave >= 2;
    const int item = kSwi ? (pwave & 1) * 64 + lane : pt;
    const int prow = item >> 1, wn_h = item & 1;  // row within its weight, block of the step
    constexpr bool kKN = LAYOUT == int(WeightLayout::kKN);
    // MatMul items: 32 k pairs x NJ column blocks.
    const int kn_c = pt >> 5, kn_kp = pt & 31;
    const bool w_thread = kKN ? pt < 32 * NJ : kSwi ? prow < BNO : (NBLK == 256 || pt < NBLK);
    const int wn_row = (up_rows ? BNO : 0) + prow;  // tile row
    const uint8_t* wsrc = up_rows ? args.seg[1].w : w;
    const int64_t wrows = min((int64_t)BNO, (int64_t)N - n0);
    const uint8_t* wtile = wsrc + n0 * row_bytes;
    const __amdgpu_buffer_rsrc_t wrs = rsrc(wtile, (uint32_t)(wrows * row_bytes));
    const uint32_t boff = (uint32_t)prow * row_bytes + (uint32_t)wn_h * kBlockBytes;
    // MatMul: B row k holds NB = N / 32 blocks; the item's blocks are column
    // block n0 / 32 + kn_c of rows 64 s + 2 kn_kp and + 1.  Rows past K read as
    // zero through the range check, column blocks past N are masked.
    const int NBK = N / kBlockElems;
    const uint32_t kn_row = (uint32_t)NBK * kBlockBytes;
    const __amdgpu_buffer_rsrc_t knrs = rsrc(wsrc, (uint32_t)((int64_t)K * kn_row));
    const bool kn_live = n0 / kBlockElems + kn_c < NBK;
    const uint32_t kn_off = (uint32_t)(2 * kn_kp) * kn_row + (uint32_t)(n0 / kBlockElems + kn_c) * kBlockBytes;
    const uint32_t kn_mis0 = (uint32_t)(((uintptr_t)wsrc + kn_off) & 2u);
    const uint32_t kn_mis1 = (uint32_t)(((uintptr_t)wsrc + kn_off + kn_row) & 2u);
    const uint32_t wmis = (uint32_t)(((uintptr_t)wtile + boff) & 2u);
    const uint32_t wv8 = boff + wmis;
    const uint32_t wv2 = boff + (wmis ? 0u : 32u);
    // Tiled weights (LAYOUT 1): the tile's rows are whole 16-row groups
    // [n0/16, n0/16 + BNO/16) of quant pieces (1 KB per group and K step) and
    // scale pieces (64 B).  Item (row, half j) reads the quant slots of lanes
    // 32 j + r and 32 j + 16 + r (r = row % 16): quants 16 j .. 16 j + 15 of
    // both blocks of the step, and the row's scale dword of the pair.
    constexpr bool kTiled = LAYOUT == int(WeightLayout::kTiled);
    const int KP = (KB + 1) >> 1;
    const int64_t G = ((int64_t)N + kTileRows - 1) / kTileRows;
    const int64_t g0 = n0 / kTileRows;
    const int64_t ngr = min((int64_t)(BNO / kTileRows), G - g0);
    const uint8_t* tq_base = wsrc + g0 * KP * kTilePieceBytes;
    const uint8_t* ts_base = wsrc + G * KP * kTilePieceBytes + g0 * KP * kTileScaleBytes;
    const __amdgpu_buffer_rsrc_t tqrs = rsrc(tq_base, (uint32_t)(ngr * KP * kTilePieceBytes));
    const __amdgpu_buffer_rsrc_t tsrs = rsrc(ts_base, (uint32_t)(ngr * KP * kTileScaleBytes));
    const uint32_t tqv = (uint32_t)(prow / kTileRows) * KP * kTilePieceBytes +
                         (uint32_t)(32 * wn_h + prow % kTileRows) * 16;
    const uint32_t tsv = (uint32_t)(prow / kTileRows) * KP * kTileScaleBytes +
                         (uint32_t)(prow % kTileRows) * 4;
    // Steps s with block 2 s + h < KB (none for threads without a W block,
    // whose loads are then all masked); tiled: every pair (the block past an
    // odd K/32 is zero in the tiled tensor).
    const int w_steps = w_thread ? (kKN ? (kn_live ? n_steps : 0)
                                         : kTiled ? KP : (KB - wn_h + 1) >> 1)
                                 : 0;
    struct TiledW {
      u32x4 a, b;  // quant slots 32 j + r, 32 j + 16 + r
      uint32_t sc;  // scales of both blocks
    };
    struct KNPair {
      RawBlock r0, r1;  // rows 2 kp and 2 kp + 1 of the step, one column block
    };
    using WItem = std::conditional_t<kTiled, TiledW, std::conditional_t<kKN, KNPair, RawBlock>>;
    auto load_kn = [&](uint32_t off, uint32_t mis, uint32_t so, bool live, RawBlock& r) {
      const uint32_t v8 = live ? off + mis : 0x80000000u;
      const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(knrs, v8, so, 0);
      const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(knrs, v8 + 16, so, 0);
      r.v0 = u32x4_a4{a.x, a.y, a.z, a.w};
      r.v1 = u32x4_a4{b.x, b.y, b.z, b.w};
      r.u = __builtin_amdgcn_raw_buffer_load_b16(
          knrs, live ? off + (mis ? 0u : 32u) : 0x80000000u, so, 0);
      r.mis = mis;
    };
    auto load_w = [&](int s, WItem& r) {
      s = min(s, s_last);
      const bool live = s < w_steps;
      if constexpr (kKN) {
        const uint32_t so = (uint32_t)s * (uint32_t)BK * kn_row;  // 64 rows of B per step
        load_kn(kn_off, kn_mis0, so, live, r.r0);
        load_kn(kn_off + kn_row, kn_mis1, so, live, r.r1);
      } else if constexpr (kTiled) {
        const uint32_t sq = (uint32_t)s * kTilePieceBytes;
        r.a = __builtin_amdgcn_raw_buffer_load_b128(tqrs, live ? tqv : 0x80000000u, sq, 0);
        r.b = __builtin_amdgcn_raw_buffer_load_b128(tqrs, live ? tqv + 256 : 0x80000000u, sq, 0);
        r.sc = __builtin_amdgcn_raw_buffer_load_b32(tsrs, live ? tsv : 0x80000000u,
                                                    (uint32_t)s * kTileScaleBytes, 0);
      } else {
        const uint32_t so = (uint32_t)s * (2 * kBlockBytes);
        const uint32_t v8 = live ? wv8 : 0x80000000u;
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8, so, 0);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8 + 16, so, 0);
        r.v0 = u32x4_a4{a.x, a.y, a.z, a.w};
        r.v1 = u32x4_a4{b.x, b.y, b.z, b.w};
        r.u = __builtin_amdgcn_raw_buffer_load_b16(wrs, live ? wv2 : 0x80000000u, so, 0);
        r.mis = wmis;
      }
    };
    auto dq8 = [](float d, uint32_t q0, uint32_t q1) {
      return u32x4{cvt_bf16x2(d * q_at(q0, 0), d * q_at(q0, 1)),
                   cvt_bf16x2(d * q_at(q0, 2), d * q_at(q0, 3)),
                   cvt_bf16x2(d * q_at(q1, 0), d * q_at(q1, 1)),
                   cvt_bf16x2(d * q_at(q1, 2), d * q_at(q1, 3))};
    };
    auto dequant = [&](const WItem& r, uint16_t* bs) {
      if (!w_thread) return;
      if constexpr (kKN) {
        // Column 32 kn_c + i of the tile, K values 2 kp and 2 kp + 1: one dword.
        const Block b0 = finish_block(r.r0), b1 = finish_block(r.r1);
        const float d0 = scale_to_f32_fast(b0.scale_bits), d1 = scale_to_f32_fast(b1.scale_bits);
        uint32_t* dst = reinterpret_cast<uint32_t*>(bs + 32 * kn_c * LDS_STRIDE + 2 * kn_kp);
#pragma unroll
        for (int i = 0; i < kBlockElems; ++i)
          dst[i * (LDS_STRIDE / 2)] =
              cvt_bf16x2(d0 * q_at(b0.q[i >> 2], i & 3), d1 * q_at(b1.q[i >> 2], i & 3));
      } else if constexpr (kTiled) {
        // Quants 16 j .. 16 j + 15 of block h go to elements 32 h + 16 j ..
        const float d0 = scale_to_f32_fast(r.sc & 0xffffu);
        const float d1 = scale_to_f32_fast(r.sc >> 16);
        u32x4* dst = reinterpret_cast<u32x4*>(bs + wn_row * LDS_STRIDE + 16 * wn_h);
        dst[0] = dq8(d0, r.a.x, r.a.y);
        dst[1] = dq8(d0, r.b.x, r.b.y);
        dst[4] = dq8(d1, r.a.z, r.a.w);
        dst[5] = dq8(d1, r.b.z, r.b.w);
      } else {
        const Block b = finish_block(r);
        const float d = scale_to_f32_fast(b.scale_bits);
        u32x4* dst = reinterpret_cast<u32x4*>(bs + wn_row * LDS_STRIDE + wn_h * kBlockElems);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = dq8(d, b.q[2 * i], b.q[2 * i + 1]);
      }
    };
    // Ring of 8 raw blocks: slot (s - s_begin) % 8 holds W of step s.  The pair
    // starting at step t dequantises W(t + 2), W(t + 3) into the other buffer.
    // The first two steps are requested alone and dequantised before the rest of
    // the ring goes out, so the first barrier does not wait behind six more loads
    // (0.97-0.99x the time of issuing all eight first, bit-identical results).
    constexpr int RING = kKN ? 4 : 8;
    WItem r[RING];
    load_w(s_begin, r[0]);
    load_w(s_begin + 1, r[1]);
    dequant(r[0], Bs);
    dequant(r[1], Bs + BUF);
#pragma unroll
    for (int u = 2; u < RING; ++u) load_w(s_begin + u, r[u]);
    __syncthreads();
    int p = 0;
    auto pair = [&](int t, int u0) {  // u0 = (t - s_begin) % RING
      load_w(t + RING, r[u0]);          // W(t), W(t + 1) are in LDS already
      load_w(t + RING + 1, r[u0 + 1]);
      dequant(r[(u0 + 2) % RING], Bs + (2 * (p ^ 1)) * BUF);
      dequant(r[(u0 + 3) % RING], Bs + (2 * (p ^ 1) + 1) * BUF);
      __syncthreads();
      p ^= 1;
    };
    int t = s_begin;
    for (; t + RING <= s_end; t += RING) {
#pragma unroll
      for (int u = 0; u < RING; u += 2) pair(t + u, u);
    }
#pragma unroll
    for (int u = 0; u < RING; u += 2)
      if (t + u < s_end) pair(t + u, u);
    f32x16 none[MW][NJ];  // never read: producers only join the barriers
    finish(std::false_type{}, none);
  }

}

struct GemmGrid {
  unsigned tn, tm, splits;
  int steps_per_split;
  GemmArgs args;
};

LinearSegs single_seg(const uint8_t* w, const float* bias, float* y, int N) {
  LinearSegs s;
  s.seg[0] = LinearSeg{w, bias, y, N};
  return s;
}

GemmGrid gemm_grid(const GemmConfig& c, int M, const LinearSegs& s, int K) {
  GemmGrid g{};
  const bool swi = s.mode == Epilogue::kSwiGLU;
  const int cols = swi ? c.bn / 2 : c.bn;
  const int count = swi ? 1 : s.count;
  unsigned end = 0;
  for (int i = 0; i < 3; ++i) {
    g.args.seg[i] = s.seg[i];
    if (i < count) end += (unsigned)((s.seg[i].N + cols - 1) / cols);
    g.args.tile_end[i] = end;
  }
  if (swi) g.args.seg[1].N = s.seg[0].N;
  g.args.count = count;
  g.tn = end;
  g.tm = (unsigned)((M + c.bm - 1) / c.bm);
  const int n_steps = padded_k(K) / BK;
  int splits = c.splits < 1 ? 1 : c.splits;
  if (splits > n_steps) splits = n_steps;
  g.steps_per_split = (n_steps + splits - 1) / splits;
  g.splits = (unsigned)((n_steps + g.steps_per_split - 1) / g.steps_per_split);
  return g;
}

template <int MI, int NJ, int L>
void launch_tile_l(const GemmGrid& g, Epilogue mode, const u32x4* xf, uint32_t xf_bytes, int M,
                   int K, const SplitKWorkspace& ws, hipStream_t stream) {
  const dim3 grid(g.tn, g.tm, g.splits);
  if constexpr (L == int(WeightLayout::kKN)) {  // MatMul: plain epilogue only
    (void)mode;
    hipLaunchKernelGGL((gemm_q8_0_mfma_kernel<MI, NJ, 0, L>), grid, dim3(Roles<MI>::kThreads), 0,
                       stream, xf, xf_bytes, g.args, M, K, g.steps_per_split, ws.partials,
                       ws.counters);
  } else if (mode == Epilogue::kSwiGLU) {
    hipLaunchKernelGGL((gemm_q8_0_mfma_kernel<MI, NJ, 1, L>), grid, dim3(Roles<MI>::kThreads), 0,
                       stream, xf, xf_bytes, g.args, M, K, g.steps_per_split, ws.partials,
                       ws.counters);
  } else {
    hipLaunchKernelGGL((gemm_q8_0_mfma_kernel<MI, NJ, 0, L>), grid, dim3(Roles<MI>::kThreads), 0,
                       stream, xf, xf_bytes, g.args, M, K, g.steps_per_split, ws.partials,
                       ws.counters);
  }
}

template <int MI, int NJ>
void launch_tile(const GemmGrid& g, Epilogue mode, WeightLayout layout, const u32x4* xf,
                 uint32_t xf_bytes, int M, int K, const SplitKWorkspace& ws,
                 hipStream_t stream) {
  if (layout == WeightLayout::kTiled)
    launch_tile_l<MI, NJ, int(WeightLayout::kTiled)>(g, mode, xf, xf_bytes, M, K, ws, stream);
  else if (layout == WeightLayout::kKN)
    launch_tile_l<MI, NJ, int(WeightLayout::kKN)>(g, mode, xf, xf_bytes, M, K, ws, stream);
  else
    launch_tile_l<MI, NJ, int(WeightLayout::kRaw)>(g, mode, xf, xf_bytes, M, K, ws, stream);
}

// Bytes of the fragment-ordered bf16 copy of X: rows rounded up to 32, K to 64.
size_t xf_bytes_of(int M, int K) { return (size_t)(M + 31) / 32 * 32 * padded_k(K) * 2; }

constexpr size_t kScratchAlign = 256;

}  // namespace

bool gemm_mfma_config_valid(const GemmConfig& c) {
  // 256 x 128 tiles would need more than the 256 registers a wave gets.
  return ((c.bm == 128 && (c.bn == 64 || c.bn == 96 || c.bn == 128)) ||
          (c.bm == 256 && (c.bn == 64 || c.bn == 96))) &&
         c.splits >= 1 && c.splits <= 64;
}

GemmConfig gemm_mfma_pick_segs(int M, const LinearSegs& s, int K) {
  // Estimated time = rounds of workgroups over the 256 CUs (one per CU) x K
  // steps per workgroup x the measured time of one K step of the tile shape
  // (MI355X, microseconds, fitted over M = 512 x {11008, 12288, 4096} x
  // {4096, 11008} sweeps), plus the split-K partial traffic (written and read
  // once per split; it mostly stays in cache, ~5.6 TB/s).  Tile heights of 256
  // only once M exceeds 128.  A SwiGLU tile holds BN/2 rows of each weight.
  struct Shape {
    int bm, bn;
    double step_us;
  };
  static const Shape shapes[] = {{256, 96, 0.90}, {256, 64, 0.75}, {128, 128, 0.85},
                                 {128, 96, 0.62}, {128, 64, 0.52}};
  const bool swi = s.mode == Epilogue::kSwiGLU;
  const int count = swi ? 1 : s.count;
  const int n_steps = padded_k(K) / BK;
  GemmConfig best{128, 64, 1};
  double best_us = 1e300;
  for (const Shape& sh : shapes) {
    if (sh.bm == 256 && (M <= 128 || s.layout == WeightLayout::kKN)) continue;  // KN: below
    const int cols = swi ? sh.bn / 2 : sh.bn;
    int64_t col_tiles = 0, out_cols = 0;
    for (int i = 0; i < count; ++i) {
      col_tiles += (s.seg[i].N + cols - 1) / cols;
      out_cols += s.seg[i].N;
    }
    const int64_t tiles = col_tiles * ((M + sh.bm - 1) / sh.bm);
    for (int splits = 1; splits <= 4; splits *= 2) {
      if (splits > n_steps) break;
      const int64_t rounds = (tiles * splits + 255) / 256;
      const int steps = (n_steps + splits - 1) / splits;
      const double split_us =
          splits > 1 ? (double)splits * M * out_cols * (swi ? 2 : 1) * 8 / 5.6e6 : 0.0;
      const double us = (double)rounds * steps * sh.step_us + split_us;
      if (us < best_us) {
        best_us = us;
        best = GemmConfig{sh.bm, sh.bn, splits};
      }
    }
  }
  // MatMul (B [K, N]): in the 12-wave 256-row tiles the producer ring (two raw
  // blocks per item and step) spills ~20 registers, and a K step costs about
  // twice a 128-row tile's, so those tiles pay only where they put the whole
  // grid in one round of workgroups and no 128-row tile does (512 rows of A with
  // 8192 < N <= 12288).  Measured on MI355X, rotated B copies, three
  // interleaved runs: 512 x 11008 x 4096 77-78 us vs 116 us on 128 x 96 tiles;
  // where 128-row tiles fit one round or neither fits, the 128-row pick stays
  // faster (512 x 4096 x 4096: 46-47 vs 49-50 us on 256 x 64 tiles with two K
  // splits; 2048 x 4096 x 4096: 127-128 vs 142-143 on 256 x 96).
  if (s.layout == WeightLayout::kKN && M > 256) {
    const int64_t N = s.seg[0].N;
    auto one_round = [&](int bm, int bn) {
      return (N + bn - 1) / bn * ((M + bm - 1) / bm) <= 256;
    };
    if (!one_round(128, 128) && !one_round(128, 96) && !one_round(128, 64) &&
        one_round(256, 96))
      return GemmConfig{256, 96, 1};
  }
  return best;
}

GemmConfig gemm_mfma_pick(int M, int N, int K) {
  return gemm_mfma_pick_segs(M, single_seg(nullptr, nullptr, nullptr, N), K);
}

SplitKNeed gemm_mfma_workspace_segs(const GemmConfig& c, int M, const LinearSegs& s, int K) {
  const GemmGrid g = gemm_grid(c, M, s, K);
  SplitKNeed need;
  need.splits = (int)g.splits;
  const size_t tiles = (size_t)g.tn * g.tm;
  need.partial_floats = g.splits > 1 ? tiles * g.splits * (size_t)c.bm * c.bn : 0;
  need.counters = g.splits > 1 ? tiles : 0;
  need.scratch_bytes = (xf_bytes_of(M, K) + kScratchAlign - 1) / kScratchAlign * kScratchAlign;
  return need;
}

SplitKNeed gemm_mfma_workspace(const GemmConfig& c, int M, int N, int K) {
  return gemm_mfma_workspace_segs(c, M, single_seg(nullptr, nullptr, nullptr, N), K);
}

bool gemm_mfma_fits(const GemmConfig& c, int M, int N, int K) {
  // 32-bit buffer offsets within the bf16 copy of X (whole) and within one
  // tile's rows of W; the X conversion grid has one y index per 32 rows.
  const int64_t row_bytes = (int64_t)(K / kBlockElems) * kBlockBytes;
  (void)N;
  return (int64_t)(M + c.bm) * padded_k(K) * 2 < (int64_t(1) << 31) &&
         (int64_t)c.bn * row_bytes < (int64_t(1) << 31) && (M + 31) / 32 <= 65535;
}

bool gemm_mfma_kn_fits(const LinearSegs& s, int K) {
  // One plain output; N a whole number of blocks; 32-bit offsets within B.
  const int N = s.seg[0].N;
  return s.count == 1 && s.mode == Epilogue::kPlain && N % kBlockElems == 0 &&
         (int64_t)K * (N / kBlockElems) * kBlockBytes < (int64_t(1) << 31);
}

GemmConfig gemm_mfma_pick_kn(int M, int N, int K) {
  LinearSegs s = single_seg(nullptr, nullptr, nullptr, N);
  s.layout = WeightLayout::kKN;
  return gemm_mfma_pick_segs(M, s, K);
}

hipError_t launch_gemm_mfma_segs(const GemmConfig& c, const float* x, const LinearSegs& s,
                                 int M, int K, const SplitKWorkspace& ws, hipStream_t stream) {
  const bool swi = s.mode == Epilogue::kSwiGLU;
  if (!gemm_mfma_config_valid(c) || !gemm_mfma_fits(c, M, 0, K) || ws.scratch == nullptr)
    return hipErrorInvalidValue;
  if (s.count < 1 || s.count > 3 || (swi && s.count != 2))
    return hipErrorInvalidValue;
  for (int i = 0; i < s.count; ++i)
    if (s.seg[i].N <= 0 || s.seg[i].w == nullptr) return hipErrorInvalidValue;
  if (s.layout == WeightLayout::kKN && !gemm_mfma_kn_fits(s, K))
    return hipErrorInvalidValue;
  const GemmGrid g = gemm_grid(c, M, s, K);
  if (g.splits > 1 && (ws.partials == nullptr || ws.counters == nullptr))
    return hipErrorInvalidValue;
  const size_t xfb = xf_bytes_of(M, K);
  u32x4* xf = static_cast<u32x4*>(ws.scratch);
  const int n_steps = padded_k(K) / BK;
  hipLaunchKernelGGL(x_to_frag_kernel, dim3((unsigned)n_steps, (unsigned)((M + 31) / 32)),
                     dim3(256), 0, stream, x, xf, M, K, n_steps);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int mi = c.bm / 128;
  switch (mi * 1000 + c.bn) {
    case 1064: launch_tile<1, 2>(g, s.mode, s.layout, xf, (uint32_t)xfb, M, K, ws, stream); break;
    case 1096: launch_tile<1, 3>(g, s.mode, s.layout, xf, (uint32_t)xfb, M, K, ws, stream); break;
    case 1128: launch_tile<1, 4>(g, s.mode, s.layout, xf, (uint32_t)xfb, M, K, ws, stream); break;
    case 2064: launch_tile<2, 2>(g, s.mode, s.layout, xf, (uint32_t)xfb, M, K, ws, stream); break;
    case 2096: launch_tile<2, 3>(g, s.mode, s.layout, xf, (uint32_t)xfb, M, K, ws, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemm_mfma(const GemmConfig& c, const float* x, const uint8_t* w,
                            const float* bias, float* y, int M, int N, int K,
                            const SplitKWorkspace& ws, hipStream_t stream) {
  return launch_gemm_mfma_segs(c, x, single_seg(w, bias, y, N), M, K, ws, stream);
}

}  // namespace mle
