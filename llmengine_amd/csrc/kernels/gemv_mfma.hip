// gemv_mfma.hip -- Q8_0 Linear decode (1 <= M <= 16 tokens per launch) on bf16
// MFMA for gfx950, with FP32-exact activations.
//
// y[m, n] = sum_k x[m, k] * d[n, k/32] * q[n, k]  (+ bias[n])
//
// Computes what cpu::sgemm_nt(const float*, const uint8_t*, ...) computes
// (src/runtime/kernels/cpu_kernels.cpp:208-218) and replaces the reference's
// sgemm_nt_q8_0_warp_kernel (src/runtime/kernels/cuda_kernels.cu:333-358) for
// small M, where an FP32 FMA path needs M FMAs per weight element and runs out of
// VALU long before HBM.
//
// Exactness.  Every fp32 activation is split into three bf16 parts
// x = hi + mid + lo, each taking the next 8 significant bits (truncation), so the
// sum is exact for every finite x.  The int8 quants are exact in bf16.  The MFMA
// forms each product q * part exactly (8 x 8 significant bits) and accumulates in
// fp32, so one v_mfma_f32_16x16x32_bf16 over a 32-wide K block yields the block
// dot product sum_k q * x to fp32 accumulation error, as an FP32 FMA chain does.
// The binary16 scale is applied once per block in fp32: acc = fma(d, s, acc).
// x = +-Inf is carried whole in `hi` (mid = lo = 0) and NaN stays NaN, so
// non-finite activations propagate with IEEE semantics.
//
// MFMA operands (16 x 16 x 32): A = 16 weight rows x one 32-quant block; B = 32 k
// x 16 "virtual columns" v = part * MT + m (token m, part 0..2); P = ceil(3 MT/16)
// chained MFMAs cover all virtual columns, and column v % 16 of the accumulator
// collects every part of its token (MT is 1, 2, 4, 5, 8 or 16 so no two tokens
// share a column).
//
// Work split.  A workgroup of W waves owns 16 W output rows (wave w: rows
// 16w .. 16w+15, so no cross-wave reduction) and a range of K chunks of KS
// blocks.  Lane l loads whole 34-byte blocks: row l % 16, blocks 4u + l / 16 of
// the chunk (u = 0 .. KS/4-1), i.e. every row's blocks in 136-byte runs.  A 4 x 4
// transpose of 8-byte quant chunks across the four 16-lane rows
// (v_permlane32_swap then v_permlane16_swap, 8 instructions per 4 blocks) turns
// those registers straight into MFMA A fragments, with no LDS round trip.
// Software pipeline: the loads of chunk c+1 (weights and the activations of its K
// slice) are in flight while chunk c is multiplied; the activation split of chunk
// c+1 goes to the other half of a double-buffered LDS B-fragment area; one
// barrier per chunk.
//
// Split K.  When there are too few row tiles to fill the GPU, the K chunks are
// split over gridDim.y workgroups.  Each stores its 16 W x MT partial sums to its
// own aligned workspace region and bumps a per-tile counter; the last workgroup
// of a tile adds the partials in split order (deterministic) plus bias, writes y
// and resets the counter to zero for the next launch on the stream.  The
// partials travel by device-scope (sc1, write-through) stores and loads, and the
// wait for every store's completion (s_waitcnt 0) precedes the counter increment,
// so the workgroup that sees the final count reads complete data.  A
// release/acquire fence pair instead would write back and invalidate the whole
// L2 of the XCD per workgroup (measured 10x slower than the whole GEMV).
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t top_halves(uint32_t lo_word, uint32_t hi_word) {
  // bf16 pair from the upper 16 bits of two fp32 bit patterns (lo in bits 0-15).
  return __builtin_amdgcn_perm(hi_word, lo_word, 0x07060302u);
}

// Splits 8 activations into packed bf16 hi / mid / lo parts (4 dwords each).
__device__ __forceinline__ void split3(const float (&v)[8], uint32_t (&hi)[4],
                                       uint32_t (&mid)[4], uint32_t (&lo)[4]) {
  uint32_t hb[8], rb[8], lb[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v[j]);
    const float h = __builtin_bit_cast(float, b & 0xffff0000u);
    // x == h covers +-Inf (x - h would be NaN) and values already exact in bf16.
    const float r = (v[j] == h) ? 0.0f : v[j] - h;
    const uint32_t r_bits = __builtin_bit_cast(uint32_t, r);
    const float m = __builtin_bit_cast(float, r_bits & 0xffff0000u);
    const float l = r - m;
    hb[j] = b;
    rb[j] = r_bits;
    lb[j] = __builtin_bit_cast(uint32_t, l);
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    hi[p] = top_halves(hb[2 * p], hb[2 * p + 1]);
    mid[p] = top_halves(rb[2 * p], rb[2 * p + 1]);
    lo[p] = top_halves(lb[2 * p], lb[2 * p + 1]);
  }
}

// 8 int8 quants (two dwords) -> 8 bf16 (exact).
__device__ __forceinline__ bf16x8_t quants_to_bf16(uint32_t q0, uint32_t q1) {
  u32x4 o;
  o.x = top_halves(__builtin_bit_cast(uint32_t, q_at(q0, 0)), __builtin_bit_cast(uint32_t, q_at(q0, 1)));
  o.y = top_halves(__builtin_bit_cast(uint32_t, q_at(q0, 2)), __builtin_bit_cast(uint32_t, q_at(q0, 3)));
  o.z = top_halves(__builtin_bit_cast(uint32_t, q_at(q1, 0)), __builtin_bit_cast(uint32_t, q_at(q1, 1)));
  o.w = top_halves(__builtin_bit_cast(uint32_t, q_at(q1, 2)), __builtin_bit_cast(uint32_t, q_at(q1, 3)));
  return __builtin_bit_cast(bf16x8_t, o);
}

// In-register 4 x 4 transpose of 8-byte chunks across the four 16-lane rows of
// the wave.  On entry the lanes of row g hold a whole block in q[0..7] (chunk j
// = q[2j], q[2j+1]); on exit they hold chunk g of the blocks of rows 0..3, the
// block of row j in q[2j], q[2j+1].
__device__ __forceinline__ void transpose_chunks(uint32_t (&q)[8]) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      // rows 2,3 of chunk j  <->  rows 0,1 of chunk j+2
      const auto s = __builtin_amdgcn_permlane32_swap(q[2 * j + d], q[2 * (j + 2) + d], false, false);
      q[2 * j + d] = s[0];
      q[2 * (j + 2) + d] = s[1];
    }
#pragma unroll
  for (int j = 0; j < 4; j += 2)
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      // rows 1,3 of chunk j  <->  rows 0,2 of chunk j+1
      const auto s = __builtin_amdgcn_permlane16_swap(q[2 * j + d], q[2 * (j + 1) + d], false, false);
      q[2 * j + d] = s[0];
      q[2 * (j + 1) + d] = s[1];
    }
}

template <int MT>
struct Cols {
  static constexpr int P = (3 * MT + 15) / 16;  // chained MFMAs per tile
  static constexpr int PADC = 16 * P - 3 * MT;  // virtual columns that stay zero
};

template <int MT, int W, int KS>
struct Shape {
  static constexpr int NT = 64 * W;               // threads
  static constexpr int R = 16 * W;                // output rows per workgroup
  static constexpr int P = Cols<MT>::P;
  static constexpr int NL = KS / 4;               // blocks per lane per chunk
  static constexpr int BBUF = KS * P * 1024;      // B fragments of one chunk (bytes)
  static constexpr int XITEMS = MT * KS * 4;      // (token, block, 8-wide k chunk)
  static constexpr int XPT = (XITEMS + NT - 1) / NT;
  static constexpr int OUTS = 16 * MT;            // outputs per wave
  static constexpr int OPL = (OUTS + 63) / 64;    // outputs per lane
};

template <int MT, int W, int KS>
__global__ __launch_bounds__(64 * W) void gemv_q8_0_mfma_kernel(
    const float* __restrict__ x, const uint8_t* __restrict__ w,
    const float* __restrict__ bias, float* __restrict__ y, int M, int N, int K,
    int chunks_per_split, float* __restrict__ partials, uint32_t* __restrict__ counters) {
  using S = Shape<MT, W, KS>;
  constexpr int P = S::P;
  constexpr int NL = S::NL;
  constexpr int XPT = S::XPT;
  static_assert(KS % 4 == 0, "chunk = whole load sets of 4 blocks");
  __shared__ __attribute__((aligned(16))) uint8_t bfr[2][S::BBUF];
  __shared__ __attribute__((aligned(16))) float scl[W][KS][16];
  __shared__ float red[W][16][17];
  __shared__ uint32_t arrived;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int KB = K / kBlockElems;
  const int n_chunks = (KB + KS - 1) / KS;
  const int c_begin = blockIdx.y * chunks_per_split;
  const int c_end = min(c_begin + chunks_per_split, n_chunks);
  const int64_t n0 = (int64_t)blockIdx.x * S::R;
  // This lane's weight row; rows past N are clamped (outputs dropped at the end).
  const int64_t my_row = min(n0 + wave * 16 + r16, (int64_t)N - 1);
  const uint8_t* wrow = w + my_row * ((int64_t)KB * kBlockBytes);

  auto load_w = [&](int c, RawBlock (&b)[NL]) {
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const int kb = min(c * KS + 4 * u + g, KB - 1);
      b[u] = load_block_raw(wrow + (int64_t)kb * kBlockBytes);
    }
  };
  auto load_x = [&](int c, float (&xv)[XPT][8]) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int it = tid + S::NT * i;
      const int m = it / (KS * 4), q = it % (KS * 4);
      const int kbg = c * KS + (q >> 2);
      if (it < S::XITEMS && m < M && kbg < KB) {
        const f32x4* xp = reinterpret_cast<const f32x4*>(
            x + (int64_t)m * K + (int64_t)kbg * kBlockElems + 8 * (q & 3));
        const f32x4 a = xp[0], b = xp[1];
        xv[i][0] = a.x; xv[i][1] = a.y; xv[i][2] = a.z; xv[i][3] = a.w;
        xv[i][4] = b.x; xv[i][5] = b.y; xv[i][6] = b.z; xv[i][7] = b.w;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[i][j] = 0.0f;
      }
    }
  };
  // B fragment (block kb, MFMA p): lane l holds virtual column l % 16, k = 8 (l/16) .. +7.
  auto prep_x = [&](const float (&xv)[XPT][8], uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int it = tid + S::NT * i;
      if (it >= S::XITEMS) continue;
      const int m = it / (KS * 4), q = it % (KS * 4);
      const int kb = q >> 2, c = q & 3;
      uint32_t parts[3][4];
      split3(xv[i], parts[0], parts[1], parts[2]);
#pragma unroll
      for (int part = 0; part < 3; ++part) {
        const int vc = part * MT + m;
        u32x4* dst = reinterpret_cast<u32x4*>(
            buf + ((kb * P + (vc >> 4)) * 64 + c * 16 + (vc & 15)) * 16);
        *dst = u32x4{parts[part][0], parts[part][1], parts[part][2], parts[part][3]};
      }
    }
  };

  // Virtual columns past 3*MT are never written by prep_x: zero them once.
  if constexpr (Cols<MT>::PADC > 0) {
    constexpr int PADC = Cols<MT>::PADC;
    for (int it = tid; it < 2 * KS * 4 * PADC; it += S::NT) {
      const int bsel = it / (KS * 4 * PADC);
      const int rest = it % (KS * 4 * PADC);
      const int kb = rest / (4 * PADC), q = rest % (4 * PADC);
      const int c = q / PADC, vc = 3 * MT + q % PADC;
      *reinterpret_cast<u32x4*>(bfr[bsel] + ((kb * P + (vc >> 4)) * 64 + c * 16 + (vc & 15)) *
                                                16) = u32x4{0u, 0u, 0u, 0u};
    }
  }

  RawBlock wc[NL];
  float xv[XPT][8];
  load_x(c_begin, xv);
  load_w(c_begin, wc);
  prep_x(xv, bfr[0]);
  __syncthreads();

  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c = c_begin; c < c_end; ++c) {
    const int buf = (c - c_begin) & 1;
    const bool more = c + 1 < c_end;
    RawBlock wn[NL];
    if (more) {
      load_x(c + 1, xv);
      load_w(c + 1, wn);
    }
    // Scales of this chunk: lane (g, r16) holds blocks 4u+g of row r16.
    Block blk[NL];
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      blk[u] = finish_block(wc[u]);
      const bool valid = c * KS + 4 * u + g < KB;
      scl[wave][4 * u + g][r16] = valid ? scale_to_f32_fast(blk[u].scale_bits) : 0.0f;
    }
    const uint8_t* bb = bfr[buf];
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      uint32_t q[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = blk[u].q[i];
      transpose_chunks(q);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kb = 4 * u + j;
        const bf16x8_t a = quants_to_bf16(q[2 * j], q[2 * j + 1]);
        f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            a, *reinterpret_cast<const bf16x8_t*>(bb + ((kb * P) * 64 + lane) * 16),
            f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int p = 1; p < P; ++p)
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              a, *reinterpret_cast<const bf16x8_t*>(bb + ((kb * P + p) * 64 + lane) * 16), d,
              0, 0, 0);
        // D layout: lane l holds rows 4 (l/16) + v (v = 0..3), virtual column l % 16.
        const f32x4 s = *reinterpret_cast<const f32x4*>(&scl[wave][kb][4 * g]);
        acc.x = __builtin_fmaf(s.x, d.x, acc.x);
        acc.y = __builtin_fmaf(s.y, d.y, acc.y);
        acc.z = __builtin_fmaf(s.z, d.z, acc.z);
        acc.w = __builtin_fmaf(s.w, d.w, acc.w);
      }
    }
    if (more) {
      prep_x(xv, bfr[buf ^ 1]);
#pragma unroll
      for (int u = 0; u < NL; ++u) wc[u] = wn[u];
    }
    __syncthreads();
  }

  // Sum the part columns of each token (within the wave).
  red[wave][4 * g + 0][r16] = acc.x;
  red[wave][4 * g + 1][r16] = acc.y;
  red[wave][4 * g + 2][r16] = acc.z;
  red[wave][4 * g + 3][r16] = acc.w;
  float outv[S::OPL];
#pragma unroll
  for (int o = 0; o < S::OPL; ++o) {
    const int idx = lane + 64 * o;  // (token m, row rr) with rows fastest
    const int m = idx >> 4, rr = idx & 15;
    float s = 0.0f;
    if (idx < S::OUTS) {
      const int c0 = m, c1 = (MT + m) & 15, c2 = (2 * MT + m) & 15;
      s = red[wave][rr][c0];
      if (c1 != c0) s += red[wave][rr][c1];
      if (c2 != c0 && c2 != c1) s += red[wave][rr][c2];
    }
    outv[o] = s;
  }

  if (gridDim.y == 1) {
#pragma unroll
    for (int o = 0; o < S::OPL; ++o) {
      const int idx = lane + 64 * o;
      const int m = idx >> 4, rr = idx & 15;
      const int64_t n = n0 + wave * 16 + rr;
      if (idx < S::OUTS && m < M && n < N) y[(int64_t)m * N + n] = outv[o] + (bias ? bias[n] : 0.0f);
    }
    return;
  }

  // Split K: partials [tile][split][wave][MT][16], then the last workgroup reduces.
  constexpr int REGION = S::R * MT;
  float* tile_part = partials + (int64_t)blockIdx.x * gridDim.y * REGION;
#pragma unroll
  for (int o = 0; o < S::OPL; ++o) {
    const int idx = lane + 64 * o;
    if (idx < S::OUTS && (idx >> 4) < M)
      __hip_atomic_store(tile_part + (int64_t)blockIdx.y * REGION + wave * S::OUTS + idx,
                         outv[o], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (tid == 0)
    arrived = __hip_atomic_fetch_add(counters + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (arrived != gridDim.y - 1) return;
#pragma unroll
  for (int o = 0; o < S::OPL; ++o) {
    const int idx = lane + 64 * o;
    const int m = idx >> 4, rr = idx & 15;
    const int64_t n = n0 + wave * 16 + rr;
    if (idx >= S::OUTS || m >= M || n >= N) continue;
    float s = 0.0f;
    for (unsigned sp = 0; sp < gridDim.y; ++sp)
      s += __hip_atomic_load(tile_part + (int64_t)sp * REGION + wave * S::OUTS + idx,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    y[(int64_t)m * N + n] = s + (bias ? bias[n] : 0.0f);
  }
  if (tid == 0)
    __hip_atomic_store(counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Grid {
  unsigned tiles, splits;
  int chunks_per_split;
};

Grid grid_of(const DecodeMfmaConfig& c, int N, int K) {
  const int KB = K / kBlockElems;
  const int n_chunks = (KB + c.ks - 1) / c.ks;
  const int rows = 16 * c.waves;
  Grid gr;
  gr.tiles = (unsigned)((N + rows - 1) / rows);
  int splits = c.splits > 0 ? c.splits : 1;
  if (splits > n_chunks) splits = n_chunks;
  gr.chunks_per_split = (n_chunks + splits - 1) / splits;
  gr.splits = (unsigned)((n_chunks + gr.chunks_per_split - 1) / gr.chunks_per_split);
  return gr;
}

template <int MT, int W, int KS>
hipError_t launch_t(const Grid& gr, const float* x, const uint8_t* w, const float* bias,
                    float* y, int M, int N, int K, const SplitKWorkspace& ws,
                    hipStream_t stream) {
  hipLaunchKernelGGL((gemv_q8_0_mfma_kernel<MT, W, KS>), dim3(gr.tiles, gr.splits),
                     dim3(64 * W), 0, stream, x, w, bias, y, M, N, K, gr.chunks_per_split,
                     ws.partials, ws.counters);
  return hipGetLastError();
}

template <int MT>
hipError_t dispatch_shape(const DecodeMfmaConfig& c, const Grid& gr, const float* x,
                          const uint8_t* w, const float* bias, float* y, int M, int N, int K,
                          const SplitKWorkspace& ws, hipStream_t stream) {
  if (c.waves == 4 && c.ks == 8) return launch_t<MT, 4, 8>(gr, x, w, bias, y, M, N, K, ws, stream);
  if (c.waves == 4 && c.ks == 16) return launch_t<MT, 4, 16>(gr, x, w, bias, y, M, N, K, ws, stream);
  if (c.waves == 2 && c.ks == 8) return launch_t<MT, 2, 8>(gr, x, w, bias, y, M, N, K, ws, stream);
  if (c.waves == 8 && c.ks == 8) return launch_t<MT, 8, 8>(gr, x, w, bias, y, M, N, K, ws, stream);
  return hipErrorInvalidValue;
}

}  // namespace

bool decode_mfma_config_valid(const DecodeMfmaConfig& c) {
  const bool mt = c.mt == 1 || c.mt == 2 || c.mt == 4 || c.mt == 5 || c.mt == 8 || c.mt == 16;
  const bool shape = (c.waves == 4 && (c.ks == 8 || c.ks == 16)) ||
                     (c.waves == 2 && c.ks == 8) || (c.waves == 8 && c.ks == 8);
  return mt && shape && c.splits >= 0 && c.splits <= 64;
}

int decode_mfma_tile(int M) {
  return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 5 ? 5 : M <= 8 ? 8 : 16;
}

DecodeMfmaConfig decode_mfma_pick(int M, int N, int K) {
  DecodeMfmaConfig c;
  c.mt = decode_mfma_tile(M);
  c.waves = 4;
  c.ks = 8;
  // Enough workgroups to give every CU about two: split K when row tiles are few.
  const int tiles = (N + 16 * c.waves - 1) / (16 * c.waves);
  const int n_chunks = (K / kBlockElems + c.ks - 1) / c.ks;
  int splits = (512 + tiles - 1) / tiles;
  if (splits > n_chunks) splits = n_chunks;
  if (splits < 1) splits = 1;
  c.splits = splits;
  return c;
}

SplitKNeed decode_mfma_workspace(const DecodeMfmaConfig& c, int N, int K) {
  const Grid gr = grid_of(c, N, K);
  SplitKNeed need;
  need.splits = (int)gr.splits;
  const size_t region = (size_t)16 * c.waves * c.mt;
  need.partial_floats = gr.splits > 1 ? (size_t)gr.tiles * gr.splits * region : 0;
  need.counters = gr.splits > 1 ? (size_t)gr.tiles : 0;
  return need;
}

hipError_t launch_gemv_mfma(const DecodeMfmaConfig& c, const float* x, const uint8_t* w,
                            const float* bias, float* y, int M, int N, int K,
                            const SplitKWorkspace& ws, hipStream_t stream) {
  const Grid gr = grid_of(c, N, K);
  switch (c.mt) {
    case 1: return dispatch_shape<1>(c, gr, x, w, bias, y, M, N, K, ws, stream);
    case 2: return dispatch_shape<2>(c, gr, x, w, bias, y, M, N, K, ws, stream);
    case 4: return dispatch_shape<4>(c, gr, x, w, bias, y, M, N, K, ws, stream);
    case 5: return dispatch_shape<5>(c, gr, x, w, bias, y, M, N, K, ws, stream);
    case 8: return dispatch_shape<8>(c, gr, x, w, bias, y, M, N, K, ws, stream);
    case 16: return dispatch_shape<16>(c, gr, x, w, bias, y, M, N, K, ws, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace mle
