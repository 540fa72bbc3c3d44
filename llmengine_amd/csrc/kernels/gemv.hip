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

constexpr int kXPad = 36;  // floats per staged 32-activation block (144 B: conflict-free)

template <int RW>
__device__ __forceinline__ void load_rows(Block (&blk)[RW], const uint8_t* const (&row)[RW],
                                          int b) {
#pragma unroll
  for (int r = 0; r < RW; ++r) blk[r] = load_block(row[r] + (int64_t)b * kBlockBytes);
}

// Output segments as the kernel sees them: segment i owns the workgroups
// [wg_end[i-1], wg_end[i]) of the grid.
struct GemvArgs {
  LinearSeg seg[3];
  unsigned wg_end[3];
  int count;
};

// silu(g) * u with the reference's operation order (cpu_kernels.cpp:848-858).
__device__ __forceinline__ float silu_mul(float g, float u) {
  return (g / (1.0f + expf(-g))) * u;
}

// One lane's contribution of block `blk[r]` (activations from LDS) to acc[m][r].
template <int MT, int RW>
__device__ __forceinline__ void consume(float (&acc)[MT][RW], const Block (&blk)[RW],
                                        const float* __restrict__ xb, int xm_stride) {
  float part[MT][RW];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) part[m][r] = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    f32x4 xv[MT][2];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const f32x4* xp = reinterpret_cast<const f32x4*>(xb + m * xm_stride + 8 * c);
      xv[m][0] = xp[0];
      xv[m][1] = xp[1];
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

// Activations are staged in LDS one K-chunk of `ckb` blocks at a time, as
// [token][block][kXPad] floats; rows of weights stream straight from HBM.
// MODE 0: plain / multi-output Linear (RT = RW rows per lane group).  MODE 1
// (SwiGLU): a lane group computes RW rows of the gate weight and the same RW
// rows of the up weight (RT = 2 RW) and writes silu(gate) * up.
template <int MT, int LPR, int RW, int MODE>
__global__ __launch_bounds__(256) void gemv_q8_0_kernel(const float* __restrict__ x,
                                                        const GemvArgs args, int M, int K,
                                                        int ckb) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  constexpr bool kSwi = MODE == 1;
  constexpr int RT = kSwi ? 2 * RW : RW;  // weight rows per lane group
  constexpr int G = 256 / LPR;            // lane groups per workgroup
  const int li = threadIdx.x % LPR;
  const int grp = threadIdx.x / LPR;
  // Segment of this workgroup (uniform selects: no indexing into the argument).
  const unsigned wg = blockIdx.x;
  const int si = (!kSwi && args.count > 1 && wg >= args.wg_end[0])
                     ? ((args.count > 2 && wg >= args.wg_end[1]) ? 2 : 1)
                     : 0;
  const unsigned wg0 = si == 0 ? 0u : si == 1 ? args.wg_end[0] : args.wg_end[1];
  const uint8_t* w = si == 0 ? args.seg[0].w : si == 1 ? args.seg[1].w : args.seg[2].w;
  const void* bias = si == 0 ? args.seg[0].bias : si == 1 ? args.seg[1].bias : args.seg[2].bias;
  const int bias_bf16 =
      si == 0 ? args.seg[0].bias_bf16 : si == 1 ? args.seg[1].bias_bf16 : args.seg[2].bias_bf16;
  float* y = si == 0 ? args.seg[0].y : si == 1 ? args.seg[1].y : args.seg[2].y;
  const int N = si == 0 ? args.seg[0].N : si == 1 ? args.seg[1].N : args.seg[2].N;
  const int64_t row0 = ((int64_t)(wg - wg0) * G + grp) * RW;
  const int KB = K / kBlockElems;
  const int64_t row_bytes = (int64_t)KB * kBlockBytes;
  const int xm_stride = ckb * kXPad;

  // Rows past N are clamped to row N-1 so that every weight load is
  // unconditional (loads issue back to back); their results are dropped.
  const uint8_t* row_ptr[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int rr = r % RW;
    const uint8_t* base = (kSwi && r >= RW) ? args.seg[1].w : w;
    row_ptr[r] = base + (row0 + rr < N ? row0 + rr : (int64_t)N - 1) * row_bytes;
  }

  float acc[MT][RT];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[m][r] = 0.0f;

  // Long rows (LPR >= 32, i.e. K >= 2048): a lane keeps two raw (not yet
  // realigned) blocks of every row in flight and realigns each only when it is
  // consumed, so no wait for a load is placed ahead of the previous block's
  // FMAs (measured on MI355X: 4-12% faster on the Llama shapes at M = 1, and
  // bitwise the same results).  Short rows keep the realigned double buffer,
  // which is faster there (the [151936, 896] lm_head: 6% slower with the ring).
  constexpr bool kRing = LPR >= 32;
  constexpr int DEPTH = 2;
  for (int c0 = 0; c0 < KB; c0 += ckb) {
    const int cend = c0 + ckb < KB ? c0 + ckb : KB;
    // Issue this lane's first weight loads before waiting on the barrier.
    int b = c0 + li;
    Block cur[RT];
    RawBlock ring[kRing ? DEPTH : 1][RT];
    if constexpr (kRing) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d)
        if (b + d * LPR < cend)
#pragma unroll
          for (int r = 0; r < RT; ++r)
            ring[d][r] = load_block_raw(row_ptr[r] + (int64_t)(b + d * LPR) * kBlockBytes);
    } else {
      if (b < cend) load_rows<RT>(cur, row_ptr, b);
    }

    __syncthreads();  // the previous chunk's readers are done with xs
    {
      const int nquads = (cend - c0) * 8;  // float4s per token in this chunk
      for (int i = threadIdx.x; i < M * nquads; i += 256) {
        const int m = i / nquads;
        const int qd = i - m * nquads;
        const int bb = qd >> 3, j = qd & 7;
        const f32x4 v = *reinterpret_cast<const f32x4*>(
            x + (int64_t)m * K + (int64_t)(c0 + bb) * kBlockElems + 4 * j);
        *reinterpret_cast<f32x4*>(xs + m * xm_stride + bb * kXPad + 4 * j) = v;
      }
    }
    __syncthreads();

    if constexpr (kRing) {
      for (; b < cend; b += DEPTH * LPR) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
          const int bb = b + d * LPR;
          if (bb < cend) {
            Block blk[RT];
#pragma unroll
            for (int r = 0; r < RT; ++r) blk[r] = finish_block(ring[d][r]);
            const int bn = bb + DEPTH * LPR;
            if (bn < cend)
#pragma unroll
              for (int r = 0; r < RT; ++r)
                ring[d][r] = load_block_raw(row_ptr[r] + (int64_t)bn * kBlockBytes);
            consume<MT, RT>(acc, blk, xs + (bb - c0) * kXPad, xm_stride);
          }
        }
      }
    } else {
      for (; b < cend; b += LPR) {
        Block nxt[RT];
        const int bn = b + LPR;
        if (bn < cend) load_rows<RT>(nxt, row_ptr, bn);
        consume<MT, RT>(acc, cur, xs + (b - c0) * kXPad, xm_stride);
#pragma unroll
        for (int r = 0; r < RT; ++r) cur[r] = nxt[r];
      }
    }
  }

  // Reduce the LPR partial sums of every (token, row) pair within the group.
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < RT; ++r) acc[m][r] += __shfl_xor(acc[m][r], off, LPR);
  }

  if (li == 0) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      if (row0 + r >= N) continue;
      const float bv = (!kSwi && bias) ? bias_at(bias, bias_bf16, row0 + r) : 0.0f;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m >= M) continue;
        if constexpr (kSwi)
          y[(int64_t)m * N + row0 + r] = silu_mul(acc[m][r], acc[m][RW + r]);
        else
          y[(int64_t)m * N + row0 + r] = acc[m][r] + bv;
      }
    }
  }
}

// Row-span GEMV on raw weights, one token, lanes along K.  A workgroup owns
// RPW = 4 consecutive rows of a weight and all of K; wave w (of up to 8) takes
// the 64-block chunks c = w, w + waves, .. and lane l block 64 c + l of every
// row.  So a wave's load instruction reads 64 consecutive blocks of one row
// (2176 contiguous bytes), and the lane loads the 32 activations of its block
// once, straight into registers, for all RPW rows: no LDS staging, no barrier
// before the first multiply.  Per row the lane realigns its block, forms
// s = sum_j x_j q_j over the 32 quants in fp32 FMAs and adds d * s; the loads of
// all RPW rows are in flight before the first multiply.  Lanes past K read zeros
// (buffer range check).  The 64 lanes' sums are added by a transposing butterfly
// (each exchange halves the values a lane holds), the waves' totals in LDS in
// wave order: deterministic.
//
// Measured on MI355X against the LDS-staged kernel above (one token, rotated
// weight copies, three interleaved runs per build): 0.92x on [4096, 11008],
// 0.82x on the [896, 4864] Qwen down projection; on rows of 4096 elements 0.95x
// on [4096, 4096] but 1.03x on [12288, 4096] and [11008, 4096].  It takes the
// one-token launches on rows of more than 4096 elements, whatever the output
// count, so that a fused q / k / v launch and its single Linears run the same
// kernel and agree bit for bit (a row's sum depends only on K's split over lanes
// and waves).  Eight or 16 rows per
// workgroup cut the activation reads (every workgroup reads all of x) but were
// slower: 1.1-1.3x with four rows in flight per lane, 1.7-1.9x with eight
// (each lane's whole share requested up front).
constexpr int kRawkRows = 4;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemv_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Sums each of the V per-lane values v[0..V) over the wave's 64 lanes (V a power
// of two, <= 64).  On return v[0] of lane l holds the total of value l >> (6 - log2 V).
template <int V>
__device__ __forceinline__ void wave_sum_transpose(float (&v)[V], int lane) {
  int n = V;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    if (n > 1) {
      const int h = n / 2;
      const bool up = (lane & o) != 0;
#pragma unroll
      for (int i = 0; i < V / 2; ++i) {
        if (i >= h) break;
        const float keep = up ? v[i + h] : v[i];
        const float give = up ? v[i] : v[i + h];
        v[i] = keep + __shfl_xor(give, o);
      }
      n = h;
    } else {
      v[0] += __shfl_xor(v[0], o);
    }
  }
}

template <int RPW>
__global__ __launch_bounds__(512) void gemv_rawk_kernel(const float* __restrict__ x,
                                                         const GemvArgs args, int K) {
  static_assert(RPW == 4 || RPW == 8 || RPW == 16, "the row sums fit one butterfly");
  constexpr int SHIFT = RPW == 16 ? 2 : RPW == 8 ? 3 : 4;
  __shared__ float red[8][RPW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const unsigned wg = blockIdx.x;
  const int si = (args.count > 1 && wg >= args.wg_end[0])
                     ? ((args.count > 2 && wg >= args.wg_end[1]) ? 2 : 1)
                     : 0;
  const unsigned wg0 = si == 0 ? 0u : si == 1 ? args.wg_end[0] : args.wg_end[1];
  const uint8_t* w = si == 0 ? args.seg[0].w : si == 1 ? args.seg[1].w : args.seg[2].w;
  const void* bias = si == 0 ? args.seg[0].bias : si == 1 ? args.seg[1].bias : args.seg[2].bias;
  const int bias_bf16 =
      si == 0 ? args.seg[0].bias_bf16 : si == 1 ? args.seg[1].bias_bf16 : args.seg[2].bias_bf16;
  float* y = si == 0 ? args.seg[0].y : si == 1 ? args.seg[1].y : args.seg[2].y;
  const int N = si == 0 ? args.seg[0].N : si == 1 ? args.seg[1].N : args.seg[2].N;
  const int64_t row0 = (int64_t)(wg - wg0) * RPW;
  const int KB = K / kBlockElems;
  const uint32_t row_bytes = (uint32_t)KB * kBlockBytes;
  // Buffer over this workgroup's rows (rows past N read as zero); a block's
  // offset is relative to the first row, so its byte phase is the base's plus
  // the offset's.
  const int64_t live_rows = N - row0 < RPW ? N - row0 : RPW;
  const uint8_t* base = w + row0 * row_bytes;
  const __amdgpu_buffer_rsrc_t wrs = gemv_rsrc(base, (uint32_t)(live_rows * row_bytes));
  const uint32_t phase = (uint32_t)((uintptr_t)base & 2u);
  const __amdgpu_buffer_rsrc_t xrs = gemv_rsrc(x, (uint32_t)K * 4u);

  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
  for (int c = wave; c * 64 < KB; c += nw) {
    const int b = c * 64 + lane;
    const bool live = b < KB;
    f32x4 xv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t off = live ? (uint32_t)((b * kBlockElems + 4 * j) * 4) : 0x80000000u;
      xv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
    }
    // Block b of row r: two 16-byte loads from the 4-aligned address at or after
    // the block and the remaining u16 (load_block_raw's cases A and B).
    RawBlock rb[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const uint32_t off = (uint32_t)r * row_bytes + (uint32_t)b * kBlockBytes;
      const uint32_t mis = (phase + off) & 2u;
      uint32_t v8 = live ? off + mis : 0x80000000u;
      uint32_t v2 = live ? off + (mis ? 0u : 32u) : 0x80000000u;
      asm volatile("" : "+v"(v8), "+v"(v2));  // the loads stay where they are written
      const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8, 0, 0);
      const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8 + 16, 0, 0);
      rb[r].v0 = u32x4_a4{v0.x, v0.y, v0.z, v0.w};
      rb[r].v1 = u32x4_a4{v1.x, v1.y, v1.z, v1.w};
      rb[r].u = __builtin_amdgcn_raw_buffer_load_b16(wrs, v2, 0, 0);
      rb[r].mis = mis;
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const Block blk = finish_block(rb[r]);
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t q = blk.q[j];
        s = __builtin_fmaf(xv[j].x, q_at(q, 0), s);
        s = __builtin_fmaf(xv[j].y, q_at(q, 1), s);
        s = __builtin_fmaf(xv[j].z, q_at(q, 2), s);
        s = __builtin_fmaf(xv[j].w, q_at(q, 3), s);
      }
      acc[r] = __builtin_fmaf(scale_to_f32_fast(blk.scale_bits), s, acc[r]);
    }
  }
  wave_sum_transpose<RPW>(acc, lane);
  if ((lane & ((1 << SHIFT) - 1)) == 0) red[wave][lane >> SHIFT] = acc[0];
  __syncthreads();
  if (wave != 0 || lane >= RPW) return;
  const int64_t n = row0 + lane;
  if (n >= N) return;
  float sum = 0.0f;
  for (int wi = 0; wi < nw; ++wi) sum += red[wi][lane];
  y[n] = sum + (bias ? bias_at(bias, bias_bf16, n) : 0.0f);
}

hipError_t launch_rawk(const float* x, const LinearSegs& s, int M, int K, hipStream_t stream) {
  if (M != 1 || s.mode != Epilogue::kPlain) return hipErrorInvalidValue;
  GemvArgs args{};
  int64_t grid = 0;
  for (int i = 0; i < 3; ++i) {
    args.seg[i] = s.seg[i];
    if (i < s.count) grid += ((int64_t)s.seg[i].N + kRawkRows - 1) / kRawkRows;
    args.wg_end[i] = (unsigned)grid;
  }
  args.count = s.count;
  const int chunks = (K / kBlockElems + 63) / 64;
  const unsigned threads = 64u * (unsigned)(chunks < 8 ? chunks : 8);
  hipLaunchKernelGGL((gemv_rawk_kernel<kRawkRows>), dim3((unsigned)grid), dim3(threads), 0,
                     stream, x, args, K);
  return hipGetLastError();
}

// Bytes of staged activations per workgroup: all of K in one chunk up to 384
// blocks at one token (the Llama down projection, K = 11008, in one pass: a
// second chunk drains the load ring behind two barriers mid-row).
constexpr int kXLdsBudget = 54 * 1024;

template <int MT, int LPR, int RW>
hipError_t launch_one(const float* x, const LinearSegs& s, int M, int K, hipStream_t stream) {
  constexpr int rows_per_wg = (256 / LPR) * RW;
  const bool swi = s.mode == Epilogue::kSwiGLU;
  GemvArgs args{};
  int64_t grid = 0;
  const int count = swi ? 1 : s.count;
  for (int i = 0; i < 3; ++i) {
    args.seg[i] = s.seg[i];
    if (i < count) grid += ((int64_t)s.seg[i].N + rows_per_wg - 1) / rows_per_wg;
    args.wg_end[i] = (unsigned)grid;
  }
  if (swi) args.seg[1].N = s.seg[0].N;
  args.count = count;
  const int KB = K / kBlockElems;
  // Chunk of blocks staged per pass: whole K if it fits, else a multiple of LPR.
  int ckb = kXLdsBudget / (MT * kXPad * 4);
  if (ckb >= KB) {
    ckb = KB;
  } else {
    ckb = ckb / LPR * LPR;
    if (ckb < LPR) ckb = LPR;
  }
  const size_t lds = (size_t)MT * ckb * kXPad * sizeof(float);
  if (swi) {
    if constexpr (MT == 1 && RW <= 4)
      hipLaunchKernelGGL((gemv_q8_0_kernel<MT, LPR, RW, 1>), dim3((unsigned)grid), dim3(256),
                         lds, stream, x, args, M, K, ckb);
    else
      return hipErrorInvalidValue;
  } else {
    hipLaunchKernelGGL((gemv_q8_0_kernel<MT, LPR, RW, 0>), dim3((unsigned)grid), dim3(256), lds,
                       stream, x, args, M, K, ckb);
  }
  return hipGetLastError();
}

template <int MT, int LPR>
hipError_t dispatch_rw(int rw, const float* x, const LinearSegs& s, int M, int K,
                       hipStream_t stream) {
  switch (rw) {
    case 1: return launch_one<MT, LPR, 1>(x, s, M, K, stream);
    case 2: return launch_one<MT, LPR, 2>(x, s, M, K, stream);
    case 4: return launch_one<MT, LPR, 4>(x, s, M, K, stream);
    case 8: return launch_one<MT, LPR, 8>(x, s, M, K, stream);
  }
  return hipErrorInvalidValue;
}

template <int MT>
hipError_t dispatch_lpr(int lpr, int rw, const float* x, const LinearSegs& s, int M, int K,
                        hipStream_t stream) {
  switch (lpr) {
    case 16: return dispatch_rw<MT, 16>(rw, x, s, M, K, stream);
    case 32: return dispatch_rw<MT, 32>(rw, x, s, M, K, stream);
    case 64: return dispatch_rw<MT, 64>(rw, x, s, M, K, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace

bool gemv_config_valid(const GemvConfig& c) {
  if (c.rpw != 0) return c.mt == 1 && c.rpw == kRawkRows;
  const bool mt = c.mt == 1 || c.mt == 2 || c.mt == 4 || c.mt == 8;
  const bool lpr = c.lpr == 16 || c.lpr == 32 || c.lpr == 64;
  const bool rw = c.rw == 1 || c.rw == 2 || c.rw == 4 || c.rw == 8;
  return mt && lpr && rw;
}

GemvConfig gemv_pick_config(int M, int N, int K) {
  GemvConfig c;
  c.mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  // Launch shapes measured best on MI355X (about 8-16 rows per workgroup):
  // narrow lane groups for short rows, wide ones for long rows; one row per
  // lane group when there are few rows (the [896, 4864] Qwen down projection:
  // 5.2 us with 64 x 1 against 5.9 with 32 x 1 and 5.8 with 64 x 2).
  const int kb = K / kBlockElems;
  c.lpr = kb < 64 ? 16 : kb <= 128 ? 32 : 64;
  // Two rows per group also for 2 tokens on 32-lane groups of wide weights (Llama
  // qkv / gate at M = 2, K = 4096: 15.9 / 15.1 us against 18.1 / 17.3 with one
  // row; o_proj 8.9 against 8.4).  The row count does not change a row's sum.
  const bool two = c.mt == 8 || (c.lpr == 64 && c.mt == 1 && N > 2048) ||
                   (c.lpr == 32 && c.mt >= 4) || (c.lpr == 32 && c.mt == 2 && N >= 8192);
  c.rw = two ? 2 : 1;
  // One token on rows of more than 4096 elements: the row-span kernel (measured
  // figures at gemv_rawk_kernel; the rule ignores N, so fused and single
  // launches agree).
  (void)N;
  if (M == 1 && K > 4096) c.rpw = kRawkRows;
  return c;
}

hipError_t launch_gemv_segs(const GemvConfig& cfg, const float* x, const LinearSegs& s, int M,
                            int K, hipStream_t stream) {
  if (s.count < 1 || s.count > 3 || (s.mode == Epilogue::kSwiGLU && s.count != 2))
    return hipErrorInvalidValue;
  if (cfg.rpw != 0) {
    if (!gemv_config_valid(cfg)) return hipErrorInvalidValue;
    return launch_rawk(x, s, M, K, stream);
  }
  switch (cfg.mt) {
    case 1: return dispatch_lpr<1>(cfg.lpr, cfg.rw, x, s, M, K, stream);
    case 2: return dispatch_lpr<2>(cfg.lpr, cfg.rw, x, s, M, K, stream);
    case 4: return dispatch_lpr<4>(cfg.lpr, cfg.rw, x, s, M, K, stream);
    case 8: return dispatch_lpr<8>(cfg.lpr, cfg.rw, x, s, M, K, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(const GemvConfig& cfg, const float* x, const uint8_t* w,
                       const float* bias, float* y, int M, int N, int K,
                       hipStream_t stream) {
  LinearSegs s;
  s.seg[0] = LinearSeg{w, bias, y, N};
  return launch_gemv_segs(cfg, x, s, M, K, stream);
}

}  // namespace mle
