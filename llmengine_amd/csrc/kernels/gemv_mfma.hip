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
// blocks.  Lane l loads whole 34-byte blocks through a buffer resource: row
// l % 16, blocks 4u + l / 16 of the chunk (u = 0 .. KS/4-1).  A 4 x 4 transpose
// of 8-byte quant chunks across the four 16-lane rows (v_permlane32_swap then
// v_permlane16_swap, 8 instructions per 4 blocks) turns those registers straight
// into MFMA A fragments, with no LDS round trip.  Order of work: the slice's
// activation loads, the first chunk's weight loads (raw weights: every chunk's),
// the activation split into LDS B fragments (shared by the waves), one barrier,
// the other chunks' weight loads, then the multiplies chunk by chunk as the
// loads land.
//
// Split K.  When there are too few row tiles to fill the GPU, the K chunks are
// split over gridDim.y workgroups.  Each stores its 16 W x MT partial sums to its
// own aligned workspace region and bumps a per-tile counter; the last workgroup
// of a tile resets the counter to zero for the next launch on the stream and
// adds the partials in a fixed order (deterministic) plus bias, all its threads
// loading 16-byte pieces of every split at once, then writes y.  The
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

// Splits 8 activations into packed bf16 hi / mid / lo parts (4 dwords each):
// hi = x with the low 16 bits cleared, r = x - hi (exact), mid = r with the low
// 16 bits cleared, lo = r - mid (exact, <= 8 significant bits).  Finite x only.
__device__ __forceinline__ void split3_finite(const float (&v)[8], uint32_t (&hi)[4],
                                              uint32_t (&mid)[4], uint32_t (&lo)[4]) {
  uint32_t hb[8], rb[8], lb[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v[j]);
    const float r = v[j] - __builtin_bit_cast(float, b & 0xffff0000u);
    const uint32_t r_bits = __builtin_bit_cast(uint32_t, r);
    const float l = r - __builtin_bit_cast(float, r_bits & 0xffff0000u);
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

// Same split for any x: +-Inf is carried whole in hi (mid = lo = 0; x - hi would
// be NaN) and NaN stays NaN in every part.
__device__ __forceinline__ void split3_any(const float (&v)[8], uint32_t (&hi)[4],
                                           uint32_t (&mid)[4], uint32_t (&lo)[4]) {
  uint32_t hb[8], rb[8], lb[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v[j]);
    const float h = __builtin_bit_cast(float, b & 0xffff0000u);
    const float r = (v[j] == h) ? 0.0f : v[j] - h;
    const uint32_t r_bits = __builtin_bit_cast(uint32_t, r);
    const float l = r - __builtin_bit_cast(float, r_bits & 0xffff0000u);
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

template <int MT, int W = 4>
struct Cols {
  static constexpr int P = (3 * MT + 15) / 16;  // chained MFMAs per tile
  // Real virtual columns of the last MFMA; when they fit in 8, its B fragment is
  // stored at half size plus one zero slot that lanes of columns 8..15 read.  The
  // smaller LDS footprint lets one more 4-wave workgroup share a CU; 8-wave
  // workgroups are register-bound already and run faster on full fragments
  // (measured on MI355X).
  static constexpr int RL = 3 * MT - 16 * (P - 1);
  static constexpr bool HALF = RL <= 8 && W <= 4;
  static constexpr int LASTC = HALF ? 8 : 16;            // stored columns, last MFMA
  static constexpr int PADC = 16 * (P - 1) + LASTC - 3 * MT;  // stored columns kept zero
  static constexpr int FB = (P - 1) * 1024 + (HALF ? 512 + 16 : 1024);  // bytes per block
};

template <int MT, int W, int KSL>
struct Shape {
  static constexpr int NT = 64 * W;               // threads
  static constexpr int R = 16 * W;                // output rows per workgroup
  static constexpr int P = Cols<MT>::P;
  static constexpr int KS = 8;                    // blocks per chunk (one load set pair)
  static constexpr int NL = KS / 4;               // blocks per lane per chunk
  static constexpr int NCH = KSL / KS;            // chunks per workgroup
  static constexpr int BBUF = KSL * Cols<MT, W>::FB;  // B fragments of the K slice (bytes)
  static constexpr int XITEMS = MT * KSL * 4;     // (token, k chunk, block)
  static constexpr int XPT = (XITEMS + NT - 1) / NT;
  static constexpr int OUTS = 16 * MT;            // outputs per wave
  static constexpr int OPL = (OUTS + 63) / 64;    // outputs per lane
};

// Byte offset of B-fragment slot (block kb, MFMA p, k chunk c, virtual column n
// of the MFMA; n < 8 for a half-size last fragment).  The 16-byte slot of lane
// (c, n) sits at position (n + ROT c) % 16 of its 16-slot row (% 8 of an 8-slot
// row in a half fragment): the activation split runs tokens fastest, so 16
// consecutive threads write (8 tokens x 2 k chunks) or (4 x 4) distinct slots of
// a 256-byte bank row, and an MFMA read of a fragment is a permutation within
// each row.  A block's fragments are FB bytes apart, so a lane's read address is
// one register plus an immediate per (block, MFMA).
template <int MT>
struct Slot {
  static constexpr int ROT = MT >= 8 ? 8 : 4;
};
template <int MT, int W, int P>
__device__ __forceinline__ int bslot(int kb, int p, int c, int n) {
  using C = Cols<MT, W>;
  if (C::HALF && p == P - 1)
    return kb * C::FB + p * 1024 + (c * 8 + ((n + 4 * c) & 7)) * 16;
  return kb * C::FB + p * 1024 + (c * 16 + ((n + Slot<MT>::ROT * c) & 15)) * 16;
}
// Read slot of lane (c, n): as bslot, except that columns 8..15 of a half-size
// last fragment read the block's zero slot.
template <int MT, int W, int P>
__device__ __forceinline__ int bslot_rd(int kb, int p, int c, int n) {
  using C = Cols<MT, W>;
  if (C::HALF && p == P - 1 && n >= 8) return kb * C::FB + p * 1024 + 512;
  return bslot<MT, W, P>(kb, p, c, n);
}

// Buffer resource over [base, base + bytes): loads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Output segments as the kernel sees them: segment i owns the row tiles
// [tile_end[i-1], tile_end[i]) of the grid.
struct DecodeArgs {
  LinearSeg seg[3];
  unsigned tile_end[3];
  int count;
};

// silu(g) * u with the reference's operation order (cpu_kernels.cpp:848-858).
__device__ __forceinline__ float silu_mul(float g, float u) {
  return (g / (1.0f + expf(-g))) * u;
}

// MODE 0: plain / multi-output Linear.  MODE 1 (SwiGLU): waves [0, W/2) take
// rows of the gate weight, waves [W/2, W) the same rows of the up weight, and
// the epilogue writes silu(gate) * up.
template <int MT, int W, int KSL, int MODE, int LAYOUT>
__global__ __launch_bounds__(64 * W) void gemv_q8_0_mfma_kernel(
    const float* __restrict__ x, const DecodeArgs args, int M, int K,
    float* __restrict__ partials, uint32_t* __restrict__ counters) {
  using S = Shape<MT, W, KSL>;
  constexpr bool kSwi = MODE == 1;
  static_assert(!kSwi || W % 2 == 0, "SwiGLU pairs gate and up waves");
  constexpr int RW = kSwi ? W / 2 : W;  // waves per weight
  constexpr int ROUT = 16 * RW;         // output rows per workgroup
  constexpr int P = S::P;
  constexpr int KS = S::KS;
  constexpr int NL = S::NL;
  constexpr int NCH = S::NCH;
  constexpr int XPT = S::XPT;
  static_assert(KSL % KS == 0, "K slice = whole chunks");
  __shared__ __attribute__((aligned(16))) uint8_t bfr[S::BBUF];
  __shared__ __attribute__((aligned(16))) float scl[W][KS][16];
  __shared__ __attribute__((aligned(16))) uint8_t xdummy[16];
  __shared__ float gate_out[kSwi ? RW : 1][kSwi ? S::OPL * 64 : 1];
  // The split-K arrival count, in the last dword of the B area (free by then;
  // the reductions below use its start): 8-token fragments of a 16-block slice
  // then take 26880 bytes of LDS in all, six 4-wave workgroups per CU.
  uint32_t& arrived = *reinterpret_cast<uint32_t*>(bfr + S::BBUF - 4);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int KB = K / kBlockElems;
  const uint32_t row_bytes = (uint32_t)KB * kBlockBytes;
  const int kb0 = blockIdx.y * KSL;                 // first block of this K slice
  const int nblk = min(KSL, KB - kb0);              // blocks in this slice

  // Segment of this row tile (uniform selects: no indexing into the argument).
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
  const int wrow = kSwi ? wave % RW : wave;  // this wave's 16-row group
  if (kSwi && wave >= RW) w = args.seg[1].w;
  const int64_t n0 = (int64_t)(tile - tile0) * ROUT;

  // Weights: one buffer resource over this workgroup's rows (rows past N read
  // as zero).  Lane (g, r16) of wave w loads row 16w + r16, blocks
  // kb0 + 8c + 4u + g: a per-lane constant offset plus a wave-uniform one.  The
  // uniform part is a multiple of 4 (34 * 4u, 34 * 8c), so each lane's block
  // alignment (the realignment case of load_block_raw) never changes.
  const uint8_t* wbase = w + n0 * row_bytes;
  const int64_t rows_here = min((int64_t)ROUT, (int64_t)N - n0);
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(wbase, (uint32_t)(rows_here * row_bytes));
  const uint32_t lane_off = (uint32_t)(wrow * 16 + r16) * row_bytes +
                            (uint32_t)(kb0 + g) * kBlockBytes;
  const uint32_t mis = (uint32_t)(((uintptr_t)wbase + lane_off) & 2u);
  const uint32_t voff = lane_off + mis;
  const uint32_t uoff = lane_off + (mis ? 0u : 32u);

  // 0. The slice's activation loads go first: vector-memory loads complete in
  //    order, so the split below then waits only for these, and it and the
  //    barrier overlap the weight loads still in flight.  Item = (token m
  //    fastest, k quarter, block); items past the end (token >= M, block >=
  //    nblk, or no item) read zeros.
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)((int64_t)M * K * 4));
  f32x4 xv[XPT][2];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int it = tid + S::NT * i;
    const int m = it % MT, q = it / MT;
    const int kb = q >> 2;
    const uint32_t off = it < S::XITEMS && kb < nblk
                             ? (uint32_t)((m * K + (kb0 + kb) * kBlockElems + 8 * (q & 3)) * 4)
                             : 0x80000000u;
    xv[i][0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
    xv[i][1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off + 16, 0, 0));
  }

  // 1. The weight loads of this wave's 16 rows x KSL blocks, in chunks of KS
  //    blocks (tiled: the first chunk before the activation split, the others
  //    right after it; raw: all up front).  Blocks past the slice's end read as
  //    zeros: their per-lane offset is put
  //    past the buffer (the range check applies to the per-lane offset), so no
  //    lane ever addresses a byte outside its slice of the weight tensor.
  constexpr bool kTiled = LAYOUT == int(WeightLayout::kTiled);
  RawBlock wr[kTiled ? 1 : NCH][NL];
  u32x4 tq[kTiled ? NCH : 1][4];  // tiled: the chunk's 4 block pairs
  uint32_t ts[kTiled ? NCH : 1];  // tiled: one scale dword per chunk
  // Chunk c's loads (raw: NL load sets of whole blocks; tiled: 4 quant pieces
  // and a scale dword).
  auto issue_chunk = [&](int c) {
  if constexpr (!kTiled) {
#pragma unroll
      for (int u = 0; u < NL; ++u) {
        const int b = KS * c + 4 * u;  // first block of the load set (lane adds g)
        const bool live = b + g < nblk;
        const uint32_t soff = b < nblk ? (uint32_t)b * kBlockBytes : 0u;  // uniform
        const uint32_t v8 = live ? voff : 0x80000000u;
        const uint32_t v2 = live ? uoff : 0x80000000u;
        const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8, soff, 0);
        const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8 + 16, soff, 0);
        wr[c][u].v0 = u32x4_a4{v0.x, v0.y, v0.z, v0.w};
        wr[c][u].v1 = u32x4_a4{v1.x, v1.y, v1.z, v1.w};
        wr[c][u].u = __builtin_amdgcn_raw_buffer_load_b16(wrs, v2, soff, 0);
        wr[c][u].mis = mis;
      }
  } else {
    // Tiled weights: the wave's row group streams its quant pieces (1 KB per
    // block pair, one 16-byte slot per lane: rows l % 16, quants 8 (l/16) .. +7
    // of both blocks) and scale pieces (lane l reads dword l of the chunk's four
    // 64-byte pieces: pair l/16, row l % 16).  Pairs past the slice read as zero.
    const int KP = (KB + 1) >> 1;
    const int64_t G = ((int64_t)N + kTileRows - 1) / kTileRows;
    const int64_t rg = n0 / kTileRows + wrow;
    const int64_t rgc = rg < G ? rg : 0;
    const uint8_t* qb = w + rgc * KP * kTilePieceBytes;
    const uint8_t* sb = w + G * KP * kTilePieceBytes + rgc * KP * kTileScaleBytes;
    const __amdgpu_buffer_rsrc_t qrs =
        make_rsrc(qb, rg < G ? (uint32_t)KP * kTilePieceBytes : 0u);
    const __amdgpu_buffer_rsrc_t srs =
        make_rsrc(sb, rg < G ? (uint32_t)KP * kTileScaleBytes : 0u);
    const int p0 = kb0 >> 1;  // KSL is even
    {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int pr = (KS / 2) * c + u;  // pair within the slice
        const uint32_t off = 2 * pr < nblk
                                 ? (uint32_t)(p0 + pr) * kTilePieceBytes + (uint32_t)lane * 16
                                 : 0x80000000u;
        tq[c][u] = __builtin_amdgcn_raw_buffer_load_b128(qrs, off, 0, kNonTemporal);
      }
      const int ps = (KS / 2) * c + g;  // scale pair of this lane
      ts[c] = __builtin_amdgcn_raw_buffer_load_b32(
          srs, 2 * ps < nblk ? (uint32_t)(p0 + (KS / 2) * c) * kTileScaleBytes + (uint32_t)lane * 4
                             : 0x80000000u,
          0, 0);
    }
  }
  };
  // Tiled weights: the first chunk before the split, the others right after it.
  // Raw weights: every chunk up front (issuing the later ones after the split
  // measured 1.04-1.15x slower on the Llama shapes at 4 and 8 tokens).
  constexpr int kPre = kTiled ? 1 : NCH;
#pragma unroll
  for (int c = 0; c < kPre; ++c) issue_chunk(c);

  // 2. B fragments of the whole K slice (activations split into bf16 parts),
  //    shared by the workgroup's waves.  B fragment (block kb, MFMA p): lane l
  //    holds virtual column l % 16, k = 8 (l/16) .. +7.  Every thread runs every
  //    item slot, those past XITEMS writing a dummy LDS slot.
  {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int it = tid + S::NT * i;
      const bool real = S::XITEMS % S::NT == 0 || it < S::XITEMS;
      const int m = it % MT, q = it / MT;
      const int kb = q >> 2, c = q & 3;
      const float v[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                          xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
      bool finite = true;
#pragma unroll
      for (int j = 0; j < 8; ++j) finite &= !__builtin_amdgcn_class(v[j], 0x207);  // NaN, +-Inf
      uint32_t parts[3][4];
      if (__builtin_expect(finite, 1))
        split3_finite(v, parts[0], parts[1], parts[2]);
      else
        split3_any(v, parts[0], parts[1], parts[2]);
#pragma unroll
      for (int part = 0; part < 3; ++part) {
        const int vc = part * MT + m;
        uint8_t* dst = real ? bfr + bslot<MT, W, P>(kb, vc >> 4, c, vc & 15) : xdummy;
        *reinterpret_cast<u32x4*>(dst) =
            u32x4{parts[part][0], parts[part][1], parts[part][2], parts[part][3]};
      }
    }
    // Virtual columns past 3*MT are never written above: zero them.
    if constexpr (Cols<MT, W>::HALF) {
      for (int kb = tid; kb < KSL; kb += S::NT)
        *reinterpret_cast<u32x4*>(bfr + kb * Cols<MT, W>::FB + (P - 1) * 1024 + 512) =
            u32x4{0u, 0u, 0u, 0u};
    }
    if constexpr (Cols<MT, W>::PADC > 0) {
      constexpr int PADC = Cols<MT, W>::PADC;
      for (int it = tid; it < KSL * 4 * PADC; it += S::NT) {
        const int kb = it / (4 * PADC), q = it % (4 * PADC);
        const int c = q / PADC, vc = 3 * MT + q % PADC;
        *reinterpret_cast<u32x4*>(bfr + bslot<MT, W, P>(kb, vc >> 4, c, vc & 15)) =
            u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  __syncthreads();
  // Tiled weights: the other chunks' loads go out once the split is done, so a
  // wave that waits on full request queues while issuing them has only
  // multiplies and the hand-off left after that wait (MI355X: o_proj 4096 x 4096
  // at 8 tokens 0.96x against issuing every chunk first).
#pragma unroll
  for (int c = kPre; c < NCH; ++c) issue_chunk(c);

  // 3. Each wave multiplies its rows chunk by chunk as the loads land: realign,
  //    scales to (wave-private) LDS, in-register transpose into A fragments,
  //    P chained MFMAs per block, fp32 scale FMA.  No barrier.
  f32x4 accs[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  // Block kc of chunk (kb = block within the slice): P chained MFMAs against
  // the token columns, then the fp32 scale FMA into an accumulator that takes
  // every other block (even blocks in accs[0], odd in accs[1], in K order).
  auto block_mma = [&](int kc, int kb, const bf16x8_t a, f32x4& a4) {
    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        a, *reinterpret_cast<const bf16x8_t*>(bfr + bslot_rd<MT, W, P>(kb, 0, g, r16)),
        f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
    for (int p = 1; p < P; ++p)
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          a, *reinterpret_cast<const bf16x8_t*>(bfr + bslot_rd<MT, W, P>(kb, p, g, r16)), d, 0,
          0, 0);
    // D layout: lane l holds rows 4 (l/16) + v (v = 0..3), virtual column l % 16.
    const f32x4 sc = *reinterpret_cast<const f32x4*>(&scl[wave][kc][4 * g]);
    a4.x = __builtin_fmaf(sc.x, d.x, a4.x);
    a4.y = __builtin_fmaf(sc.y, d.y, a4.y);
    a4.z = __builtin_fmaf(sc.z, d.z, a4.z);
    a4.w = __builtin_fmaf(sc.w, d.w, a4.w);
  };
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if constexpr (kTiled) {
      // Scales of pair g (blocks 2g, 2g+1 of the chunk) for row r16; the quant
      // slots are A fragments already.
      scl[wave][2 * g][r16] = scale_to_f32_fast(ts[c] & 0xffffu);
      scl[wave][2 * g + 1][r16] = scale_to_f32_fast(ts[c] >> 16);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const u32x4 q = tq[c][u];
        block_mma(2 * u, KS * c + 2 * u, quants_to_bf16(q.x, q.y), accs[0]);
        block_mma(2 * u + 1, KS * c + 2 * u + 1, quants_to_bf16(q.z, q.w), accs[1]);
      }
    } else {
      Block blk[NL];
#pragma unroll
      for (int u = 0; u < NL; ++u) {
        blk[u] = finish_block(wr[c][u]);
        const bool valid = KS * c + 4 * u + g < nblk;
        scl[wave][4 * u + g][r16] = valid ? scale_to_f32_fast(blk[u].scale_bits) : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < NL; ++u) {
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = blk[u].q[i];
        transpose_chunks(q);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          block_mma(4 * u + j, KS * c + 4 * u + j, quants_to_bf16(q[2 * j], q[2 * j + 1]),
                    accs[j & 1]);
      }
    }
  }
  const f32x4 acc = accs[0] + accs[1];

  // Sum the part columns of each token (within the wave), in a wave-private
  // slice of the B-fragment area once every wave is done with the fragments:
  // no LDS of its own, which lets a sixth 4-wave workgroup of 8-token fragments
  // onto a CU.
  static_assert(W * 16 * 17 * 4 <= S::BBUF - 4, "the part sums fit the B area");
  __syncthreads();
  float (*red)[16][17] = reinterpret_cast<float (*)[16][17]>(bfr);
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

  // Final values of this wave's outputs -> y (plain: + bias; SwiGLU: the up
  // waves combine with the gate waves' values through LDS).
  auto write_out = [&](const float (&v)[S::OPL]) {
    if constexpr (kSwi) {
      if (wave < RW) {
#pragma unroll
        for (int o = 0; o < S::OPL; ++o) gate_out[wrow][64 * o + lane] = v[o];
      }
      __syncthreads();
      if (wave < RW) return;
    }
#pragma unroll
    for (int o = 0; o < S::OPL; ++o) {
      const int idx = lane + 64 * o;
      const int m = idx >> 4, rr = idx & 15;
      const int64_t n = n0 + wrow * 16 + rr;
      if (idx >= S::OUTS || m >= M || n >= N) continue;
      if constexpr (kSwi)
        y[(int64_t)m * N + n] = silu_mul(gate_out[wrow][64 * o + lane], v[o]);
      else
        y[(int64_t)m * N + n] = v[o] + (bias ? bias_at(bias, bias_bf16, n) : 0.0f);
    }
  };

  if (gridDim.y == 1) {
    write_out(outv);
    return;
  }

  // Split K: partials [tile][split][wave][MT][16], then the last workgroup
  // reduces.  The partials travel by device-scope (sc1: L2 write-through /
  // coherent) buffer stores and loads; plain (non-atomic) accesses, so the S
  // loads of the reduction issue together instead of one round trip each.
  constexpr int REGION = S::R * MT;
  constexpr int SC1 = 16;  // cache-policy bit: device scope
  const __amdgpu_buffer_rsrc_t prs =
      make_rsrc(partials + (int64_t)blockIdx.x * gridDim.y * REGION,
                (uint32_t)(gridDim.y * REGION * 4));
#pragma unroll
  for (int o = 0; o < S::OPL; ++o) {
    const int idx = lane + 64 * o;
    if (idx < S::OUTS && (idx >> 4) < M)
      __builtin_amdgcn_raw_buffer_store_b32(
          __builtin_bit_cast(uint32_t, outv[o]), prs,
          (uint32_t)((blockIdx.y * REGION + wave * S::OUTS + idx) * 4), 0, SC1);
  }
  // Each tile's counter sits alone in a 128-byte line (kCounterStride), so the
  // tiles' arrivals do not queue on one line.
  uint32_t* const counter = counters + (size_t)blockIdx.x * kCounterStride;
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

  if (gridDim.y <= 8) {
    // Up to 8 splits: each lane sums its outputs' partials in split order, the
    // loads of all splits issued together.
    float total[S::OPL];
#pragma unroll
    for (int o = 0; o < S::OPL; ++o) {
      const int idx = lane + 64 * o;
      float v[8];
#pragma unroll
      for (int sp = 0; sp < 8; ++sp)
        v[sp] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(
                       prs,
                       idx < S::OUTS && (idx >> 4) < M && sp < (int)gridDim.y
                           ? (uint32_t)((sp * REGION + wave * S::OUTS + idx) * 4)
                           : 0x80000000u,
                       0, SC1));
      float s = 0.0f;
#pragma unroll
      for (int sp = 0; sp < 8; ++sp)
        if (sp < (int)gridDim.y) s += v[sp];
      total[o] = s;
    }
    write_out(total);
    return;
  }

  // More splits: the last workgroup reduces with every thread at once. The tile's partials
  // are CHUNKS 16-byte pieces per split; TPC threads share a piece, thread
  // (h, c) summing piece c of splits [h SPT, (h+1) SPT) in split order with all
  // loads of a batch of 8 issued together (one round trip per batch instead of
  // one per split), then the TPC sums of a piece are added in h order in LDS.
  // The B-fragment LDS area is free by now (every wave has passed the barrier
  // after its MFMAs) and holds the sums, then the tile's totals.
  constexpr int CHUNKS = REGION / 4;
  constexpr int TPC = S::NT / CHUNKS;  // 16 / MT threads per piece, rounded down
  static_assert(TPC >= 1, "one thread per piece at least");
  static_assert((4 * S::NT + REGION) * 4 <= S::BBUF - 4, "reduction scratch fits the B area");
  float* const sums = reinterpret_cast<float*>(bfr);  // [TPC][CHUNKS] x 4
  float* const tot = sums + 4 * S::NT;                // [REGION]
  {
    const int c = tid % CHUNKS, h = tid / CHUNKS;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    const int off = 4 * c;  // float offset inside a split's region: wave, token, 4 rows
    if (h < TPC && ((off % S::OUTS) >> 4) < M) {
      const unsigned nspl = gridDim.y, spt = (nspl + TPC - 1) / TPC;
      const unsigned s0 = h * spt, s1 = min(nspl, s0 + spt);
      for (unsigned sp = s0; sp < s1; sp += 8) {
        f32x4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          v[j] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         prs, sp + j < s1 ? (uint32_t)(((sp + j) * REGION + off) * 4) : 0x80000000u,
                         0, SC1));
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (sp + j < s1) s += v[j];
      }
    }
    if (h < TPC) *reinterpret_cast<f32x4*>(sums + 4 * tid) = s;
  }
  __syncthreads();
  for (int c = tid; c < CHUNKS; c += S::NT) {
    f32x4 t = *reinterpret_cast<const f32x4*>(sums + 4 * c);
    for (int h = 1; h < TPC; ++h) t += *reinterpret_cast<const f32x4*>(sums + 4 * (h * CHUNKS + c));
    *reinterpret_cast<f32x4*>(tot + 4 * c) = t;
  }
  __syncthreads();
  float total[S::OPL];
#pragma unroll
  for (int o = 0; o < S::OPL; ++o) {
    const int idx = lane + 64 * o;
    total[o] = idx < S::OUTS ? tot[wave * S::OUTS + idx] : 0.0f;
  }
  write_out(total);
}

// Row-range decode (below): 16-row groups per workgroup for G groups on the
// GPU's 256 CUs.
int rows_groups_per_workgroup(int64_t G) { return (int)((G + 255) / 256); }

// Row-range MFMA decode without split K (3-8 tokens; tiled weights, and raw
// weights at 3-4 tokens and in the SwiGLU launches).  The
// split-K kernel above needs a hand-off between the workgroups of a row tile
// (partial stores, their completion, a counter, the read-back), about 3 us at
// the end of every launch.  Here a workgroup owns whole rows instead: NG 16-row
// groups of WG waves each and all of K, so its waves add their sums in LDS and
// nothing crosses workgroups.  The price is that every workgroup splits all of
// K's activations: that pays where 2-4 groups share each workgroup's split
// (11008 or 12288 outputs over 256 CUs), or for 4096 outputs at 4 tokens with 16
// waves on the one group (o_proj); not for K = 11008 (down).
//
// K is walked in phases of PHB blocks: a phase's activations are split once into
// LDS B fragments (the layout and arithmetic of the kernel above) shared by every
// group; wave (group lg, index qw) multiplies block pairs
// [PHB/2 ph + PHB/(2 WG) qw, + PHB/(2 WG)) of its group, 4 pairs (one 16-byte
// quant slot and one scale dword per lane each) at a time.  RING 4-pair chunks of
// loads are in flight ahead of the chunk being multiplied: issuing a whole share
// up front stalls a wave on the full request queue before its first multiply
// (10-15% slower), and deeper rings measured slower too.  With NBUF = 2 the
// fragments of phase ph + 1 are split into the second buffer while phase ph is
// multiplied (one barrier per phase); with NBUF = 1 the split waits for the
// phase before it.  Per block and wave the arithmetic is the split-K kernel's
// (P chained MFMAs, fp32 scale FMA into even/odd accumulators); the WG waves of
// a group then add their sums in wave order, so results are deterministic
// (rel-L2 ~1e-7 from the split-K kernel, which groups the K sum differently).
// Output segments of a row-range launch: segment i owns the 16-row groups
// [grp_end[i-1], grp_end[i]) of the grid (multi-output Linear: q, k, v).
struct RowsArgs {
  LinearSeg seg[3];
  unsigned grp_end[3];
  int count;
};

// MODE 1 (SwiGLU): groups [0, NG/2) of a workgroup hold rows of the gate weight
// (seg[0]) and groups [NG/2, NG) the same rows of the up weight (seg[1]); the
// first wave of each gate group writes silu(gate) * up to seg[0].y.  grp_end[0]
// then counts the gate weight's groups.
template <int MT, int NG, int NPH, int PHB, int NBUF, int RING, int WG, int MODE, int LAYOUT>
__global__ __launch_bounds__(64 * WG * NG) void gemv_mfma_rows_kernel(
    const float* __restrict__ x, const RowsArgs args, int M, int K) {
  constexpr bool kSwi = MODE == 1;
  constexpr bool kTiled = LAYOUT == int(WeightLayout::kTiled);
  static_assert(!kSwi || NG % 2 == 0, "SwiGLU pairs gate and up groups");
  constexpr int NGH = kSwi ? NG / 2 : NG;  // output groups per workgroup
  constexpr int W = WG * NG;
  constexpr int NT = 64 * W;
  constexpr int P = Cols<MT>::P;
  using C = Cols<MT, 4>;                // half-size last fragment when it fits
  constexpr int PHP = PHB / 2;          // block pairs per phase
  constexpr int WPP = PHP / WG;         // pairs per wave per phase
  static_assert(WPP % 4 == 0, "whole 4-pair chunks per wave");
  constexpr int NCK = WPP / 4;          // chunks per wave per phase
  constexpr int TC = NPH * NCK;         // chunks per wave
  constexpr int BBUF = PHB * C::FB;
  constexpr int XITEMS = MT * PHB * 4;  // (token, k quarter, block) per phase
  static_assert(XITEMS % 64 == 0, "activation items fill whole waves");
  constexpr int XPT = (XITEMS + NT - 1) / NT;
  constexpr int OUTS = 16 * MT;
  constexpr int OPL = (OUTS + 63) / 64;
  static_assert(W * 16 * 17 * 4 <= BBUF, "the group reduction fits the B area");
  __shared__ __attribute__((aligned(16))) uint8_t bfr[NBUF * BBUF];
  __shared__ __attribute__((aligned(16))) float scl[W][8][16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r16 = lane & 15;
  const int lg = wave / WG, qw = wave % WG;
  const int KB = K / kBlockElems;
  const int KP = (KB + 1) >> 1;
  // This wave's group: global index -> segment (uniform selects: no indexing
  // into the argument) and its group within the segment's weight.
  const unsigned grp = blockIdx.x * NGH + (kSwi ? lg % NGH : lg);
  const int si = kSwi ? (lg >= NGH ? 1 : 0)
                      : (args.count > 1 && grp >= args.grp_end[0])
                            ? ((args.count > 2 && grp >= args.grp_end[1]) ? 2 : 1)
                            : 0;
  const unsigned grp0 = kSwi || si == 0 ? 0u : si == 1 ? args.grp_end[0] : args.grp_end[1];
  const uint8_t* w = si == 0 ? args.seg[0].w : si == 1 ? args.seg[1].w : args.seg[2].w;
  const void* bias = si == 0 ? args.seg[0].bias : si == 1 ? args.seg[1].bias : args.seg[2].bias;
  const int bias_bf16 =
      si == 0 ? args.seg[0].bias_bf16 : si == 1 ? args.seg[1].bias_bf16 : args.seg[2].bias_bf16;
  float* y = si == 0 ? args.seg[0].y : si == 1 ? args.seg[1].y : args.seg[2].y;
  const int N = si == 0 ? args.seg[0].N : si == 1 ? args.seg[1].N : args.seg[2].N;
  const int64_t G = ((int64_t)N + kTileRows - 1) / kTileRows;
  const unsigned grp_total = kSwi || args.count == 1 ? args.grp_end[0]
                             : args.count == 2      ? args.grp_end[1]
                                                    : args.grp_end[2];
  const bool live_g = grp < grp_total;
  const int64_t rg = live_g ? (int64_t)(grp - grp0) : 0;  // group within the segment's weight
  const int64_t rgc = rg;

  // Activations of one phase: item (token m fastest, k quarter, block), 8 fp32.
  // Items past M or K read zeros through the range check of the per-lane offset.
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)((int64_t)M * K * 4));
  f32x4 xv[NPH][XPT][2];
  auto load_x = [&](int ph) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int it = tid + NT * i;
      const int m = it % MT, q = it / MT;
      const int kb = ph * PHB + (q >> 2);
      uint32_t off = it < XITEMS && kb < KB && m < M
                         ? (uint32_t)((m * K + kb * kBlockElems + 8 * (q & 3)) * 4)
                         : 0x80000000u;
      asm volatile("" : "+v"(off));  // the load stays where it is written
      xv[ph][i][0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
      xv[ph][i][1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off + 16, 0, 0));
    }
  };

  // Tiled: quant slots (lane l: rows l % 16, quants 8 (l/16) .. +7 of both
  // blocks of a pair) and scale dwords (lane l: pair l/16 of the chunk, row
  // l % 16) of this wave's group; a group past N reads zeros (empty buffer).
  // Raw (SwiGLU launches; plain ones at 4 tokens): a chunk's 8 blocks as two load sets of whole 34-byte
  // blocks, lane (g, r16) taking block 4u + g of the chunk in row r16 of the
  // group, as the split-K kernel's raw path (rows past N and blocks past K read
  // as zeros).  A wave's chunks start 8-block (272-byte) steps apart, so each
  // lane's 4-byte alignment phase is fixed.
  const uint8_t* qb = w + rgc * KP * kTilePieceBytes;
  const uint8_t* sb = w + G * KP * kTilePieceBytes + rgc * KP * kTileScaleBytes;
  const __amdgpu_buffer_rsrc_t qrs = make_rsrc(qb, live_g ? (uint32_t)KP * kTilePieceBytes : 0u);
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(sb, live_g ? (uint32_t)KP * kTileScaleBytes : 0u);
  const uint32_t row_bytes = (uint32_t)KB * kBlockBytes;
  const uint8_t* gbase = w + rgc * kTileRows * (int64_t)row_bytes;
  const int64_t grows = live_g ? min((int64_t)kTileRows, (int64_t)N - rgc * kTileRows) : 0;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(gbase, (uint32_t)(grows * row_bytes));
  const uint32_t lane_off = (uint32_t)r16 * row_bytes + (uint32_t)(2 * qw * WPP + g) * kBlockBytes;
  const uint32_t mis = (uint32_t)(((uintptr_t)gbase + lane_off) & 2u);
  const uint32_t voff = lane_off + mis;
  const uint32_t uoff = lane_off + (mis ? 0u : 32u);
  u32x4 tq[kTiled ? TC : 1][4];
  uint32_t ts[kTiled ? TC : 1];
  RawBlock wr[kTiled ? 1 : TC][2];
  auto load_chunk = [&](int cg) {  // chunk cg = ph * NCK + ck
    const int ph = cg / NCK, ck = cg % NCK;
    const int p0 = ph * PHP + qw * WPP + 4 * ck;
    if constexpr (kTiled) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int pr = p0 + u;
        uint32_t off =
            pr < KP ? (uint32_t)pr * kTilePieceBytes + (uint32_t)lane * 16 : 0x80000000u;
        asm volatile("" : "+v"(off));
        tq[cg][u] = __builtin_amdgcn_raw_buffer_load_b128(qrs, off, 0, kNonTemporal);
      }
      const int ps = p0 + g;
      uint32_t soff = ps < KP ? (uint32_t)ps * kTileScaleBytes + (uint32_t)r16 * 4 : 0x80000000u;
      asm volatile("" : "+v"(soff));
      ts[cg] = __builtin_amdgcn_raw_buffer_load_b32(srs, soff, 0, 0);
    } else {
      // Blocks 2 p0 + 4u + g: the lane's own offset plus a wave-uniform 4-byte multiple.
      const int bw = 2 * (p0 - qw * WPP);  // first block of the chunk past the wave's start
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const bool live = 2 * p0 + 4 * u + g < KB;
        const uint32_t soff = (uint32_t)(bw + 4 * u) * kBlockBytes;  // uniform
        uint32_t v8 = live ? voff + soff : 0x80000000u;
        uint32_t v2 = live ? uoff + soff : 0x80000000u;
        asm volatile("" : "+v"(v8), "+v"(v2));
        const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8, 0, 0);
        const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8 + 16, 0, 0);
        wr[cg][u].v0 = u32x4_a4{v0.x, v0.y, v0.z, v0.w};
        wr[cg][u].v1 = u32x4_a4{v1.x, v1.y, v1.z, v1.w};
        wr[cg][u].u = __builtin_amdgcn_raw_buffer_load_b16(wrs, v2, 0, 0);
        wr[cg][u].mis = mis;
      }
    }
  };
  load_x(0);  // first: the split waits only for these
  if constexpr (NBUF == 2) {
    if (NPH > 1) load_x(1);
  }
#pragma unroll
  for (int cg = 0; cg < RING && cg < TC; ++cg) load_chunk(cg);

  // Stored virtual columns past 3 MT are never written by the split: zero once.
  if constexpr (C::HALF) {
    for (int kb = tid; kb < NBUF * PHB; kb += NT)
      *reinterpret_cast<u32x4*>(bfr + kb * C::FB + (P - 1) * 1024 + 512) = u32x4{0u, 0u, 0u, 0u};
  }
  if constexpr (C::PADC > 0) {
    constexpr int PADC = C::PADC;
    for (int it = tid; it < NBUF * PHB * 4 * PADC; it += NT) {
      const int kb = it / (4 * PADC), q = it % (4 * PADC);
      const int c = q / PADC, vc = 3 * MT + q % PADC;
      *reinterpret_cast<u32x4*>(bfr + bslot<MT, 4, P>(kb, vc >> 4, c, vc & 15)) =
          u32x4{0u, 0u, 0u, 0u};
    }
  }

  f32x4 accs[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  auto block_mma = [&](const uint8_t* bb, int kc, int kb, const bf16x8_t a, f32x4& a4) {
    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        a, *reinterpret_cast<const bf16x8_t*>(bb + bslot_rd<MT, 4, P>(kb, 0, g, r16)),
        f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
    for (int p = 1; p < P; ++p)
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          a, *reinterpret_cast<const bf16x8_t*>(bb + bslot_rd<MT, 4, P>(kb, p, g, r16)), d, 0,
          0, 0);
    const f32x4 sc = *reinterpret_cast<const f32x4*>(&scl[wave][kc][4 * g]);
    a4.x = __builtin_fmaf(sc.x, d.x, a4.x);
    a4.y = __builtin_fmaf(sc.y, d.y, a4.y);
    a4.z = __builtin_fmaf(sc.z, d.z, a4.z);
    a4.w = __builtin_fmaf(sc.w, d.w, a4.w);
  };

  auto split_phase = [&](int ph) {
    uint8_t* bb = bfr + (ph % NBUF) * BBUF;
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int it = tid + NT * i;
      if (XITEMS % NT != 0 && it >= XITEMS) continue;  // whole waves
      const int m = it % MT, q = it / MT;
      const int kb = q >> 2, c = q & 3;
      float v[8] = {xv[ph][i][0].x, xv[ph][i][0].y, xv[ph][i][0].z, xv[ph][i][0].w,
                    xv[ph][i][1].x, xv[ph][i][1].y, xv[ph][i][1].z, xv[ph][i][1].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(v[j]));  // the split stays in its phase
      bool finite = true;
#pragma unroll
      for (int j = 0; j < 8; ++j) finite &= !__builtin_amdgcn_class(v[j], 0x207);
      uint32_t parts[3][4];
      if (__builtin_expect(finite, 1))
        split3_finite(v, parts[0], parts[1], parts[2]);
      else
        split3_any(v, parts[0], parts[1], parts[2]);
#pragma unroll
      for (int part = 0; part < 3; ++part) {
        const int vc = part * MT + m;
        *reinterpret_cast<u32x4*>(bb + bslot<MT, 4, P>(kb, vc >> 4, c, vc & 15)) =
            u32x4{parts[part][0], parts[part][1], parts[part][2], parts[part][3]};
      }
    }
  };
  auto compute_phase = [&](int ph) {
    const uint8_t* bb = bfr + (ph % NBUF) * BBUF;
#pragma unroll
    for (int ck = 0; ck < NCK; ++ck) {
      const int cg = ph * NCK + ck;
      const int kb0 = 2 * (qw * WPP + 4 * ck);
      if constexpr (kTiled) {
        scl[wave][2 * g][r16] = scale_to_f32_fast(ts[cg] & 0xffffu);
        scl[wave][2 * g + 1][r16] = scale_to_f32_fast(ts[cg] >> 16);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const u32x4 q = tq[cg][u];
          block_mma(bb, 2 * u, kb0 + 2 * u, quants_to_bf16(q.x, q.y), accs[0]);
          block_mma(bb, 2 * u + 1, kb0 + 2 * u + 1, quants_to_bf16(q.z, q.w), accs[1]);
        }
      } else {
        // Realign, scales to (wave-private) LDS, in-register transpose into A
        // fragments; blocks in K order into the even / odd accumulators, as above.
        Block blk[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          blk[u] = finish_block(wr[cg][u]);
          scl[wave][4 * u + g][r16] = scale_to_f32_fast(blk[u].scale_bits);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          uint32_t q[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) q[i] = blk[u].q[i];
          transpose_chunks(q);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            block_mma(bb, 4 * u + j, kb0 + 4 * u + j, quants_to_bf16(q[2 * j], q[2 * j + 1]),
                      accs[j & 1]);
        }
      }
      if (cg + RING < TC) load_chunk(cg + RING);
    }
  };
  if constexpr (NBUF == 1) {
#pragma unroll
    for (int ph = 0; ph < NPH; ++ph) {
      if (ph > 0) {
        // The previous phase's sums are complete before the barrier: otherwise the
        // compiler defers its scale FMAs past the split and holds every MFMA
        // result of the phase in registers (spills).
        asm volatile("" : "+v"(accs[0]), "+v"(accs[1]));
        __syncthreads();  // every wave is done with the phase's fragments
      }
      split_phase(ph);
      __syncthreads();
      if (ph + 1 < NPH) load_x(ph + 1);
      compute_phase(ph);
    }
  } else {
    split_phase(0);
    __syncthreads();
#pragma unroll
    for (int ph = 0; ph < NPH; ++ph) {
      if (ph + 1 < NPH) split_phase(ph + 1);  // the other buffer: last read in phase ph - 1
      if (ph + 2 < NPH) load_x(ph + 2);
      compute_phase(ph);
      if (ph + 1 < NPH) {
        asm volatile("" : "+v"(accs[0]), "+v"(accs[1]));  // as above
        __syncthreads();  // phase ph + 1 split, phase ph fragments no longer read
      }
    }
  }
  const f32x4 acc = accs[0] + accs[1];

  // The group's WG waves add their sums in LDS (the B area is free after the
  // barrier), then the first wave of the group writes y.
  __syncthreads();
  float (*red)[16][17] = reinterpret_cast<float (*)[16][17]>(bfr);
  red[wave][4 * g + 0][r16] = acc.x;
  red[wave][4 * g + 1][r16] = acc.y;
  red[wave][4 * g + 2][r16] = acc.z;
  red[wave][4 * g + 3][r16] = acc.w;
  __syncthreads();
  if (qw != 0 || !live_g || (kSwi && lg >= NGH)) return;
  // The sum of group g's waves for (token m, row rr), in wave order.
  auto group_sum = [&](int gl, int m, int rr) {
    const int c0 = m, c1 = (MT + m) & 15, c2 = (2 * MT + m) & 15;
    float t = 0.0f;
#pragma unroll
    for (int q4 = 0; q4 < WG; ++q4) {
      const int wv = WG * gl + q4;
      float s = red[wv][rr][c0];
      if (c1 != c0) s += red[wv][rr][c1];
      if (c2 != c0 && c2 != c1) s += red[wv][rr][c2];
      t = q4 == 0 ? s : t + s;
    }
    return t;
  };
#pragma unroll
  for (int o = 0; o < OPL; ++o) {
    const int idx = lane + 64 * o;  // (token m, row rr), rows fastest
    const int m = idx >> 4, rr = idx & 15;
    const int64_t n = rg * 16 + rr;
    if (idx >= OUTS || m >= M || n >= N) continue;
    const float t = group_sum(lg, m, rr);
    if constexpr (kSwi)
      y[(int64_t)m * N + n] = silu_mul(t, group_sum(lg + NGH, m, rr));
    else
      y[(int64_t)m * N + n] = t + (bias ? bias_at(bias, bias_bf16, n) : 0.0f);
  }
}

// Launch shapes of the row-range decode (MI355X, Llama-7B shapes at K = 4096):
//  * 4 tokens, 512-1024 groups: NG = ceil(G / 256) groups of 4 waves, K in one
//    128-block phase (128 KB of fragments), 2 chunks in flight;
//  * 4 tokens, 240-256 groups (o_proj): one group of 16 waves per workgroup;
//  * 8 tokens, 512-1024 groups: 4 waves per group, 32-block phases in two
//    buffers (2 x 50 KB; 0.95-0.97x the 64-block single buffer), 2 chunks in
//    flight (0.98-0.99x one chunk on the Llama qkv / gate shapes; 3 or 4 chunks
//    1.01-1.12x).
template <int MT, int NG, int WG, int PHB, int NBUF, int RING, int MODE = 0,
          int L = int(WeightLayout::kTiled)>
hipError_t launch_rows_k(const float* x, const RowsArgs& a, int M, int K, hipStream_t stream) {
  constexpr int NGH = MODE == 1 ? NG / 2 : NG;  // output groups per workgroup
  const unsigned groups = MODE == 1 ? a.grp_end[0] : a.grp_end[a.count - 1];
  const dim3 grid((groups + NGH - 1) / NGH), block(64 * WG * NG);
  const int nph = (K / kBlockElems + PHB - 1) / PHB;
#define MLE_ROWS(NPH)                                                                         \
  hipLaunchKernelGGL((gemv_mfma_rows_kernel<MT, NG, NPH, PHB, NBUF, RING, WG, MODE, L>), grid, \
                     block, 0, stream, x, a, M, K)
  switch (nph) {
    case 1: MLE_ROWS(1); break;
    case 2: if constexpr (PHB < 128) MLE_ROWS(2); else return hipErrorInvalidValue; break;
    case 3: if constexpr (PHB < 64) MLE_ROWS(3); else return hipErrorInvalidValue; break;
    case 4: if constexpr (PHB < 64) MLE_ROWS(4); else return hipErrorInvalidValue; break;
    default: return hipErrorInvalidValue;
  }
#undef MLE_ROWS
  return hipGetLastError();
}

// The 16-row groups of 1-3 output segments, numbered segment after segment
// (SwiGLU: the gate weight's groups; the up weight has the same rows).
RowsArgs rows_args(const LinearSegs& s) {
  RowsArgs a{};
  const bool swi = s.mode == Epilogue::kSwiGLU;
  unsigned end = 0;
  for (int i = 0; i < 3; ++i) {
    a.seg[i] = s.seg[i];
    if (i < (swi ? 1 : s.count)) end += (unsigned)((s.seg[i].N + kTileRows - 1) / kTileRows);
    a.grp_end[i] = end;
  }
  if (swi) a.seg[1].N = s.seg[0].N;
  a.count = swi ? 1 : s.count;
  return a;
}

template <int MT>
hipError_t launch_rows(const float* x, const LinearSegs& s, int M, int K, hipStream_t stream) {
  const RowsArgs a = rows_args(s);
  const int64_t G = a.grp_end[a.count - 1];
  if (s.mode == Epilogue::kSwiGLU) {
    // Gate and up groups of the same rows side by side, two waves each: 2-4 pairs
    // per workgroup (8-16 waves) for 512-1024 groups per weight on 256 CUs; tiled
    // or raw weights.
    constexpr int PB = MT == 4 ? 128 : 32, NB = MT == 4 ? 1 : 2;
    constexpr int T = int(WeightLayout::kTiled), R = int(WeightLayout::kRaw);
    const bool tiled = s.layout == WeightLayout::kTiled;
    switch (rows_groups_per_workgroup(G)) {
      case 2: return tiled ? launch_rows_k<MT, 4, 2, PB, NB, 2, 1, T>(x, a, M, K, stream)
                           : launch_rows_k<MT, 4, 2, PB, NB, 2, 1, R>(x, a, M, K, stream);
      case 3: return tiled ? launch_rows_k<MT, 6, 2, PB, NB, 2, 1, T>(x, a, M, K, stream)
                           : launch_rows_k<MT, 6, 2, PB, NB, 2, 1, R>(x, a, M, K, stream);
      case 4: return tiled ? launch_rows_k<MT, 8, 2, PB, NB, 2, 1, T>(x, a, M, K, stream)
                           : launch_rows_k<MT, 8, 2, PB, NB, 2, 1, R>(x, a, M, K, stream);
    }
    return hipErrorInvalidValue;
  }
  if constexpr (MT == 4) {
    constexpr int R = int(WeightLayout::kRaw);
    if (s.layout == WeightLayout::kRaw) {
      switch (rows_groups_per_workgroup(G)) {
        case 2: return launch_rows_k<4, 2, 4, 128, 1, 2, 0, R>(x, a, M, K, stream);
        case 3: return launch_rows_k<4, 3, 4, 128, 1, 2, 0, R>(x, a, M, K, stream);
        case 4: return launch_rows_k<4, 4, 4, 128, 1, 2, 0, R>(x, a, M, K, stream);
      }
      return hipErrorInvalidValue;
    }
    switch (rows_groups_per_workgroup(G)) {
      case 1: return launch_rows_k<4, 1, 16, 128, 1, 1>(x, a, M, K, stream);
      case 2: return launch_rows_k<4, 2, 4, 128, 1, 2>(x, a, M, K, stream);
      case 3: return launch_rows_k<4, 3, 4, 128, 1, 2>(x, a, M, K, stream);
      case 4: return launch_rows_k<4, 4, 4, 128, 1, 2>(x, a, M, K, stream);
    }
  } else {
    switch (rows_groups_per_workgroup(G)) {
      case 2: return launch_rows_k<8, 2, 4, 32, 2, 2>(x, a, M, K, stream);
      case 3: return launch_rows_k<8, 3, 4, 32, 2, 2>(x, a, M, K, stream);
      case 4: return launch_rows_k<8, 4, 4, 32, 2, 2>(x, a, M, K, stream);
    }
  }
  return hipErrorInvalidValue;
}

// Row groups with a short K split ("hybrid" decode, tiled or raw weights, 4 or
// 8 tokens, plain outputs).  The split-K kernel above gives a workgroup 16 W rows
// x 16 blocks, so every output row's activations are read and split once per
// row tile (64 times for down's 4096 rows) and 22 partial sums meet per output;
// the row-range kernel reads and splits all of K once per workgroup.  Here a
// workgroup owns NG 16-row groups x one split of SPB blocks (NG = 8, SPB = 44 on
// down 4096 x 11008: 32 x 8 = 256 workgroups, one per CU): its split's
// activations are loaded and split once into LDS B fragments (the layout and
// arithmetic of the kernels above) and shared by all NG groups, every weight
// load of the workgroup (RING chunks of 4 block pairs per wave, all of them when
// RING covers the wave's share) is issued before the split, and the splits of a
// row tile meet in one hand-off (partials, completion wait, counter, read-back
// by the last workgroup in split order: deterministic).  Wave (group lg, index
// qw) multiplies pairs [qw WPP, (qw + 1) WPP) of the split for its group; the
// WG waves of a group add their sums in LDS in wave order.
//
// Raw weights (LAYOUT kRaw): lane (g, r16) loads blocks 4 u + g (u = 0, 1) of each
// 8-block chunk of row r16 of its group as whole 34-byte blocks and transposes
// them in registers into the same A fragments (the row-range kernel's raw path);
// blocks meet the same accumulators in the same order, so raw and tiled launches
// give the same bits.
template <int MT, int NG, int WG, int SPB, int RING, int LAYOUT>
__global__ __launch_bounds__(64 * WG * NG) void gemv_mfma_hyb_kernel(
    const float* __restrict__ x, const RowsArgs args, int M, int K,
    float* __restrict__ partials, uint32_t* __restrict__ counters) {
  constexpr int W = WG * NG;
  constexpr int NT = 64 * W;
  constexpr int P = Cols<MT>::P;
  using C = Cols<MT, 4>;                  // half-size last fragment when it fits
  static_assert(SPB % 2 == 0, "whole block pairs per split");
  constexpr int SPP = SPB / 2;            // pairs per split
  constexpr int WPP = (SPP + WG - 1) / WG;  // pairs per wave
  constexpr int NCK = (WPP + 3) / 4;      // 4-pair chunks per wave
  constexpr int PADB = 8 * NCK * WG;      // blocks of the B area (>= SPB)
  constexpr int BBUF = PADB * C::FB;
  constexpr int XITEMS = MT * PADB * 4;   // (token, k quarter, block)
  constexpr int XPT = (XITEMS + NT - 1) / NT;
  constexpr int OUTS = 16 * MT;           // outputs per group
  constexpr int OPL = (OUTS + 63) / 64;
  constexpr int REGION = NG * OUTS;       // partial floats per workgroup
  constexpr int RPT = (REGION + NT - 1) / NT;
  constexpr int RG = RING < NCK ? RING : NCK;
  static_assert(W * 16 * 17 * 4 <= BBUF, "the group reduction fits the B area");
  __shared__ __attribute__((aligned(16))) uint8_t bfr[BBUF];
  __shared__ __attribute__((aligned(16))) float scl[W][8][16];
  __shared__ uint32_t arrived;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r16 = lane & 15;
  const int lg = wave / WG, qw = wave % WG;
  const int KB = K / kBlockElems;
  const int KP = (KB + 1) >> 1;
  const int kb0 = blockIdx.y * SPB;       // first block of this split
  const int pp0 = kb0 >> 1;               // first pair of this split

  const unsigned grp_total = args.count == 1 ? args.grp_end[0]
                             : args.count == 2 ? args.grp_end[1]
                                               : args.grp_end[2];
  // Segment of a group (uniform selects: no indexing into the argument).
  auto seg_of = [&](unsigned gr) {
    return (args.count > 1 && gr >= args.grp_end[0])
               ? ((args.count > 2 && gr >= args.grp_end[1]) ? 2 : 1)
               : 0;
  };
  const unsigned grp = blockIdx.x * NG + lg;
  const int si = seg_of(grp);
  const unsigned grp0 = si == 0 ? 0u : si == 1 ? args.grp_end[0] : args.grp_end[1];
  const uint8_t* w = si == 0 ? args.seg[0].w : si == 1 ? args.seg[1].w : args.seg[2].w;
  const int N = si == 0 ? args.seg[0].N : si == 1 ? args.seg[1].N : args.seg[2].N;
  const int64_t G = ((int64_t)N + kTileRows - 1) / kTileRows;
  const bool live_g = grp < grp_total;
  const int64_t rg = live_g ? (int64_t)(grp - grp0) : 0;

  // 0. This split's activations first: item (token m fastest, k quarter, block
  //    of the B area); items past M, past the split or past K read zeros.
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)((int64_t)M * K * 4));
  f32x4 xv[XPT][2];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int it = tid + NT * i;
    const int m = it % MT, q = it / MT;
    const int kb = q >> 2;
    uint32_t off = it < XITEMS && kb < SPB && kb0 + kb < KB && m < M
                       ? (uint32_t)((m * K + (kb0 + kb) * kBlockElems + 8 * (q & 3)) * 4)
                       : 0x80000000u;
    asm volatile("" : "+v"(off));  // the load stays where it is written
    xv[i][0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
    xv[i][1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off + 16, 0, 0));
  }

  // 1. Weights: quant slots (lane l: rows l % 16, quants 8 (l/16) .. +7 of both
  //    blocks of a pair) and scale dwords (lane l: pair l/16 of the chunk, row
  //    l % 16) of this wave's group; pairs past the wave's share, the split or K,
  //    and groups past N, read zeros.
  constexpr bool kTiled = LAYOUT == int(WeightLayout::kTiled);
  const uint8_t* qb = w + rg * KP * kTilePieceBytes;
  const uint8_t* sb = w + G * KP * kTilePieceBytes + rg * KP * kTileScaleBytes;
  const __amdgpu_buffer_rsrc_t qrs = make_rsrc(qb, live_g ? (uint32_t)KP * kTilePieceBytes : 0u);
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(sb, live_g ? (uint32_t)KP * kTileScaleBytes : 0u);
  // Raw: one buffer over the group's rows (rows past N read as zero); a chunk's
  // blocks start 8-block (272-byte) steps apart, so each lane's 4-byte alignment
  // phase is fixed.
  const uint32_t row_bytes = (uint32_t)KB * kBlockBytes;
  const uint8_t* gbase = w + rg * kTileRows * (int64_t)row_bytes;
  const int64_t grows = live_g ? min((int64_t)kTileRows, (int64_t)N - rg * kTileRows) : 0;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(gbase, (uint32_t)(grows * row_bytes));
  const uint32_t lane_off =
      (uint32_t)r16 * row_bytes + (uint32_t)(kb0 + 2 * qw * WPP + g) * kBlockBytes;
  const uint32_t mis = (uint32_t)(((uintptr_t)gbase + lane_off) & 2u);
  const uint32_t voff = lane_off + mis;
  const uint32_t uoff = lane_off + (mis ? 0u : 32u);
  u32x4 tq[kTiled ? NCK : 1][4];
  uint32_t ts[kTiled ? NCK : 1];
  RawBlock wr[kTiled ? 1 : NCK][2];
  auto pair_live = [&](int j) {  // pair j of this wave's share
    return j < WPP && qw * WPP + j < SPP && pp0 + qw * WPP + j < KP;
  };
  auto load_chunk = [&](int ck) {
    if constexpr (kTiled) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = 4 * ck + u;
        uint32_t off = pair_live(j)
                           ? (uint32_t)(pp0 + qw * WPP + j) * kTilePieceBytes + (uint32_t)lane * 16
                           : 0x80000000u;
        asm volatile("" : "+v"(off));
        tq[ck][u] = __builtin_amdgcn_raw_buffer_load_b128(qrs, off, 0, kNonTemporal);
      }
      const int j = 4 * ck + g;
      uint32_t soff = pair_live(j)
                          ? (uint32_t)(pp0 + qw * WPP + j) * kTileScaleBytes + (uint32_t)r16 * 4
                          : 0x80000000u;
      asm volatile("" : "+v"(soff));
      ts[ck] = __builtin_amdgcn_raw_buffer_load_b32(srs, soff, 0, 0);
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int jb = 8 * ck + 4 * u + g;  // block of this wave's share
        const bool live = jb < 2 * WPP && 2 * qw * WPP + jb < SPB && kb0 + 2 * qw * WPP + jb < KB;
        const uint32_t soff = (uint32_t)(8 * ck + 4 * u) * kBlockBytes;  // multiple of 4
        uint32_t v8 = live ? voff + soff : 0x80000000u;
        uint32_t v2 = live ? uoff + soff : 0x80000000u;
        asm volatile("" : "+v"(v8), "+v"(v2));
        const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8, 0, 0);
        const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(wrs, v8 + 16, 0, 0);
        wr[ck][u].v0 = u32x4_a4{v0.x, v0.y, v0.z, v0.w};
        wr[ck][u].v1 = u32x4_a4{v1.x, v1.y, v1.z, v1.w};
        wr[ck][u].u = __builtin_amdgcn_raw_buffer_load_b16(wrs, v2, 0, 0);
        wr[ck][u].mis = mis;
      }
    }
  };
#pragma unroll
  for (int ck = 0; ck < RG; ++ck) load_chunk(ck);

  // 2. B fragments of the split (stored columns past 3 MT zeroed once).
  if constexpr (C::HALF) {
    for (int kb = tid; kb < PADB; kb += NT)
      *reinterpret_cast<u32x4*>(bfr + kb * C::FB + (P - 1) * 1024 + 512) = u32x4{0u, 0u, 0u, 0u};
  }
  if constexpr (C::PADC > 0) {
    constexpr int PADC = C::PADC;
    for (int it = tid; it < PADB * 4 * PADC; it += NT) {
      const int kb = it / (4 * PADC), q = it % (4 * PADC);
      const int c = q / PADC, vc = 3 * MT + q % PADC;
      *reinterpret_cast<u32x4*>(bfr + bslot<MT, 4, P>(kb, vc >> 4, c, vc & 15)) =
          u32x4{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int it = tid + NT * i;
    if (XITEMS % NT != 0 && it >= XITEMS) continue;
    const int m = it % MT, q = it / MT;
    const int kb = q >> 2, c = q & 3;
    const float v[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                        xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
    bool finite = true;
#pragma unroll
    for (int j = 0; j < 8; ++j) finite &= !__builtin_amdgcn_class(v[j], 0x207);  // NaN, +-Inf
    uint32_t parts[3][4];
    if (__builtin_expect(finite, 1))
      split3_finite(v, parts[0], parts[1], parts[2]);
    else
      split3_any(v, parts[0], parts[1], parts[2]);
#pragma unroll
    for (int part = 0; part < 3; ++part) {
      const int vc = part * MT + m;
      *reinterpret_cast<u32x4*>(bfr + bslot<MT, 4, P>(kb, vc >> 4, c, vc & 15)) =
          u32x4{parts[part][0], parts[part][1], parts[part][2], parts[part][3]};
    }
  }
  __syncthreads();

  // 3. Chunks in order as their loads land: P chained MFMAs per block, fp32
  //    scale FMA into the even / odd accumulators (the kernels' arithmetic).
  f32x4 accs[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  auto block_mma = [&](int kc, int kb, const bf16x8_t a, f32x4& a4) {
    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        a, *reinterpret_cast<const bf16x8_t*>(bfr + bslot_rd<MT, 4, P>(kb, 0, g, r16)),
        f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
    for (int p = 1; p < P; ++p)
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          a, *reinterpret_cast<const bf16x8_t*>(bfr + bslot_rd<MT, 4, P>(kb, p, g, r16)), d, 0,
          0, 0);
    const f32x4 sc = *reinterpret_cast<const f32x4*>(&scl[wave][kc][4 * g]);
    a4.x = __builtin_fmaf(sc.x, d.x, a4.x);
    a4.y = __builtin_fmaf(sc.y, d.y, a4.y);
    a4.z = __builtin_fmaf(sc.z, d.z, a4.z);
    a4.w = __builtin_fmaf(sc.w, d.w, a4.w);
  };
#pragma unroll
  for (int ck = 0; ck < NCK; ++ck) {
    const int kbw = 2 * (qw * WPP + 4 * ck);  // first B-area block of the chunk
    if constexpr (kTiled) {
      scl[wave][2 * g][r16] = scale_to_f32_fast(ts[ck] & 0xffffu);
      scl[wave][2 * g + 1][r16] = scale_to_f32_fast(ts[ck] >> 16);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (4 * ck + u >= WPP) break;  // past the wave's share: nothing to add
        const u32x4 q = tq[ck][u];
        block_mma(2 * u, kbw + 2 * u, quants_to_bf16(q.x, q.y), accs[0]);
        block_mma(2 * u + 1, kbw + 2 * u + 1, quants_to_bf16(q.z, q.w), accs[1]);
      }
    } else {
      // Realign, scales to (wave-private) LDS, in-register transpose into A
      // fragments; blocks in K order into the even / odd accumulators.
      Block blk[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        blk[u] = finish_block(wr[ck][u]);
        scl[wave][4 * u + g][r16] = scale_to_f32_fast(blk[u].scale_bits);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = blk[u].q[i];
        transpose_chunks(q);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // past the wave's share: nothing to add (those B blocks are other waves')
          if (8 * ck + 4 * u + j >= 2 * WPP) break;
          block_mma(4 * u + j, kbw + 4 * u + j, quants_to_bf16(q[2 * j], q[2 * j + 1]),
                    accs[j & 1]);
        }
      }
    }
    if (ck + RG < NCK) load_chunk(ck + RG);
  }
  const f32x4 acc = accs[0] + accs[1];

  // 4. The WG waves of a group add their sums in LDS (the B area is free after
  //    the barrier); group sums of (token, row) in wave order.
  __syncthreads();
  float (*red)[16][17] = reinterpret_cast<float (*)[16][17]>(bfr);
  red[wave][4 * g + 0][r16] = acc.x;
  red[wave][4 * g + 1][r16] = acc.y;
  red[wave][4 * g + 2][r16] = acc.z;
  red[wave][4 * g + 3][r16] = acc.w;
  __syncthreads();
  auto group_sum = [&](int gl, int idx) {
    const int m = idx >> 4, rr = idx & 15;
    const int c0 = m, c1 = (MT + m) & 15, c2 = (2 * MT + m) & 15;
    float t = 0.0f;
#pragma unroll
    for (int q4 = 0; q4 < WG; ++q4) {
      const int wv = WG * gl + q4;
      float s = red[wv][rr][c0];
      if (c1 != c0) s += red[wv][rr][c1];
      if (c2 != c0 && c2 != c1) s += red[wv][rr][c2];
      t = q4 == 0 ? s : t + s;
    }
    return t;
  };
  // Output (group-local index idx = token m x 16 + row) of group gl -> y.
  auto write_y = [&](int gl, int idx, float t) {
    const unsigned gr = blockIdx.x * NG + gl;
    if (gr >= grp_total) return;
    const int s2 = seg_of(gr);
    const unsigned g0 = s2 == 0 ? 0u : s2 == 1 ? args.grp_end[0] : args.grp_end[1];
    float* y = s2 == 0 ? args.seg[0].y : s2 == 1 ? args.seg[1].y : args.seg[2].y;
    const int n2 = s2 == 0 ? args.seg[0].N : s2 == 1 ? args.seg[1].N : args.seg[2].N;
    const void* bias = s2 == 0 ? args.seg[0].bias : s2 == 1 ? args.seg[1].bias : args.seg[2].bias;
    const int bias_bf16 =
        s2 == 0 ? args.seg[0].bias_bf16 : s2 == 1 ? args.seg[1].bias_bf16 : args.seg[2].bias_bf16;
    const int m = idx >> 4;
    const int64_t n = (int64_t)(gr - g0) * 16 + (idx & 15);
    if (m >= M || n >= n2) return;
    y[(int64_t)m * n2 + n] = t + (bias ? bias_at(bias, bias_bf16, n) : 0.0f);
  };

  if (gridDim.y == 1) {
    if (qw != 0) return;
#pragma unroll
    for (int o = 0; o < OPL; ++o) {
      const int idx = lane + 64 * o;
      if (idx < OUTS) write_y(lg, idx, group_sum(lg, idx));
    }
    return;
  }

  // 5. Split K: partials [tile][split][REGION] by device-scope stores, their
  //    completion, the tile's counter; the last workgroup resets the counter and
  //    adds the splits of every output in split order.
  constexpr int SC1 = 16;  // cache-policy bit: device scope
  const unsigned nspl = gridDim.y;
  const __amdgpu_buffer_rsrc_t prs =
      make_rsrc(partials + (int64_t)blockIdx.x * nspl * REGION, (uint32_t)(nspl * REGION * 4));
  if (qw == 0) {
#pragma unroll
    for (int o = 0; o < OPL; ++o) {
      const int idx = lane + 64 * o;
      if (idx < OUTS)
        __builtin_amdgcn_raw_buffer_store_b32(
            __builtin_bit_cast(uint32_t, group_sum(lg, idx)), prs,
            (uint32_t)((blockIdx.y * REGION + lg * OUTS + idx) * 4), 0, SC1);
    }
  }
  uint32_t* const counter = counters + (size_t)blockIdx.x * kCounterStride;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // every partial has reached the coherence point
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (tid == 0)
    arrived = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (arrived != nspl - 1) return;
  if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int o = 0; o < RPT; ++o) {
    const int r = tid + NT * o;
    if (REGION % NT != 0 && r >= REGION) break;
    float s = 0.0f;
    for (unsigned sp = 0; sp < nspl; sp += 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v[j] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(
                       prs, sp + j < nspl ? (uint32_t)(((sp + j) * REGION + r) * 4) : 0x80000000u,
                       0, SC1));
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (sp + j < nspl) s += v[j];
    }
    write_y(r / OUTS, r % OUTS, s);
  }
}

// Launch shapes of the hybrid decode (index = DecodeMfmaConfig::hyb): row
// groups per workgroup, waves per group, blocks per split, 4-pair load chunks in
// flight per wave.  Measured on MI355X (tiled weights, rotated copies), against
// the split-K kernel's 13.0-13.5 / 14.5-15.5 us on down 4096 x 11008 at 4 / 8
// tokens:
//   1: 4 groups x 2 waves, 44-block splits, 2 chunks in flight: 64 x 8 = 512
//      workgroups, two per CU: 11.98-12.21 / 13.68-13.81 us (picked);
//      the same with 1 chunk in flight 15.3 / 17.2, all 3 up front 12.6 / 15.1;
//   2: 8 groups x 1 wave, 44-block splits, 3 of 6 chunks in flight (256
//      workgroups): 12.1-12.3 / 14.2-14.8 (all 6 up front: 14.5 / 16.1);
//   3: 16 groups x 1 wave, 22-block splits, 2 of 3 chunks in flight: 13.4 / 16.6;
//   4: 4 groups x 4 waves, 32-block splits, 1 chunk: 64 x 11 workgroups.
// Other measured shapes (kept out): 9-10 splits (288-320 workgroups, more than
// fit at once) 15.8-16.7 / 20-20.7; 2 groups per workgroup (1024 workgroups)
// 14.4 / 18.7; 16 waves over 4 groups 12.5 / 17.0; 16 waves over 4 groups with
// 88-block splits (4 splits, 256 workgroups, 157 KB of LDS at 8 tokens) 12.8 /
// 14.1 with 2 chunks in flight, 14.0 / 15.6 with 3.  On K = 4096 (o_proj, gate,
// qkv) every shape tried was slower than the kernels above.
struct HybShape {
  int ng, wg, spb, ring;
};
constexpr HybShape kHybShapes[] = {
    {0, 0, 0, 0},
    {4, 2, 44, 2},
    {8, 1, 44, 3},
    {16, 1, 22, 2},
    {4, 4, 32, 1},
};
constexpr int kHybCount = sizeof(kHybShapes) / sizeof(kHybShapes[0]);

template <int MT, int NG, int WG, int SPB, int RING>
hipError_t launch_hyb_k(const float* x, const RowsArgs& a, WeightLayout layout, int M, int K,
                        const SplitKWorkspace& ws, hipStream_t stream) {
  const unsigned groups = a.grp_end[a.count - 1];
  const int KB = K / kBlockElems;
  const dim3 grid((groups + NG - 1) / NG, (unsigned)((KB + SPB - 1) / SPB)), block(64 * WG * NG);
  if (grid.y > 1 && (ws.partials == nullptr || ws.counters == nullptr))
    return hipErrorInvalidValue;
  if (layout == WeightLayout::kTiled)
    hipLaunchKernelGGL((gemv_mfma_hyb_kernel<MT, NG, WG, SPB, RING, int(WeightLayout::kTiled)>),
                       grid, block, 0, stream, x, a, M, K, ws.partials, ws.counters);
  else
    hipLaunchKernelGGL((gemv_mfma_hyb_kernel<MT, NG, WG, SPB, RING, int(WeightLayout::kRaw)>),
                       grid, block, 0, stream, x, a, M, K, ws.partials, ws.counters);
  return hipGetLastError();
}

template <int MT>
hipError_t launch_hyb(int hyb, const float* x, const LinearSegs& s, int M, int K,
                      const SplitKWorkspace& ws, hipStream_t stream) {
  const RowsArgs a = rows_args(s);
  switch (hyb) {
    case 1: return launch_hyb_k<MT, 4, 2, 44, 2>(x, a, s.layout, M, K, ws, stream);
    case 2: return launch_hyb_k<MT, 8, 1, 44, 3>(x, a, s.layout, M, K, ws, stream);
    case 3: return launch_hyb_k<MT, 16, 1, 22, 2>(x, a, s.layout, M, K, ws, stream);
    case 4: return launch_hyb_k<MT, 4, 4, 32, 1>(x, a, s.layout, M, K, ws, stream);
  }
  return hipErrorInvalidValue;
}

struct Grid {
  unsigned tiles, splits;
  DecodeArgs args;
};

// Row tiles of each segment (SwiGLU: 8 W output rows per tile, else 16 W).
Grid grid_of(const DecodeMfmaConfig& c, const LinearSegs& s, int K) {
  const int KB = K / kBlockElems;
  const int rows = s.mode == Epilogue::kSwiGLU ? 8 * c.waves : 16 * c.waves;
  Grid gr{};
  unsigned end = 0;
  const int count = s.mode == Epilogue::kSwiGLU ? 1 : s.count;
  for (int i = 0; i < 3; ++i) {
    gr.args.seg[i] = s.seg[i];
    if (i < count) end += (unsigned)((s.seg[i].N + rows - 1) / rows);
    gr.args.tile_end[i] = end;
  }
  if (s.mode == Epilogue::kSwiGLU) gr.args.seg[1].N = s.seg[0].N;
  gr.args.count = count;
  gr.tiles = end;
  gr.splits = (unsigned)((KB + c.kslice - 1) / c.kslice);
  return gr;
}

template <int MT, int W, int KSL, int L>
hipError_t launch_l(const Grid& gr, Epilogue mode, const float* x, int M, int K,
                    const SplitKWorkspace& ws, hipStream_t stream) {
  if (mode == Epilogue::kSwiGLU) {
    if constexpr (W % 2 == 0)
      hipLaunchKernelGGL((gemv_q8_0_mfma_kernel<MT, W, KSL, 1, L>), dim3(gr.tiles, gr.splits),
                         dim3(64 * W), 0, stream, x, gr.args, M, K, ws.partials, ws.counters);
  } else {
    hipLaunchKernelGGL((gemv_q8_0_mfma_kernel<MT, W, KSL, 0, L>), dim3(gr.tiles, gr.splits),
                       dim3(64 * W), 0, stream, x, gr.args, M, K, ws.partials, ws.counters);
  }
  return hipGetLastError();
}

template <int MT, int W, int KSL>
hipError_t launch_t(const Grid& gr, Epilogue mode, WeightLayout layout, const float* x, int M,
                    int K, const SplitKWorkspace& ws, hipStream_t stream) {
  if (layout == WeightLayout::kTiled)
    return launch_l<MT, W, KSL, int(WeightLayout::kTiled)>(gr, mode, x, M, K, ws, stream);
  return launch_l<MT, W, KSL, int(WeightLayout::kRaw)>(gr, mode, x, M, K, ws, stream);
}

template <int MT>
hipError_t dispatch_shape(const DecodeMfmaConfig& c, const Grid& gr, Epilogue mode,
                          WeightLayout layout, const float* x, int M, int K,
                          const SplitKWorkspace& ws, hipStream_t stream) {
  if (c.kslice == 16) {
    if (c.waves == 2) return launch_t<MT, 2, 16>(gr, mode, layout, x, M, K, ws, stream);
    if (c.waves == 4) return launch_t<MT, 4, 16>(gr, mode, layout, x, M, K, ws, stream);
    if (c.waves == 8) return launch_t<MT, 8, 16>(gr, mode, layout, x, M, K, ws, stream);
  }
  if constexpr (Cols<MT>::P <= 2) {
    if (c.kslice == 32) {
      if (c.waves == 2) return launch_t<MT, 2, 32>(gr, mode, layout, x, M, K, ws, stream);
      if (c.waves == 4) return launch_t<MT, 4, 32>(gr, mode, layout, x, M, K, ws, stream);
      if (c.waves == 8) return launch_t<MT, 8, 32>(gr, mode, layout, x, M, K, ws, stream);
    }
  }
  return hipErrorInvalidValue;
}

LinearSegs single(const uint8_t* w, const float* bias, float* y, int N) {
  LinearSegs s;
  s.seg[0] = LinearSeg{w, bias, y, N};
  return s;
}

}  // namespace

bool decode_mfma_config_valid(const DecodeMfmaConfig& c) {
  const bool mt = c.mt == 1 || c.mt == 2 || c.mt == 4 || c.mt == 5 || c.mt == 8 || c.mt == 16;
  const bool waves = c.waves == 2 || c.waves == 4 || c.waves == 8;
  // A 32-block K slice of 3-MFMA (16-token) fragments would need 96 KB of LDS.
  const bool kslice = c.kslice == 16 || (c.kslice == 32 && c.mt <= 8);
  return mt && waves && kslice;
}

int decode_mfma_tile(int M) {
  return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 5 ? 5 : M <= 8 ? 8 : 16;
}

DecodeMfmaConfig decode_mfma_pick(int M, int N, int K, WeightLayout layout) {
  // Measured on MI355X over the Llama-7B decode shapes: 16-block K slices
  // (one-shot workgroups of ~35 KB) beat 32 unless K fits one 32-block slice
  // (no split-K hand-off at all); 8 waves per workgroup pay off for 4+ tokens
  // on wide weights (qkv / gate at M = 4: 16.9 / 16.4 us vs 18.4 / 17.6 with 4
  // waves), 4 otherwise.
  DecodeMfmaConfig c;
  c.mt = decode_mfma_tile(M);
  const int KB = K / kBlockElems;
  c.kslice = (c.mt <= 8 && KB <= 32) ? 32 : 16;
  if (layout == WeightLayout::kTiled) {
    // Tiled weights (MI355X sweep over the Llama-7B and Qwen2.5-0.5B projections
    // and the Qwen lm_head, M = 1..16): short rows (one 32-block slice) run best
    // in 4-wave workgroups, except at 16 tokens and for a vocabulary-sized
    // weight from 8 tokens (lm_head M = 8: 33.0 us vs 38.4); long rows in 8-wave
    // workgroups, except 4 for 12288+ outputs at 8 tokens (fused q/k/v 15.9 us
    // vs 16.6, gate/up 24.1 vs 24.3) and for rows of 8192+ elements, where twice
    // the row tiles balance better (down 4096 x 11008 with non-temporal weight
    // loads: 14.7-15.0 us vs 15.8-15.9 at M = 8, 12.85 vs 13.15 at M = 4; o_proj
    // at K = 4096 stays faster with 8: 7.8 vs 8.55).  The K slice follows the raw
    // rule, so raw and tiled launches accumulate in the same order.
    if (KB <= 32)
      c.waves = (c.mt >= 16 || (c.mt >= 8 && N >= 65536)) ? 8 : 4;
    else
      c.waves = ((c.mt == 8 && N >= 12288) || K >= 8192) ? 4 : 8;
    // The row-range kernel where it was measured to win (MI355X, Llama-7B
    // shapes at K = 4096, time against the split-K kernel): gate / up / qkv
    // (512-1024 row groups, 2-4 per workgroup sharing its activation split) at
    // M = 4 0.83-0.86x and M = 8 0.91-0.93x; o_proj (256 groups, one per
    // workgroup) at M = 4 0.91x.  o_proj at M = 8 (1.06x) and down (K = 11008:
    // 1.07x at M = 4, 1.35x at M = 8) keep the split-K kernel.
    const int64_t G = ((int64_t)N + kTileRows - 1) / kTileRows;
    const bool k_ok = K % 64 == 0 && K >= 2048 && K <= 4096;
    if (k_ok && (c.mt == 4 || c.mt == 8) && G >= 512 && G <= 1024) c.rows = 1;
    if (k_ok && c.mt == 4 && G >= 240 && G <= 256) c.rows = 1;
    // Long rows over few row groups (down 4096 x 11008): the hybrid kernel, 4
    // groups x 44-block splits per workgroup (at most 8 splits, so the 512
    // workgroups of a 256-group weight are resident at once).
    if ((c.mt == 4 || c.mt == 8) && K >= 8192 && KB <= 8 * 44 && G <= 256) c.hyb = 1;
    return c;
  }
  c.waves = (c.mt >= 4 && N >= 8192) ? 8 : 4;
  // Raw weights: the row-range kernel at 4 tokens on 512-1024 row groups of rows of
  // 2048-4096 elements (Llama qkv / gate / up; whole 34-byte blocks per lane,
  // transposed into the A fragments in registers): 0.89x the split-K launch.  Not
  // at 8 tokens (1.00-1.01x) or on 256 groups (o_proj at 4 tokens: 1.01x).
  const int64_t G = ((int64_t)N + kTileRows - 1) / kTileRows;
  if (K % 64 == 0 && K >= 2048 && K <= 4096 && c.mt == 4 && G >= 512 && G <= 1024) c.rows = 1;
  // and the hybrid kernel where it runs on tiled weights (raw down 4096 x 11008,
  // three interleaved runs: 0.96x at 4 tokens, 0.94x at 8; the tiled launch's bits).
  if ((c.mt == 4 || c.mt == 8) && K >= 8192 && KB <= 8 * 44 && G <= 256) c.hyb = 1;
  return c;
}

DecodeMfmaConfig decode_mfma_pick_segs(int M, const LinearSegs& s, int K) {
  int total_n = 0;
  for (int i = 0; i < s.count; ++i) total_n += s.seg[i].N;
  DecodeMfmaConfig c = decode_mfma_pick(M, total_n, K, s.layout);
  if (s.mode == Epilogue::kSwiGLU) {
    // Measured on MI355X (Llama gate/up, 2 x 11008 x 4096, tiled and raw weights):
    // see the row-range launch shapes above.
    const int64_t G = ((int64_t)s.seg[0].N + kTileRows - 1) / kTileRows;
    const bool k_ok = K % 64 == 0 && K >= 2048 && K <= 4096;
    c.rows = k_ok && (c.mt == 4 || c.mt == 8) && G >= 512 && G <= 1024 ? 1 : 0;
  }
  return c;
}

SplitKNeed decode_mfma_workspace(const DecodeMfmaConfig& c, int N, int K) {
  return decode_mfma_workspace_segs(c, single(nullptr, nullptr, nullptr, N), K);
}

// The launches the row-range kernel takes: 1-3 plain outputs (tiled weights; raw
// weights at 4 tokens on 512-1024 groups) and the gate/up SwiGLU pair.
static bool rows_takes(const DecodeMfmaConfig& c, const LinearSegs& s) {
  if (c.rows != 1 || s.count < 1 || s.count > 3) return false;
  if (s.mode == Epilogue::kSwiGLU) {  // tiled or raw weights
    // gate + up of 512-1024 row groups each, no bias (the SwiGLU launch has none)
    const int64_t G = rows_args(s).grp_end[0];
    return s.count == 2 && (c.mt == 4 || c.mt == 8) && G >= 512 && G <= 1024;
  }
  if (s.mode != Epilogue::kPlain) return false;
  // The launch shapes exist for these group counts (segments rounded up to whole
  // groups each, as the grid numbers them); raw weights: 4 tokens on 512-1024.
  const int64_t G = rows_args(s).grp_end[s.count - 1];
  if (s.layout != WeightLayout::kTiled)
    return s.layout == WeightLayout::kRaw && c.mt == 4 && G >= 512 && G <= 1024;
  return (G >= 512 && G <= 1024) || (c.mt == 4 && G >= 240 && G <= 256);
}

// The launches the hybrid kernel takes: 1-3 plain outputs on tiled or raw
// weights, 4 or 8 tokens.
static bool hyb_takes(const DecodeMfmaConfig& c, const LinearSegs& s) {
  return c.hyb > 0 && c.hyb < kHybCount && (c.mt == 4 || c.mt == 8) && s.count >= 1 &&
         s.count <= 3 && s.mode == Epilogue::kPlain &&
         (s.layout == WeightLayout::kTiled || s.layout == WeightLayout::kRaw);
}

SplitKNeed decode_mfma_workspace_segs(const DecodeMfmaConfig& c, const LinearSegs& s, int K) {
  if (hyb_takes(c, s)) {
    const HybShape h = kHybShapes[c.hyb];
    const RowsArgs a = rows_args(s);
    const size_t tiles = (a.grp_end[a.count - 1] + h.ng - 1) / h.ng;
    const int splits = (K / kBlockElems + h.spb - 1) / h.spb;
    SplitKNeed need;
    need.splits = splits;
    if (splits > 1) {
      need.partial_floats = tiles * splits * (size_t)h.ng * 16 * c.mt;
      need.counters = tiles * kCounterStride;
    }
    return need;
  }
  if (rows_takes(c, s)) return SplitKNeed{};  // no split K, no workspace
  const Grid gr = grid_of(c, s, K);
  SplitKNeed need;
  need.splits = (int)gr.splits;
  const size_t region = (size_t)16 * c.waves * c.mt;
  need.partial_floats = gr.splits > 1 ? (size_t)gr.tiles * gr.splits * region : 0;
  need.counters = gr.splits > 1 ? (size_t)gr.tiles * kCounterStride : 0;
  return need;
}

bool decode_mfma_fits(const DecodeMfmaConfig& c, int M, int N, int K) {
  // Buffer offsets are 32-bit: one workgroup's rows of weights and all M rows of
  // activations must stay below 2^31 bytes.
  const int64_t row_bytes = (int64_t)(K / kBlockElems) * kBlockBytes;
  (void)N;
  return (int64_t)16 * c.waves * row_bytes < (int64_t(1) << 31) &&
         (int64_t)M * K * 4 < (int64_t(1) << 31);
}

hipError_t launch_gemv_mfma(const DecodeMfmaConfig& c, const float* x, const uint8_t* w,
                            const float* bias, float* y, int M, int N, int K,
                            const SplitKWorkspace& ws, hipStream_t stream) {
  return launch_gemv_mfma_segs(c, x, single(w, bias, y, N), M, K, ws, stream);
}

hipError_t launch_gemv_mfma_segs(const DecodeMfmaConfig& c, const float* x,
                                 const LinearSegs& s, int M, int K, const SplitKWorkspace& ws,
                                 hipStream_t stream) {
  const bool swi = s.mode == Epilogue::kSwiGLU;
  if (s.count < 1 || s.count > 3 || (swi && (s.count != 2 || c.waves % 2 != 0)))
    return hipErrorInvalidValue;
  for (int i = 0; i < s.count; ++i)
    if (!decode_mfma_fits(c, M, s.seg[i].N, K) || s.seg[i].N <= 0) return hipErrorInvalidValue;
  if (hyb_takes(c, s)) {
    if (M > c.mt) return hipErrorInvalidValue;
    if (c.mt == 4) return launch_hyb<4>(c.hyb, x, s, M, K, ws, stream);
    return launch_hyb<8>(c.hyb, x, s, M, K, ws, stream);
  }
  if (rows_takes(c, s)) {
    if (M > c.mt || K % 64 != 0) return hipErrorInvalidValue;
    if (c.mt == 4) return launch_rows<4>(x, s, M, K, stream);
    if (c.mt == 8) return launch_rows<8>(x, s, M, K, stream);
    return hipErrorInvalidValue;
  }
  const Grid gr = grid_of(c, s, K);
  switch (c.mt) {
    case 1: return dispatch_shape<1>(c, gr, s.mode, s.layout, x, M, K, ws, stream);
    case 2: return dispatch_shape<2>(c, gr, s.mode, s.layout, x, M, K, ws, stream);
    case 4: return dispatch_shape<4>(c, gr, s.mode, s.layout, x, M, K, ws, stream);
    case 5: return dispatch_shape<5>(c, gr, s.mode, s.layout, x, M, K, ws, stream);
    case 8: return dispatch_shape<8>(c, gr, s.mode, s.layout, x, M, K, ws, stream);
    case 16: return dispatch_shape<16>(c, gr, s.mode, s.layout, x, M, K, ws, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace mle
