// launch.hpp -- internal launchers behind the C ABI (not exported).
//
// Every launcher assumes the caller (capi.hip) has validated pointers and
// shapes; each only enqueues work on `stream` and returns the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mle {

// Linear GEMV (M <= 8 tokens per launch): y[M,N] = x[M,K] . W^T (+ bias).
struct GemvConfig {
  int mt;   // token tile: 1, 2, 4 or 8 (>= M)
  int lpr;  // lanes cooperating on one output row: 16, 32 or 64
  int rw;   // output rows per lane group: 1, 2, 4 or 8
  // Nonzero: the row-span kernel on raw weights instead (one token, lanes along
  // K, rpw = 4 rows per workgroup; lpr and rw unused).
  int rpw = 0;
};
GemvConfig gemv_pick_config(int M, int N, int K);
bool gemv_config_valid(const GemvConfig& c);
hipError_t launch_gemv(const GemvConfig& cfg, const float* x, const uint8_t* w,
                       const float* bias, float* y, int M, int N, int K,
                       hipStream_t stream);

// Linear decode on bf16 MFMA with FP32-exact activations (1 <= M <= 16 per
// launch; larger M in chunks).  A workgroup of `waves` waves owns 16*waves output
// rows and a K slice of `kslice` blocks; the K slices of a row tile meet in a
// split-K workspace.
struct DecodeMfmaConfig {
  int mt;        // token tile: 1, 2, 4, 5, 8 or 16 (>= M)
  int waves;     // waves per workgroup: 2, 4 or 8
  int kslice;    // K blocks per workgroup: 16 or 32 (32 only for mt <= 8)
  int rows = 0;  // 1: row-range kernel, no split K (tiled Linears with 1-3 plain
                 // outputs, mt 4 or 8, see decode_mfma_pick); the fields above then
                 // serve launches it does not take (SwiGLU, other group counts)
  int hyb = 0;   // > 0: launch shape of the hybrid kernel (row groups x a short K
                 // split; tiled Linears with 1-3 plain outputs, mt 4 or 8)
};
struct SplitKNeed {
  int splits = 1;             // workgroups along K
  size_t partial_floats = 0;  // workspace floats (0 when splits == 1)
  size_t counters = 0;        // per-tile arrival counters (0 when splits == 1)
  size_t scratch_bytes = 0;   // other device scratch (256-byte multiple)
};
// Split-K tile counters of the MFMA decode are kCounterStride uint32 apart (one
// 128-byte line each).
constexpr int kCounterStride = 32;
struct SplitKWorkspace {
  float* partials = nullptr;     // split-K partial sums
  uint32_t* counters = nullptr;  // zero between launches (the kernel resets them)
  void* scratch = nullptr;       // 256-byte aligned, scratch_bytes long
};
int decode_mfma_tile(int M);
// Output segments of one Linear launch: 1 to 3 weights read against the same
// activations (a multi-output Linear: q/k/v), or, in kSwiGLU mode, exactly two
// (gate, up) combined into y = silu(x.Wg^T) * (x.Wu^T) in seg[0].y.
struct LinearSeg {
  const uint8_t* w = nullptr;
  const void* bias = nullptr;  // optional [N], fp32 (bf16 when bias_bf16); not in kSwiGLU mode
  float* y = nullptr;
  int N = 0;
  int bias_bf16 = 0;
};
enum class Epilogue { kPlain = 0, kSwiGLU = 1 };
// Byte layout of the weights of a launch.
//   kRaw: GGUF Q8_0, row n at byte n*(K/32)*34, 34-byte blocks along K.
//   kTiled: Q8_0 16-row tiles.  With KB = K/32 blocks, KP = ceil(KB/2) block
//     pairs and G = ceil(N/16) row groups, the tensor is
//       quant pieces  [G][KP] x 1024 B, then
//       scale pieces  [G][KP] x 64 B   (at byte G*KP*1024),
//     G*KP*1088 bytes in all (34 per block, as raw, plus zero padding of rows
//     past N and of the block past KB when KB is odd).  Slot l (0..63) of quant
//     piece (g, p) holds, at bytes 16l .. 16l+7, quants 8(l/16) .. +7 of block
//     2p of row 16g + l%16, and at bytes 16l+8 .. +15 the same quants of block
//     2p+1: the bf16 MFMA A-fragment order, so one 16-byte load per lane feeds
//     two 16x16x32 MFMAs.  Dword r of scale piece (g, p) holds the binary16
//     scale of block 2p (low half) and 2p+1 (high half) of row 16g + r.
//   kKN (prefill GEMM only, the MatMul's B operand): B[K, N] raw Q8_0 with
//     blocks along N, element (k, n) at flat index k*N + n.
enum class WeightLayout { kRaw = 0, kTiled = 1, kKN = 2 };
constexpr int kTileRows = 16;
constexpr int kTilePieceBytes = 1024;
constexpr int kTileScaleBytes = 64;
// Bytes of a kTiled tensor of N rows and K columns (K % 32 == 0).
inline size_t tiled_bytes(int64_t N, int64_t K) {
  const int64_t KP = (K / 32 + 1) / 2, G = (N + kTileRows - 1) / kTileRows;
  return (size_t)(G * KP * (kTilePieceBytes + kTileScaleBytes));
}
struct LinearSegs {
  LinearSeg seg[3];
  int count = 1;
  Epilogue mode = Epilogue::kPlain;
  WeightLayout layout = WeightLayout::kRaw;
};
// FP32 GEMV on kTiled weights (M <= 4 tokens per launch): a workgroup per
// 16-row group, its waves splitting K in chunks of `ppw` block pairs.
struct TiledGemvConfig {
  int mt;   // token tile: 1, 2 or 4 (>= M)
  int ppw;  // block pairs per wave chunk: 4, 8 or 16
  int wpg;  // waves per weight in a workgroup (SwiGLU: 2 wpg waves), <= 16 in all
};
TiledGemvConfig gemv_tiled_pick(int M, int rows, int K, bool swiglu);
// Whether an M-token launch of `rows` output rows on tiled weights takes this
// GEMV rather than the MFMA decode.
bool gemv_tiled_wins(int M, int rows, int K);
bool gemv_tiled_config_valid(const TiledGemvConfig& c, bool swiglu);
hipError_t launch_gemv_tiled_segs(const TiledGemvConfig& c, const float* x,
                                  const LinearSegs& s, int M, int K, hipStream_t stream);

// Raw Q8_0 [N, K] -> kTiled (one pass; `tiled` holds tiled_bytes(N, K)).
hipError_t launch_tile_q8_0(const uint8_t* raw, uint8_t* tiled, int N, int K,
                            hipStream_t stream);

// FP32 GEMV over segments (kSwiGLU only with a token tile of 1 and rw <= 4).
hipError_t launch_gemv_segs(const GemvConfig& cfg, const float* x, const LinearSegs& s, int M,
                            int K, hipStream_t stream);

DecodeMfmaConfig decode_mfma_pick(int M, int N, int K,
                                  WeightLayout layout = WeightLayout::kRaw);
// The pick for a launch over segments: decode_mfma_pick on all output rows, and
// for a gate/up SwiGLU pair (tiled or raw weights) the row-range kernel where it
// applies (rows of 512-1024 groups per weight at 3-8 tokens, K 2048-4096).
DecodeMfmaConfig decode_mfma_pick_segs(int M, const LinearSegs& s, int K);
bool decode_mfma_config_valid(const DecodeMfmaConfig& c);
SplitKNeed decode_mfma_workspace(const DecodeMfmaConfig& c, int N, int K);
// False when the shape's buffer offsets would not fit 32 bits (the caller then
// takes the FP32 GEMV path, which uses 64-bit addressing).
bool decode_mfma_fits(const DecodeMfmaConfig& c, int M, int N, int K);
hipError_t launch_gemv_mfma(const DecodeMfmaConfig& c, const float* x, const uint8_t* w,
                            const float* bias, float* y, int M, int N, int K,
                            const SplitKWorkspace& ws, hipStream_t stream);
// Segmented / fused form: `N` of the workspace and fits checks is the largest
// segment N; kSwiGLU needs an even wave count.
SplitKNeed decode_mfma_workspace_segs(const DecodeMfmaConfig& c, const LinearSegs& s, int K);
hipError_t launch_gemv_mfma_segs(const DecodeMfmaConfig& c, const float* x,
                                 const LinearSegs& s, int M, int K, const SplitKWorkspace& ws,
                                 hipStream_t stream);

// Linear GEMM on bf16 MFMA (prefill): same contract as launch_gemv, any M.
// X is first converted to bf16 into the workspace scratch; `splits` K splits
// (1 = none) meet in the split-K partials.
struct GemmConfig {
  int bm;      // tile rows: 128 or 256
  int bn;      // tile columns: 64, 96 or 128
  int splits;  // K splits, 1..64
};
GemmConfig gemm_mfma_pick(int M, int N, int K);
bool gemm_mfma_config_valid(const GemmConfig& c);
SplitKNeed gemm_mfma_workspace(const GemmConfig& c, int M, int N, int K);
bool gemm_mfma_fits(const GemmConfig& c, int M, int N, int K);
hipError_t launch_gemm_mfma(const GemmConfig& c, const float* x, const uint8_t* w,
                            const float* bias, float* y, int M, int N, int K,
                            const SplitKWorkspace& ws, hipStream_t stream);
// Segmented / fused form (kSwiGLU: BN/2 rows of each weight per tile).
GemmConfig gemm_mfma_pick_segs(int M, const LinearSegs& s, int K);
SplitKNeed gemm_mfma_workspace_segs(const GemmConfig& c, int M, const LinearSegs& s, int K);
hipError_t launch_gemm_mfma_segs(const GemmConfig& c, const float* x, const LinearSegs& s,
                                 int M, int K, const SplitKWorkspace& ws, hipStream_t stream);
// Whether a MatMul (layout kKN: one plain segment, seg[0].w = B[K, N]) fits the
// GEMM's 32-bit offsets within B.
bool gemm_mfma_kn_fits(const LinearSegs& s, int K);
// Tile choice of a MatMul on the GEMM (128-row tiles only).
GemmConfig gemm_mfma_pick_kn(int M, int N, int K);

// MatMul C[M,N] = A[M,K] . B[K,N] with B in Q8_0 blocks along N.  When the
// launch spreads K over several workgroups per tile it needs the workspace
// matmul_workspace(M, N, K) names: `partials` floats and, for M <= 8, tile
// counters (zero between launches; the kernel resets them).
struct MatmulNeed {
  size_t partial_floats = 0;
  size_t counters = 0;
};
MatmulNeed matmul_workspace(int M, int N, int K);
hipError_t launch_matmul(const float* a, const uint8_t* b, float* c, int M, int N, int K,
                         float* partials, uint32_t* counters, hipStream_t stream);

// Greedy argmax of `rows` rows of n fp32 logits: idx (and val, if non-null) per
// row; `keys` is a workspace of rows * argmax_chunks(n) 64-bit entries.
int argmax_chunks(int64_t n);
hipError_t launch_argmax(const float* x, int rows, int64_t n, int32_t* idx, float* val,
                         uint64_t* keys, hipStream_t stream);

// Top-n tokens of `rows` rows of n fp32 logits with their softmax
// probabilities (temperature applied when > 0 and != 1): ids / probs are
// [rows][min(top_n, n)], largest probability first, ties to the lower index;
// `workspace` holds top_tokens_workspace_floats() floats.  Needs
// 1 <= top_n <= kTopTokensMax and n <= topk_max_n(min(top_n, n)).
constexpr int kTopTokensMax = 128;
int topk_chunks(int64_t n);
int topk_max_n(int k);
size_t top_tokens_workspace_floats(int rows, int64_t n, int top_n);
hipError_t launch_top_tokens(const float* x, int rows, int64_t n, int top_n, float temperature,
                             int32_t* ids, float* probs, float* workspace, hipStream_t stream);

// p[i] = v for i < n (clears workspace counters: a kernel, so that a captured
// call records no memset node).
hipError_t launch_fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t stream);

// y = silu(g) * u over n fp32 elements.
hipError_t launch_swiglu(const float* g, const float* u, float* y, int64_t n,
                         hipStream_t stream);
// Streaming-read probe: reads `bytes` (a multiple of 16) of src once; `sink` is
// one device word that is practically never written.
hipError_t launch_stream_read(const void* src, int64_t bytes, uint32_t* sink,
                              hipStream_t stream);

// Embedding gather-dequantise; ids outside [0, vocab) give rows of +0.0f.
hipError_t launch_embedding(const uint8_t* w, const int32_t* ids, float* out,
                            int64_t seq_len, int vocab, int hidden,
                            hipStream_t stream);

// The same gather from a [vocab, hidden] table in 16-row tiles (kTiled, 16-byte
// aligned); bit-identical to launch_embedding on the raw bytes.
hipError_t launch_embedding_tiled(const uint8_t* w_tiled, const int32_t* ids, float* out,
                                  int64_t seq_len, int vocab, int hidden, hipStream_t stream);

// dst[e] = q * d over the flat element stream of a Q8_0 tensor of n elements
// (the weight loader's Float32 branch); dst 16-byte aligned.
hipError_t launch_dequantize_q8_0(const uint8_t* w, float* out, int64_t n, hipStream_t stream);

// Scale decode of raw binary16 patterns (test hook).
hipError_t launch_f16_decode(const uint16_t* bits, float* out, int64_t n,
                             hipStream_t stream);

}  // namespace mle
