/*
 * mle_q8_0.h -- C ABI of the MI355X (gfx950) Q8_0 weight-only Linear / MatMul /
 * Embedding kernels: the drop-in boundary for MiniLLMEngine's Q8_0 path.
 *
 * Library: llmengine_amd/libmle_q8_0.so (hand-written HIP kernels for gfx950).
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are DEVICE pointers (HIP device memory).  Q8_0 data is
 *     the raw GGUF block_q8_0 stream: per 34-byte block a little-endian binary16
 *     scale d followed by 32 int8 quants q; value = d * q.
 *   - Work is enqueued on `stream` (NULL = the default stream) and is
 *     asynchronous; the caller synchronises.  The Linear entry points keep a
 *     split-K workspace (partial sums + tile counters) per (device, stream),
 *     and a second one per (device, stream) for calls made while the stream
 *     is capturing a HIP graph, so a captured call never shares buffers with
 *     eager calls (graphs captured on one stream share theirs: replays of two
 *     such graphs must not overlap in time).  A caller that must not allocate
 *     on its hot path reserves both beforehand (mle_q8_0_workspace_size +
 *     mle_workspace_reserve), and capture requires it; otherwise the eager one
 *     is allocated with hipMalloc on first need.  It only grows: a buffer too
 *     small for a call is replaced by one of max(need, 2 x capacity, 4 MiB) bytes
 *     (counters: at least 4096) and
 *     the old one is kept (launches already enqueued, or captured in a HIP
 *     graph, still use it), so growth never synchronises; everything lives
 *     until process exit.  Nothing else is allocated.  Entry points are
 *     re-entrant and may be called from several host threads, also on one
 *     stream; calls writing the same output buffer on different streams race,
 *     as with any kernel.
 *   - Return value: 0 on success, else a value of the reference's ErrorCode
 *     enum (include/minillm/core/status.h:20-32): 1 InvalidArgument,
 *     2 OutOfRange, 3 ShapeMismatch, 4 Unsupported, 6 RuntimeError.  The
 *     message of the last failure on the calling thread is mle_last_error().
 *   - Alignment: fp32 activation/output buffers must be 16-byte aligned (any
 *     hipMalloc'd buffer is), Q8_0 buffers 2-byte aligned (16-byte for weights in
 *     16-row tiles, mle_q8_0_tile), ids 4-byte aligned.
 */
#ifndef MLE_Q8_0_H
#define MLE_Q8_0_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLE_OK 0
#define MLE_INVALID_ARGUMENT 1
#define MLE_OUT_OF_RANGE 2
#define MLE_SHAPE_MISMATCH 3
#define MLE_UNSUPPORTED 4
#define MLE_RUNTIME_ERROR 6

/* ABI revision of this header; bumped on any signature change. */
int mle_q8_0_abi_version(void);

/*
 * Q8_0 Linear: y[M,N] = x[M,K] . W^T (+ bias[N]), W = [N,K] Q8_0 (blocks along K,
 * row n starts at byte n*(K/32)*34).  FP32 activations, FP32 accumulation.
 *
 * Replaces minillm::cuda::sgemm_nt(const float* A, const uint8_t* B_q8_0,
 * float* C, int M, int N, int K)  (reference include/minillm/runtime/kernels/
 * cuda_kernels.h:16, src/runtime/kernels/cuda_kernels.cu:918-936) followed by
 * minillm::cuda::add_bias(float*, const float*, int, int) (cuda_kernels.h:22),
 * which this entry point fuses when `bias` is non-NULL (NULL = no bias).
 *
 * Paths: M == 1, M <= 4 with K <= 1024 and N <= 32768, and M == 2 with
 * 2048 <= K <= 4096 and N <= 32768, run the FP32 decode GEMV; other
 * M < 64 run the MFMA decode kernel in chunks of up to 16 tokens (FP32
 * activations split exactly into three bf16 parts, so it matches FP32 to about
 * 1e-7 relative L2);
 * M >= 64 runs the bf16-MFMA prefill GEMM (relative L2 error vs FP32 about
 * 2e-3).  Both MFMA paths may split K over workgroups and reduce the partials
 * in a fixed order, so results are deterministic run to run.
 * Errors: NULL x/w/y -> InvalidArgument; M, N or K <= 0 -> InvalidArgument;
 * K % 32 != 0 -> Unsupported ("... requires K to be a multiple of 32").
 */
int mle_q8_0_linear(const float* x, const uint8_t* w_q8_0, const float* bias,
                    float* y, int M, int N, int K, hipStream_t stream);

/*
 * mle_q8_0_linear with a BFloat16 bias: y[M,N] = x . W^T + (float)bias_bf16[N],
 * the bias widened exactly and added in fp32 once, after the dot product, as
 * the reference's CUDA adapter does for a BFloat16 bias on a Q8_0 Linear
 * (cuda_kernel_adapter.cpp:204-218: sgemm_nt, then add_bias(float*, const
 * uint16_t*, rows, cols), cuda_kernels.cu:229-233, 963-969), fused into the
 * Linear's epilogue.  bias_bf16 may be NULL (no bias), else 2-byte aligned.
 * The _tiled form takes weights in 16-row tiles (mle_q8_0_tile).  Paths,
 * precision and errors as mle_q8_0_linear / mle_q8_0_linear_tiled.
 */
int mle_q8_0_linear_bias_bf16(const float* x, const uint8_t* w_q8_0, const uint16_t* bias_bf16,
                              float* y, int M, int N, int K, hipStream_t stream);
int mle_q8_0_linear_tiled_bias_bf16(const float* x, const uint8_t* w_tiled,
                                    const uint16_t* bias_bf16, float* y, int M, int N, int K,
                                    hipStream_t stream);

/*
 * Fused gate/up Linear + SwiGLU: y[M,N] = silu(x . Wg^T) * (x . Wu^T), with
 * silu(g) = g / (1 + exp(-g)) evaluated as the reference does
 * (src/runtime/kernels/cpu_kernels.cpp:848-858).  Wg and Wu are [N,K] Q8_0.
 *
 * Replaces the three ops of the reference's FFN front
 * (src/model/transformer_graph_builder.cpp:261-268): Linear(gate), Linear(up) and
 * SwiGLU (cuda_kernels.cu:245-248), i.e. two sgemm_nt launches, one swiglu launch
 * and two [M,N] fp32 intermediates written and read back.  One launch reads
 * both weights against one copy of the activations.  Paths and precision as for
 * mle_q8_0_linear (FP32 GEMV for M == 1, FP32-exact MFMA decode for M < 64,
 * bf16 MFMA GEMM otherwise).  No bias.
 * Errors: as mle_q8_0_linear; a NULL w_up -> InvalidArgument.
 */
int mle_q8_0_linear_swiglu(const float* x, const uint8_t* w_gate, const uint8_t* w_up,
                           float* y, int M, int N, int K, hipStream_t stream);

/*
 * Multi-output Q8_0 Linear: y[i][M,N[i]] = x[M,K] . W[i]^T (+ bias[i][N[i]]) for
 * i < count (1..3), in one launch that reads x once for all weights.
 *
 * Replaces the q/k/v projections of one layer, three Linears on the same input
 * (src/model/transformer_graph_builder.cpp:214-221).  `bias` may be NULL (no
 * bias anywhere) or hold NULL entries.  For M < 64 each output is bit-identical
 * to mle_q8_0_linear on the same operands (same kernel arithmetic); M >= 64
 * takes the bf16 MFMA GEMM with a tile choice of its own.
 * Errors: count outside 1..3 or NULL w / y / N arrays -> InvalidArgument; each
 * output is validated as mle_q8_0_linear validates its operands.
 */
int mle_q8_0_linear_multi(const float* x, int count, const uint8_t* const* w,
                          const float* const* bias, float* const* y, const int* N, int M,
                          int K, hipStream_t stream);

/*
 * Q8_0 MatMul: c[M,N] = a[M,K] . B[K,N], B = [K,N] Q8_0 stored row-major, so
 * element (k,n) is flat index k*N+n and blocks run along N.
 *
 * Replaces minillm::cuda::sgemm(const float* A, const uint8_t* B_q8_0, float* C,
 * int M, int N, int K)  (reference cuda_kernels.h:13, cuda_kernels.cu:852-868).
 * Elements as the reference CPU kernel cpu::sgemm(q8_0) forms them
 * (src/runtime/kernels/cpu_kernels.cpp:116-130), v = d*q in fp32.
 *   M < 64 (or A not 16-byte aligned): FP32 FMAs; the K sum is split into
 *   fixed pieces added in a fixed order (as the reference's device kernel
 *   splits K over warps), so results are deterministic and within fp32
 *   rounding of the CPU kernel (relative L2 <= 1e-5; small exact cases match it
 *   bit for bit).
 *   M >= 64: the bf16 MFMA GEMM of the Linear prefill, B dequantised
 *   transposed into its W tile: A and d*q rounded once to bf16, fp32
 *   accumulation, deterministic; relative L2 <= 1e-2 (about 2e-3 on N(0,1)
 *   data), as the Linear GEMM.
 * Uses the per-(device, stream) workspace of the Linear calls (split-K
 * partials, the GEMM's bf16 copy of A).
 * Errors: NULL pointers, non-positive sizes -> InvalidArgument;
 * K % 32 != 0 or N % 32 != 0, or more than 524280 rows -> Unsupported.
 */
int mle_q8_0_matmul(const float* a, const uint8_t* b_q8_0, float* c, int M,
                    int N, int K, hipStream_t stream);

/*
 * Q8_0 Embedding: out[s,h] = d*q of element h of table row ids[s]
 * (table = [vocab, hidden] Q8_0, blocks along hidden).  Bit-identical to the
 * reference CPU kernel cpu::embedding(q8_0) (cpu_kernels.cpp:286-295) for ids
 * in [0, vocab); an id outside that range gives a row of +0.0f, as the
 * reference device kernel does (cuda_kernels.cu:410-415).
 *
 * Replaces minillm::cuda::embedding(const uint8_t* weight_q8_0, const int* ids,
 * float* out, int seq_len, int vocab_size, int hidden)  (reference
 * cuda_kernels.h:37-38, cuda_kernels.cu:1054-1073).
 * Errors: NULL pointers, seq_len < 0, vocab or hidden <= 0 -> InvalidArgument;
 * hidden % 32 != 0 -> Unsupported.  seq_len == 0 is a no-op (as on the CPU path).
 */
int mle_q8_0_embedding(const uint8_t* table_q8_0, const int32_t* ids, float* out,
                       int seq_len, int vocab, int hidden, hipStream_t stream);

/*
 * mle_q8_0_embedding on a table in Q8_0 16-row tiles (mle_q8_0_tile of the
 * [vocab, hidden] table; 16-byte aligned): the same output, bit for bit, so a
 * table shared with a Linear (a tied lm_head) needs only its tiled copy.  No
 * counterpart in the reference (its tables are raw GGUF bytes).  Errors as
 * mle_q8_0_embedding, plus a table not 16-byte aligned -> InvalidArgument.
 */
int mle_q8_0_embedding_tiled(const uint8_t* table_tiled, const int32_t* ids, float* out,
                             int seq_len, int vocab, int hidden, hipStream_t stream);

/*
 * Q8_0 -> fp32 dequantisation of a whole tensor on the device: dst[e] = q * d
 * for the n elements of the raw block stream (ceil(n/32) blocks; a partial last
 * block reads only its first n % 32 quants).  Replaces the Q8_0 case of
 * WeightLoader::dequantize_to_f32 (reference src/io/gguf_weight_loader.cpp:446-463),
 * which the loader runs on the host for Float32 tensors; bit-identical to it
 * (one fp32 multiply of an exactly decoded binary16 scale).
 * Errors: NULL pointers or n < 0 -> InvalidArgument; src must be 2-byte and dst
 * 16-byte aligned.  n == 0 is a no-op.
 */
int mle_q8_0_dequantize(const uint8_t* src_q8_0, float* dst, int64_t n, hipStream_t stream);

/*
 * Unfused SwiGLU: y[i] = silu(gate[i]) * up[i] for i < n (n == 0: no-op),
 * evaluated as the reference does ((g / (1 + exp(-g))) * u).  Replaces the
 * reference's swiglu launcher (src/runtime/kernels/cuda_kernels.cu:245-248) for
 * the HIP backend's SwiGLU op.
 * Errors: NULL pointers or n < 0 -> InvalidArgument.
 */
int mle_swiglu_f32(const float* gate, const float* up, float* y, int64_t n,
                   hipStream_t stream);

/*
 * Greedy argmax of lm_head logits on the device: idx[r] = the first index of the
 * largest value of logits[r*n : (r+1)*n] (ties -> lower index; -0 == +0; NaN
 * entries ignored, a row of NaN only gives 0), val[r] = that value (val may be
 * NULL).  Deterministic.  Replaces the device-to-host copy of every logits row
 * that the reference's CUDA generator makes for its host-side greedy pick
 * (examples/generate_cuda.cpp:81-94, 305-314; src/runtime/sampler.cpp:108-118):
 * the caller copies back 4 (or 8) bytes per row instead.
 * Errors: NULL logits / idx, rows or n <= 0 -> InvalidArgument; rows > 65535 ->
 * Unsupported.  Uses the per-(device, stream) workspace of the Linear calls.
 */
int mle_argmax_f32(const float* logits, int rows, int n, int32_t* idx, float* val,
                   hipStream_t stream);

/*
 * The top_n tokens of each logits row with their softmax probabilities, on the
 * device: Sampler::get_top_tokens (src/runtime/sampler.cpp:141-197).  Row r of
 * n logits is scaled by 1 / temperature when temperature > 0 and != 1, then
 * p = exp(v - max) * (1 / sum); ids[r*k + j], probs[r*k + j] (k = min(top_n, n))
 * are the top k tokens, largest probability first, ties to the lower index.  A
 * row with a NaN, a non-finite maximum or a non-finite or zero sum gives the
 * uniform 1/n (ids 0, 1, ...), as the reference does.  With the k candidates
 * on the host, Sampler::sample's top-k / top-p / draw (:65-138) runs on k
 * values instead of the whole row the reference's generator copies back
 * (examples/generate_cuda.cpp:81-94).  Deterministic.
 * Errors: NULL logits / ids / probs, rows or n <= 0 -> InvalidArgument;
 * top_n <= 0 -> nothing written (the reference's empty list); rows > 65535,
 * top_n > 128, or n > (16384 / k) * 2048 -> Unsupported.  Uses the
 * per-(device, stream) workspace of the Linear calls.
 */
int mle_top_tokens_f32(const float* logits, int rows, int n, int top_n, float temperature,
                       int32_t* ids, float* probs, hipStream_t stream);

/*
 * Q8_0 16-row tiles: the bytes of a raw Q8_0 weight [N,K] reordered once, at
 * weight-load time, for the MI355X matrix cores.  No counterpart in the
 * reference: its loader copies GGUF bytes to the device as they are
 * (src/io/gguf_weight_loader.cpp:102-116); a loader that calls
 * mle_q8_0_tile after that copy keeps the same bytes per block (34) and gets
 * decode launches whose weight loads are contiguous 1 KB pieces per wave.
 *
 * Layout, with KB = K/32 blocks, KP = ceil(KB/2) block pairs, G = ceil(N/16)
 * row groups: G*KP quant pieces of 1024 bytes ((g, p) at (g*KP + p)*1024),
 * then G*KP scale pieces of 64 bytes ((g, p) at G*KP*1024 + (g*KP + p)*64).
 * Bytes 16l .. 16l+7 of quant piece (g, p) (l = 0..63) are quants
 * 8(l/16) .. 8(l/16)+7 of block 2p of row 16g + l%16, bytes 16l+8 .. 16l+15
 * the same quants of block 2p+1; dword r of scale piece (g, p) is the binary16
 * scale of block 2p (low half) and 2p+1 (high half) of row 16g + r.  Rows past
 * N and the block past an odd KB are zero.
 *
 * mle_q8_0_tiled_bytes: G*KP*1088; 0 for N <= 0, K <= 0 or K % 32 != 0.
 * mle_q8_0_tile: raw -> tiled on `stream`.  w_tiled is 16-byte aligned, holds
 *   mle_q8_0_tiled_bytes(N, K) bytes and does not overlap w_q8_0.
 *   Errors: NULL pointers, N or K <= 0, misalignment, overlap ->
 *   InvalidArgument; K % 32 != 0 -> Unsupported.
 * mle_q8_0_linear_tiled / _swiglu_tiled / _multi_tiled: mle_q8_0_linear /
 *   _swiglu / _multi on tiled weights (16-byte aligned), same errors.  Paths:
 *   an FP32 GEMV for M == 1, M == 2 below 65536 output rows and M <= 4 with
 *   K <= 1024 and at most 32768 output rows (the K split stays inside a
 *   workgroup: no workspace); otherwise the MFMA decode (M < 64) and the bf16
 *   MFMA GEMM (M >= 64), each bit-identical to the raw entry point on the same
 *   path.  Where one side runs an FP32 GEMV the two agree to about 1e-7
 *   relative L2; a fused multi-output launch on the GEMV agrees with the single
 *   tiled Linear to fp32 rounding (its K split follows the launch shape).
 */
size_t mle_q8_0_tiled_bytes(int N, int K);
int mle_q8_0_tile(const uint8_t* w_q8_0, uint8_t* w_tiled, int N, int K, hipStream_t stream);
int mle_q8_0_linear_tiled(const float* x, const uint8_t* w_tiled, const float* bias, float* y,
                          int M, int N, int K, hipStream_t stream);
int mle_q8_0_linear_swiglu_tiled(const float* x, const uint8_t* w_gate, const uint8_t* w_up,
                                 float* y, int M, int N, int K, hipStream_t stream);
int mle_q8_0_linear_multi_tiled(const float* x, int count, const uint8_t* const* w,
                                const float* const* bias, float* const* y, const int* N, int M,
                                int K, hipStream_t stream);

/*
 * Workspace reservation (no counterpart in the reference: its CUDA kernels need
 * no workspace, cuda_kernels.cu:918-936; this keeps allocation off the hot path
 * as the reference's RuntimeContext keeps it off for outputs,
 * runtime_context.cpp:78-220).
 *
 * mle_q8_0_workspace_size: *bytes / *counters = the workspace a call would use
 *   on the per-stream workspace: op MLE_OP_LINEAR (count 1, mle_q8_0_linear),
 *   MLE_OP_LINEAR_SWIGLU (count 2, N[0] == N[1], mle_q8_0_linear_swiglu) or
 *   MLE_OP_LINEAR_MULTI (count 1..3, mle_q8_0_linear_multi), with M tokens,
 *   output sizes N[0..count), input size K, on raw (tiled == 0) or 16-row
 *   tiled weights (0 / 0 for launches that need none: the FP32 GEMVs, and the
 *   decode of tiled plain Linears by whole row ranges), or MLE_OP_MATMUL
 *   (count 1, mle_q8_0_matmul: A [M, K], B [K, N[0]]; tiled ignored).  Launches
 *   nothing.  Errors: NULL outputs / N, M or K or an
 *   N <= 0, a bad count or op -> InvalidArgument; K % 32 != 0 (MatMul: or
 *   N % 32 != 0) -> Unsupported.
 * mle_workspace_reserve: grows the eager and the graph workspace of (current
 *   device, stream) to hold at least `bytes` and `counters` each (a no-op when
 *   they already do); later calls within those sizes allocate and synchronise
 *   nothing, eager or captured.  When the graph workspace grows, the call
 *   synchronises `stream` once (its counters are cleared by a kernel there, and
 *   a graph captured later may be replayed on any stream).  A call captured on
 *   a stream whose graph workspace is too small returns RuntimeError ("reserve
 *   it before capture").
 * mle_workspace_info: capacity of (current device, stream)'s eager workspace
 *   and the number of (re)allocations it has had (0 / 0 / 0 when it has none
 *   yet).
 * mle_workspace_plan_growth (test hook): the growth rule, applied to
 *   capacities and a need without allocating: returns 1 and the new capacities
 *   when the need does not fit (a buffer too small takes max(need,
 *   2 x capacity, minimum), the other keeps its capacity), else 0 and the
 *   capacities unchanged; -1 for NULL outputs.
 */
#define MLE_OP_LINEAR 0
#define MLE_OP_LINEAR_SWIGLU 1
#define MLE_OP_LINEAR_MULTI 2
#define MLE_OP_MATMUL 3
int mle_q8_0_workspace_size(int op, int M, int count, const int* N, int K, int tiled,
                            size_t* bytes, size_t* counters);
int mle_workspace_reserve(size_t bytes, size_t counters, hipStream_t stream);
int mle_workspace_info(hipStream_t stream, size_t* bytes, size_t* counters,
                       uint64_t* generation);
int mle_workspace_plan_growth(size_t cap_bytes, size_t cap_counters, size_t need_bytes,
                              size_t need_counters, size_t* new_bytes, size_t* new_counters);

/*
 * mle_q8_0_linear without any allocation, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same operands, paths,
 * kernels, results (bit-identical to mle_q8_0_linear) and errors, but the
 * split-K partials, tile counters and prefill scratch live in one static device
 * array per GPU (32 MiB + 65536 counters, held from library load until process
 * exit) instead of the per-stream workspace; nothing is allocated or freed.
 * A shape needing more scratch than that is rejected with Unsupported before
 * any launch (every benchmark shape fits: prefill [512 x 4096 x 11008] takes
 * 28 MB).  All calls on one GPU share the array: calls that overlap in time on
 * one GPU (different streams, or threads without ordering) race and give wrong
 * results; calls ordered on one stream do not.  The first call on a GPU clears
 * the array's counters with a kernel on `stream`; it returns RuntimeError if
 * `stream` is capturing a graph (make one call outside capture first).
 */
int mle_q8_0_linear_noalloc(const float* x, const uint8_t* w_q8_0, const float* bias,
                            float* y, int M, int N, int K, hipStream_t stream);

/*
 * Message of the last failed call on this thread ("" if none).  Stands in for
 * the message of the reference's Status return (status.h:34-59).  The pointer
 * stays valid until the next call on the same thread.
 */
const char* mle_last_error(void);

/*
 * Raw Q8_0 byte size of a tensor with `numel` elements: ceil(numel/32)*34.
 * Same rule as the reference's q8_required_bytes (src/runtime/kernels/
 * cuda_kernel_adapter.cpp:86-97) and GGUFTensorInfo::bytes()
 * (src/io/gguf_parser.cpp:226-243).  Returns 0 on overflow or numel < 0.
 */
size_t mle_q8_0_bytes(int64_t numel);

/*
 * Test / tuning hooks (no counterpart in the reference).
 *
 * mle_q8_0_f16_decode: out[i] = the scale value the kernels use for the
 *   binary16 pattern bits[i] (exact; NaN canonicalised as the reference CPU
 *   decode does, cpu_kernels.cpp:21-37).  Used for the exhaustive decode check.
 * mle_q8_0_linear_ex: mle_q8_0_linear with the path forced (path 1 = FP32 GEMV
 *   for any M, path 2 = bf16-MFMA GEMM for any M, path 3 = MFMA decode with
 *   FP32-exact activations for any M, 0 = automatic) and an optional launch
 *   shape t0..t3 (all four 0 = automatic):
 *     path 1: t0 = token tile mt in {1,2,4,8} >= min(M,8), t1 = lanes per row
 *             in {16,32,64}, t2 = rows per lane group in {1,2,4,8}, t3 = 0,
 *             or t0 = 1 and t3 = 4: the row-span kernel on raw weights (one
 *             token, 4 rows per workgroup, lanes along K; t1, t2 unused);
 *     path 2: t0 = K splits in [1, 64], t1 = tile rows in {128, 256},
 *             t2 = tile columns in {64, 96, 128} (at most 96 for 256 rows),
 *             t3 = 0 (a 0 among t0..t2 keeps that field automatic);
 *     path 3: t0 = token tile in {1,2,4,5,8,16} >= min(M,16), t1 = waves per
 *             workgroup in {2,4,8} (16 rows each), t2 = K blocks per
 *             workgroup in {16, 32} (32 only for a token tile <= 8), t3 = 0,
 *             or t3 in 1..4 = a launch shape of the hybrid kernel (row groups x
 *             a short K split; token tile 4 or 8, t1 and t2 then unused but
 *             valid).
 * mle_q8_0_linear_tiled_ex: the same hook on kTiled weights (path 0 or 3).
 */
int mle_q8_0_f16_decode(const uint16_t* bits, float* out, int64_t n,
                        hipStream_t stream);
int mle_q8_0_linear_ex(const float* x, const uint8_t* w_q8_0, const float* bias,
                       float* y, int M, int N, int K, int path, int t0, int t1,
                       int t2, int t3, hipStream_t stream);
int mle_q8_0_linear_tiled_ex(const float* x, const uint8_t* w_tiled, const float* bias,
                             float* y, int M, int N, int K, int path, int t0, int t1,
                             int t2, int t3, hipStream_t stream);

/*
 * Streaming-read probe, a measurement aid with no counterpart in the reference:
 * reads `bytes` of src once from HBM with nothing else to do (non-temporal
 * 16-byte loads over a fixed grid).  The benchmark times it over the same weight
 * buffers a decode Linear reads, so the Linear's time can be set against a pure
 * read of the same bytes as well as against the HBM peak.  `sink` is one device
 * word, practically never written.
 * Errors: NULL src / sink, bytes < 0 or not a multiple of 16, src not 16-byte
 * aligned -> InvalidArgument.  bytes == 0: no launch.
 */
int mle_probe_stream_read(const void* src, int64_t bytes, uint32_t* sink, hipStream_t stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* MLE_Q8_0_H */
