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
};
GemvConfig gemv_pick_config(int M, int N, int K);
bool gemv_config_valid(const GemvConfig& c);
hipError_t launch_gemv(const GemvConfig& cfg, const float* x, const uint8_t* w,
                       const float* bias, float* y, int M, int N, int K,
                       hipStream_t stream);

// Linear GEMM on bf16 MFMA (prefill): same contract as launch_gemv, any M.
hipError_t launch_gemm_mfma(const float* x, const uint8_t* w, const float* bias,
                            float* y, int M, int N, int K, hipStream_t stream);

// MatMul C[M,N] = A[M,K] . B[K,N] with B in Q8_0 blocks along N.
hipError_t launch_matmul(const float* a, const uint8_t* b, float* c, int M,
                         int N, int K, hipStream_t stream);

// Embedding gather-dequantise; ids outside [0, vocab) give rows of +0.0f.
hipError_t launch_embedding(const uint8_t* w, const int32_t* ids, float* out,
                            int64_t seq_len, int vocab, int hidden,
                            hipStream_t stream);

// Scale decode of raw binary16 patterns (test hook).
hipError_t launch_f16_decode(const uint16_t* bits, float* out, int64_t n,
                             hipStream_t stream);

}  // namespace mle
