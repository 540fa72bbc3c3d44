// capi.hip -- extern "C" entry points of libmle_q8_0.so (see include/mle_q8_0.h).
//
// Validation mirrors the reference's device launchers
// (src/runtime/kernels/cuda_kernels.cu:53-130 helpers, :852-868 sgemm(q8_0),
// :918-936 sgemm_nt(q8_0), :1054-1073 embedding(q8_0)): null pointers and
// non-positive sizes are InvalidArgument, a packed dimension that is not a
// multiple of 32 is Unsupported, and a failed launch is RuntimeError carrying
// the HIP error string.  Codes are the reference's ErrorCode values.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <string>

#include "../../include/mle_q8_0.h"
#include "launch.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, std::string msg) {
  g_last_error = std::move(msg);
  return code;
}

int ok() {
  g_last_error.clear();
  return MLE_OK;
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int check_launch(hipError_t err, const char* what) {
  if (err == hipSuccess) return ok();
  return fail(MLE_RUNTIME_ERROR, std::string(what) + ": " + hipGetErrorString(err));
}

int check_ptrs(const char* ctx, const void* a, const char* an, const void* b,
               const char* bn, const void* c, const char* cn) {
  const void* ps[3] = {a, b, c};
  const char* ns[3] = {an, bn, cn};
  for (int i = 0; i < 3; ++i)
    if (ps[i] == nullptr)
      return fail(MLE_INVALID_ARGUMENT, std::string("hip ") + ctx + ": " + ns[i] +
                                            " pointer must not be null");
  return MLE_OK;
}

int check_positive(const char* ctx, int v, const char* name) {
  if (v <= 0)
    return fail(MLE_INVALID_ARGUMENT,
                std::string("hip ") + ctx + ": " + name + " must be positive");
  return MLE_OK;
}

int check_align(const char* ctx, const void* p, uintptr_t a, const char* name) {
  if (p != nullptr && !aligned(p, a))
    return fail(MLE_INVALID_ARGUMENT, std::string("hip ") + ctx + ": " + name +
                                          " must be " + std::to_string(a) +
                                          "-byte aligned");
  return MLE_OK;
}

#define MLE_TRY(expr)          \
  do {                         \
    const int _rc = (expr);    \
    if (_rc != MLE_OK) return _rc; \
  } while (0)

int validate_linear(const float* x, const uint8_t* w, const float* bias, float* y,
                    int M, int N, int K) {
  const char* ctx = "sgemm_nt_q8_0_weight";
  MLE_TRY(check_ptrs(ctx, x, "A", w, "B", y, "C"));
  MLE_TRY(check_positive(ctx, M, "M"));
  MLE_TRY(check_positive(ctx, N, "N"));
  MLE_TRY(check_positive(ctx, K, "K"));
  if (K % 32 != 0)
    return fail(MLE_UNSUPPORTED, "hip sgemm_nt Q8_0 requires K to be a multiple of 32");
  MLE_TRY(check_align(ctx, x, 16, "A"));
  MLE_TRY(check_align(ctx, w, 2, "B"));
  MLE_TRY(check_align(ctx, y, 16, "C"));
  MLE_TRY(check_align(ctx, bias, 4, "bias"));
  return MLE_OK;
}

int run_linear(const float* x, const uint8_t* w, const float* bias, float* y, int M,
               int N, int K, int path, mle::GemvConfig cfg, hipStream_t stream) {
  if (path == 0) path = M >= 64 ? 2 : 1;
  if (path == 2)
    return check_launch(mle::launch_gemm_mfma(x, w, bias, y, M, N, K, stream),
                        "hip sgemm_nt Q8_0 launch failed");
  // FP32 GEMV in chunks of at most 8 tokens.
  for (int m0 = 0; m0 < M; m0 += 8) {
    const int mc = M - m0 < 8 ? M - m0 : 8;
    mle::GemvConfig c = cfg;
    if (c.mt == 0) {
      c = mle::gemv_pick_config(mc, N, K);
    } else if (c.mt < mc) {
      return fail(MLE_INVALID_ARGUMENT, "hip sgemm_nt_q8_0_weight: GEMV token tile " +
                                            std::to_string(c.mt) + " is smaller than M");
    }
    const hipError_t err = mle::launch_gemv(c, x + (int64_t)m0 * K, w, bias,
                                            y + (int64_t)m0 * N, mc, N, K, stream);
    if (err != hipSuccess) return check_launch(err, "hip sgemm_nt Q8_0 launch failed");
  }
  return ok();
}

}  // namespace

extern "C" {

int mle_q8_0_abi_version(void) { return 1; }

const char* mle_last_error(void) { return g_last_error.c_str(); }

size_t mle_q8_0_bytes(int64_t numel) {
  if (numel < 0) return 0;
  const uint64_t blocks = ((uint64_t)numel + 31u) / 32u;
  if (blocks > SIZE_MAX / 34u) return 0;
  return (size_t)(blocks * 34u);
}

int mle_q8_0_linear(const float* x, const uint8_t* w_q8_0, const float* bias, float* y,
                    int M, int N, int K, hipStream_t stream) {
  MLE_TRY(validate_linear(x, w_q8_0, bias, y, M, N, K));
  return run_linear(x, w_q8_0, bias, y, M, N, K, 0, mle::GemvConfig{0, 0, 0}, stream);
}

int mle_q8_0_linear_ex(const float* x, const uint8_t* w_q8_0, const float* bias,
                       float* y, int M, int N, int K, int path, int mt, int lpr, int rw,
                       hipStream_t stream) {
  MLE_TRY(validate_linear(x, w_q8_0, bias, y, M, N, K));
  if (path < 0 || path > 2)
    return fail(MLE_INVALID_ARGUMENT, "hip sgemm_nt_q8_0_weight: path must be 0, 1 or 2");
  mle::GemvConfig cfg{mt, lpr, rw};
  const bool all_zero = mt == 0 && lpr == 0 && rw == 0;
  if (!all_zero && !mle::gemv_config_valid(cfg))
    return fail(MLE_INVALID_ARGUMENT,
                "hip sgemm_nt_q8_0_weight: invalid GEMV launch shape (mt " +
                    std::to_string(mt) + ", lpr " + std::to_string(lpr) + ", rw " +
                    std::to_string(rw) + ")");
  if (all_zero) cfg = mle::GemvConfig{0, 0, 0};
  return run_linear(x, w_q8_0, bias, y, M, N, K, path, cfg, stream);
}

int mle_q8_0_matmul(const float* a, const uint8_t* b_q8_0, float* c, int M, int N, int K,
                    hipStream_t stream) {
  const char* ctx = "sgemm_q8_0_weight";
  MLE_TRY(check_ptrs(ctx, a, "A", b_q8_0, "B", c, "C"));
  MLE_TRY(check_positive(ctx, M, "M"));
  MLE_TRY(check_positive(ctx, N, "N"));
  MLE_TRY(check_positive(ctx, K, "K"));
  if (K % 32 != 0 || N % 32 != 0)
    return fail(MLE_UNSUPPORTED, "hip sgemm Q8_0 requires K and N to be multiples of 32");
  MLE_TRY(check_align(ctx, a, 4, "A"));
  MLE_TRY(check_align(ctx, b_q8_0, 2, "B"));
  MLE_TRY(check_align(ctx, c, 16, "C"));
  return check_launch(mle::launch_matmul(a, b_q8_0, c, M, N, K, stream),
                      "hip sgemm Q8_0 launch failed");
}

int mle_q8_0_embedding(const uint8_t* table_q8_0, const int32_t* ids, float* out,
                       int seq_len, int vocab, int hidden, hipStream_t stream) {
  const char* ctx = "embedding_q8_0_weight";
  MLE_TRY(check_ptrs(ctx, table_q8_0, "weight", ids, "ids", out, "out"));
  if (seq_len < 0)
    return fail(MLE_INVALID_ARGUMENT,
                std::string("hip ") + ctx + ": seq_len must not be negative");
  MLE_TRY(check_positive(ctx, vocab, "vocab_size"));
  MLE_TRY(check_positive(ctx, hidden, "hidden"));
  if (hidden % 32 != 0)
    return fail(MLE_UNSUPPORTED,
                "hip embedding Q8_0 requires hidden to be a multiple of 32");
  MLE_TRY(check_align(ctx, table_q8_0, 2, "weight"));
  MLE_TRY(check_align(ctx, ids, 4, "ids"));
  MLE_TRY(check_align(ctx, out, 16, "out"));
  if (seq_len == 0) return ok();
  return check_launch(
      mle::launch_embedding(table_q8_0, ids, out, seq_len, vocab, hidden, stream),
      "hip embedding Q8_0 launch failed");
}

int mle_q8_0_f16_decode(const uint16_t* bits, float* out, int64_t n, hipStream_t stream) {
  if (bits == nullptr || out == nullptr)
    return fail(MLE_INVALID_ARGUMENT, "hip f16_decode: pointers must not be null");
  if (n < 0) return fail(MLE_INVALID_ARGUMENT, "hip f16_decode: n must not be negative");
  return check_launch(mle::launch_f16_decode(bits, out, n, stream),
                      "hip f16_decode launch failed");
}

}  // extern "C"
