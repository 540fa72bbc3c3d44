// capi.hip -- extern "C" entry points of libmle_q8_0.so (see include/mle_q8_0.h).
//
// Validation mirrors the reference's device launchers
// (src/runtime/kernels/cuda_kernels.cu:53-130 helpers, :852-868 sgemm(q8_0),
// :918-936 sgemm_nt(q8_0), :1054-1073 embedding(q8_0)): null pointers and
// non-positive sizes are InvalidArgument, a packed dimension that is not a
// multiple of 32 is Unsupported, and a failed launch is RuntimeError carrying
// the HIP error string.  Codes are the reference's ErrorCode values.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <map>
#include <vector>
#include <mutex>
#include <string>
#include <tuple>
#include <utility>

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

int validate_linear(const float* x, const uint8_t* w, const void* bias, float* y,
                    int M, int N, int K, uintptr_t bias_align = 4) {
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
  MLE_TRY(check_align(ctx, bias, bias_align, "bias"));
  return MLE_OK;
}

// Workspace of the MFMA paths, two per (device, stream): split-K partial sums
// and tile counters, and the prefill GEMM's bf16 copy of X.  Eager calls use
// the stream's eager workspace; calls made while the stream is capturing a HIP
// graph use its graph workspace, which no eager call touches, so a graph
// replayed on any stream cannot race eager calls on the capturing stream.
// Eager calls on one stream run in order, so the eager workspace is never used
// by two launches at once; graphs captured on one stream share the graph
// workspace, so their replays must not overlap each other.  Both are reserved
// ahead of the hot path (mle_workspace_reserve, which minillm::HipExecutor
// calls from compile() and tile_weights() for its graph's largest shapes); the
// eager one is otherwise allocated on the first call that needs it, while the
// graph one is never allocated during capture (a capture that needs more than
// the reservation is refused).  A buffer that must grow is replaced by a new
// one of at least twice its capacity; the old one is kept (launches already
// enqueued on the stream, or captured in a HIP graph, may still use it), so
// growth never synchronises, and the kept buffers add up to less than the live
// capacity.  Everything lives until the process ends.
struct StreamWorkspace {
  uint8_t* buf = nullptr;  // partial sums, then scratch
  size_t buf_cap = 0;      // bytes
  uint32_t* counters = nullptr;
  size_t counter_cap = 0;  // uint32 entries
  uint64_t generation = 0;  // (re)allocations so far
  uint64_t synced_generation = 0;  // graph workspace: the generation last waited for
  std::vector<void*> retired;  // replaced buffers, never freed (see above)
};
std::mutex g_ws_mu;
// Key: (device, stream, graph workspace?).
std::map<std::tuple<int, hipStream_t, bool>, StreamWorkspace> g_ws;

bool stream_capturing(hipStream_t stream) {
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone;
}

constexpr size_t kMinWorkspaceBytes = size_t(4) << 20;
constexpr size_t kMinWorkspaceCounters = 4096;

// Growth rule, per buffer: capacities never shrink, and a buffer too small for
// the need takes max(need, 2 x capacity, minimum).  Returns whether either
// buffer must grow.
bool plan_growth(size_t cap_bytes, size_t cap_counters, size_t need_bytes, size_t need_counters,
                 size_t* new_bytes, size_t* new_counters) {
  *new_bytes = need_bytes > cap_bytes ? std::max({need_bytes, 2 * cap_bytes, kMinWorkspaceBytes})
                                      : cap_bytes;
  *new_counters = need_counters > cap_counters
                      ? std::max({need_counters, 2 * cap_counters, kMinWorkspaceCounters})
                      : cap_counters;
  return *new_bytes != cap_bytes || *new_counters != cap_counters;
}

// Bytes of the workspace buffer a launch needs: partial sums (256-byte
// multiple), then scratch.
size_t need_bytes(const mle::SplitKNeed& need) {
  if (need.partial_floats == 0 && need.scratch_bytes == 0) return 0;
  return (need.partial_floats * sizeof(float) + 255) / 256 * 256 + need.scratch_bytes;
}

int ensure_workspace(size_t bytes, size_t counters, hipStream_t stream, bool graph,
                     StreamWorkspace** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return check_launch(err, "hip Q8_0 workspace");
  StreamWorkspace& e = g_ws[{dev, stream, graph}];
  size_t nb = 0, nc = 0;
  if (plan_growth(e.buf_cap, e.counter_cap, bytes, counters, &nb, &nc)) {
    if (stream_capturing(stream))
      return fail(MLE_RUNTIME_ERROR,
                  "hip Q8_0 workspace: this call needs " + std::to_string(bytes) + " bytes and " +
                      std::to_string(counters) +
                      " counters, more than the stream's workspace holds, while the stream is "
                      "capturing a graph; reserve it before capture (mle_q8_0_workspace_size, "
                      "mle_workspace_reserve)");
    uint8_t* buf = e.buf;
    uint32_t* cnt = e.counters;
    if (nb != e.buf_cap) err = hipMalloc(&buf, nb);
    if (err == hipSuccess && nc != e.counter_cap) {
      err = hipMalloc(&cnt, nc * sizeof(uint32_t));
      // Counters start at zero (the kernels leave them at zero); cleared by a
      // kernel rather than a memset node, so a captured first call replays too.
      if (err == hipSuccess) err = mle::launch_fill_u32(cnt, nc, 0u, stream);
    }
    if (err != hipSuccess) {
      if (buf != e.buf) (void)hipFree(buf);
      if (cnt != e.counters) (void)hipFree(cnt);
      return check_launch(err, "hip Q8_0 workspace allocation failed");
    }
    if (buf != e.buf && e.buf != nullptr) e.retired.push_back(e.buf);
    if (cnt != e.counters && e.counters != nullptr) e.retired.push_back(e.counters);
    e.buf = buf;
    e.counters = cnt;
    e.buf_cap = nb;
    e.counter_cap = nc;
    ++e.generation;
  }
  *out = &e;
  return MLE_OK;
}

// `hold` keeps the workspace table locked until the caller has enqueued the
// launch that uses the buffers, so launches from several host threads take the
// buffers in the order they enqueue.
int get_workspace(const mle::SplitKNeed& need, hipStream_t stream, mle::SplitKWorkspace* out,
                  std::unique_lock<std::mutex>* hold) {
  *out = mle::SplitKWorkspace{};
  const size_t bytes = need_bytes(need);
  if (bytes == 0) return MLE_OK;
  const size_t partial_bytes = (need.partial_floats * sizeof(float) + 255) / 256 * 256;
  std::unique_lock<std::mutex> lock(g_ws_mu);
  StreamWorkspace* e = nullptr;
  MLE_TRY(ensure_workspace(bytes, need.counters, stream, stream_capturing(stream), &e));
  out->partials = reinterpret_cast<float*>(e->buf);
  out->counters = e->counters;
  out->scratch = need.scratch_bytes ? e->buf + partial_bytes : nullptr;
  *hold = std::move(lock);
  return MLE_OK;
}

// Where a Linear-family call takes its workspace: the per-stream one, or (plan
// mode) nowhere: the call only records the largest need of its launches and
// launches nothing.
struct Exec {
  hipStream_t stream = nullptr;
  size_t* plan_bytes = nullptr;     // non-null: plan mode
  size_t* plan_counters = nullptr;
  // A caller-fixed workspace (the no-allocation entry point): the launches use
  // these buffers and nothing is allocated.
  bool fixed = false;
  uint8_t* fixed_buf = nullptr;
  size_t fixed_bytes = 0;
  uint32_t* fixed_counters = nullptr;
  size_t fixed_counter_count = 0;
  bool planning() const { return plan_bytes != nullptr; }
};

int workspace_for(const mle::SplitKNeed& need, const Exec& ex, mle::SplitKWorkspace* out,
                  std::unique_lock<std::mutex>* hold) {
  if (ex.planning()) {
    *out = mle::SplitKWorkspace{};
    *ex.plan_bytes = std::max(*ex.plan_bytes, need_bytes(need));
    *ex.plan_counters = std::max(*ex.plan_counters, need.counters);
    return MLE_OK;
  }
  if (ex.fixed) {
    *out = mle::SplitKWorkspace{};
    const size_t bytes = need_bytes(need);
    if (bytes > ex.fixed_bytes || need.counters > ex.fixed_counter_count)
      return fail(MLE_UNSUPPORTED, "hip Q8_0 fixed workspace too small: need " +
                                       std::to_string(bytes) + " bytes and " +
                                       std::to_string(need.counters) + " counters");
    if (bytes == 0) return MLE_OK;
    if (ex.fixed_buf == nullptr)
      return fail(MLE_RUNTIME_ERROR, "hip Q8_0 fixed workspace missing");
    const size_t partial_bytes = (need.partial_floats * sizeof(float) + 255) / 256 * 256;
    out->partials = reinterpret_cast<float*>(ex.fixed_buf);
    out->counters = ex.fixed_counters;
    out->scratch = need.scratch_bytes ? ex.fixed_buf + partial_bytes : nullptr;
    return MLE_OK;
  }
  return get_workspace(need, ex.stream, out, hold);
}

// Linear path numbers (mle_q8_0_linear_ex): 1 FP32 GEMV, 2 bf16-MFMA prefill GEMM,
// 3 MFMA decode with FP32-exact activations.
// The FP32 GEMV also wins for a few tokens on short rows (K <= 1024, e.g. the
// 896-wide Qwen projections: 4.5-5.1 us vs 5.5-7.0 us at M = 2..4, MI355X),
// and for two tokens on rows of 2048-4096 elements (Llama qkv / gate / o_proj
// at M = 2: 15.9 / 15.1 / 8.4 us vs 17.2 / 16.4 / 8.5 for the MFMA decode; not
// down at K = 11008, 19.8 vs 15.6).  The rule looks at M and K only (and the
// vocabulary bound), so a fused q/k/v launch and its three single Linears take
// the same path and agree bit for bit.  Not on a vocabulary-sized weight (the
// [151936, 896] lm_head at M = 4: 50.9 us vs 34.5 us for the MFMA decode).
int pick_path(int M, int N, int K) {
  if (M >= 64) return 2;
  if (M == 1 || (M <= 4 && K <= 1024 && N <= 32768) ||
      (M == 2 && K >= 2048 && K <= 4096 && N <= 32768))
    return 1;
  return 3;
}

struct Tune {
  mle::GemvConfig gemv{0, 0, 0};
  mle::DecodeMfmaConfig dec{0, 0, 0};
  mle::GemmConfig gemm{0, 0, 0};  // 0 fields = automatic
};

// Tiled weights (mle::WeightLayout::kTiled): the tiled FP32 GEMV where
// mle::gemv_tiled_wins (one token; two below vocabulary-sized outputs; up to
// four on short rows), else the MFMA decode below 64 tokens and the MFMA GEMM
// from 64.
int run_linear(const float* x, const uint8_t* w, const void* bias, float* y, int M,
               int N, int K, int path, const Tune& tune, const Exec& ex,
               mle::WeightLayout layout = mle::WeightLayout::kRaw, bool bias_bf16 = false) {
  const bool tiled = layout == mle::WeightLayout::kTiled;
  if (path == 0) {
    path = tiled ? (M >= 64 ? 2 : 3) : pick_path(M, N, K);
    const int mc = M < 16 ? M : 16;
    if (path == 3 && !mle::decode_mfma_fits(mle::decode_mfma_pick(mc, N, K, layout), mc, N, K)) {
      if (tiled)
        return fail(MLE_UNSUPPORTED, "hip sgemm_nt Q8_0: K too large for the MFMA decode");
      path = 1;
    }
  }
  mle::LinearSegs one;
  one.seg[0] = mle::LinearSeg{w, bias, y, N};
  one.seg[0].bias_bf16 = bias_bf16 ? 1 : 0;
  one.layout = layout;
  if (tiled && path == 3 && tune.dec.mt == 0 && M <= 4 && mle::gemv_tiled_wins(M, N, K)) {
    const mle::TiledGemvConfig c = mle::gemv_tiled_pick(M, N, K, false);
    return check_launch((ex.planning() ? hipSuccess : mle::launch_gemv_tiled_segs(c, x, one, M, K, ex.stream)),
                        "hip sgemm_nt Q8_0 launch failed");
  }
  if (path == 2) {
    mle::GemmConfig c = mle::gemm_mfma_pick(M, N, K);
    if (tune.gemm.bm) c.bm = tune.gemm.bm;
    if (tune.gemm.bn) {
      c.bn = tune.gemm.bn;
      if (!tune.gemm.bm && !mle::gemm_mfma_config_valid(c)) c.bm = 128;
    }
    if (tune.gemm.splits) c.splits = tune.gemm.splits;
    if (!mle::gemm_mfma_config_valid(c))
      return fail(MLE_INVALID_ARGUMENT, "hip sgemm_nt_q8_0_weight: invalid MFMA GEMM shape (bm " +
                                            std::to_string(c.bm) + ", bn " +
                                            std::to_string(c.bn) + ")");
    if (!mle::gemm_mfma_fits(c, M, N, K))
      return fail(MLE_UNSUPPORTED, "hip sgemm_nt Q8_0: K too large for the MFMA GEMM");
    mle::SplitKWorkspace ws;
    std::unique_lock<std::mutex> hold;  // released after the launch is enqueued
    MLE_TRY(workspace_for(mle::gemm_mfma_workspace(c, M, N, K), ex, &ws, &hold));
    return check_launch((ex.planning() ? hipSuccess : mle::launch_gemm_mfma_segs(c, x, one, M, K, ws, ex.stream)),
                        "hip sgemm_nt Q8_0 launch failed");
  }
  if (path == 3) {
    // MFMA decode in chunks of at most 16 tokens.
    for (int m0 = 0; m0 < M; m0 += 16) {
      const int mc = M - m0 < 16 ? M - m0 : 16;
      mle::DecodeMfmaConfig c = tune.dec;
      if (c.mt == 0) {
        c = mle::decode_mfma_pick(mc, N, K, layout);
      } else if (c.mt < mc) {
        return fail(MLE_INVALID_ARGUMENT, "hip sgemm_nt_q8_0_weight: MFMA token tile " +
                                              std::to_string(c.mt) + " is smaller than M");
      }
      mle::LinearSegs chunk = one;
      chunk.seg[0].y = y + (int64_t)m0 * N;
      mle::SplitKWorkspace ws;
      std::unique_lock<std::mutex> hold;  // released after the launch is enqueued
      MLE_TRY(workspace_for(mle::decode_mfma_workspace_segs(c, chunk, K), ex, &ws, &hold));
      const hipError_t err =
          (ex.planning() ? hipSuccess : mle::launch_gemv_mfma_segs(c, x + (int64_t)m0 * K, chunk, mc, K, ws, ex.stream));
      if (err != hipSuccess) return check_launch(err, "hip sgemm_nt Q8_0 launch failed");
    }
    return ok();
  }
  // FP32 GEMV in chunks of at most 8 tokens.
  for (int m0 = 0; m0 < M; m0 += 8) {
    const int mc = M - m0 < 8 ? M - m0 : 8;
    mle::GemvConfig c = tune.gemv;
    if (c.mt == 0) {
      c = mle::gemv_pick_config(mc, N, K);
    } else if (c.mt < mc) {
      return fail(MLE_INVALID_ARGUMENT, "hip sgemm_nt_q8_0_weight: GEMV token tile " +
                                            std::to_string(c.mt) + " is smaller than M");
    }
    mle::LinearSegs chunk = one;
    chunk.seg[0].y = y + (int64_t)m0 * N;
    const hipError_t err =
        ex.planning() ? hipSuccess
                      : mle::launch_gemv_segs(c, x + (int64_t)m0 * K, chunk, mc, K, ex.stream);
    if (err != hipSuccess) return check_launch(err, "hip sgemm_nt Q8_0 launch failed");
  }
  return ok();
}

// One launch over 1-3 output segments (multi-output Linear) or a gate/up pair
// (SwiGLU): the same path choice as a single Linear (bf16 MFMA GEMM for
// M >= 64, FP32 GEMV for M == 1, for M <= 4 on short rows and for M == 2 on
// rows of 2048-4096 elements, else the MFMA
// decode kernel in chunks of up to 16 tokens with FP32-exact activations);
// SwiGLU takes the GEMV for M == 1 only.
int run_segs(const char* ctx, const float* x, const mle::LinearSegs& s, int M, int K,
             const Exec& ex) {
  const bool swi = s.mode == mle::Epilogue::kSwiGLU;
  int total_n = 0;
  for (int i = 0; i < s.count; ++i) total_n += s.seg[i].N;
  if (M >= 64) {
    const mle::GemmConfig c = mle::gemm_mfma_pick_segs(M, s, K);
    if (!mle::gemm_mfma_fits(c, M, 0, K))
      return fail(MLE_UNSUPPORTED, std::string("hip ") + ctx + ": K too large for the MFMA GEMM");
    mle::SplitKWorkspace ws;
    std::unique_lock<std::mutex> hold;  // released after the launch is enqueued
    MLE_TRY(workspace_for(mle::gemm_mfma_workspace_segs(c, M, s, K), ex, &ws, &hold));
    return check_launch((ex.planning() ? hipSuccess : mle::launch_gemm_mfma_segs(c, x, s, M, K, ws, ex.stream)),
                        "hip Q8_0 fused Linear launch failed");
  }
  const bool tiled = s.layout == mle::WeightLayout::kTiled;
  const int rows = swi ? s.seg[0].N : total_n;
  if (tiled && M <= 4 && mle::gemv_tiled_wins(M, rows, K)) {
    const mle::TiledGemvConfig c = mle::gemv_tiled_pick(M, rows, K, swi);
    return check_launch((ex.planning() ? hipSuccess : mle::launch_gemv_tiled_segs(c, x, s, M, K, ex.stream)),
                        "hip Q8_0 fused Linear launch failed");
  }
  if (!tiled && (swi ? M == 1 : pick_path(M, total_n, K) == 1)) {
    mle::GemvConfig c = mle::gemv_pick_config(M, total_n, K);
    if (swi) c.rpw = 0;  // the row-span kernel has no SwiGLU epilogue
    return check_launch((ex.planning() ? hipSuccess : mle::launch_gemv_segs(c, x, s, M, K, ex.stream)),
                        "hip Q8_0 fused Linear launch failed");
  }
  for (int m0 = 0; m0 < M; m0 += 16) {
    const int mc = M - m0 < 16 ? M - m0 : 16;
    const mle::DecodeMfmaConfig c = mle::decode_mfma_pick_segs(mc, s, K);
    if (!mle::decode_mfma_fits(c, mc, 1, K))
      return fail(MLE_UNSUPPORTED, std::string("hip ") + ctx + ": K too large for the MFMA decode");
    mle::LinearSegs chunk = s;
    for (int i = 0; i < s.count; ++i) {
      if (swi && i == 1) break;  // the up segment has no output of its own
      chunk.seg[i].y = s.seg[i].y + (int64_t)m0 * s.seg[i].N;
    }
    mle::SplitKWorkspace ws;
    std::unique_lock<std::mutex> hold;  // released after the launch is enqueued
    MLE_TRY(workspace_for(mle::decode_mfma_workspace_segs(c, chunk, K), ex, &ws, &hold));
    const hipError_t err =
        (ex.planning() ? hipSuccess : mle::launch_gemv_mfma_segs(c, x + (int64_t)m0 * K, chunk, mc, K, ws, ex.stream));
    if (err != hipSuccess) return check_launch(err, "hip Q8_0 fused Linear launch failed");
  }
  return ok();
}

}  // namespace

namespace {

int linear_swiglu(const float* x, const uint8_t* w_gate, const uint8_t* w_up, float* y, int M,
                  int N, int K, hipStream_t stream, mle::WeightLayout layout) {
  const bool tiled = layout == mle::WeightLayout::kTiled;
  const char* ctx = tiled ? "linear_swiglu_q8_0_tiled" : "linear_swiglu_q8_0";
  MLE_TRY(validate_linear(x, w_gate, nullptr, y, M, N, K));
  if (w_up == nullptr)
    return fail(MLE_INVALID_ARGUMENT, std::string("hip ") + ctx + ": up pointer must not be null");
  MLE_TRY(check_align(ctx, w_gate, tiled ? 16 : 2, "gate"));
  MLE_TRY(check_align(ctx, w_up, tiled ? 16 : 2, "up"));
  mle::LinearSegs s;
  s.layout = layout;
  s.mode = mle::Epilogue::kSwiGLU;
  s.count = 2;
  s.seg[0] = mle::LinearSeg{w_gate, nullptr, y, N};
  s.seg[1] = mle::LinearSeg{w_up, nullptr, y, N};
  return run_segs(ctx, x, s, M, K, Exec{stream});
}

int linear_multi(const float* x, int count, const uint8_t* const* w, const float* const* bias,
                 float* const* y, const int* N, int M, int K, hipStream_t stream,
                 mle::WeightLayout layout) {
  const bool tiled = layout == mle::WeightLayout::kTiled;
  const char* ctx = tiled ? "linear_multi_q8_0_tiled" : "linear_multi_q8_0";
  if (count < 1 || count > 3)
    return fail(MLE_INVALID_ARGUMENT, std::string("hip ") + ctx + ": count must be 1, 2 or 3");
  if (w == nullptr || y == nullptr || N == nullptr)
    return fail(MLE_INVALID_ARGUMENT,
                std::string("hip ") + ctx + ": weight, output and N arrays must not be null");
  mle::LinearSegs s;
  s.count = count;
  s.layout = layout;
  for (int i = 0; i < count; ++i) {
    const float* b = bias ? bias[i] : nullptr;
    MLE_TRY(validate_linear(x, w[i], b, y[i], M, N[i], K));
    if (tiled) MLE_TRY(check_align(ctx, w[i], 16, "B"));
    s.seg[i] = mle::LinearSeg{w[i], b, y[i], N[i]};
  }
  return run_segs(ctx, x, s, M, K, Exec{stream});
}

// Workspace of mle_q8_0_linear_noalloc: a file-scope device array (each GPU
// holds its own copy from module load until the process ends), bytes
// [0, kNoAllocBytes) for partial sums and scratch, then kNoAllocCounters tile
// counters.  Host code reaches it only through the address that
// hipGetSymbolAddress returns for the current device (the array's name in host
// code is a stand-in, not a device address).
constexpr size_t kNoAllocBytes = size_t(32) << 20;
constexpr size_t kNoAllocCounters = 65536;
__device__ __align__(256) uint8_t scratch[kNoAllocBytes + kNoAllocCounters * sizeof(uint32_t)];

struct NoAllocScratch {
  uint8_t* base = nullptr;  // device address of `scratch` on that device
};
std::mutex g_noalloc_mu;
std::map<int, NoAllocScratch> g_noalloc;  // device -> its scratch

// Device address of `scratch` on the current device; on the first call there,
// its counters are cleared on `stream` (a fill kernel, enqueued before the
// caller's launch).  Later launches leave the counters at zero.  That first
// call is refused while `stream` is capturing a graph: the clearing would
// become a node of the graph and the eager calls after it would find the
// counters uncleared.
int noalloc_scratch(hipStream_t stream, uint8_t** base) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return check_launch(err, "hip linear_noalloc");
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  auto it = g_noalloc.find(dev);
  if (it == g_noalloc.end()) {
    if (stream_capturing(stream))
      return fail(MLE_RUNTIME_ERROR,
                  "hip linear_noalloc: the first call on a device clears the scratch "
                  "counters and must not be captured; make one call outside capture first");
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr)
      return check_launch(err == hipSuccess ? hipErrorInvalidSymbol : err,
                          "hip linear_noalloc: scratch address");
    err = mle::launch_fill_u32(reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p) + kNoAllocBytes),
                               kNoAllocCounters, 0u, stream);
    if (err != hipSuccess) return check_launch(err, "hip linear_noalloc: clearing counters");
    it = g_noalloc.emplace(dev, NoAllocScratch{static_cast<uint8_t*>(p)}).first;
  }
  *base = it->second.base;
  return MLE_OK;
}

// MatMul from 64 rows of A on the bf16 MFMA GEMM (B[K, N] dequantised
// transposed into its W tile); below that, and where B's offsets would not fit
// 32 bits, the FP32 kernel of matmul.hip.  Fills the GEMM's tile choice and
// segment (B and C are set by the caller).
bool matmul_on_gemm(int M, int N, int K, mle::GemmConfig* c, mle::LinearSegs* s) {
  if (M < 64) return false;
  *s = mle::LinearSegs{};
  s->seg[0].N = N;
  s->layout = mle::WeightLayout::kKN;
  *c = mle::gemm_mfma_pick_kn(M, N, K);
  return mle::gemm_mfma_fits(*c, M, N, K) && mle::gemm_mfma_kn_fits(*s, K);
}

}  // namespace

extern "C" {

int mle_q8_0_abi_version(void) { return 7; }

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
  return run_linear(x, w_q8_0, bias, y, M, N, K, 0, Tune{}, Exec{stream});
}

namespace {

int linear_ex(const float* x, const uint8_t* w_q8_0, const float* bias, float* y, int M, int N,
              int K, int path, int t0, int t1, int t2, int t3, hipStream_t stream,
              mle::WeightLayout layout) {
  if (path < 0 || path > 3)
    return fail(MLE_INVALID_ARGUMENT,
                "hip sgemm_nt_q8_0_weight: path must be 0, 1, 2 or 3");
  Tune tune;
  const bool all_zero = t0 == 0 && t1 == 0 && t2 == 0 && t3 == 0;
  if (!all_zero) {
    if (path == 1) {
      tune.gemv = mle::GemvConfig{t0, t1, t2, t3};
      if (!mle::gemv_config_valid(tune.gemv))
        return fail(MLE_INVALID_ARGUMENT,
                    "hip sgemm_nt_q8_0_weight: invalid GEMV launch shape (mt " +
                        std::to_string(t0) + ", lpr " + std::to_string(t1) + ", rw " +
                        std::to_string(t2) + ", rpw " + std::to_string(t3) + ")");
    } else if (path == 3) {
      tune.dec = mle::DecodeMfmaConfig{t0, t1, t2};
      tune.dec.hyb = t3;
      if (t3 != 0 && t0 != 4 && t0 != 8)
        return fail(MLE_INVALID_ARGUMENT,
                    "hip sgemm_nt_q8_0_weight: a hybrid MFMA decode shape needs a token tile "
                    "of 4 or 8");
      if (t3 < 0 || t3 > 4 || !mle::decode_mfma_config_valid(tune.dec))
        return fail(MLE_INVALID_ARGUMENT,
                    "hip sgemm_nt_q8_0_weight: invalid MFMA decode shape (mt " +
                        std::to_string(t0) + ", waves " + std::to_string(t1) + ", kslice " +
                        std::to_string(t2) + ")");
    } else if (path == 2) {
      tune.gemm = mle::GemmConfig{t1, t2, t0};
      const mle::GemmConfig probe{t1 ? t1 : 128, t2 ? t2 : 64, t0 ? t0 : 1};
      if (t3 != 0 || !mle::gemm_mfma_config_valid(probe))
        return fail(MLE_INVALID_ARGUMENT,
                    "hip sgemm_nt_q8_0_weight: invalid MFMA GEMM shape (splits " +
                        std::to_string(t0) + ", bm " + std::to_string(t1) + ", bn " +
                        std::to_string(t2) + ")");
    } else {
      return fail(MLE_INVALID_ARGUMENT,
                  "hip sgemm_nt_q8_0_weight: a launch shape needs path 1, 2 or 3");
    }
  }
  return run_linear(x, w_q8_0, bias, y, M, N, K, path, tune, Exec{stream}, layout);
}

}  // namespace

int mle_q8_0_linear_ex(const float* x, const uint8_t* w_q8_0, const float* bias,
                       float* y, int M, int N, int K, int path, int t0, int t1, int t2,
                       int t3, hipStream_t stream) {
  MLE_TRY(validate_linear(x, w_q8_0, bias, y, M, N, K));
  return linear_ex(x, w_q8_0, bias, y, M, N, K, path, t0, t1, t2, t3, stream,
                   mle::WeightLayout::kRaw);
}

int mle_q8_0_linear_tiled_ex(const float* x, const uint8_t* w_tiled, const float* bias,
                             float* y, int M, int N, int K, int path, int t0, int t1, int t2,
                             int t3, hipStream_t stream) {
  MLE_TRY(validate_linear(x, w_tiled, bias, y, M, N, K));
  MLE_TRY(check_align("sgemm_nt_q8_0_tiled", w_tiled, 16, "B"));
  if (path == 1 || path == 2)
    return fail(MLE_INVALID_ARGUMENT,
                "hip sgemm_nt_q8_0_tiled: a forced path on tiled weights is 0 or 3");
  return linear_ex(x, w_tiled, bias, y, M, N, K, path, t0, t1, t2, t3, stream,
                   mle::WeightLayout::kTiled);
}


int mle_q8_0_linear_swiglu(const float* x, const uint8_t* w_gate, const uint8_t* w_up,
                           float* y, int M, int N, int K, hipStream_t stream) {
  return linear_swiglu(x, w_gate, w_up, y, M, N, K, stream, mle::WeightLayout::kRaw);
}

int mle_q8_0_linear_multi(const float* x, int count, const uint8_t* const* w,
                          const float* const* bias, float* const* y, const int* N, int M, int K,
                          hipStream_t stream) {
  return linear_multi(x, count, w, bias, y, N, M, K, stream, mle::WeightLayout::kRaw);
}

size_t mle_q8_0_tiled_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || K % 32 != 0) return 0;
  return mle::tiled_bytes(N, K);
}

int mle_q8_0_tile(const uint8_t* w_q8_0, uint8_t* w_tiled, int N, int K, hipStream_t stream) {
  const char* ctx = "tile_q8_0";
  MLE_TRY(check_ptrs(ctx, w_q8_0, "w_q8_0", w_tiled, "w_tiled", w_tiled, "w_tiled"));
  MLE_TRY(check_positive(ctx, N, "N"));
  MLE_TRY(check_positive(ctx, K, "K"));
  if (K % 32 != 0)
    return fail(MLE_UNSUPPORTED, std::string("hip ") + ctx + " requires K to be a multiple of 32");
  MLE_TRY(check_align(ctx, w_q8_0, 2, "w_q8_0"));
  MLE_TRY(check_align(ctx, w_tiled, 16, "w_tiled"));
  const uintptr_t r0 = (uintptr_t)w_q8_0, r1 = r0 + (uintptr_t)N * (K / 32) * 34;
  const uintptr_t t0 = (uintptr_t)w_tiled, t1 = t0 + mle::tiled_bytes(N, K);
  if (r0 < t1 && t0 < r1)
    return fail(MLE_INVALID_ARGUMENT,
                std::string("hip ") + ctx + ": w_q8_0 and w_tiled must not overlap");
  return check_launch(mle::launch_tile_q8_0(w_q8_0, w_tiled, N, K, stream),
                      "hip tile_q8_0 launch failed");
}

int mle_q8_0_linear_bias_bf16(const float* x, const uint8_t* w_q8_0, const uint16_t* bias_bf16,
                              float* y, int M, int N, int K, hipStream_t stream) {
  MLE_TRY(validate_linear(x, w_q8_0, bias_bf16, y, M, N, K, 2));
  return run_linear(x, w_q8_0, bias_bf16, y, M, N, K, 0, Tune{}, Exec{stream},
                    mle::WeightLayout::kRaw, true);
}

int mle_q8_0_linear_tiled_bias_bf16(const float* x, const uint8_t* w_tiled,
                                    const uint16_t* bias_bf16, float* y, int M, int N, int K,
                                    hipStream_t stream) {
  MLE_TRY(validate_linear(x, w_tiled, bias_bf16, y, M, N, K, 2));
  MLE_TRY(check_align("sgemm_nt_q8_0_tiled", w_tiled, 16, "B"));
  return run_linear(x, w_tiled, bias_bf16, y, M, N, K, 0, Tune{}, Exec{stream},
                    mle::WeightLayout::kTiled, true);
}

int mle_q8_0_linear_tiled(const float* x, const uint8_t* w_tiled, const float* bias, float* y,
                          int M, int N, int K, hipStream_t stream) {
  MLE_TRY(validate_linear(x, w_tiled, bias, y, M, N, K));
  MLE_TRY(check_align("sgemm_nt_q8_0_tiled", w_tiled, 16, "B"));
  return run_linear(x, w_tiled, bias, y, M, N, K, 0, Tune{}, Exec{stream},
                    mle::WeightLayout::kTiled);
}

int mle_q8_0_linear_swiglu_tiled(const float* x, const uint8_t* w_gate, const uint8_t* w_up,
                                 float* y, int M, int N, int K, hipStream_t stream) {
  return linear_swiglu(x, w_gate, w_up, y, M, N, K, stream, mle::WeightLayout::kTiled);
}

int mle_q8_0_linear_multi_tiled(const float* x, int count, const uint8_t* const* w,
                                const float* const* bias, float* const* y, const int* N, int M,
                                int K, hipStream_t stream) {
  return linear_multi(x, count, w, bias, y, N, M, K, stream, mle::WeightLayout::kTiled);
}

int mle_q8_0_linear_noalloc(const float* x, const uint8_t* w_q8_0, const float* bias,
                            float* y, int M, int N, int K, hipStream_t stream) {
  MLE_TRY(validate_linear(x, w_q8_0, bias, y, M, N, K));
  size_t bytes = 0, counters = 0;
  {
    Exec plan;
    plan.plan_bytes = &bytes;
    plan.plan_counters = &counters;
    MLE_TRY(run_linear(x, w_q8_0, bias, y, M, N, K, 0, Tune{}, plan));
  }
  if (bytes > kNoAllocBytes || counters > kNoAllocCounters)
    return fail(MLE_UNSUPPORTED,
                "hip linear_noalloc: this shape needs " + std::to_string(bytes) +
                    " bytes and " + std::to_string(counters) +
                    " counters of scratch; the no-allocation entry point holds " +
                    std::to_string(kNoAllocBytes) + " bytes and " +
                    std::to_string(kNoAllocCounters) + " counters (use mle_q8_0_linear)");
  Exec ex;
  ex.stream = stream;
  ex.fixed = true;  // launches needing no workspace get none
  if (bytes != 0 || counters != 0) {
    uint8_t* base = nullptr;
    MLE_TRY(noalloc_scratch(stream, &base));
    ex.fixed_buf = base;
    ex.fixed_bytes = kNoAllocBytes;
    ex.fixed_counters = reinterpret_cast<uint32_t*>(base + kNoAllocBytes);
    ex.fixed_counter_count = kNoAllocCounters;
  }
  return run_linear(x, w_q8_0, bias, y, M, N, K, 0, Tune{}, ex);
}

int mle_q8_0_workspace_size(int op, int M, int count, const int* N, int K, int tiled,
                            size_t* bytes, size_t* counters) {
  const char* ctx = "q8_0_workspace_size";
  if (bytes == nullptr || counters == nullptr || N == nullptr)
    return fail(MLE_INVALID_ARGUMENT,
                std::string("hip ") + ctx + ": N, bytes and counters must not be null");
  *bytes = 0;
  *counters = 0;
  MLE_TRY(check_positive(ctx, M, "M"));
  MLE_TRY(check_positive(ctx, K, "K"));
  if (K % 32 != 0)
    return fail(MLE_UNSUPPORTED, std::string("hip ") + ctx + " requires K to be a multiple of 32");
  const mle::WeightLayout layout = tiled ? mle::WeightLayout::kTiled : mle::WeightLayout::kRaw;
  Exec ex;
  ex.plan_bytes = bytes;
  ex.plan_counters = counters;
  mle::LinearSegs s;
  s.layout = layout;
  if (op == MLE_OP_LINEAR) {
    if (count != 1) return fail(MLE_INVALID_ARGUMENT, std::string("hip ") + ctx + ": a Linear has count 1");
    MLE_TRY(check_positive(ctx, N[0], "N"));
    return run_linear(nullptr, nullptr, nullptr, nullptr, M, N[0], K, 0, Tune{}, ex, layout);
  }
  if (op == MLE_OP_LINEAR_SWIGLU) {
    if (count != 2 || N[0] != N[1])
      return fail(MLE_INVALID_ARGUMENT,
                  std::string("hip ") + ctx + ": a gate/up pair has count 2 and equal N");
    MLE_TRY(check_positive(ctx, N[0], "N"));
    s.mode = mle::Epilogue::kSwiGLU;
    s.count = 2;
    s.seg[0].N = s.seg[1].N = N[0];
    return run_segs(ctx, nullptr, s, M, K, ex);
  }
  if (op == MLE_OP_LINEAR_MULTI) {
    if (count < 1 || count > 3)
      return fail(MLE_INVALID_ARGUMENT, std::string("hip ") + ctx + ": count must be 1, 2 or 3");
    s.count = count;
    for (int i = 0; i < count; ++i) {
      MLE_TRY(check_positive(ctx, N[i], "N"));
      s.seg[i].N = N[i];
    }
    return run_segs(ctx, nullptr, s, M, K, ex);
  }
  if (op == MLE_OP_MATMUL) {
    if (count != 1) return fail(MLE_INVALID_ARGUMENT, std::string("hip ") + ctx + ": a MatMul has count 1");
    MLE_TRY(check_positive(ctx, N[0], "N"));
    if (N[0] % 32 != 0)
      return fail(MLE_UNSUPPORTED, std::string("hip ") + ctx + " requires a MatMul's N to be a multiple of 32");
    mle::GemmConfig gc;
    mle::LinearSegs gs;
    if (matmul_on_gemm(M, N[0], K, &gc, &gs)) {
      const mle::SplitKNeed need = mle::gemm_mfma_workspace_segs(gc, M, gs, K);
      *bytes = need_bytes(need);
      *counters = need.counters;
      return ok();
    }
    const mle::MatmulNeed mm = mle::matmul_workspace(M, N[0], K);
    mle::SplitKNeed need;
    need.partial_floats = mm.partial_floats;
    need.counters = mm.counters;
    *bytes = need_bytes(need);
    *counters = need.counters;
    return ok();
  }
  return fail(MLE_INVALID_ARGUMENT, std::string("hip ") + ctx + ": unknown op " + std::to_string(op));
}

int mle_workspace_reserve(size_t bytes, size_t counters, hipStream_t stream) {
  if (bytes == 0 && counters == 0) return ok();
  std::lock_guard<std::mutex> lock(g_ws_mu);
  StreamWorkspace* e = nullptr;
  MLE_TRY(ensure_workspace(bytes, counters, stream, false, &e));
  MLE_TRY(ensure_workspace(bytes, counters, stream, true, &e));
  // A graph workspace that grew had its counters cleared by a kernel on
  // `stream`; a graph captured later may be replayed on another stream, which is
  // not ordered after that kernel, so wait for it here.
  const uint64_t gen = e->generation;
  if (gen != e->synced_generation) {
    const hipError_t err = hipStreamSynchronize(stream);
    if (err != hipSuccess) return check_launch(err, "hip workspace_reserve: synchronise");
    e->synced_generation = gen;
  }
  return ok();
}

int mle_workspace_info(hipStream_t stream, size_t* bytes, size_t* counters,
                       uint64_t* generation) {
  if (bytes == nullptr || counters == nullptr || generation == nullptr)
    return fail(MLE_INVALID_ARGUMENT, "hip workspace_info: output pointers must not be null");
  int dev = 0;
  const hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return check_launch(err, "hip workspace_info");
  std::lock_guard<std::mutex> lock(g_ws_mu);
  auto it = g_ws.find({dev, stream, false});
  *bytes = it == g_ws.end() ? 0 : it->second.buf_cap;
  *counters = it == g_ws.end() ? 0 : it->second.counter_cap;
  *generation = it == g_ws.end() ? 0 : it->second.generation;
  return ok();
}

int mle_workspace_plan_growth(size_t cap_bytes, size_t cap_counters, size_t need_bytes_,
                              size_t need_counters, size_t* new_bytes, size_t* new_counters) {
  if (new_bytes == nullptr || new_counters == nullptr) return -1;
  return plan_growth(cap_bytes, cap_counters, need_bytes_, need_counters, new_bytes,
                     new_counters)
             ? 1
             : 0;
}

int mle_swiglu_f32(const float* gate, const float* up, float* y, int64_t n,
                   hipStream_t stream) {
  const char* ctx = "swiglu_f32";
  MLE_TRY(check_ptrs(ctx, gate, "gate", up, "up", y, "output"));
  if (n < 0) return fail(MLE_INVALID_ARGUMENT, std::string("hip ") + ctx + ": n must be >= 0");
  MLE_TRY(check_align(ctx, gate, 4, "gate"));
  MLE_TRY(check_align(ctx, up, 4, "up"));
  MLE_TRY(check_align(ctx, y, 4, "output"));
  return check_launch(mle::launch_swiglu(gate, up, y, n, stream), "hip swiglu launch failed");
}

int mle_probe_stream_read(const void* src, int64_t bytes, uint32_t* sink, hipStream_t stream) {
  const char* ctx = "probe_stream_read";
  MLE_TRY(check_ptrs(ctx, src, "src", sink, "sink", sink, "sink"));
  if (bytes < 0 || bytes % 16 != 0)
    return fail(MLE_INVALID_ARGUMENT,
                std::string("hip ") + ctx + ": bytes must be a non-negative multiple of 16");
  MLE_TRY(check_align(ctx, src, 16, "src"));
  MLE_TRY(check_align(ctx, sink, 4, "sink"));
  return check_launch(mle::launch_stream_read(src, bytes, sink, stream),
                      "hip stream-read probe launch failed");
}

int mle_argmax_f32(const float* logits, int rows, int n, int32_t* idx, float* val,
                   hipStream_t stream) {
  const char* ctx = "argmax_f32";
  MLE_TRY(check_ptrs(ctx, logits, "logits", idx, "idx", idx, "idx"));
  MLE_TRY(check_positive(ctx, rows, "rows"));
  MLE_TRY(check_positive(ctx, n, "n"));
  if (rows > 65535)
    return fail(MLE_UNSUPPORTED, std::string("hip ") + ctx + ": at most 65535 rows per call");
  MLE_TRY(check_align(ctx, logits, 4, "logits"));
  MLE_TRY(check_align(ctx, idx, 4, "idx"));
  MLE_TRY(check_align(ctx, val, 4, "val"));
  mle::SplitKNeed need;
  need.partial_floats = (size_t)rows * mle::argmax_chunks(n) * 2;  // 64-bit keys
  mle::SplitKWorkspace ws;
  std::unique_lock<std::mutex> hold;  // released after the launch is enqueued
  MLE_TRY(get_workspace(need, stream, &ws, &hold));
  return check_launch(mle::launch_argmax(logits, rows, n, idx, val,
                                         reinterpret_cast<uint64_t*>(ws.partials), stream),
                      "hip argmax launch failed");
}

int mle_top_tokens_f32(const float* logits, int rows, int n, int top_n, float temperature,
                       int32_t* ids, float* probs, hipStream_t stream) {
  const char* ctx = "top_tokens_f32";
  MLE_TRY(check_ptrs(ctx, logits, "logits", ids, "ids", probs, "probs"));
  MLE_TRY(check_positive(ctx, rows, "rows"));
  MLE_TRY(check_positive(ctx, n, "n"));
  if (top_n <= 0) return ok();  // an empty list, as Sampler::get_top_tokens returns
  if (rows > 65535)
    return fail(MLE_UNSUPPORTED, std::string("hip ") + ctx + ": at most 65535 rows per call");
  if (top_n > mle::kTopTokensMax)
    return fail(MLE_UNSUPPORTED, std::string("hip ") + ctx + ": top_n must be at most " +
                                     std::to_string(mle::kTopTokensMax) + ", got " +
                                     std::to_string(top_n));
  const int kk = top_n < n ? top_n : n;
  if (n > mle::topk_max_n(kk))
    return fail(MLE_UNSUPPORTED, std::string("hip ") + ctx + ": n must be at most " +
                                     std::to_string(mle::topk_max_n(kk)) + " for top_n " +
                                     std::to_string(kk));
  MLE_TRY(check_align(ctx, logits, 4, "logits"));
  MLE_TRY(check_align(ctx, ids, 4, "ids"));
  MLE_TRY(check_align(ctx, probs, 4, "probs"));
  mle::SplitKNeed need;
  need.partial_floats = mle::top_tokens_workspace_floats(rows, n, top_n);
  mle::SplitKWorkspace ws;
  std::unique_lock<std::mutex> hold;  // released after the launch is enqueued
  MLE_TRY(get_workspace(need, stream, &ws, &hold));
  return check_launch(mle::launch_top_tokens(logits, rows, n, top_n, temperature, ids, probs,
                                             ws.partials, stream),
                      "hip top_tokens launch failed");
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
  if ((M + 7) / 8 > 65535)
    return fail(MLE_UNSUPPORTED, "hip sgemm Q8_0: at most 524280 rows of A per call");
  mle::GemmConfig gc;
  mle::LinearSegs gs;
  // The GEMM's X pre-pass reads A in 16-byte pieces (any hipMalloc'd A qualifies).
  if (((uintptr_t)a & 15u) == 0 && matmul_on_gemm(M, N, K, &gc, &gs)) {
    gs.seg[0].w = b_q8_0;
    gs.seg[0].y = c;
    mle::SplitKWorkspace ws;
    std::unique_lock<std::mutex> hold;  // released after the launch is enqueued
    MLE_TRY(get_workspace(mle::gemm_mfma_workspace_segs(gc, M, gs, K), stream, &ws, &hold));
    return check_launch(mle::launch_gemm_mfma_segs(gc, a, gs, M, K, ws, stream),
                        "hip sgemm Q8_0 launch failed");
  }
  const mle::MatmulNeed mm = mle::matmul_workspace(M, N, K);
  mle::SplitKNeed need;
  need.partial_floats = mm.partial_floats;
  need.counters = mm.counters;
  mle::SplitKWorkspace ws;
  std::unique_lock<std::mutex> hold;  // released after the launch is enqueued
  MLE_TRY(get_workspace(need, stream, &ws, &hold));
  return check_launch(
      mle::launch_matmul(a, b_q8_0, c, M, N, K, ws.partials, ws.counters, stream),
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

int mle_q8_0_embedding_tiled(const uint8_t* table_tiled, const int32_t* ids, float* out,
                             int seq_len, int vocab, int hidden, hipStream_t stream) {
  const char* ctx = "embedding_q8_0_tiled";
  MLE_TRY(check_ptrs(ctx, table_tiled, "weight", ids, "ids", out, "out"));
  if (seq_len < 0)
    return fail(MLE_INVALID_ARGUMENT,
                std::string("hip ") + ctx + ": seq_len must not be negative");
  MLE_TRY(check_positive(ctx, vocab, "vocab_size"));
  MLE_TRY(check_positive(ctx, hidden, "hidden"));
  if (hidden % 32 != 0)
    return fail(MLE_UNSUPPORTED,
                "hip embedding Q8_0 requires hidden to be a multiple of 32");
  MLE_TRY(check_align(ctx, table_tiled, 16, "weight"));
  MLE_TRY(check_align(ctx, ids, 4, "ids"));
  MLE_TRY(check_align(ctx, out, 16, "out"));
  if (seq_len == 0) return ok();
  return check_launch(
      mle::launch_embedding_tiled(table_tiled, ids, out, seq_len, vocab, hidden, stream),
      "hip embedding Q8_0 tiled launch failed");
}

int mle_q8_0_dequantize(const uint8_t* src_q8_0, float* dst, int64_t n, hipStream_t stream) {
  const char* ctx = "dequantize_q8_0";
  MLE_TRY(check_ptrs(ctx, src_q8_0, "src", dst, "dst", dst, "dst"));
  if (n < 0) return fail(MLE_INVALID_ARGUMENT, std::string("hip ") + ctx + ": n must not be negative");
  MLE_TRY(check_align(ctx, src_q8_0, 2, "src"));
  MLE_TRY(check_align(ctx, dst, 16, "dst"));
  return check_launch(mle::launch_dequantize_q8_0(src_q8_0, dst, n, stream),
                      "hip dequantize_q8_0 launch failed");
}

int mle_q8_0_f16_decode(const uint16_t* bits, float* out, int64_t n, hipStream_t stream) {
  if (bits == nullptr || out == nullptr)
    return fail(MLE_INVALID_ARGUMENT, "hip f16_decode: pointers must not be null");
  if (n < 0) return fail(MLE_INVALID_ARGUMENT, "hip f16_decode: n must not be negative");
  return check_launch(mle::launch_f16_decode(bits, out, n, stream),
                      "hip f16_decode launch failed");
}

}  // extern "C"
