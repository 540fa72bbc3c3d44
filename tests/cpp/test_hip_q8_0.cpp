// test_hip_q8_0.cpp -- the HIP backend end to end on an MI355X.
//
// Mirrors the reference's device tests of the Q8_0 path with the HIP names:
//   tests/test_cuda_kernels.cpp:409-529   low-level sgemm_nt / sgemm / embedding
//   tests/test_cuda_kernels.cpp:953-1061  executor Linear + MatMul on Q8_0 weights
//   tests/test_cuda_kernels.cpp:1063-1123 rejects K % 32 != 0 and short storage
//   tests/test_runtime.cpp:561-626        Linear with bias through the executor
// plus embedding through the executor (device semantics for bad ids), a
// caller-owned stream, a prefill-sized Linear (bf16 MFMA path), and a synthetic
// GGUF model loaded by the weight loader's HIP branch (raw Q8_0 host-to-device
// copy, reference src/io/gguf_weight_loader.cpp:100-117, 526-541) and run end
// to end: Embedding -> Linear -> Linear -> tied lm_head Linear.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gguf_writer.h"
#include "mle_q8_0.h"
#include "minillm_hip/io.h"
#include "minillm_hip/runtime.h"

using namespace minillm;

#define CHECK(cond)                                                              \
  do {                                                                           \
    if (!(cond)) {                                                               \
      std::fprintf(stderr, "CHECK failed at %s:%d: %s\n", __FILE__, __LINE__, #cond); \
      std::abort();                                                              \
    }                                                                            \
  } while (0)

static void check_hip(hipError_t e) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "HIP error: %s\n", hipGetErrorString(e));
    std::abort();
  }
}

static Status from_hip(int rc) {
  return rc == 0 ? Status::make_ok() : Status::runtime_error(mle_last_error());
}

static void check_status(const Status& st) {
  if (!st.ok()) {
    std::fprintf(stderr, "%s\n", st.to_string().c_str());
    std::abort();
  }
}

static void near(float got, float want, float tol) {
  if (!(std::fabs(got - want) <= tol)) {
    std::fprintf(stderr, "got %.9g want %.9g (tol %g)\n", got, want, tol);
    std::abort();
  }
}

// Packs int8 values into Q8_0 blocks with one fp16 scale (reference test helper
// semantics, tests/test_cuda_kernels.cpp:51-65).
static std::vector<uint8_t> pack_q8_0(const std::vector<int8_t>& v, uint16_t scale_bits) {
  const size_t blocks = (v.size() + 31) / 32;
  std::vector<uint8_t> out(blocks * 34, 0);
  for (size_t b = 0; b < blocks; ++b) {
    out[b * 34] = static_cast<uint8_t>(scale_bits & 0xff);
    out[b * 34 + 1] = static_cast<uint8_t>(scale_bits >> 8);
    for (size_t i = 0; i < 32 && b * 32 + i < v.size(); ++i)
      out[b * 34 + 2 + i] = static_cast<uint8_t>(v[b * 32 + i]);
  }
  return out;
}

template <typename T>
struct DevBuf {
  T* p = nullptr;
  size_t n = 0;
  explicit DevBuf(size_t count) : n(count) { check_hip(hipMalloc(&p, n * sizeof(T) + 1)); }
  ~DevBuf() { (void)hipFree(p); }
  void put(const std::vector<T>& h) { check_hip(hipMemcpy(p, h.data(), n * sizeof(T), hipMemcpyHostToDevice)); }
  std::vector<T> get() const {
    std::vector<T> h(n);
    check_hip(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
  }
};

static void upload(Tensor& t, const void* host, size_t bytes) {
  check_hip(hipMemcpy(t.data(), host, bytes, hipMemcpyHostToDevice));
}

static std::vector<float> download(const Tensor* t, size_t count) {
  std::vector<float> h(count);
  check_hip(hipMemcpy(h.data(), t->data(), count * 4, hipMemcpyDeviceToHost));
  return h;
}

static void test_low_level_kernels() {
  {  // Linear M=1 N=2 K=32, scale 1.0
    const int M = 1, N = 2, K = 32;
    std::vector<float> A(M * K);
    std::vector<int8_t> B(N * K);
    for (int i = 0; i < M * K; ++i) A[i] = float((i % 7) - 3) * 0.25f;
    for (int i = 0; i < N * K; ++i) B[i] = int8_t((i * 5) % 17 - 8);
    auto packed = pack_q8_0(B, 0x3c00);
    DevBuf<float> dA(A.size()), dC(M * N);
    DevBuf<uint8_t> dB(packed.size());
    dA.put(A);
    dB.put(packed);
    check_status(hip::sgemm_nt(dA.p, dB.p, dC.p, M, N, K));
    check_hip(hipDeviceSynchronize());
    auto C = dC.get();
    for (int n = 0; n < N; ++n) {
      float e = 0.f;
      for (int k = 0; k < K; ++k) e += A[k] * float(B[n * K + k]);
      near(C[n], e, 1e-5f);
    }
  }
  {  // Linear M=2 N=3 K=64, scale 0.5
    const int M = 2, N = 3, K = 64;
    std::vector<float> A(M * K);
    std::vector<int8_t> B(N * K);
    for (int i = 0; i < M * K; ++i) A[i] = float((i % 11) - 5) * 0.125f;
    for (int i = 0; i < N * K; ++i) B[i] = int8_t((i * 7) % 23 - 11);
    auto packed = pack_q8_0(B, 0x3800);
    DevBuf<float> dA(A.size()), dC(M * N);
    DevBuf<uint8_t> dB(packed.size());
    dA.put(A);
    dB.put(packed);
    check_status(hip::sgemm_nt(dA.p, dB.p, dC.p, M, N, K));
    check_hip(hipDeviceSynchronize());
    auto C = dC.get();
    for (int m = 0; m < M; ++m)
      for (int n = 0; n < N; ++n) {
        float e = 0.f;
        for (int k = 0; k < K; ++k) e += A[m * K + k] * float(B[n * K + k]) * 0.5f;
        near(C[m * N + n], e, 1e-4f);
      }
  }
  {  // MatMul M=2 N=64 K=32, scale 0.5 (blocks along N)
    const int M = 2, N = 64, K = 32;
    std::vector<float> A(M * K);
    std::vector<int8_t> B(K * N);
    for (int i = 0; i < M * K; ++i) A[i] = float((i % 13) - 6) * 0.125f;
    for (int i = 0; i < K * N; ++i) B[i] = int8_t((i * 3) % 29 - 14);
    auto packed = pack_q8_0(B, 0x3800);
    DevBuf<float> dA(A.size()), dC(M * N);
    DevBuf<uint8_t> dB(packed.size());
    dA.put(A);
    dB.put(packed);
    check_status(hip::sgemm(dA.p, dB.p, dC.p, M, N, K));
    check_hip(hipDeviceSynchronize());
    auto C = dC.get();
    for (int m = 0; m < M; ++m)
      for (int n = 0; n < N; ++n) {
        float e = 0.f;
        for (int k = 0; k < K; ++k) e += A[m * K + k] * float(B[k * N + n]) * 0.5f;
        near(C[m * N + n], e, 1e-4f);
      }
  }
  {  // Embedding vocab 3, hidden 64, ids {2, 0, 1}, scale 0.5
    const int vocab = 3, hidden = 64;
    std::vector<int8_t> W(vocab * hidden);
    for (int i = 0; i < vocab * hidden; ++i) W[i] = int8_t((i * 5) % 31 - 15);
    auto packed = pack_q8_0(W, 0x3800);
    const std::vector<int> ids{2, 0, 1};
    DevBuf<uint8_t> dW(packed.size());
    DevBuf<int> dids(ids.size());
    DevBuf<float> dout(ids.size() * hidden);
    dW.put(packed);
    dids.put(ids);
    check_status(hip::embedding(dW.p, dids.p, dout.p, int(ids.size()), vocab, hidden));
    check_hip(hipDeviceSynchronize());
    auto out = dout.get();
    for (size_t s = 0; s < ids.size(); ++s)
      for (int h = 0; h < hidden; ++h)
        CHECK(out[s * hidden + h] == float(W[ids[s] * hidden + h]) * 0.5f);  // exact
  }
  {  // low-level error path: K not a multiple of 32
    const Status st = hip::sgemm_nt(reinterpret_cast<const float*>(16),
                                    reinterpret_cast<const uint8_t*>(16),
                                    reinterpret_cast<float*>(16), 1, 2, 31);
    CHECK(st.code() == ErrorCode::Unsupported);
    CHECK(std::string(st.message()).find("multiple of 32") != std::string::npos);
  }
  std::printf("  PASS test_low_level_kernels\n");
}

static void test_executor_linear_and_matmul() {
  KernelRegistry registry;
  register_hip_kernels(registry);
  {
    Graph graph;
    GraphBuilder gb(graph);
    auto x = gb.input("x", Shape({2, 32}), DType::Float32, Device::hip(0));
    auto w = gb.constant("w", Shape({3, 32}), DType::Float32, Device::hip(0));
    auto y = gb.linear(*x, *w, std::nullopt, "linear_q8");
    CHECK(x && w && y && gb.output(*y, "out"));
    Tensor tx("x", Shape({2, 32}), DType::Float32, Device::hip(0));
    Tensor tw("w", Shape({3, 32}), DType::Q8_0, Device::hip(0));
    check_status(tx.allocate_hip());
    std::vector<float> hx(64);
    for (int i = 0; i < 64; ++i) hx[i] = float((i % 11) - 5) * 0.125f;
    std::vector<int8_t> hw(96);
    for (int i = 0; i < 96; ++i) hw[i] = int8_t((i * 7) % 19 - 9);
    auto packed = pack_q8_0(hw, 0x3c00);
    check_status(tw.allocate_hip_bytes(packed.size()));
    upload(tx, hx.data(), hx.size() * 4);
    upload(tw, packed.data(), packed.size());
    RuntimeContext ctx;
    check_status(ctx.bind(*x, &tx));
    check_status(ctx.bind(*w, &tw));
    check_status(ctx.allocate_intermediates(graph));
    HipExecutor ex(std::make_shared<HipBackend>(), registry);
    check_status(ex.compile(graph));
    check_status(ex.run(ctx));
    check_hip(hipDeviceSynchronize());
    Tensor* yt = ctx.get(*y);
    CHECK(yt && yt->device().type == DeviceType::HIP && yt->dtype() == DType::Float32);
    auto got = download(yt, 6);
    for (int m = 0; m < 2; ++m)
      for (int n = 0; n < 3; ++n) {
        float e = 0.f;
        for (int k = 0; k < 32; ++k) e += hx[m * 32 + k] * float(hw[n * 32 + k]);
        near(got[m * 3 + n], e, 1e-4f);
      }
  }
  {
    Graph graph;
    GraphBuilder gb(graph);
    auto a = gb.input("a", Shape({2, 32}), DType::Float32, Device::hip(0));
    auto b = gb.constant("b", Shape({32, 32}), DType::Float32, Device::hip(0));
    auto y = gb.matmul(*a, *b, "matmul_q8");
    CHECK(a && b && y);
    Tensor ta("a", Shape({2, 32}), DType::Float32, Device::hip(0));
    Tensor tb("b", Shape({32, 32}), DType::Q8_0, Device::hip(0));
    check_status(ta.allocate_hip());
    std::vector<float> ha(64);
    for (int i = 0; i < 64; ++i) ha[i] = float((i % 13) - 6) * 0.125f;
    std::vector<int8_t> hb(1024);
    for (int i = 0; i < 1024; ++i) hb[i] = int8_t((i * 5) % 17 - 8);
    auto packed = pack_q8_0(hb, 0x3c00);
    check_status(tb.allocate_hip_bytes(packed.size()));
    upload(ta, ha.data(), ha.size() * 4);
    upload(tb, packed.data(), packed.size());
    RuntimeContext ctx;
    check_status(ctx.bind(*a, &ta));
    check_status(ctx.bind(*b, &tb));
    check_status(ctx.allocate_intermediates(graph));
    HipExecutor ex(std::make_shared<HipBackend>(), registry);
    check_status(ex.compile(graph));
    check_status(ex.run(ctx));
    check_hip(hipDeviceSynchronize());
    auto got = download(ctx.get(*y), 64);
    for (int m = 0; m < 2; ++m)
      for (int n = 0; n < 32; ++n) {
        float e = 0.f;
        for (int k = 0; k < 32; ++k) e += ha[m * 32 + k] * float(hb[k * 32 + n]);
        CHECK(got[m * 32 + n] == e);  // exact: integer quants x dyadic activations
      }
  }
  std::printf("  PASS test_executor_linear_and_matmul\n");
}

static void test_executor_linear_bias_rank3() {
  // x [1,2,32], w [3,32] Q8_0 scale 1, bias [3]  (tests/test_runtime.cpp:561-626)
  Graph g;
  GraphBuilder gb(g);
  auto x = gb.input("x", Shape({1, 2, 32}), DType::Float32, Device::hip(0));
  auto w = gb.constant("w", Shape({3, 32}), DType::Float32, Device::hip(0));
  auto b = gb.constant("b", Shape({3}), DType::Float32, Device::hip(0));
  auto y = gb.linear(*x, *w, *b, "linear_q8");
  CHECK(y && gb.output(*y, "out"));
  Tensor tx("x", Shape({1, 2, 32}), DType::Float32, Device::hip(0));
  Tensor tw("w", Shape({3, 32}), DType::Q8_0, Device::hip(0));
  Tensor tb("b", Shape({3}), DType::Float32, Device::hip(0));
  check_status(tx.allocate_hip());
  check_status(tb.allocate_hip());
  std::vector<float> hx(64), hb{0.5f, -1.0f, 1.5f};
  for (int i = 0; i < 64; ++i) hx[i] = float((i % 11) - 5) * 0.125f;
  std::vector<int8_t> hw(96);
  for (int i = 0; i < 96; ++i) hw[i] = int8_t((i * 7) % 19 - 9);
  auto packed = pack_q8_0(hw, 0x3c00);
  check_status(tw.allocate_hip_bytes(packed.size()));
  upload(tx, hx.data(), 256);
  upload(tb, hb.data(), 12);
  upload(tw, packed.data(), packed.size());
  RuntimeContext ctx;
  check_status(ctx.bind(*x, &tx));
  check_status(ctx.bind(*w, &tw));
  check_status(ctx.bind(*b, &tb));
  check_status(ctx.allocate_intermediates(g));
  KernelRegistry reg;
  register_hip_kernels(reg);
  HipExecutor ex(std::make_shared<HipBackend>(), reg);
  check_status(ex.compile(g));
  check_status(ex.run(ctx));
  check_hip(hipDeviceSynchronize());
  CHECK(ctx.get(*y)->shape() == Shape({1, 2, 3}));
  auto got = download(ctx.get(*y), 6);
  for (int t = 0; t < 2; ++t)
    for (int o = 0; o < 3; ++o) {
      float e = hb[o];
      for (int k = 0; k < 32; ++k) e += hx[t * 32 + k] * float(hw[o * 32 + k]);
      near(got[t * 3 + o], e, 1e-5f);
    }
  std::printf("  PASS test_executor_linear_bias_rank3\n");
}

static void test_executor_embedding_and_stream() {
  // ids [2,3] (rank 2) -> out [2,3,64]; id 7 is outside vocab 5 -> zero row.
  hipStream_t stream;
  check_hip(hipStreamCreate(&stream));
  Graph g;
  GraphBuilder gb(g);
  auto ids = gb.input("ids", Shape({2, 3}), DType::Int32, Device::hip(0));
  auto w = gb.constant("emb", Shape({5, 64}), DType::Float32, Device::hip(0));
  auto y = gb.embedding(*ids, *w, "embed");
  CHECK(y && gb.output(*y, "out"));
  Tensor tids("ids", Shape({2, 3}), DType::Int32, Device::hip(0));
  Tensor tw("emb", Shape({5, 64}), DType::Q8_0, Device::hip(0));
  check_status(tids.allocate_hip());
  check_status(tw.allocate_hip());
  CHECK(tw.allocated_bytes() == q8_0_bytes(320));
  std::vector<int8_t> hw(320);
  for (int i = 0; i < 320; ++i) hw[i] = int8_t((i * 13) % 255 - 127);
  auto packed = pack_q8_0(hw, 0x1401);  // a non-trivial scale (~0.00101)
  std::vector<int> hids{4, 0, 7, 2, 2, 1};
  upload(tids, hids.data(), 24);
  upload(tw, packed.data(), packed.size());
  RuntimeContext ctx;
  check_status(ctx.bind(*ids, &tids));
  check_status(ctx.bind(*w, &tw));
  check_status(ctx.allocate_intermediates(g));
  KernelRegistry reg;
  register_hip_kernels(reg);
  HipExecutor ex(std::make_shared<HipBackend>(), reg, stream);
  CHECK(ex.stream() == stream);
  check_status(ex.compile(g));
  check_status(ex.run(ctx));
  check_hip(hipStreamSynchronize(stream));
  CHECK(ctx.get(*y)->shape() == Shape({2, 3, 64}));
  auto got = download(ctx.get(*y), 6 * 64);
  const float d = std::ldexp(1025.0f, -20);  // fp16 0x1401 = (1 + 1/1024) * 2^-10
  for (int s = 0; s < 6; ++s)
    for (int h = 0; h < 64; ++h) {
      const float want = (hids[s] < 0 || hids[s] >= 5) ? 0.0f : d * float(hw[hids[s] * 64 + h]);
      CHECK(got[s * 64 + h] == want);
    }
  check_hip(hipStreamDestroy(stream));
  std::printf("  PASS test_executor_embedding_and_stream\n");
}

static void test_executor_rejects_invalid_inputs() {
  KernelRegistry reg;
  register_hip_kernels(reg);
  {  // K = 31
    Graph g;
    GraphBuilder gb(g);
    auto x = gb.input("x", Shape({1, 31}), DType::Float32, Device::hip(0));
    auto w = gb.constant("w", Shape({2, 31}), DType::Float32, Device::hip(0));
    auto y = gb.linear(*x, *w, std::nullopt, "linear_q8_bad_k");
    CHECK(y);
    Tensor tx("x", Shape({1, 31}), DType::Float32, Device::hip(0));
    Tensor tw("w", Shape({2, 31}), DType::Q8_0, Device::hip(0));
    check_status(tx.allocate_hip());
    check_status(tw.allocate_hip_bytes(q8_0_bytes(62)));
    RuntimeContext ctx;
    check_status(ctx.bind(*x, &tx));
    check_status(ctx.bind(*w, &tw));
    check_status(ctx.allocate_intermediates(g));
    HipExecutor ex(std::make_shared<HipBackend>(), reg);
    check_status(ex.compile(g));
    const Status st = ex.run(ctx);
    CHECK(!st.ok() && std::string(st.message()).find("Q8_0") != std::string::npos);
  }
  {  // raw storage too small
    Graph g;
    GraphBuilder gb(g);
    auto x = gb.input("x", Shape({1, 32}), DType::Float32, Device::hip(0));
    auto w = gb.constant("w", Shape({1, 32}), DType::Float32, Device::hip(0));
    auto y = gb.linear(*x, *w, std::nullopt, "linear_q8_short_storage");
    CHECK(y);
    Tensor tx("x", Shape({1, 32}), DType::Float32, Device::hip(0));
    Tensor tw("w", Shape({1, 32}), DType::Q8_0, Device::hip(0));
    check_status(tx.allocate_hip());
    check_status(tw.allocate_hip_bytes(1));
    RuntimeContext ctx;
    check_status(ctx.bind(*x, &tx));
    check_status(ctx.bind(*w, &tw));
    check_status(ctx.allocate_intermediates(g));
    HipExecutor ex(std::make_shared<HipBackend>(), reg);
    check_status(ex.compile(g));
    const Status st = ex.run(ctx);
    CHECK(!st.ok() && std::string(st.message()).find("too small") != std::string::npos);
  }
  std::printf("  PASS test_executor_rejects_invalid_inputs\n");
}

static void test_executor_prefill_linear() {
  // x [2,64,256] -> M = 128 tokens: the bf16 MFMA path; checked in FP64.
  const int M = 128, N = 160, K = 256;
  Graph g;
  GraphBuilder gb(g);
  auto x = gb.input("x", Shape({2, 64, K}), DType::Float32, Device::hip(0));
  auto w = gb.constant("w", Shape({N, K}), DType::Float32, Device::hip(0));
  auto y = gb.linear(*x, *w, std::nullopt, "prefill");
  CHECK(y);
  std::vector<float> hx(size_t(M) * K);
  uint32_t s = 12345;
  auto rnd = [&]() { s = s * 1664525u + 1013904223u; return s; };
  for (auto& v : hx) v = float(int(rnd() >> 16) % 2001 - 1000) / 500.0f;
  std::vector<int8_t> hq(size_t(N) * K);
  for (auto& q : hq) q = int8_t(int(rnd() >> 20) % 255 - 127);
  auto packed = pack_q8_0(hq, 0x2200);  // scale 2^-7 * 1.5
  Tensor tx("x", Shape({2, 64, K}), DType::Float32, Device::hip(0));
  Tensor tw("w", Shape({N, K}), DType::Q8_0, Device::hip(0));
  check_status(tx.allocate_hip());
  check_status(tw.allocate_hip());
  upload(tx, hx.data(), hx.size() * 4);
  upload(tw, packed.data(), packed.size());
  RuntimeContext ctx;
  check_status(ctx.bind(*x, &tx));
  check_status(ctx.bind(*w, &tw));
  check_status(ctx.allocate_intermediates(g));
  KernelRegistry reg;
  register_hip_kernels(reg);
  HipExecutor ex(std::make_shared<HipBackend>(), reg);
  check_status(ex.compile(g));
  check_status(ex.run(ctx));
  check_hip(hipDeviceSynchronize());
  auto got = download(ctx.get(*y), size_t(M) * N);
  const double d = 1.5 / 128.0;
  double num = 0, den = 0;
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      double e = 0;
      for (int k = 0; k < K; ++k) e += double(hx[size_t(m) * K + k]) * d * hq[size_t(n) * K + k];
      num += (got[size_t(m) * N + n] - e) * (got[size_t(m) * N + n] - e);
      den += e * e;
    }
  const double rel = std::sqrt(num / den);
  std::printf("    prefill rel_l2 = %.3e\n", rel);
  CHECK(rel <= 1e-2);
  std::printf("  PASS test_executor_prefill_linear\n");
}

// Seeded Q8_0 blocks: q uniform in [-127, 127], scale |z| * 0.02 / 127 rounded
// to binary16 (the benchmark's weight distribution, here from a small LCG).
static std::vector<uint8_t> synth_q8(size_t rows, size_t cols, uint32_t seed) {
  std::vector<uint8_t> out(rows * (cols / 32) * 34);
  uint32_t s = seed;
  auto next = [&]() { s = s * 1664525u + 1013904223u; return s; };
  for (size_t b = 0; b < out.size() / 34; ++b) {
    const float d = float((next() >> 8) % 1000 + 1) * 1e-3f * 0.02f / 127.0f;
    const _Float16 hd = static_cast<_Float16>(d);  // round to nearest even
    uint16_t h;
    std::memcpy(&h, &hd, 2);
    out[b * 34] = uint8_t(h & 0xff);
    out[b * 34 + 1] = uint8_t(h >> 8);
    for (int i = 0; i < 32; ++i) out[b * 34 + 2 + i] = uint8_t(int8_t(int(next() >> 24) % 255 - 127));
  }
  return out;
}

static float host_half(uint16_t h) {
  const int e = (h >> 10) & 0x1f, m = h & 0x3ff;
  const float mag = e == 0 ? float(m) * 0x1p-24f : std::ldexp(float(m | 0x400), e - 25);
  return (h & 0x8000) ? -mag : mag;
}

// Element (row, col) of a row-major Q8_0 matrix with `cols` columns: d * q.
static float q8_at(const std::vector<uint8_t>& w, size_t cols, size_t row, size_t col) {
  const uint8_t* blk = w.data() + (row * (cols / 32) + col / 32) * 34;
  return float(int8_t(blk[2 + col % 32])) * host_half(uint16_t(blk[0] | (blk[1] << 8)));
}

// y = x . W^T in double from the same fp32 inputs; relative L2 of `got` against it.
static double linear_rel_l2(const std::vector<float>& x, const std::vector<uint8_t>& w,
                            const std::vector<float>& got, int M, int N, int K) {
  double num = 0, den = 0;
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      double acc = 0;
      for (int k = 0; k < K; ++k) acc += double(x[size_t(m) * K + k]) * q8_at(w, K, n, k);
      const double e = double(got[size_t(m) * N + n]) - acc;
      num += e * e;
      den += acc * acc;
    }
  return std::sqrt(num / den);
}

static void test_gguf_model_end_to_end() {
  const int V = 320, H = 128, I = 256;
  const auto embd = synth_q8(V, H, 11), up = synth_q8(I, H, 12), down = synth_q8(H, I, 13);
  GgufWriter w;
  w.kv_str("general.architecture", "llama");
  w.kv_u32("llama.embedding_length", H);
  w.tensor("token_embd.weight", {V, H}, 8, embd);
  w.tensor("blk.0.ffn_up.weight", {I, H}, 8, up);
  w.tensor("blk.0.ffn_down.weight", {H, I}, 8, down);  // no output.weight: lm_head is tied
  const std::string path = w.write("mle_e2e");

  KernelRegistry registry;
  register_hip_kernels(registry);
  for (int T : {5, 70}) {  // MFMA decode path (FP32-exact) and the bf16 MFMA GEMM path
    Graph g;
    GraphBuilder gb(g);
    const Device dev = Device::hip(0);
    auto ids = gb.input("input_ids", Shape({1, T}), DType::Int32, dev);
    auto tok = gb.constant("tok_embeddings.weight", Shape({V, H}), DType::Float32, dev);
    auto wup = gb.constant("layer_0.up_proj.weight", Shape({I, H}), DType::Float32, dev);
    auto wdn = gb.constant("layer_0.down_proj.weight", Shape({H, I}), DType::Float32, dev);
    auto lm = gb.constant("lm_head.weight", Shape({V, H}), DType::Float32, dev);
    CHECK(ids && tok && wup && wdn && lm);
    auto x = gb.embedding(*ids, *tok, "embed");
    CHECK(x);
    auto h = gb.linear(*x, *wup, std::nullopt, "up");
    CHECK(h);
    auto o = gb.linear(*h, *wdn, std::nullopt, "down");
    CHECK(o);
    auto logits = gb.linear(*o, *lm, std::nullopt, "lm_head");
    CHECK(logits && gb.output(*logits, "logits"));

    WeightLoader loader(path);
    auto file = loader.open();
    CHECK(file);
    auto store = loader.load_shared_weights(*file, g);
    CHECK(store);
    CHECK(store->tensor_count() == 3 && store->alias_count() == 4);
    // Raw Q8_0 bytes on the device, unchanged; the tied lm_head shares the table.
    const std::pair<const char*, const std::vector<uint8_t>*> raw[] = {
        {"tok_embeddings.weight", &embd}, {"layer_0.up_proj.weight", &up},
        {"layer_0.down_proj.weight", &down}};
    for (const auto& [name, bytes] : raw) {
      Tensor* t = store->get(name);
      CHECK(t && t->device().type == DeviceType::HIP && t->dtype() == DType::Q8_0);
      CHECK(t->allocated_bytes() == bytes->size());
      std::vector<uint8_t> back(bytes->size());
      check_hip(hipMemcpy(back.data(), t->data(), back.size(), hipMemcpyDeviceToHost));
      CHECK(back == *bytes);
    }
    CHECK(store->get("lm_head.weight") == store->get("tok_embeddings.weight"));

    std::vector<int32_t> hid(T);
    for (int i = 0; i < T; ++i) hid[i] = (i * 37 + 5) % V;
    Tensor tids("input_ids", Shape({1, T}), DType::Int32, dev);
    check_status(tids.allocate_hip());
    upload(tids, hid.data(), hid.size() * 4);
    RuntimeContext ctx;
    check_status(ctx.bind(*ids, &tids));
    check_status(store->bind(g, ctx));
    check_status(ctx.allocate_intermediates(g));
    HipExecutor ex(std::make_shared<HipBackend>(), registry);
    check_status(ex.compile(g));
    check_status(ex.run(ctx));
    check_hip(hipDeviceSynchronize());

    // Each stage against a double-precision reference fed with the GPU's own
    // input to that stage: the embedding bit for bit, the Linears within the
    // per-path bound (1e-5 FP32-exact decode for M < 64, 1e-2 bf16 GEMM otherwise).
    const auto ex_ = download(ctx.get(*x), size_t(T) * H);
    for (int t = 0; t < T; ++t)
      for (int c = 0; c < H; ++c) {
        const float want = q8_at(embd, H, hid[t], c);
        CHECK(std::memcmp(&ex_[size_t(t) * H + c], &want, 4) == 0);
      }
    const double tol = T < 64 ? 1e-5 : 1e-2;
    const auto eh = download(ctx.get(*h), size_t(T) * I);
    const auto eo = download(ctx.get(*o), size_t(T) * H);
    const auto el = download(ctx.get(*logits), size_t(T) * V);
    const double e1 = linear_rel_l2(ex_, up, eh, T, I, H);
    const double e2 = linear_rel_l2(eh, down, eo, T, H, I);
    const double e3 = linear_rel_l2(eo, embd, el, T, V, H);
    std::printf("    T=%d rel L2: up %.2e down %.2e lm_head %.2e (bound %.0e)\n", T, e1, e2, e3, tol);
    CHECK(e1 <= tol && e2 <= tol && e3 <= tol);

    // The loader's Linear-only tensors re-tiled in place, the tied table tiled
    // by copy (its raw bytes stay for the gather): same bits from every stage.
    check_status(ex.tile_weights(ctx, true));
    CHECK(ex.tiled_in_place() == 2u && ex.tiled_weights() == 1u);
    CHECK(store->get("layer_0.up_proj.weight")->storage_layout() == StorageLayout::Q8_0Tiled);
    CHECK(store->get("layer_0.up_proj.weight")->allocated_bytes() ==
          hip::q8_0_tiled_bytes(I, H));
    CHECK(store->get("lm_head.weight")->storage_layout() == StorageLayout::Raw);
    check_status(ex.run(ctx));
    check_hip(hipDeviceSynchronize());
    const std::vector<float>* before[4] = {&ex_, &eh, &eo, &el};
    const ValueId vals[4] = {*x, *h, *o, *logits};
    const size_t cnt[4] = {size_t(T) * H, size_t(T) * I, size_t(T) * H, size_t(T) * V};
    for (int i = 0; i < 4; ++i) {
      const auto after = download(ctx.get(vals[i]), cnt[i]);
      CHECK(std::memcmp(after.data(), before[i]->data(), cnt[i] * 4) == 0);
    }
    // Raw GGUF bytes are not written into storage that now holds 16-row tiles
    // (they would be read as tiles): InvalidArgument, and the tiles are kept.
    const Status reload = loader.load_weights(*file, g, ctx);
    CHECK(reload.code() == ErrorCode::InvalidArgument &&
          reload.message().find("16-row tiles") != std::string::npos);
    CHECK(store->get("layer_0.up_proj.weight")->storage_layout() == StorageLayout::Q8_0Tiled);
    check_status(ex.run(ctx));
    check_hip(hipDeviceSynchronize());
    const auto again = download(ctx.get(*logits), cnt[3]);
    CHECK(std::memcmp(again.data(), el.data(), cnt[3] * 4) == 0);
  }
  std::remove(path.c_str());
  std::printf("  PASS test_gguf_model_end_to_end\n");
}

static void test_fused_launchers() {
  // M=3, N=40, K=64, scale 1.0, integer quants x dyadic activations: every
  // Linear sum is exact, so gate/up are known exactly; silu in double.
  const int M = 3, N = 40, K = 64;
  std::vector<float> x(M * K);
  for (int i = 0; i < M * K; ++i) x[i] = float((i * 7) % 9 - 4) * 0.125f;
  std::vector<int8_t> qg(N * K), qu(N * K), qv(N * K);
  for (int i = 0; i < N * K; ++i) {
    qg[i] = int8_t((i * 5) % 11 - 5);
    qu[i] = int8_t((i * 3) % 13 - 6);
    qv[i] = int8_t((i * 11) % 7 - 3);
  }
  const auto pg = pack_q8_0(qg, 0x3c00), pu = pack_q8_0(qu, 0x3c00), pv = pack_q8_0(qv, 0x3c00);
  DevBuf<float> dx(x.size()), dy(M * N), dy2(M * N), dy3(M * N);
  DevBuf<uint8_t> dg(pg.size()), du(pu.size()), dv(pv.size());
  dx.put(x);
  dg.put(pg);
  du.put(pu);
  dv.put(pv);
  auto dot = [&](const std::vector<int8_t>& q, int m, int n) {
    double s = 0;
    for (int k = 0; k < K; ++k) s += double(x[m * K + k]) * q[n * K + k];
    return s;
  };
  check_status(hip::linear_swiglu(dx.p, dg.p, du.p, dy.p, M, N, K));
  const uint8_t* ws[3] = {dg.p, du.p, dv.p};
  float* ys[3] = {dy.p, dy2.p, dy3.p};
  const int Ns[3] = {N, N, N};
  const auto sw = dy.get();
  check_status(hip::linear_multi(dx.p, 3, ws, nullptr, ys, Ns, M, K));
  const auto g = dy.get(), u = dy2.get(), v = dy3.get();
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      const double gg = dot(qg, m, n), uu = dot(qu, m, n);
      CHECK(g[m * N + n] == float(gg) && u[m * N + n] == float(uu));
      CHECK(v[m * N + n] == float(dot(qv, m, n)));
      const double want = gg / (1.0 + std::exp(-gg)) * uu;
      near(sw[m * N + n], float(want), 1e-5f * float(std::fabs(want)) + 1e-6f);
    }
  // Argmax of the gate outputs per row.
  DevBuf<int32_t> di(M);
  DevBuf<float> dval(M);
  check_status(hip::argmax(dy.p, M, N, di.p, dval.p));
  const auto ix = di.get();
  const auto vx = dval.get();
  for (int m = 0; m < M; ++m) {
    int best = 0;
    for (int n = 1; n < N; ++n)
      if (g[m * N + n] > g[m * N + best]) best = n;
    CHECK(ix[m] == best && vx[m] == g[m * N + best]);
  }
  CHECK(hip::argmax(dy.p, 0, N, di.p).code() == ErrorCode::InvalidArgument);
  // Top tokens of the gate outputs (Sampler::get_top_tokens restated on the host:
  // softmax after 1/temperature, probability order, ties to the lower index).
  {
    const int top = 7;
    const float temp = 0.5f;
    DevBuf<int32_t> tid(M * top);
    DevBuf<float> tpr(M * top);
    check_status(hip::top_tokens(dy.p, M, N, top, temp, tid.p, tpr.p));
    const auto ti = tid.get();
    const auto tp = tpr.get();
    for (int m = 0; m < M; ++m) {
      std::vector<float> v(N);
      float mx = -INFINITY;
      for (int n = 0; n < N; ++n) {
        v[n] = g[m * N + n] * (1.0f / temp);
        mx = std::max(mx, v[n]);
      }
      double sum = 0;
      for (int n = 0; n < N; ++n) sum += std::exp(double(v[n] - mx));
      std::vector<int> order(N);
      for (int n = 0; n < N; ++n) order[n] = n;
      std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return v[a] > v[b]; });
      for (int j = 0; j < top; ++j) {
        CHECK(ti[m * top + j] == order[j]);
        const float want = float(std::exp(double(v[order[j]] - mx)) / sum);
        near(tp[m * top + j], want, 1e-5f * want + 1e-7f);
      }
    }
    CHECK(hip::top_tokens(dy.p, M, N, top, temp, nullptr, tpr.p).code() ==
          ErrorCode::InvalidArgument);
    CHECK(hip::top_tokens(dy.p, M, N, 129, temp, tid.p, tpr.p).code() ==
          ErrorCode::Unsupported);
  }
  CHECK(hip::linear_swiglu(dx.p, dg.p, nullptr, dy.p, M, N, K).code() ==
        ErrorCode::InvalidArgument);
  std::printf("  PASS test_fused_launchers\n");
}

static void test_executor_fusion_end_to_end() {
  // x -> {gate, up} -> SwiGLU -> down, plus q / k / v on x; the fused executor
  // against the unfused one (bitwise for M < 64, the same kernels' arithmetic;
  // within 1e-5 of each other at M = 70, where split choices may differ).
  const int K = 128, I = 96, Q = 64, KV = 32;
  std::vector<std::vector<uint8_t>> w;
  const int rows[6] = {I, I, K, Q, KV, KV};
  const int cols[6] = {K, K, I, K, K, K};
  for (int i = 0; i < 6; ++i) w.push_back(synth_q8(rows[i], cols[i], 40 + i));
  KernelRegistry registry;
  register_hip_kernels(registry);
  for (int M : {5, 70}) {
    std::vector<float> hx(size_t(M) * K);
    for (size_t i = 0; i < hx.size(); ++i) hx[i] = float(int(i * 37 % 101) - 50) * 0.02f;
    std::vector<std::vector<float>> outs[2];
    for (int fuse = 0; fuse < 2; ++fuse) {
      Graph g;
      GraphBuilder gb(g);
      const Device dev = Device::hip(0);
      auto x = gb.input("x", Shape({M, K}), DType::Float32, dev);
      CHECK(x);
      std::vector<ValueId> cw;
      const char* names[6] = {"wg", "wu", "wd", "wq", "wk", "wv"};
      for (int i = 0; i < 6; ++i) {
        auto c = gb.constant(names[i], Shape({rows[i], cols[i]}), DType::Float32, dev);
        CHECK(c);
        cw.push_back(*c);
      }
      auto gate = gb.linear(*x, cw[0], std::nullopt, "gate");
      auto up = gb.linear(*x, cw[1], std::nullopt, "up");
      CHECK(gate && up);
      auto act = gb.swiglu(*gate, *up, "swiglu");
      CHECK(act);
      auto down = gb.linear(*act, cw[2], std::nullopt, "down");
      auto q = gb.linear(*x, cw[3], std::nullopt, "q");
      auto k = gb.linear(*x, cw[4], std::nullopt, "k");
      auto v = gb.linear(*x, cw[5], std::nullopt, "v");
      CHECK(down && q && k && v);
      CHECK(gb.output(*down, "o_down") && gb.output(*q, "o_q") && gb.output(*k, "o_k") &&
            gb.output(*v, "o_v"));
      std::vector<std::unique_ptr<Tensor>> tw;
      RuntimeContext ctx;
      for (int i = 0; i < 6; ++i) {
        tw.push_back(std::make_unique<Tensor>(names[i], Shape({rows[i], cols[i]}), DType::Q8_0,
                                              dev));
        check_status(tw.back()->allocate_hip_bytes(w[i].size()));
        upload(*tw.back(), w[i].data(), w[i].size());
        check_status(ctx.bind(cw[i], tw.back().get()));
      }
      Tensor tx("x", Shape({M, K}), DType::Float32, dev);
      check_status(tx.allocate_hip());
      upload(tx, hx.data(), hx.size() * 4);
      check_status(ctx.bind(*x, &tx));
      check_status(ctx.allocate_intermediates(g));
      HipExecutor ex(std::make_shared<HipBackend>(), registry);
      ex.set_fusion(fuse == 1);
      check_status(ex.compile(g));
      check_status(ex.run(ctx));
      check_hip(hipDeviceSynchronize());
      CHECK(ex.fused_launches() == (fuse ? 2u : 0u));
      outs[fuse] = {download(ctx.get(*down), size_t(M) * K), download(ctx.get(*q), size_t(M) * Q),
                    download(ctx.get(*k), size_t(M) * KV), download(ctx.get(*v), size_t(M) * KV)};
    }
    for (int o = 0; o < 4; ++o) {
      const auto& a = outs[0][o];
      const auto& b = outs[1][o];
      double num = 0, den = 0;
      for (size_t i = 0; i < a.size(); ++i) {
        num += double(a[i] - b[i]) * (a[i] - b[i]);
        den += double(a[i]) * a[i];
      }
      if (M < 64) CHECK(std::memcmp(a.data(), b.data(), a.size() * 4) == 0);
      else CHECK(std::sqrt(num / den) <= 1e-5);
    }
  }
  // The unfused SwiGLU op on its own: silu(g) * u in the reference's order.
  {
    const int n = 1001;
    std::vector<float> hg(n), hu(n);
    for (int i = 0; i < n; ++i) {
      hg[i] = float(i - 500) * 0.013f;
      hu[i] = float((i * 7) % 23 - 11) * 0.25f;
    }
    DevBuf<float> dg(n), du(n), dy(n);
    dg.put(hg);
    du.put(hu);
    check_status(from_hip(mle_swiglu_f32(dg.p, du.p, dy.p, n, nullptr)));
    const auto hy = dy.get();
    for (int i = 0; i < n; ++i) {
      const double want = double(hg[i]) / (1.0 + std::exp(-double(hg[i]))) * hu[i];
      near(hy[i], float(want), 2e-6f * float(std::fabs(want)) + 1e-7f);
    }
  }
  std::printf("  PASS test_executor_fusion_end_to_end\n");
}

static void test_executor_tiled_weights() {
  // The same graph as the fusion test, run on the raw bytes and then on tiled
  // copies (HipExecutor::tile_weights): bitwise equal where both run the MFMA
  // decode (M = 5) or the GEMM (M = 70); within 1e-6 relative L2 where the
  // tiled FP32 GEMV replaces the raw one (M = 1).  Fused and unfused plans.
  const int K = 128, I = 96, Q = 64, KV = 32;
  std::vector<std::vector<uint8_t>> w;
  const int rows[6] = {I, I, K, Q, KV, KV};
  const int cols[6] = {K, K, I, K, K, K};
  for (int i = 0; i < 6; ++i) w.push_back(synth_q8(rows[i], cols[i], 60 + i));
  KernelRegistry registry;
  register_hip_kernels(registry);
  for (int fuse = 0; fuse < 2; ++fuse) {
    for (int M : {1, 5, 70}) {
      std::vector<float> hx(size_t(M) * K);
      for (size_t i = 0; i < hx.size(); ++i) hx[i] = float(int(i * 41 % 103) - 51) * 0.02f;
      Graph g;
      GraphBuilder gb(g);
      const Device dev = Device::hip(0);
      auto x = gb.input("x", Shape({M, K}), DType::Float32, dev);
      CHECK(x);
      std::vector<ValueId> cw;
      const char* names[6] = {"wg", "wu", "wd", "wq", "wk", "wv"};
      for (int i = 0; i < 6; ++i) {
        auto c = gb.constant(names[i], Shape({rows[i], cols[i]}), DType::Float32, dev);
        CHECK(c);
        cw.push_back(*c);
      }
      auto gate = gb.linear(*x, cw[0], std::nullopt, "gate");
      auto up = gb.linear(*x, cw[1], std::nullopt, "up");
      CHECK(gate && up);
      auto act = gb.swiglu(*gate, *up, "swiglu");
      CHECK(act);
      auto down = gb.linear(*act, cw[2], std::nullopt, "down");
      auto q = gb.linear(*x, cw[3], std::nullopt, "q");
      auto k = gb.linear(*x, cw[4], std::nullopt, "k");
      auto v = gb.linear(*x, cw[5], std::nullopt, "v");
      CHECK(down && q && k && v);
      CHECK(gb.output(*down, "o_down") && gb.output(*q, "o_q") && gb.output(*k, "o_k") &&
            gb.output(*v, "o_v"));
      std::vector<std::unique_ptr<Tensor>> tw;
      RuntimeContext ctx;
      for (int i = 0; i < 6; ++i) {
        tw.push_back(std::make_unique<Tensor>(names[i], Shape({rows[i], cols[i]}), DType::Q8_0,
                                              dev));
        check_status(tw.back()->allocate_hip_bytes(w[i].size()));
        upload(*tw.back(), w[i].data(), w[i].size());
        check_status(ctx.bind(cw[i], tw.back().get()));
      }
      Tensor tx("x", Shape({M, K}), DType::Float32, dev);
      check_status(tx.allocate_hip());
      upload(tx, hx.data(), hx.size() * 4);
      check_status(ctx.bind(*x, &tx));
      check_status(ctx.allocate_intermediates(g));
      HipExecutor ex(std::make_shared<HipBackend>(), registry);
      ex.set_fusion(fuse == 1);
      check_status(ex.compile(g));
      std::vector<std::vector<float>> outs[2];
      for (int tiled = 0; tiled < 2; ++tiled) {
        if (tiled) {
          check_status(ex.tile_weights(ctx));
          CHECK(ex.tiled_weights() == 6u);
        }
        check_status(ex.run(ctx));
        check_hip(hipDeviceSynchronize());
        // fused: gate/up + SwiGLU, q/k/v, down; unfused: six Linears
        CHECK(ex.tiled_launches() == (tiled ? (fuse ? 3u : 6u) : 0u));
        outs[tiled] = {download(ctx.get(*down), size_t(M) * K),
                       download(ctx.get(*q), size_t(M) * Q),
                       download(ctx.get(*k), size_t(M) * KV),
                       download(ctx.get(*v), size_t(M) * KV)};
      }
      for (int o = 0; o < 4; ++o) {
        const auto& a = outs[0][o];
        const auto& b = outs[1][o];
        double num = 0, den = 0;
        for (size_t i = 0; i < a.size(); ++i) {
          num += double(a[i] - b[i]) * (a[i] - b[i]);
          den += double(a[i]) * a[i];
        }
        if (M == 1) CHECK(std::sqrt(num / den) <= 1e-6);
        else CHECK(std::memcmp(a.data(), b.data(), a.size() * 4) == 0);
      }
      ex.release_tiled_weights();
      CHECK(ex.tiled_weights() == 0u);
      check_status(ex.run(ctx));
      check_hip(hipDeviceSynchronize());
      CHECK(ex.tiled_launches() == 0u);
      const auto again = download(ctx.get(*q), size_t(M) * Q);
      CHECK(std::memcmp(again.data(), outs[0][1].data(), again.size() * 4) == 0);
    }
  }
  std::printf("  PASS test_executor_tiled_weights\n");
}

static void test_executor_rows_decode() {
  // Llama-7B q / k / v (3 x 4096 x 4096) at 4 and 8 tokens through the executor,
  // fused (one multi-output launch, 768 row groups) and unfused (three launches,
  // 256 groups each at 4 tokens): on tiled weights these take the row-range MFMA
  // decode, on the raw bytes the split-K decode.  Both sum the same exact block
  // products, grouped differently over K: within 1e-6 relative L2 of each other,
  // repeatable bit for bit, and sampled rows within 1e-5 of an fp64 sum.
  const int K = 4096, N = 4096;
  std::vector<std::vector<uint8_t>> w;
  for (int i = 0; i < 3; ++i) w.push_back(synth_q8(N, K, 80 + i));
  KernelRegistry registry;
  register_hip_kernels(registry);
  for (int M : {4, 8}) {
    for (int fuse = 0; fuse < 2; ++fuse) {
      std::vector<float> hx(size_t(M) * K);
      for (size_t i = 0; i < hx.size(); ++i) hx[i] = float(int(i * 53 % 211) - 105) * 0.01f;
      Graph g;
      GraphBuilder gb(g);
      const Device dev = Device::hip(0);
      auto x = gb.input("x", Shape({M, K}), DType::Float32, dev);
      CHECK(x);
      const char* names[3] = {"wq", "wk", "wv"};
      std::vector<ValueId> cw, outs;
      for (int i = 0; i < 3; ++i) {
        auto c = gb.constant(names[i], Shape({N, K}), DType::Float32, dev);
        CHECK(c);
        cw.push_back(*c);
        auto y = gb.linear(*x, *c, std::nullopt, names[i] + 1);
        CHECK(y);
        CHECK(gb.output(*y, std::string("o_") + (names[i] + 1)));
        outs.push_back(*y);
      }
      std::vector<std::unique_ptr<Tensor>> tw;
      RuntimeContext ctx;
      for (int i = 0; i < 3; ++i) {
        tw.push_back(std::make_unique<Tensor>(names[i], Shape({N, K}), DType::Q8_0, dev));
        check_status(tw.back()->allocate_hip_bytes(w[i].size()));
        upload(*tw.back(), w[i].data(), w[i].size());
        check_status(ctx.bind(cw[i], tw.back().get()));
      }
      Tensor tx("x", Shape({M, K}), DType::Float32, dev);
      check_status(tx.allocate_hip());
      upload(tx, hx.data(), hx.size() * 4);
      check_status(ctx.bind(*x, &tx));
      check_status(ctx.allocate_intermediates(g));
      HipExecutor ex(std::make_shared<HipBackend>(), registry);
      ex.set_fusion(fuse == 1);
      check_status(ex.compile(g));
      std::vector<std::vector<float>> got[3];  // raw, tiled, tiled again
      for (int pass = 0; pass < 3; ++pass) {
        if (pass == 1) check_status(ex.tile_weights(ctx));
        check_status(ex.run(ctx));
        check_hip(hipDeviceSynchronize());
        CHECK(ex.tiled_launches() == (pass == 0 ? 0u : (fuse ? 1u : 3u)));
        for (int i = 0; i < 3; ++i) got[pass].push_back(download(ctx.get(outs[i]), size_t(M) * N));
      }
      for (int i = 0; i < 3; ++i) {
        const auto& a = got[0][i];
        const auto& b = got[1][i];
        CHECK(std::memcmp(b.data(), got[2][i].data(), b.size() * 4) == 0);
        double num = 0, den = 0;
        for (size_t e = 0; e < a.size(); ++e) {
          num += double(a[e] - b[e]) * (a[e] - b[e]);
          den += double(a[e]) * a[e];
        }
        CHECK(std::sqrt(num / den) <= 1e-6);
        // rows 0, 1, N / 2 and N - 1 of every token against an fp64 sum
        num = den = 0;
        for (int n : {0, 1, N / 2, N - 1})
          for (int m = 0; m < M; ++m) {
            double e = 0;
            for (int kb = 0; kb < K / 32; ++kb) {
              const uint8_t* blk = w[i].data() + (size_t(n) * (K / 32) + kb) * 34;
              const double d = host_half(uint16_t(blk[0] | (blk[1] << 8)));
              for (int j = 0; j < 32; ++j)
                e += double(hx[size_t(m) * K + 32 * kb + j]) * d * double(int8_t(blk[2 + j]));
            }
            const double gv = b[size_t(m) * N + n];
            num += (gv - e) * (gv - e);
            den += e * e;
          }
        CHECK(std::sqrt(num / den) <= 1e-5);
      }
    }
  }
  std::printf("  PASS test_executor_rows_decode\n");
}

static std::vector<uint8_t> random_q8(int64_t N, int64_t K, uint32_t seed) {
  std::vector<uint8_t> w(size_t(N) * (K / 32) * 34);
  uint32_t st = seed;
  for (size_t b = 0; b < w.size() / 34; ++b) {
    w[b * 34] = 0x00;
    w[b * 34 + 1] = 0x1c;  // scale 2^-8
    for (int i = 0; i < 32; ++i) {
      st = st * 1664525u + 1013904223u;
      w[b * 34 + 2 + i] = static_cast<uint8_t>(int8_t((st >> 24) % 255) - 127);
    }
  }
  return w;
}

static void test_workspace_no_regrowth() {
  // A counter-heavy launch (many row tiles, few K splits) and a partial-heavy
  // one (few tiles, many splits) alternating on one stream: the workspace grows
  // at most once for each, then never again (each buffer keeps
  // max(capacity, need)); results stay the same run to run.
  hipStream_t stream;
  check_hip(hipStreamCreate(&stream));
  struct Shape3 { int M, N, K; };
  const Shape3 a{4, 32768, 2048}, b{16, 1024, 65536};
  size_t ab = 0, ac = 0, bb = 0, bc = 0;
  CHECK(mle_q8_0_workspace_size(MLE_OP_LINEAR, a.M, 1, &a.N, a.K, 0, &ab, &ac) == 0);
  CHECK(mle_q8_0_workspace_size(MLE_OP_LINEAR, b.M, 1, &b.N, b.K, 0, &bb, &bc) == 0);
  CHECK(ac > 4096 && bc < ac);  // a needs more counters than the minimum, b fewer
  CHECK(bb > ab && bb > (size_t(4) << 20));
  std::vector<DevBuf<uint8_t>*> w;
  std::vector<DevBuf<float>*> x, y;
  for (const Shape3& s : {a, b}) {
    const auto hw = random_q8(s.N, s.K, 7u + s.N);
    w.push_back(new DevBuf<uint8_t>(hw.size()));
    w.back()->put(hw);
    std::vector<float> hx(size_t(s.M) * s.K);
    for (size_t i = 0; i < hx.size(); ++i) hx[i] = float(int(i * 37 % 201) - 100) * 0.01f;
    x.push_back(new DevBuf<float>(hx.size()));
    x.back()->put(hx);
    y.push_back(new DevBuf<float>(size_t(s.M) * s.N));
  }
  size_t cap_b = 0, cap_c = 0;
  uint64_t gen0 = 0, gen = 0;
  CHECK(mle_workspace_info(stream, &cap_b, &cap_c, &gen0) == 0);
  CHECK(gen0 == 0 && cap_b == 0 && cap_c == 0);  // a fresh stream has none yet
  std::vector<float> first;
  for (int it = 0; it < 6; ++it) {
    const Shape3& s = it % 2 ? b : a;
    const int i = it % 2;
    CHECK(mle_q8_0_linear(x[i]->p, w[i]->p, nullptr, y[i]->p, s.M, s.N, s.K, stream) == 0);
    check_hip(hipStreamSynchronize(stream));
    CHECK(mle_workspace_info(stream, &cap_b, &cap_c, &gen) == 0);
    if (it == 0) first = y[0]->get();
    CHECK(gen == uint64_t(it < 2 ? it + 1 : 2));  // grows on the first a and the first b only
    CHECK(cap_b >= (it == 0 ? ab : bb) && cap_c >= ac);
  }
  CHECK(cap_b >= bb && cap_c == ac);
  CHECK(y[0]->get() == first);  // deterministic
  for (auto* p : w) delete p;
  for (auto* p : x) delete p;
  for (auto* p : y) delete p;
  // A reservation that covers both up front: no growth at all afterwards.
  hipStream_t s2;
  check_hip(hipStreamCreate(&s2));
  CHECK(mle_workspace_reserve(std::max(ab, bb), std::max(ac, bc), s2) == 0);
  CHECK(mle_workspace_info(s2, &cap_b, &cap_c, &gen) == 0);
  CHECK(gen == 1 && cap_b >= bb && cap_c >= ac);
  CHECK(mle_workspace_reserve(ab, ac, s2) == 0);  // within capacity: nothing happens
  CHECK(mle_workspace_info(s2, &cap_b, &cap_c, &gen) == 0 && gen == 1);
  check_hip(hipStreamDestroy(s2));
  check_hip(hipStreamDestroy(stream));
  std::printf("  workspace_no_regrowth ok\n");
}

static void test_executor_reserves_workspace() {
  // compile() reserves the executor stream's workspace for the plan's largest
  // Linear (here a split-K MFMA decode at M = 8), so run() allocates nothing:
  // the workspace generation does not move across runs.
  const int M = 8, N = 4096, K = 11008;
  hipStream_t stream;
  check_hip(hipStreamCreate(&stream));
  Graph g;
  GraphBuilder gb(g);
  const Device dev = Device::hip(0);
  auto x = gb.input("x", Shape({M, K}), DType::Float32, dev);
  auto w = gb.constant("w", Shape({N, K}), DType::Float32, dev);
  CHECK(x && w);
  auto y = gb.linear(*x, *w, std::nullopt, "down");
  CHECK(y && gb.output(*y, "out"));
  KernelRegistry registry;
  register_hip_kernels(registry);
  HipExecutor ex(std::make_shared<HipBackend>(), registry, stream);
  check_status(ex.compile(g));
  size_t need_b = 0, need_c = 0, cap_b = 0, cap_c = 0;
  CHECK(mle_q8_0_workspace_size(MLE_OP_LINEAR, M, 1, &N, K, 0, &need_b, &need_c) == 0);
  CHECK(need_b > 0 && need_c > 0);
  CHECK(ex.workspace_bytes() >= need_b && ex.workspace_counters() >= need_c);
  uint64_t gen = 0, gen2 = 0;
  CHECK(mle_workspace_info(stream, &cap_b, &cap_c, &gen) == 0);
  CHECK(gen >= 1 && cap_b >= need_b && cap_c >= need_c);
  const auto hw = random_q8(N, K, 99);
  Tensor tw("w", Shape({N, K}), DType::Q8_0, dev);
  check_status(tw.allocate_hip_bytes(hw.size()));
  upload(tw, hw.data(), hw.size());
  std::vector<float> hx(size_t(M) * K);
  for (size_t i = 0; i < hx.size(); ++i) hx[i] = float(int(i * 13 % 97) - 48) * 0.03f;
  Tensor tx("x", Shape({M, K}), DType::Float32, dev);
  check_status(tx.allocate_hip());
  upload(tx, hx.data(), hx.size() * 4);
  RuntimeContext ctx;
  check_status(ctx.bind(*x, &tx));
  check_status(ctx.bind(*w, &tw));
  check_status(ctx.allocate_intermediates(g));
  for (int r = 0; r < 3; ++r) check_status(ex.run(ctx));
  check_hip(hipStreamSynchronize(stream));
  CHECK(mle_workspace_info(stream, &cap_b, &cap_c, &gen2) == 0);
  CHECK(gen2 == gen);
  // and after tiling the weight (the tiled launch fits the same reservation)
  check_status(ex.tile_weights(ctx));
  check_status(ex.run(ctx));
  check_hip(hipStreamSynchronize(stream));
  CHECK(ex.tiled_launches() == 1u);
  CHECK(mle_workspace_info(stream, &cap_b, &cap_c, &gen2) == 0 && gen2 == gen);
  check_hip(hipStreamDestroy(stream));
  std::printf("  executor_reserves_workspace ok\n");
}

static void test_executor_reserves_matmul_workspace() {
  // A decode-size MatMul (A [1, 4096] . B [4096, 4096]) spreads K over several
  // workgroups per column tile and needs workspace (partial sums and one arrival
  // counter per column tile): compile() reserves it, run() allocates nothing, and
  // sampled outputs match an fp64 sum within 1e-5.
  const int M = 1, K = 4096, N = 4096;
  hipStream_t stream;
  check_hip(hipStreamCreate(&stream));
  Graph g;
  GraphBuilder gb(g);
  const Device dev = Device::hip(0);
  auto a = gb.input("a", Shape({M, K}), DType::Float32, dev);
  auto b = gb.constant("b", Shape({K, N}), DType::Float32, dev);
  CHECK(a && b);
  auto y = gb.matmul(*a, *b, "mm");
  CHECK(y && gb.output(*y, "out"));
  KernelRegistry registry;
  register_hip_kernels(registry);
  HipExecutor ex(std::make_shared<HipBackend>(), registry, stream);
  check_status(ex.compile(g));
  size_t need_b = 0, need_c = 0, cap_b = 0, cap_c = 0;
  CHECK(mle_q8_0_workspace_size(MLE_OP_MATMUL, M, 1, &N, K, 0, &need_b, &need_c) == 0);
  CHECK(need_b > 0 && need_c >= 16);
  CHECK(ex.workspace_bytes() >= need_b);
  uint64_t gen = 0, gen2 = 0;
  CHECK(mle_workspace_info(stream, &cap_b, &cap_c, &gen) == 0);
  CHECK(gen >= 1 && cap_b >= need_b && cap_c >= need_c);
  const auto hb = random_q8(K, N, 77);  // K rows of N: blocks along N
  Tensor tb("b", Shape({K, N}), DType::Q8_0, dev);
  check_status(tb.allocate_hip_bytes(hb.size()));
  upload(tb, hb.data(), hb.size());
  std::vector<float> ha(size_t(M) * K);
  for (size_t i = 0; i < ha.size(); ++i) ha[i] = float(int(i * 29 % 113) - 56) * 0.02f;
  Tensor ta("a", Shape({M, K}), DType::Float32, dev);
  check_status(ta.allocate_hip());
  upload(ta, ha.data(), ha.size() * 4);
  RuntimeContext ctx;
  check_status(ctx.bind(*a, &ta));
  check_status(ctx.bind(*b, &tb));
  check_status(ctx.allocate_intermediates(g));
  for (int r = 0; r < 3; ++r) check_status(ex.run(ctx));
  check_hip(hipStreamSynchronize(stream));
  CHECK(mle_workspace_info(stream, &cap_b, &cap_c, &gen2) == 0);
  CHECK(gen2 == gen);
  const auto got = download(ctx.get(*y), size_t(M) * N);
  double num = 0, den = 0;
  for (int n : {0, 31, 32, 1000, N / 2, N - 1}) {
    double e = 0;
    for (int k = 0; k < K; ++k) {
      const uint8_t* blk = hb.data() + (size_t(k) * (N / 32) + n / 32) * 34;
      e += double(ha[k]) * host_half(uint16_t(blk[0] | (blk[1] << 8))) *
           double(int8_t(blk[2 + n % 32]));
    }
    num += (got[n] - e) * (got[n] - e);
    den += e * e;
  }
  CHECK(std::sqrt(num / den) <= 1e-5);
  check_hip(hipStreamDestroy(stream));
  std::printf("  executor_reserves_matmul_workspace ok\n");
}

static void test_tiled_copy_shape_guard() {
  // A tiled copy is used only for the weight shape it was made for: after the
  // executor is recompiled for a graph that views the same weight buffer as
  // [N/2, 2K], its Linear runs on the raw bytes and matches the raw launcher.
  const int M = 2, N = 64, K = 128;
  const auto hw = random_q8(N, K, 5);
  DevBuf<uint8_t> buf(hw.size());
  buf.put(hw);
  KernelRegistry registry;
  register_hip_kernels(registry);
  HipExecutor exe(std::make_shared<HipBackend>(), registry);
  Graph graphs[2];
  const Device dev = Device::hip(0);
  for (int pass = 0; pass < 2; ++pass) {
    const int n = pass ? N / 2 : N, k = pass ? 2 * K : K;
    Graph& g = graphs[pass];
    GraphBuilder gb(g);
    auto x = gb.input("x", Shape({M, k}), DType::Float32, dev);
    auto w = gb.constant("w", Shape({n, k}), DType::Float32, dev);
    CHECK(x && w);
    auto y = gb.linear(*x, *w, std::nullopt, "lin");
    CHECK(y && gb.output(*y, "out"));
    std::vector<float> hx(size_t(M) * k);
    for (size_t i = 0; i < hx.size(); ++i) hx[i] = float(int(i * 7 % 31) - 15) * 0.1f;
    Tensor tx("x", Shape({M, k}), DType::Float32, dev);
    check_status(tx.allocate_hip());
    upload(tx, hx.data(), hx.size() * 4);
    Tensor tw("w", Shape({n, k}), DType::Q8_0, dev);
    check_status(tw.bind_hip_data(buf.p, hw.size()));
    RuntimeContext ctx;
    check_status(ctx.bind(*x, &tx));
    check_status(ctx.bind(*w, &tw));
    check_status(ctx.allocate_intermediates(g));
    check_status(exe.compile(g));
    if (pass == 0) check_status(exe.tile_weights(ctx));
    CHECK(exe.tiled_weights() == 1u);  // the copy of pass 0 is still held in pass 1
    check_status(exe.run(ctx));
    check_hip(hipDeviceSynchronize());
    CHECK(exe.tiled_launches() == (pass == 0 ? 1u : 0u));
    DevBuf<float> ref(size_t(M) * n);
    DevBuf<float> dx(hx.size());
    dx.put(hx);
    CHECK(mle_q8_0_linear(dx.p, buf.p, nullptr, ref.p, M, n, k, nullptr) == 0);
    check_hip(hipDeviceSynchronize());
    const auto got = download(ctx.get(*y), size_t(M) * n);
    const auto want = ref.get();
    double num = 0, den = 0;
    for (size_t i = 0; i < got.size(); ++i) {
      num += double(got[i] - want[i]) * (got[i] - want[i]);
      den += double(want[i]) * want[i];
    }
    CHECK(std::sqrt(num / den) <= 1e-6);
  }
  std::printf("  tiled_copy_shape_guard ok\n");
}

static void test_loader_dequantizes_q8_0_on_device() {
  // WeightLoader::load_weights into a Float32 HIP tensor bound to a Q8_0 GGUF
  // tensor: the raw blocks go to the device and are dequantised there
  // (hip::dequantize_q8_0); the bits equal the loader's host loop
  // WeightLoader::dequantize_to_f32 (reference gguf_weight_loader.cpp:446-463),
  // special binary16 scales included.
  const int R = 96, C = 160;
  auto q = synth_q8(R, C, 21);
  const uint16_t special[] = {0x0001, 0x03ff, 0x0000, 0x8000, 0x7c00, 0xfc00, 0x7e00, 0x3c00};
  for (int i = 0; i < 8; ++i) {
    q[size_t(i) * 7 * 34] = uint8_t(special[i] & 0xff);
    q[size_t(i) * 7 * 34 + 1] = uint8_t(special[i] >> 8);
  }
  GgufWriter w;
  w.kv_str("general.architecture", "llama");
  w.kv_u32("llama.embedding_length", C);
  w.tensor("blk.0.ffn_up.weight", {R, C}, 8, q);
  const std::string path = w.write("mle_dequant");
  Graph g;
  GraphBuilder gb(g);
  const Device dev = Device::hip(0);
  auto wv = gb.constant("layer_0.up_proj.weight", Shape({R, C}), DType::Float32, dev);
  CHECK(wv);
  WeightLoader loader(path);
  auto file = loader.open();
  CHECK(file);
  Tensor t("layer_0.up_proj.weight", Shape({R, C}), DType::Float32, dev);
  check_status(t.allocate_hip());
  RuntimeContext ctx;
  check_status(ctx.bind(*wv, &t));
  check_status(loader.load_weights(*file, g, ctx));
  const auto got = download(&t, size_t(R) * C);
  std::vector<float> want(size_t(R) * C);
  check_status(WeightLoader::dequantize_to_f32(GgmlDataType::Q8_0, q.data(), want.data(), want.size()));
  for (size_t i = 0; i < want.size(); ++i) {
    if (std::isnan(want[i])) {
      CHECK(std::isnan(got[i]));
      continue;
    }
    uint32_t a, b;
    std::memcpy(&a, &got[i], 4);
    std::memcpy(&b, &want[i], 4);
    CHECK(a == b);
  }
  std::printf("  loader_dequantizes_q8_0_on_device ok\n");
}

static void test_executor_linear_bf16_bias() {
  // Linear nodes with a BFloat16 bias (the reference CUDA adapter's accepted
  // bias dtypes, cuda_kernel_adapter.cpp:204-218): the same bits as the bias
  // widened to Float32, on raw and tiled weights; two sibling Linears with BF16
  // biases run node by node (no fused launch) and still agree.
  const int M = 5, N = 96, K = 256;
  const Device dev = Device::hip(0);
  const auto hw = random_q8(N, K, 41);
  std::vector<uint16_t> b16(N);
  std::vector<float> b32(N);
  for (int i = 0; i < N; ++i) {
    const float v = float(i % 13 - 6) * 0.37f + 0.01f * i;
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    b16[i] = uint16_t(bits >> 16);
    const uint32_t wide = uint32_t(b16[i]) << 16;
    std::memcpy(&b32[i], &wide, 4);
  }
  std::vector<float> hx(size_t(M) * K);
  for (size_t i = 0; i < hx.size(); ++i) hx[i] = float(int(i * 29 % 83) - 41) * 0.05f;
  KernelRegistry registry;
  register_hip_kernels(registry);
  std::vector<float> outs[2][2];  // [bias dtype][tiled]
  for (int bf = 0; bf < 2; ++bf) {
    Graph g;
    GraphBuilder gb(g);
    auto x = gb.input("x", Shape({M, K}), DType::Float32, dev);
    auto w = gb.constant("w", Shape({N, K}), DType::Float32, dev);
    auto w2 = gb.constant("w2", Shape({N, K}), DType::Float32, dev);
    auto b = gb.constant("b", Shape({N}), DType::Float32, dev);
    CHECK(x && w && w2 && b);
    auto y = gb.linear(*x, *w, *b, "lin");
    auto y2 = gb.linear(*x, *w2, *b, "lin2");  // sibling on the same input
    CHECK(y && y2 && gb.output(*y, "out") && gb.output(*y2, "out2"));
    Tensor tx("x", Shape({M, K}), DType::Float32, dev), tw("w", Shape({N, K}), DType::Q8_0, dev);
    Tensor tw2("w2", Shape({N, K}), DType::Q8_0, dev);
    Tensor tb("b", Shape({N}), bf ? DType::BFloat16 : DType::Float32, dev);
    check_status(tx.allocate_hip());
    check_status(tw.allocate_hip_bytes(hw.size()));
    check_status(tw2.allocate_hip_bytes(hw.size()));
    check_status(tb.allocate_hip());
    upload(tx, hx.data(), hx.size() * 4);
    upload(tw, hw.data(), hw.size());
    upload(tw2, hw.data(), hw.size());
    if (bf) upload(tb, b16.data(), N * 2); else upload(tb, b32.data(), N * 4);
    RuntimeContext ctx;
    check_status(ctx.bind(*x, &tx));
    check_status(ctx.bind(*w, &tw));
    check_status(ctx.bind(*w2, &tw2));
    check_status(ctx.bind(*b, &tb));
    check_status(ctx.allocate_intermediates(g));
    HipExecutor ex(std::make_shared<HipBackend>(), registry);
    check_status(ex.compile(g));
    CHECK(ex.fused_groups() == 1u);
    for (int tiled = 0; tiled < 2; ++tiled) {
      if (tiled) check_status(ex.tile_weights(ctx));
      check_status(ex.run(ctx));
      check_hip(hipDeviceSynchronize());
      CHECK(ex.fused_launches() == (bf ? 0u : 1u));
      outs[bf][tiled] = download(ctx.get(*y), size_t(M) * N);
      CHECK(download(ctx.get(*y2), size_t(M) * N) == outs[bf][tiled]);
    }
  }
  CHECK(outs[1][0] == outs[0][0]);
  CHECK(outs[1][1] == outs[0][1]);
  std::printf("  executor_linear_bf16_bias ok\n");
}

static void test_executor_tiles_in_place() {
  // tile_weights(ctx, release_raw = true): the Linear-only weights (gate, up,
  // down, q) are re-tiled in place -- the tensors adopt 16-row tiles and their
  // raw bytes are freed -- while the table read by both an Embedding and a
  // Linear (a tied lm_head, bound to two values) keeps its raw bytes and gets a
  // copy.  Outputs match the raw run (bitwise on the MFMA paths and the
  // embedding, 1e-6 relative L2 where the tiled FP32 GEMV runs, M = 1), also
  // from a second executor that never tiled anything (the registered Linear
  // kernel reads the layout tag); an Embedding over an in-place tiled tensor
  // gives the raw gather's bits, and a MatMul over one is rejected.
  const int K = 128, I = 96, Q = 64, V = 80, T = 4;
  KernelRegistry registry;
  register_hip_kernels(registry);
  const Device dev = Device::hip(0);
  for (int fuse = 0; fuse < 2; ++fuse) {
    for (int M : {1, 5, 70}) {
      Graph g;
      GraphBuilder gb(g);
      auto x = gb.input("x", Shape({M, K}), DType::Float32, dev);
      auto ids = gb.input("ids", Shape({T}), DType::Int32, dev);
      CHECK(x && ids);
      const char* names[6] = {"wg", "wu", "wd", "wq", "table_e", "table_l"};
      const int rows[6] = {I, I, K, Q, V, V};
      const int cols[6] = {K, K, I, K, K, K};
      std::vector<ValueId> cw;
      for (int i = 0; i < 6; ++i) {
        auto c = gb.constant(names[i], Shape({rows[i], cols[i]}), DType::Float32, dev);
        CHECK(c);
        cw.push_back(*c);
      }
      auto gate = gb.linear(*x, cw[0], std::nullopt, "gate");
      auto up = gb.linear(*x, cw[1], std::nullopt, "up");
      CHECK(gate && up);
      auto act = gb.swiglu(*gate, *up, "swiglu");
      CHECK(act);
      auto down = gb.linear(*act, cw[2], std::nullopt, "down");
      auto q = gb.linear(*x, cw[3], std::nullopt, "q");
      auto emb = gb.embedding(*ids, cw[4], "embed");
      auto logits = gb.linear(*x, cw[5], std::nullopt, "lm_head");
      CHECK(down && q && emb && logits);
      CHECK(gb.output(*down, "o_down") && gb.output(*q, "o_q") && gb.output(*emb, "o_emb") &&
            gb.output(*logits, "o_logits"));
      std::vector<std::unique_ptr<Tensor>> tw;
      RuntimeContext ctx;
      for (int i = 0; i < 5; ++i) {
        tw.push_back(std::make_unique<Tensor>(names[i], Shape({rows[i], cols[i]}), DType::Q8_0,
                                              dev));
        const auto hw = synth_q8(rows[i], cols[i], 90 + i);
        check_status(tw.back()->allocate_hip_bytes(hw.size()));
        upload(*tw.back(), hw.data(), hw.size());
        check_status(ctx.bind(cw[i], tw.back().get()));
      }
      check_status(ctx.bind(cw[5], tw[4].get()));  // tied: one table, two values
      std::vector<float> hx(size_t(M) * K);
      for (size_t i = 0; i < hx.size(); ++i) hx[i] = float(int(i * 37 % 101) - 50) * 0.02f;
      Tensor tx("x", Shape({M, K}), DType::Float32, dev);
      check_status(tx.allocate_hip());
      upload(tx, hx.data(), hx.size() * 4);
      std::vector<int> hids{3, 0, 79, 41};
      Tensor tids("ids", Shape({T}), DType::Int32, dev);
      check_status(tids.allocate_hip());
      upload(tids, hids.data(), hids.size() * 4);
      check_status(ctx.bind(*x, &tx));
      check_status(ctx.bind(*ids, &tids));
      check_status(ctx.allocate_intermediates(g));
      const size_t counts[4] = {size_t(M) * K, size_t(M) * Q, size_t(T) * K, size_t(M) * V};
      const ValueId outs_id[4] = {*down, *q, *emb, *logits};
      auto outputs = [&]() {
        std::vector<std::vector<float>> o;
        for (int i = 0; i < 4; ++i) o.push_back(download(ctx.get(outs_id[i]), counts[i]));
        return o;
      };
      auto same = [&](const std::vector<std::vector<float>>& a,
                      const std::vector<std::vector<float>>& b) {
        for (int o = 0; o < 4; ++o) {
          if (o == 2 || M > 1) {  // embedding always, Linears on the MFMA paths: bitwise
            CHECK(std::memcmp(a[o].data(), b[o].data(), a[o].size() * 4) == 0);
            continue;
          }
          double num = 0, den = 0;
          for (size_t i = 0; i < a[o].size(); ++i) {
            num += double(a[o][i] - b[o][i]) * (a[o][i] - b[o][i]);
            den += double(a[o][i]) * a[o][i];
          }
          CHECK(std::sqrt(num / den) <= 1e-6);
        }
      };
      HipExecutor ex(std::make_shared<HipBackend>(), registry);
      ex.set_fusion(fuse == 1);
      check_status(ex.compile(g));
      check_status(ex.run(ctx));
      check_hip(hipDeviceSynchronize());
      const auto ref = outputs();

      check_status(ex.tile_weights(ctx, true));
      CHECK(ex.tiled_in_place() == 4u);
      CHECK(ex.tiled_weights() == 1u);  // the tied table: a copy, raw bytes kept
      for (int i = 0; i < 4; ++i) {
        CHECK(tw[i]->storage_layout() == StorageLayout::Q8_0Tiled);
        CHECK(tw[i]->allocated_bytes() == hip::q8_0_tiled_bytes(rows[i], cols[i]));
      }
      CHECK(tw[4]->storage_layout() == StorageLayout::Raw);
      check_status(ex.run(ctx));
      check_hip(hipDeviceSynchronize());
      // fused: gate+up+SwiGLU, q+lm_head, down; unfused: five Linears
      CHECK(ex.tiled_launches() == (fuse ? 3u : 5u));
      same(ref, outputs());

      // An executor that never tiled: the registered Linear kernel follows the tag.
      HipExecutor ex2(std::make_shared<HipBackend>(), registry);
      ex2.set_fusion(fuse == 1);
      check_status(ex2.compile(g));
      check_status(ex2.run(ctx));
      check_hip(hipDeviceSynchronize());
      same(ref, outputs());

      // Dropping the copies leaves the in-place tiles (the raw bytes are gone).
      ex.release_tiled_weights();
      CHECK(tw[0]->storage_layout() == StorageLayout::Q8_0Tiled);
      check_status(ex.run(ctx));
      check_hip(hipDeviceSynchronize());
      same(ref, outputs());

      if (fuse == 0 && M == 1) {
        // An Embedding over an in-place tiled tensor (wq read as a [64, 128]
        // table) gives the bits of the raw gather, computed before tiling.
        {
          Graph g3;
          GraphBuilder gb3(g3);
          auto ids3 = gb3.input("ids", Shape({T}), DType::Int32, dev);
          auto tab3 = gb3.constant("wq", Shape({Q, K}), DType::Float32, dev);
          CHECK(ids3 && tab3);
          auto e3 = gb3.embedding(*ids3, *tab3, "embed");
          CHECK(e3 && gb3.output(*e3, "o"));
          const auto hq = synth_q8(Q, K, 93);
          std::vector<int> qids{5, 0, 63, 17};
          upload(tids, qids.data(), qids.size() * 4);
          RuntimeContext ctx3;
          check_status(ctx3.bind(*ids3, &tids));
          check_status(ctx3.bind(*tab3, tw[3].get()));
          check_status(ctx3.allocate_intermediates(g3));
          HipExecutor ex4(std::make_shared<HipBackend>(), registry);
          check_status(ex4.compile(g3));
          check_status(ex4.run(ctx3));
          check_hip(hipDeviceSynchronize());
          const auto got = download(ctx3.get(*e3), size_t(T) * K);
          for (int t = 0; t < T; ++t)
            for (int c = 0; c < K; ++c) {
              const float want = q8_at(hq, K, qids[t], c);
              CHECK(std::memcmp(&got[size_t(t) * K + c], &want, 4) == 0);
            }
          upload(tids, hids.data(), hids.size() * 4);
        }
        // MatMul over an in-place tiled tensor (read as B [64, 128]) is refused.
        Graph g2;
        GraphBuilder gb2(g2);
        auto a2 = gb2.input("a", Shape({2, Q}), DType::Float32, dev);
        auto b2 = gb2.constant("wq", Shape({Q, K}), DType::Float32, dev);
        CHECK(a2 && b2);
        auto e2 = gb2.matmul(*a2, *b2, "mm");
        CHECK(e2 && gb2.output(*e2, "o"));
        Tensor ta2("a", Shape({2, Q}), DType::Float32, dev);
        check_status(ta2.allocate_hip());
        RuntimeContext ctx2;
        check_status(ctx2.bind(*a2, &ta2));
        check_status(ctx2.bind(*b2, tw[3].get()));
        check_status(ctx2.allocate_intermediates(g2));
        HipExecutor ex3(std::make_shared<HipBackend>(), registry);
        check_status(ex3.compile(g2));
        const Status st = ex3.run(ctx2);
        CHECK(!st.ok());
        CHECK(st.to_string().find("16-row tiles") != std::string::npos);
      }
    }
  }
  std::printf("  PASS test_executor_tiles_in_place\n");
}

static void test_tile_in_place_skips_viewed_buffers() {
  // tile_weights(ctx, release_raw = true) re-tiles in place only a weight whose
  // bytes no other tensor bound in the context views.  Here weight A owns its
  // buffer and tensor B views A's bytes (bind_hip_data), each the weight of a
  // Linear; tensor C views the second half of D's buffer, and D is a Linear
  // weight.  Freeing A's or D's raw bytes would leave B or C dangling, so both
  // get copies (A and B share one: same bytes), while E, owned and viewed by
  // nothing else, is re-tiled in place.  Every output equals the raw run bit for
  // bit (M = 8: the MFMA decode), before and after.
  const int M = 8, K = 256, N = 64;
  KernelRegistry registry;
  register_hip_kernels(registry);
  const Device dev = Device::hip(0);
  Graph g;
  GraphBuilder gb(g);
  auto x = gb.input("x", Shape({M, K}), DType::Float32, dev);
  CHECK(x);
  const char* names[5] = {"wa", "wb", "wc", "wd", "we"};
  const int rows[5] = {N, N, N / 2, N, N};
  std::vector<ValueId> cw;
  for (int i = 0; i < 5; ++i) {
    auto c = gb.constant(names[i], Shape({rows[i], K}), DType::Float32, dev);
    CHECK(c);
    cw.push_back(*c);
  }
  std::vector<ValueId> outs;
  for (int i = 0; i < 5; ++i) {
    auto y = gb.linear(*x, cw[i], std::nullopt, std::string("lin_") + names[i]);
    CHECK(y && gb.output(*y, std::string("o_") + names[i]));
    outs.push_back(*y);
  }
  const size_t row_bytes = size_t(K / 32) * 34;
  Tensor ta("wa", Shape({N, K}), DType::Q8_0, dev), td("wd", Shape({N, K}), DType::Q8_0, dev),
      te("we", Shape({N, K}), DType::Q8_0, dev);
  Tensor tb("wb", Shape({N, K}), DType::Q8_0, dev), tc("wc", Shape({N / 2, K}), DType::Q8_0, dev);
  Tensor* owners[3] = {&ta, &td, &te};
  for (int i = 0; i < 3; ++i) {
    const auto hw = synth_q8(N, K, 300 + i);
    check_status(owners[i]->allocate_hip_bytes(hw.size()));
    upload(*owners[i], hw.data(), hw.size());
  }
  check_status(tb.bind_hip_data(ta.data(), ta.allocated_bytes()));
  check_status(tc.bind_hip_data(static_cast<uint8_t*>(td.data()) + row_bytes * (N / 2),
                                row_bytes * (N / 2)));
  RuntimeContext ctx;
  Tensor* bound[5] = {&ta, &tb, &tc, &td, &te};
  for (int i = 0; i < 5; ++i) check_status(ctx.bind(cw[i], bound[i]));
  std::vector<float> hx(size_t(M) * K);
  for (size_t i = 0; i < hx.size(); ++i) hx[i] = float(int(i * 53 % 97) - 48) * 0.03f;
  Tensor tx("x", Shape({M, K}), DType::Float32, dev);
  check_status(tx.allocate_hip());
  upload(tx, hx.data(), hx.size() * 4);
  check_status(ctx.bind(*x, &tx));
  check_status(ctx.allocate_intermediates(g));
  auto outputs = [&]() {
    std::vector<std::vector<float>> o;
    for (int i = 0; i < 5; ++i) o.push_back(download(ctx.get(outs[i]), size_t(M) * rows[i]));
    return o;
  };
  HipExecutor ex(std::make_shared<HipBackend>(), registry);
  ex.set_fusion(false);
  check_status(ex.compile(g));
  check_status(ex.run(ctx));
  check_hip(hipDeviceSynchronize());
  const auto ref = outputs();
  check_status(ex.tile_weights(ctx, true));
  CHECK(ex.tiled_in_place() == 1u);  // E
  CHECK(ex.tiled_weights() == 3u);   // A (shared with B), C, D
  CHECK(te.storage_layout() == StorageLayout::Q8_0Tiled);
  for (const Tensor* t : {&ta, &tb, &tc, &td}) CHECK(t->storage_layout() == StorageLayout::Raw);
  check_status(ex.run(ctx));
  check_hip(hipDeviceSynchronize());
  CHECK(ex.tiled_launches() == 5u);
  const auto got = outputs();
  for (int i = 0; i < 5; ++i)
    CHECK(std::memcmp(ref[i].data(), got[i].data(), ref[i].size() * 4) == 0);
  std::printf("  PASS test_tile_in_place_skips_viewed_buffers\n");
}

int main() {
  int count = 0;
  check_hip(hipGetDeviceCount(&count));
  CHECK(count > 0);
  check_hip(hipSetDevice(0));
  std::printf("test_hip_q8_0:\n");
  test_low_level_kernels();
  test_executor_linear_and_matmul();
  test_executor_linear_bias_rank3();
  test_executor_embedding_and_stream();
  test_executor_rejects_invalid_inputs();
  test_executor_prefill_linear();
  test_gguf_model_end_to_end();
  test_fused_launchers();
  test_executor_fusion_end_to_end();
  test_executor_tiled_weights();
  test_executor_rows_decode();
  test_workspace_no_regrowth();
  test_executor_reserves_workspace();
  test_executor_reserves_matmul_workspace();
  test_tiled_copy_shape_guard();
  test_loader_dequantizes_q8_0_on_device();
  test_executor_linear_bf16_bias();
  test_executor_tiles_in_place();
  test_tile_in_place_skips_viewed_buffers();
  std::printf("test_hip_q8_0: all passed\n");
  return 0;
}
