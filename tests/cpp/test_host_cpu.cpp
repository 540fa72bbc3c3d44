// test_host_cpu.cpp -- host-side checks of the HIP backend that need no GPU.
//
// Graph building and shape rules, registry and executor contracts, and every
// adapter validation path that fails before a kernel is launched (tensors are
// bound to placeholder device addresses that are never dereferenced: each case
// here is rejected by validation first).  Mirrors the reference's runtime
// tests where they apply (tests/test_runtime.cpp:686-756,
// tests/test_cuda_kernels.cpp:1063-1091).
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <stdexcept>
#include <string>

#include "minillm_hip/runtime.h"

using namespace minillm;

#define CHECK(cond)                                                              \
  do {                                                                           \
    if (!(cond)) {                                                               \
      std::fprintf(stderr, "CHECK failed at %s:%d: %s\n", __FILE__, __LINE__, #cond); \
      std::abort();                                                              \
    }                                                                            \
  } while (0)

static bool contains(std::string_view s, std::string_view sub) {
  return s.find(sub) != std::string_view::npos;
}

// Placeholder device address: validation must reject every use before launch.
static void* fake_ptr() { return reinterpret_cast<void*>(uintptr_t{0x10000}); }

static void test_core_types() {
  CHECK(Status::make_ok().ok());
  const Status st = Status::unsupported("x");
  CHECK(st.code() == ErrorCode::Unsupported && st.to_string() == "Unsupported: x");
  CHECK(!dtype_size(DType::Q8_0));
  CHECK(*dtype_size(DType::Float32) == 4);
  CHECK(q8_0_bytes(32) == 34 && q8_0_bytes(33) == 68 && q8_0_bytes(4096 * 4096) == 4096 * 128 * 34);
  CHECK(*Shape({2, 3, 4}).numel() == 24);
  CHECK(!Shape({2, -1}).numel());
  bool threw = false;
  try {
    Shape bad({2, 0});
  } catch (const std::invalid_argument&) {
    threw = true;
  }
  CHECK(threw);
  CHECK(Device::hip(1).to_string() == "hip:1");
  Tensor t("w", Shape({3, 32}), DType::Q8_0, Device::hip(0));
  CHECK(!t.allocate_cpu().ok());  // Q8_0 has no element size: use *_bytes
  CHECK(t.allocate_cpu_bytes(q8_0_bytes(96)).ok() && t.allocated_bytes() == 102);
  CHECK(t.device().type == DeviceType::CPU);
  Tensor h("h", Shape({4, 32}), DType::Q8_0, Device::hip(0));
  CHECK(!h.bind_hip_data(fake_ptr(), 135).ok());  // needs 136 bytes
  CHECK(h.bind_hip_data(fake_ptr(), 136).ok() && h.device().type == DeviceType::HIP);
  std::printf("  PASS test_core_types\n");
}

static void test_graph_and_shapes() {
  Graph g;
  GraphBuilder gb(g);
  auto ids = gb.input("ids", Shape({2, 5}), DType::Int32, Device::hip(0));
  auto emb = gb.constant("emb", Shape({100, 64}), DType::Float32, Device::hip(0));
  auto w = gb.constant("w", Shape({96, 64}), DType::Float32, Device::hip(0));
  auto b = gb.constant("b", Shape({96}), DType::Float32, Device::hip(0));
  auto mm = gb.constant("mm", Shape({96, 32}), DType::Float32, Device::hip(0));
  CHECK(ids && emb && w && b && mm);
  auto e = gb.embedding(*ids, *emb, "tok");
  CHECK(e);
  CHECK((*g.value(*e))->shape == Shape({2, 5, 64}));
  auto y = gb.linear(*e, *w, *b, "proj");
  CHECK(y);
  CHECK((*g.value(*y))->shape == Shape({2, 5, 96}));
  // logical dtype / device come from the weight Value
  CHECK((*g.value(*y))->dtype == DType::Float32 && (*g.value(*y))->device == Device::hip(0));
  auto bad_bias = gb.constant("bb", Shape({95}), DType::Float32, Device::hip(0));
  auto y2 = gb.linear(*e, *w, *bad_bias, "bad");
  CHECK(!y2 && y2.error().code() == ErrorCode::ShapeMismatch);
  auto bad_w = gb.constant("bw", Shape({96, 63}), DType::Float32);
  CHECK(!gb.linear(*e, *bad_w, std::nullopt, "bad2"));
  auto a2 = gb.input("a2", Shape({4, 96}), DType::Float32, Device::hip(0));
  auto z = gb.matmul(*a2, *mm, "mm");
  CHECK(z && (*g.value(*z))->shape == Shape({4, 32}));
  CHECK(!gb.matmul(*a2, *emb, "bad_mm"));  // [4,96] x [100,64]: inner dims differ
  auto out = gb.output(*y, "out");
  CHECK(out && (*g.value(*y))->kind == ValueKind::Output);
  auto order = g.topological_sort();
  CHECK(order && order->size() == g.nodes().size());
  CHECK(g.nodes()[(*order)[0].value].op_type() == OpType::Embedding ||
        g.nodes()[(*order)[0].value].op_type() == OpType::MatMul);
  std::printf("  PASS test_graph_and_shapes\n");
}

static void test_registry_and_executor_contract() {
  KernelRegistry reg;
  CHECK(!reg.has(DeviceType::HIP, OpType::Linear));
  register_hip_kernels(reg);
  CHECK(reg.has(DeviceType::HIP, OpType::Linear) && reg.has(DeviceType::HIP, OpType::MatMul) &&
        reg.has(DeviceType::HIP, OpType::Embedding));
  CHECK(!reg.has(DeviceType::HIP, OpType::Add) && !reg.has(DeviceType::CUDA, OpType::Linear));
  auto f = reg.find(DeviceType::HIP, OpType::Add);
  CHECK(!f && f.error().code() == ErrorCode::NotImplemented &&
        contains(f.error().message(), "no kernel registered for op Add"));

  auto backend = std::make_shared<HipBackend>();
  CHECK(backend->device_type() == DeviceType::HIP && backend->name() == "HipBackend");
  CHECK(backend->supports(OpType::Linear) && !backend->supports(OpType::Softmax));

  // an op outside the Q8_0 path is rejected at compile time
  Graph g;
  auto a = g.add_value("a", Shape({4}), DType::Float32, Device::hip(0), ValueKind::Input);
  auto c = g.add_value("c", Shape({4}), DType::Float32, Device::hip(0), ValueKind::Intermediate);
  CHECK(g.add_node(OpType::Add, "add", {*a, *a}, {*c}));
  HipExecutor ex(backend, reg);
  const Status st = ex.compile(g);
  CHECK(st.code() == ErrorCode::Unsupported &&
        contains(st.message(), "backend HipBackend does not support op Add"));

  // a supported op without a registered kernel
  Graph g2;
  GraphBuilder gb(g2);
  auto x = gb.input("x", Shape({1, 32}), DType::Float32, Device::hip(0));
  auto w = gb.constant("w", Shape({2, 32}), DType::Float32, Device::hip(0));
  CHECK(gb.linear(*x, *w, std::nullopt, "lin"));
  KernelRegistry empty;
  HipExecutor ex2(backend, empty);
  const Status st2 = ex2.compile(g2);
  CHECK(st2.code() == ErrorCode::NotImplemented &&
        contains(st2.message(), "no HIP kernel registered for op Linear"));
  RuntimeContext ctx;
  CHECK(ex2.run(ctx).code() == ErrorCode::RuntimeError);  // not compiled

  // a dangling ValueId fails validation
  Graph g3;
  auto v = g3.add_value("v", Shape({1}), DType::Float32, Device::hip(0), ValueKind::Input);
  CHECK(g3.add_node(OpType::Linear, "dangling", {*v, ValueId{7}}, {ValueId{8}}));
  CHECK(g3.validate().code() == ErrorCode::InvalidArgument);
  std::printf("  PASS test_registry_and_executor_contract\n");
}

// Builds x[M,K] . W[N,K]^T with every tensor bound to placeholder device storage,
// runs the executor, returns its status (validation must fail before launch).
struct LinearCase {
  int M = 1, N = 2, K = 31;
  DType w_dtype = DType::Q8_0;
  Device w_device = Device::hip(0);
  bool with_bias = false;
  int64_t bias_len = 2;
};

static Status run_linear_case(const LinearCase& c) {
  Graph g;
  GraphBuilder gb(g);
  auto x = gb.input("x", Shape({c.M, c.K}), DType::Float32, Device::hip(0));
  auto w = gb.constant("w", Shape({c.N, c.K}), DType::Float32, Device::hip(0));
  std::optional<ValueId> bias;
  if (c.with_bias) bias = *gb.constant("b", Shape({c.N}), DType::Float32, Device::hip(0));
  auto y = gb.linear(*x, *w, bias, "linear_q8");
  CHECK(y);
  Tensor tx("x", Shape({c.M, c.K}), DType::Float32, Device::hip(0));
  Tensor tw("w", Shape({c.N, c.K}), c.w_dtype, c.w_device);
  Tensor tb("b", Shape({c.bias_len}), DType::Float32, Device::hip(0));
  Tensor ty("y", Shape({c.M, c.N}), DType::Float32, Device::hip(0));
  CHECK(tx.bind_hip_data(fake_ptr(), size_t(c.M) * c.K * 4).ok());
  CHECK(ty.bind_hip_data(fake_ptr(), size_t(c.M) * c.N * 4).ok());
  CHECK(tb.bind_hip_data(fake_ptr(), size_t(c.bias_len) * 4).ok());
  const size_t wbytes = c.w_dtype == DType::Q8_0 ? q8_0_bytes(size_t(c.N) * c.K)
                                                 : size_t(c.N) * c.K * 4;
  if (c.w_device.type == DeviceType::HIP) {
    CHECK(tw.bind_hip_data(fake_ptr(), wbytes).ok());
  } else {
    CHECK(tw.allocate_cpu_bytes(wbytes).ok());
  }
  RuntimeContext ctx;
  CHECK(ctx.bind(*x, &tx).ok() && ctx.bind(*w, &tw).ok() && ctx.bind(*y, &ty).ok());
  if (bias) CHECK(ctx.bind(*bias, &tb).ok());
  KernelRegistry reg;
  register_hip_kernels(reg);
  HipExecutor ex(std::make_shared<HipBackend>(), reg);
  CHECK(ex.compile(g).ok());
  return ex.run(ctx);
}

static void test_linear_validation() {
  LinearCase c;  // K = 31
  Status st = run_linear_case(c);
  CHECK(st.code() == ErrorCode::RuntimeError);
  CHECK(contains(st.message(), "Q8_0") && contains(st.message(), "32"));
  CHECK(contains(st.message(), "HIP kernel Linear failed for node #0 (linear_q8)"));

  c = LinearCase{};
  c.K = 64;
  c.w_dtype = DType::Float32;
  st = run_linear_case(c);
  CHECK(contains(st.message(), "supports Q8_0 weights on the HIP backend, got Float32"));

  c = LinearCase{};
  c.K = 64;
  c.w_device = Device::cpu();
  st = run_linear_case(c);
  CHECK(contains(st.message(), "weight must be a HIP tensor, got cpu:0"));

  c = LinearCase{};
  c.K = 64;
  c.with_bias = true;
  c.bias_len = 3;  // tensor bound with a shape that does not match N = 2
  st = run_linear_case(c);
  CHECK(contains(st.message(), "Linear bias shape must match output features"));
  std::printf("  PASS test_linear_validation\n");
}

static void test_matmul_and_embedding_validation() {
  KernelRegistry reg;
  register_hip_kernels(reg);
  {
    Graph g;
    GraphBuilder gb(g);
    auto a = gb.input("a", Shape({2, 32}), DType::Float32, Device::hip(0));
    auto b = gb.constant("b", Shape({32, 48}), DType::Float32, Device::hip(0));
    auto y = gb.matmul(*a, *b, "mm_bad_n");
    CHECK(y);
    Tensor ta("a", Shape({2, 32}), DType::Float32, Device::hip(0));
    Tensor tb("b", Shape({32, 48}), DType::Q8_0, Device::hip(0));
    Tensor ty("y", Shape({2, 48}), DType::Float32, Device::hip(0));
    CHECK(ta.bind_hip_data(fake_ptr(), 256).ok() && ty.bind_hip_data(fake_ptr(), 384).ok());
    CHECK(tb.bind_hip_data(fake_ptr(), q8_0_bytes(32 * 48)).ok());
    RuntimeContext ctx;
    CHECK(ctx.bind(*a, &ta).ok() && ctx.bind(*b, &tb).ok() && ctx.bind(*y, &ty).ok());
    HipExecutor ex(std::make_shared<HipBackend>(), reg);
    CHECK(ex.compile(g).ok());
    const Status st = ex.run(ctx);
    CHECK(contains(st.message(), "matmul output dimension Q8_0 weights require the packed "
                                 "dimension to be a multiple of 32, got 48"));
  }
  {
    Graph g;
    GraphBuilder gb(g);
    auto ids = gb.input("ids", Shape({3}), DType::Int32, Device::hip(0));
    auto w = gb.constant("w", Shape({10, 32}), DType::Float32, Device::hip(0));
    auto y = gb.embedding(*ids, *w, "emb");
    CHECK(y);
    Tensor tids("ids", Shape({3}), DType::Int64, Device::hip(0));
    Tensor tw("w", Shape({10, 32}), DType::Q8_0, Device::hip(0));
    Tensor ty("y", Shape({3, 32}), DType::Float32, Device::hip(0));
    CHECK(tids.bind_hip_data(fake_ptr(), 24).ok() && ty.bind_hip_data(fake_ptr(), 384).ok());
    CHECK(tw.bind_hip_data(fake_ptr(), q8_0_bytes(320)).ok());
    RuntimeContext ctx;
    CHECK(ctx.bind(*ids, &tids).ok() && ctx.bind(*w, &tw).ok() && ctx.bind(*y, &ty).ok());
    HipExecutor ex(std::make_shared<HipBackend>(), reg);
    CHECK(ex.compile(g).ok());
    const Status st = ex.run(ctx);
    CHECK(contains(st.message(), "input_ids only supports Int32, got Int64"));
  }
  std::printf("  PASS test_matmul_and_embedding_validation\n");
}

int main() {
  std::printf("test_host_cpu:\n");
  test_core_types();
  test_graph_and_shapes();
  test_registry_and_executor_contract();
  test_linear_validation();
  test_matmul_and_embedding_validation();
  std::printf("test_host_cpu: all passed\n");
  return 0;
}
