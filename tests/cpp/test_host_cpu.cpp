// test_host_cpu.cpp -- host-side checks of the HIP backend that need no GPU.
//
// Graph building and shape rules, registry and executor contracts, and every
// adapter validation path that fails before a kernel is launched (tensors are
// bound to placeholder device addresses that are never dereferenced: each case
// here is rejected by validation first).  Mirrors the reference's runtime
// tests where they apply (tests/test_runtime.cpp:686-756,
// tests/test_cuda_kernels.cpp:1063-1091), and the GGUF reader / weight loader
// on the host (tests/test_gguf_parser.cpp:334-340, 569-592, 855-899).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <memory>
#include <stdexcept>
#include <string>

#include "gguf_writer.h"
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
  DType bias_dtype = DType::Float32;
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
  Tensor tb("b", Shape({c.bias_len}), c.bias_dtype, Device::hip(0));
  Tensor ty("y", Shape({c.M, c.N}), DType::Float32, Device::hip(0));
  CHECK(tx.bind_hip_data(fake_ptr(), size_t(c.M) * c.K * 4).ok());
  CHECK(ty.bind_hip_data(fake_ptr(), size_t(c.M) * c.N * 4).ok());
  const size_t bias_elem = c.bias_dtype == DType::BFloat16 ? 2 : 4;
  CHECK(tb.bind_hip_data(fake_ptr(), size_t(c.bias_len) * bias_elem).ok());
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

  // Bias dtypes: Float32 or BFloat16 (reference cuda_kernel_adapter.cpp:48-59, 204-218).
  c = LinearCase{};
  c.K = 64;
  c.with_bias = true;
  c.bias_dtype = DType::Int32;
  st = run_linear_case(c);
  CHECK(st.code() == ErrorCode::RuntimeError);
  CHECK(contains(st.message(), "bias supports Float32 or BFloat16, got Int32"));
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

// Q8_0 blocks for `n` elements from a seeded generator: q in [-127, 127],
// scale bits cycling through normal and subnormal binary16 values.
static std::vector<uint8_t> q8_blocks(size_t n, uint32_t seed) {
  const size_t blocks = (n + 31) / 32;
  std::vector<uint8_t> out(blocks * 34);
  uint32_t s = seed;
  const uint16_t scales[4] = {0x3800, 0x1c00, 0x0203, 0x2e66};  // 0.5, 2^-8, subnormal, ~0.1
  for (size_t b = 0; b < blocks; ++b) {
    const uint16_t d = scales[b % 4];
    out[b * 34] = uint8_t(d & 0xff);
    out[b * 34 + 1] = uint8_t(d >> 8);
    for (int i = 0; i < 32; ++i) {
      s = s * 1664525u + 1013904223u;
      out[b * 34 + 2 + i] = uint8_t(int8_t(int((s >> 24) % 255) - 127));
    }
  }
  return out;
}

static void test_gguf_parse_and_host_load() {
  // F16 known answers: 1, -0, 65504, smallest subnormal, largest subnormal, +Inf.
  const uint16_t f16[6] = {0x3c00, 0x8000, 0x7bff, 0x0001, 0x03ff, 0x7c00};
  const float f16_want[6] = {1.0f, -0.0f, 65504.0f, 0x1p-24f, 1023.0f * 0x1p-24f, INFINITY};
  std::vector<uint8_t> f16_bytes(64 * 2, 0);
  for (int i = 0; i < 64; ++i) {
    f16_bytes[2 * i] = uint8_t(f16[i % 6] & 0xff);
    f16_bytes[2 * i + 1] = uint8_t(f16[i % 6] >> 8);
  }
  std::vector<uint8_t> f32_bytes(64 * 4);
  for (int i = 0; i < 64; ++i) {
    const float v = 0.25f * float(i) - 3.0f;
    std::memcpy(&f32_bytes[4 * i], &v, 4);
  }
  const auto embd = q8_blocks(6 * 64, 7);

  GgufWriter w;
  w.alignment = 64;
  w.kv_str("general.architecture", "llama");
  w.kv_u32("llama.block_count", 1);
  w.kv_u32("general.alignment", 64);
  w.kv_f32("llama.attention.layer_norm_rms_epsilon", 1e-5f);
  w.kv_str_array("tokenizer.ggml.tokens", {"a", "b", "c", "d", "e"});
  w.tensor("token_embd.weight", {6, 64}, 8, embd);
  w.tensor("blk.0.ffn_norm.weight", {64}, 1, f16_bytes);
  w.tensor("output_norm.weight", {64}, 0, f32_bytes);
  const std::string path = w.write("mle_host_gguf");

  auto file = GGUFParser::parse(path);
  CHECK(file);
  CHECK(file->version == 3 && file->tensor_count == 3 && file->metadata_kv_count == 5);
  CHECK(file->alignment == 64 && file->data_offset % 64 == 0);
  CHECK(get_metadata_or<std::string>(file->metadata, "general.architecture", "") == "llama");
  CHECK(get_metadata_or<uint32_t>(file->metadata, "llama.block_count", 0) == 1);
  CHECK(*get_metadata_array_size(file->metadata, "tokenizer.ggml.tokens") == 5);
  CHECK(get_metadata_array_size(file->metadata, "llama.block_count").error().code() ==
        ErrorCode::TypeError);
  CHECK(get_metadata(file->metadata, "nope").error().code() == ErrorCode::NotFound);
  const GGUFTensorInfo* te = file->find_tensor("token_embd.weight");
  CHECK(te && te->dtype == GgmlDataType::Q8_0);
  CHECK(te->dimensions.size() == 2 && te->dimensions[0] == 6 && te->dimensions[1] == 64);
  CHECK(*te->num_elements() == 384 && *te->bytes() == 12 * 34);
  CHECK(ggml_dtype_size(GgmlDataType::Q8_0) == 34 && ggml_blck_size(GgmlDataType::Q8_0) == 32);
  CHECK(!map_ggml_dtype(GgmlDataType::Q4_0));
  GGUFTensorInfo q4{"x", GgmlDataType::Q4_0, {32}, 0};
  CHECK(q4.bytes().error().code() == ErrorCode::Unsupported);

  // Name mapping (the graph's naming contract).
  CHECK(*WeightLoader::gguf_name_to_value_name("blk.12.ffn_gate.weight") ==
        "layer_12.gate_proj.weight");
  CHECK(*WeightLoader::gguf_name_to_value_name("output.weight") == "lm_head.weight");
  CHECK(WeightLoader::gguf_name_to_value_name("blk.x.ffn_up.weight").error().code() ==
        ErrorCode::InvalidArgument);
  CHECK(WeightLoader::gguf_name_to_value_name("rope_freqs").error().code() ==
        ErrorCode::NotFound);

  // Shared host load: Q8_0 keeps its raw bytes (also for the tied lm_head), F16
  // and F32 become Float32.
  Graph g;
  GraphBuilder gb(g);
  auto tok = gb.constant("tok_embeddings.weight", Shape({6, 64}), DType::Float32);
  auto lm = gb.constant("lm_head.weight", Shape({6, 64}), DType::Float32);
  auto norm = gb.constant("layer_0.ffn_norm.weight", Shape({64}), DType::Float32);
  auto onorm = gb.constant("output_norm.weight", Shape({64}), DType::Float32);
  CHECK(tok && lm && norm && onorm);
  WeightLoader loader(path);
  auto store = loader.load_shared_weights(*file, g);
  CHECK(store);
  CHECK(store->tensor_count() == 3 && store->alias_count() == 4);
  CHECK(store->total_bytes() == 12 * 34 + 64 * 4 + 64 * 4);
  Tensor* t = store->get("tok_embeddings.weight");
  CHECK(t && t == store->get("lm_head.weight") && t->dtype() == DType::Q8_0);
  CHECK(t->allocated_bytes() == embd.size() &&
        std::memcmp(t->data(), embd.data(), embd.size()) == 0);
  const float* nv = static_cast<const float*>(store->get("layer_0.ffn_norm.weight")->data());
  for (int i = 0; i < 64; ++i) {
    const float want = f16_want[i % 6];
    CHECK(std::memcmp(&nv[i], &want, 4) == 0);
  }
  const float* ov = static_cast<const float*>(store->get("output_norm.weight")->data());
  CHECK(std::memcmp(ov, f32_bytes.data(), f32_bytes.size()) == 0);
  RuntimeContext ctx;
  CHECK(store->bind(g, ctx).ok() && ctx.get(*tok) == t && ctx.get(*lm) == t);

  // Q8_0 dequantisation: value = (float)q * d.
  std::vector<float> deq(384);
  CHECK(WeightLoader::dequantize_to_f32(GgmlDataType::Q8_0, embd.data(), deq.data(), 384).ok());
  for (int i = 0; i < 384; ++i) {
    const uint8_t* blk = embd.data() + (i / 32) * 34;
    const uint16_t bits = uint16_t(blk[0] | (blk[1] << 8));
    float d;
    if ((bits & 0x7c00) == 0) d = float(bits & 0x3ff) * 0x1p-24f;
    else d = std::ldexp(float((bits & 0x3ff) | 0x400), int((bits >> 10) & 0x1f) - 25);
    CHECK(deq[i] == float(int8_t(blk[2 + i % 32])) * d);
  }

  // load_weights into tensors bound beforehand; a too-small tensor is rejected.
  {
    RuntimeContext c2;
    Tensor small("tok_embeddings.weight", Shape({6, 64}), DType::Q8_0);
    CHECK(small.allocate_cpu_bytes(100).ok());
    CHECK(c2.bind(*tok, &small).ok());
    const Status st = loader.load_weights(*file, g, c2);
    CHECK(st.code() == ErrorCode::OutOfRange && contains(st.message(), "too small"));
  }

  // Error paths.
  CHECK(GGUFParser::parse(path + ".missing").error().code() == ErrorCode::IOError);
  {
    GgufWriter bad = w;
    bad.magic = "GGUX";
    auto r = GGUFParser::parse(bad.write("mle_bad_magic"));
    CHECK(r.error().code() == ErrorCode::InvalidArgument && contains(r.error().message(), "magic"));
  }
  {
    GgufWriter bad = w;
    bad.version = 2;
    CHECK(GGUFParser::parse(bad.write("mle_bad_version")).error().code() == ErrorCode::Unsupported);
  }
  {
    GgufWriter bad;
    bad.tensor("blk.0.ffn_up.weight", {4, 0}, 8, {});
    CHECK(GGUFParser::parse(bad.write("mle_zero_dim")).error().code() ==
          ErrorCode::InvalidArgument);
  }
  {
    auto bytes = w.bytes();
    bytes.resize(40);  // cut inside the metadata
    const std::string cut = path + ".cut";
    std::FILE* f = std::fopen(cut.c_str(), "wb");
    CHECK(f && std::fwrite(bytes.data(), 1, bytes.size(), f) == bytes.size());
    std::fclose(f);
    CHECK(GGUFParser::parse(cut).error().code() == ErrorCode::IOError);
    std::remove(cut.c_str());
  }
  {
    std::vector<uint8_t> buf(16);
    CHECK(GGUFParser::read_tensor_data(path, file->data_offset, 1u << 20, buf.data(), 16).code() ==
          ErrorCode::OutOfRange);
  }
  std::remove(path.c_str());
  std::printf("  PASS test_gguf_parse_and_host_load\n");
}

static void test_executor_fusion_plan() {
  // x -> {gate, up} -> SwiGLU -> down, and q / k / v on x: one fused SwiGLU
  // group and one multi-output group; with the gate value also a graph output
  // the SwiGLU cannot fuse and the five sibling Linears group as 3 + 2.
  for (int variant = 0; variant < 3; ++variant) {
    Graph g;
    GraphBuilder gb(g);
    const Device dev = Device::hip(0);
    auto x = gb.input("x", Shape({4, 64}), DType::Float32, dev);
    auto wg = gb.constant("wg", Shape({96, 64}), DType::Float32, dev);
    auto wu = gb.constant("wu", Shape({96, 64}), DType::Float32, dev);
    auto wd = gb.constant("wd", Shape({64, 96}), DType::Float32, dev);
    auto wq = gb.constant("wq", Shape({64, 64}), DType::Float32, dev);
    auto wk = gb.constant("wk", Shape({32, 64}), DType::Float32, dev);
    auto wv = gb.constant("wv", Shape({32, 64}), DType::Float32, dev);
    CHECK(x && wg && wu && wd && wq && wk && wv);
    auto gate = gb.linear(*x, *wg, std::nullopt, "gate");
    auto up = gb.linear(*x, *wu, std::nullopt, "up");
    CHECK(gate && up);
    auto act = gb.swiglu(*gate, *up, "swiglu");
    CHECK(act);
    auto down = gb.linear(*act, *wd, std::nullopt, "down");
    auto q = gb.linear(*x, *wq, std::nullopt, "q");
    auto k = gb.linear(*x, *wk, std::nullopt, "k");
    auto v = gb.linear(*x, *wv, std::nullopt, "v");
    CHECK(down && q && k && v);
    CHECK(gb.output(*down, "o1") && gb.output(*q, "o2") && gb.output(*k, "o3") &&
          gb.output(*v, "o4"));
    if (variant == 1) CHECK(gb.output(*gate, "o5"));
    KernelRegistry reg;
    register_hip_kernels(reg);
    HipExecutor ex(std::make_shared<HipBackend>(), reg);
    if (variant == 2) ex.set_fusion(false);
    CHECK(ex.compile(g).ok());
    if (variant == 0) CHECK(ex.fused_groups() == 2);
    if (variant == 1) CHECK(ex.fused_groups() == 2);  // {gate, up, q}, {k, v}: no SwiGLU group
    if (variant == 2) CHECK(ex.fused_groups() == 0);
  }
  {  // shape rule of the SwiGLU builder
    Graph g;
    GraphBuilder gb(g);
    auto a = gb.input("a", Shape({2, 8}), DType::Float32);
    auto b = gb.input("b", Shape({2, 9}), DType::Float32);
    CHECK(a && b);
    auto r = gb.swiglu(*a, *b, "bad");
    CHECK(!r && r.error().code() == ErrorCode::ShapeMismatch);
  }
  std::printf("  PASS test_executor_fusion_plan\n");
}

int main() {
  std::printf("test_host_cpu:\n");
  test_core_types();
  test_graph_and_shapes();
  test_registry_and_executor_contract();
  test_linear_validation();
  test_matmul_and_embedding_validation();
  test_gguf_parse_and_host_load();
  test_executor_fusion_plan();
  std::printf("test_host_cpu: all passed\n");
  return 0;
}
