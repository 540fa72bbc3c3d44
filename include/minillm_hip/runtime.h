// runtime.h -- kernel registry, backends, runtime context and executors of the
// MiniLLMEngine host API, with the HIP backend and executor.
//
// Same plugin contract as the reference runtime:
//   KernelFn = Status(*)(const Node&, RuntimeContext&)    (kernel_registry.h:18)
//   KernelRegistry::register_kernel/find/has              (kernel_registry.h:20-35)
//   Backend(DeviceType, name)::supports(OpType)           (backend.h:10-21, backend.cpp:9-30)
//   Executor::compile(const Graph&) / run(RuntimeContext&) (executor.h:16-51,
//                                                           executor.cpp:86-142)
//   RuntimeContext::bind/emplace/get/allocate_intermediates (runtime_context.h:19-97)
// HipBackend and HipExecutor stand where CudaBackend and CudaExecutor stand.
// The executor enqueues every kernel on its HIP stream (carried to the kernels
// through RuntimeContext::hip_stream()) and never synchronises: as with the
// reference device executor, the caller synchronises before reading outputs.
#pragma once

#include <hip/hip_runtime_api.h>

#include <map>
#include <memory>
#include <string_view>
#include <unordered_map>
#include <utility>
#include <vector>

#include "minillm_hip/core.h"
#include "minillm_hip/graph.h"

namespace minillm {

class RuntimeContext;

using KernelFn = Status (*)(const Node&, RuntimeContext&);

class KernelRegistry {
 public:
  void register_kernel(DeviceType device, OpType op, KernelFn fn);
  expected<KernelFn, Status> find(DeviceType device, OpType op) const;
  bool has(DeviceType device, OpType op) const;

 private:
  std::map<std::pair<int, int>, KernelFn> kernels_;
};

class Backend {
 public:
  Backend(DeviceType dt, std::string_view n);
  virtual ~Backend() = default;
  DeviceType device_type() const;
  // Ops the backend can run (graph plumbing ops included).
  virtual bool supports(OpType op) const;
  std::string_view name() const;

 private:
  DeviceType device_type_;
  std::string_view name_;
};

// MI355X backend: the ops of the Q8_0 path (Embedding, MatMul, Linear) plus
// Output.  Graphs using other ops are rejected by HipExecutor::compile.
class HipBackend final : public Backend {
 public:
  HipBackend() : Backend(DeviceType::HIP, "HipBackend") {}
  bool supports(OpType op) const override;
};

// ValueId -> Tensor* binding for one execution.
class RuntimeContext {
 public:
  RuntimeContext() = default;
  ~RuntimeContext();
  RuntimeContext(const RuntimeContext&) = delete;
  RuntimeContext& operator=(const RuntimeContext&) = delete;

  Status bind(ValueId id, Tensor* tensor);
  Status emplace(ValueId id, std::unique_ptr<Tensor> tensor);
  Tensor* get(ValueId id) const;
  // Allocates every non-Input, non-Constant value that has no binding yet, on
  // the value's device (HIP values: hipMalloc'd device storage).
  Status allocate_intermediates(const Graph& graph);
  // No KV cache on this path; kept for executor parity (reference
  // runtime_context.cpp:222-243).
  Status advance_kv_cache_step();

  hipStream_t hip_stream() const { return hip_stream_; }
  void set_hip_stream(hipStream_t s) { hip_stream_ = s; }

 private:
  std::unordered_map<size_t, Tensor*> bindings_;
  std::vector<std::unique_ptr<Tensor>> owned_;
  hipStream_t hip_stream_{nullptr};
};

namespace detail {
// Raw Q8_0 weight buffer (device pointer) -> its copy in 16-row tiles, with the
// shape it was made for.  A node whose bound weight has another shape (a buffer
// freed and its address reused, or one buffer viewed with two shapes) does not
// match and runs on the raw bytes.
struct TiledCopy {
  const uint8_t* data = nullptr;
  int64_t N = 0, K = 0;
  size_t bytes = 0;
};
using TiledWeights = std::unordered_map<const void*, TiledCopy>;
}  // namespace detail

class Executor {
 public:
  virtual ~Executor() = default;
  virtual Status compile(const Graph& graph) = 0;
  virtual Status run(RuntimeContext& ctx) = 0;
};

class HipExecutor final : public Executor {
 public:
  // `stream` = the HIP stream every kernel is enqueued on (nullptr = default stream).
  HipExecutor(std::shared_ptr<Backend> backend, KernelRegistry& registry,
              hipStream_t stream = nullptr);

  Status compile(const Graph& graph) override;
  Status run(RuntimeContext& ctx) override;
  hipStream_t stream() const { return stream_; }

  // Split-K workspace of the Q8_0 Linear kernels (no counterpart in the
  // reference, whose CUDA kernels use none): reserves the executor stream's
  // workspace for the largest Linear launch of the compiled plan (fused groups
  // included, raw or tiled weights), with shapes from the tensors bound in
  // `ctx` where given, else from the graph's static value shapes.  compile()
  // (on a machine with a HIP device) and tile_weights() call it, so run()
  // allocates and synchronises nothing; a bound tensor larger than the graph's
  // shapes makes its launch grow the workspace once.
  Status reserve_workspace(const RuntimeContext* ctx = nullptr);
  // Bytes / counters of the last reservation (0 / 0 before any).
  size_t workspace_bytes() const { return ws_bytes_; }
  size_t workspace_counters() const { return ws_counters_; }

  // Linear epilogue fusion (on by default; takes effect at the next compile):
  //  * Linear(gate) + Linear(up) + SwiGLU, where both Linears read one input,
  //    have no bias and feed only the SwiGLU, run as one fused launch at the
  //    SwiGLU's place (the two Linear outputs are then not written);
  //  * 2-3 other Linears reading one input (q/k/v) run as one multi-output
  //    launch at the first one's place.
  // A group whose bound tensors do not fit the fused kernels (e.g. non-Q8_0
  // weights) runs node by node.  Off: one launch per node in topological
  // order, exactly the reference executor's schedule.
  void set_fusion(bool on) { fusion_ = on; }
  bool fusion() const { return fusion_; }
  // Fused groups in the compiled plan, and fused launches made by the last run.
  size_t fused_groups() const;
  size_t fused_launches() const { return fused_launches_; }

  // Weights in Q8_0 16-row tiles (no counterpart in the reference executor; a
  // loader step): makes a tiled copy (mle_q8_0_tile, on this executor's stream)
  // of every Q8_0 Linear weight of the compiled graph bound in `ctx` on a HIP
  // device, once per weight buffer.  Later runs give those Linears (and their
  // fused groups) the tiled copy while the same buffer stays bound; a node
  // whose bound weight buffer has no copy runs on the raw bytes.  The copies
  // live until release_tiled_weights() or the executor's destruction; call
  // again after overwriting a bound weight in place.  Memory: one more copy of
  // each Linear weight (the raw buffer stays with the caller).
  //
  // release_raw: a weight whose tensor owns its device storage
  // (allocate_hip*), whose buffer the graph reads only as Linear weights and
  // whose bytes no other tensor bound in `ctx` views (bind_hip_data on the same
  // or an overlapping range) is re-tiled in place instead: the tensor adopts the tiled buffer
  // (StorageLayout::Q8_0Tiled) and its raw bytes are freed after a synchronise
  // of this stream, so the weight costs no extra memory.  Such a tensor stays
  // tiled for good: any executor's Linear and Embedding kernels run it on the
  // tiled entry points, MatMul rejects it, and it must not be refilled with
  // raw bytes (reallocate it first).  Other weights get copies as above; an
  // Embedding table shared with a Linear (a tied lm_head) keeps its raw bytes,
  // whose gather is twice as fast as the gather from tiles.
  Status tile_weights(RuntimeContext& ctx, bool release_raw = false);
  void release_tiled_weights();
  size_t tiled_weights() const { return tiled_.size(); }
  // Weights the last tile_weights re-tiled in place.
  size_t tiled_in_place() const { return in_place_; }
  // Linear launches of the last run on 16-row tiles (a copy or in place).
  size_t tiled_launches() const { return tiled_launches_; }
  ~HipExecutor() override;

 private:
  struct Step {
    enum Kind { kNode, kSwiGLU, kMulti } kind;
    std::vector<NodeId> nodes;  // kSwiGLU: gate, up, swiglu; kMulti: 2-3 Linears
  };
  Status run_nodes(const std::vector<NodeId>& ids, RuntimeContext& ctx);

  const Graph* graph_{nullptr};
  std::shared_ptr<Backend> backend_;
  KernelRegistry& registry_;
  std::vector<NodeId> execution_order_;
  std::vector<Step> plan_;
  bool fusion_{true};
  size_t fused_launches_{0};
  size_t tiled_launches_{0};
  hipStream_t stream_;
  detail::TiledWeights tiled_;  // raw buffer -> tiled copy
  std::vector<void*> tiled_bufs_;
  size_t in_place_{0};
  size_t ws_bytes_{0}, ws_counters_{0};
  bool ws_pending_{false};  // a reservation compile() could not make (no HIP device)
};

// Registers the HIP Q8_0 kernels (Embedding, Linear, MatMul) under
// DeviceType::HIP; stands where register_cuda_kernels stands
// (reference src/runtime/kernels/cuda_kernel_adapter.cpp:700-715).
void register_hip_kernels(KernelRegistry& registry);

// Low-level launchers (device pointers, async on `stream`), the counterparts of
// minillm::cuda::sgemm_nt / sgemm / embedding for Q8_0 weights
// (reference include/minillm/runtime/kernels/cuda_kernels.h:13,16,37-38).
namespace hip {
Status sgemm_nt(const float* A, const uint8_t* B_q8_0, float* C, int M, int N, int K,
                const float* bias = nullptr, hipStream_t stream = nullptr);
// Linear with a BFloat16 bias (mle_q8_0_linear_bias_bf16): the reference's
// sgemm_nt + add_bias(float*, const uint16_t*, ...) for a BF16 bias
// (cuda_kernel_adapter.cpp:204-218), fused.
Status sgemm_nt_bias_bf16(const float* A, const uint8_t* B_q8_0, float* C, int M, int N, int K,
                          const uint16_t* bias_bf16, hipStream_t stream = nullptr);
Status sgemm_nt_tiled_bias_bf16(const float* A, const uint8_t* B_tiled, float* C, int M, int N,
                                int K, const uint16_t* bias_bf16, hipStream_t stream = nullptr);
Status sgemm(const float* A, const uint8_t* B_q8_0, float* C, int M, int N, int K,
             hipStream_t stream = nullptr);
Status embedding(const uint8_t* weight_q8_0, const int* ids, float* out, int seq_len,
                 int vocab_size, int hidden, hipStream_t stream = nullptr);
// The same gather from a table in 16-row tiles (mle_q8_0_embedding_tiled).
Status embedding_tiled(const uint8_t* weight_tiled, const int* ids, float* out, int seq_len,
                       int vocab_size, int hidden, hipStream_t stream = nullptr);
// WeightLoader::dequantize_to_f32's Q8_0 case on the device (mle_q8_0_dequantize;
// reference src/io/gguf_weight_loader.cpp:446-463): out[e] = q * d, e < n.
Status dequantize_q8_0(const uint8_t* src_q8_0, float* out, int64_t n,
                       hipStream_t stream = nullptr);

// Fused launchers with no counterpart among the reference's kernels (see
// mle_q8_0.h): y = silu(x.Wg^T) * (x.Wu^T) in place of Linear + Linear +
// SwiGLU (transformer_graph_builder.cpp:261-268); up to three Linears on one
// input (q/k/v, :214-221); the greedy argmax of logits rows on the device
// (generate_cuda.cpp:305-314 copies the whole row to the host instead).
Status linear_swiglu(const float* x, const uint8_t* w_gate_q8_0, const uint8_t* w_up_q8_0,
                     float* y, int M, int N, int K, hipStream_t stream = nullptr);
Status linear_multi(const float* x, int count, const uint8_t* const* w_q8_0,
                    const float* const* bias, float* const* y, const int* N, int M, int K,
                    hipStream_t stream = nullptr);
// Weights in Q8_0 16-row tiles (mle_q8_0_tile / mle_q8_0_*_tiled; no
// counterpart in the reference).
size_t q8_0_tiled_bytes(int N, int K);
Status tile_q8_0(const uint8_t* w_q8_0, uint8_t* w_tiled, int N, int K,
                 hipStream_t stream = nullptr);
Status sgemm_nt_tiled(const float* A, const uint8_t* B_tiled, float* C, int M, int N, int K,
                      const float* bias = nullptr, hipStream_t stream = nullptr);
Status linear_swiglu_tiled(const float* x, const uint8_t* w_gate_tiled,
                           const uint8_t* w_up_tiled, float* y, int M, int N, int K,
                           hipStream_t stream = nullptr);
Status linear_multi_tiled(const float* x, int count, const uint8_t* const* w_tiled,
                          const float* const* bias, float* const* y, const int* N, int M,
                          int K, hipStream_t stream = nullptr);
Status argmax(const float* logits, int rows, int n, int32_t* idx, float* val = nullptr,
              hipStream_t stream = nullptr);
// Sampler::get_top_tokens (sampler.cpp:141-197) on the device: ids / probs
// [rows][min(top_n, n)] of each logits row, largest probability first.
Status top_tokens(const float* logits, int rows, int n, int top_n, float temperature,
                  int32_t* ids, float* probs, hipStream_t stream = nullptr);
}  // namespace hip

}  // namespace minillm
