// runtime.cpp -- registry, backends, runtime context, HIP executor
// (see include/minillm_hip/runtime.h).
#include "minillm_hip/runtime.h"

namespace minillm {

// ---------------------------------------------------------------- registry
void KernelRegistry::register_kernel(DeviceType device, OpType op, KernelFn fn) {
  kernels_[{static_cast<int>(device), static_cast<int>(op)}] = fn;
}

expected<KernelFn, Status> KernelRegistry::find(DeviceType device, OpType op) const {
  auto it = kernels_.find({static_cast<int>(device), static_cast<int>(op)});
  if (it != kernels_.end()) return it->second;
  return unexpected(
      Status::not_implemented("no kernel registered for op " + std::string(op_type_name(op))));
}

bool KernelRegistry::has(DeviceType device, OpType op) const {
  return kernels_.count({static_cast<int>(device), static_cast<int>(op)}) != 0;
}

// ---------------------------------------------------------------- backends
Backend::Backend(DeviceType dt, std::string_view n) : device_type_(dt), name_(n) {}
DeviceType Backend::device_type() const { return device_type_; }
std::string_view Backend::name() const { return name_; }

// The reference backend's op list (src/runtime/backend.cpp:9-30).
bool Backend::supports(OpType op) const {
  switch (op) {
    case OpType::Embedding:
    case OpType::MatMul:
    case OpType::Linear:
    case OpType::Add:
    case OpType::Mul:
    case OpType::RMSNorm:
    case OpType::SiLU:
    case OpType::SwiGLU:
    case OpType::RoPE:
    case OpType::Attention:
    case OpType::QKNorm:
    case OpType::Softmax:
    case OpType::Reshape:
    case OpType::Transpose:
    case OpType::Output:
      return true;
    default:
      return false;
  }
}

bool HipBackend::supports(OpType op) const {
  return op == OpType::Embedding || op == OpType::MatMul || op == OpType::Linear ||
         op == OpType::Output;
}

// ---------------------------------------------------------------- context
RuntimeContext::~RuntimeContext() = default;

Status RuntimeContext::bind(ValueId id, Tensor* tensor) {
  if (!tensor)
    return Status::invalid_argument("cannot bind null Tensor to ValueId %" +
                                    std::to_string(id.value));
  bindings_[id.value] = tensor;
  return Status::make_ok();
}

Status RuntimeContext::emplace(ValueId id, std::unique_ptr<Tensor> tensor) {
  if (!tensor)
    return Status::invalid_argument("cannot emplace null Tensor for ValueId %" +
                                    std::to_string(id.value));
  bindings_[id.value] = tensor.get();
  owned_.push_back(std::move(tensor));
  return Status::make_ok();
}

Tensor* RuntimeContext::get(ValueId id) const {
  auto it = bindings_.find(id.value);
  return it == bindings_.end() ? nullptr : it->second;
}

Status RuntimeContext::allocate_intermediates(const Graph& graph) {
  for (const Value& v : graph.values()) {
    if (v.kind == ValueKind::Input || v.kind == ValueKind::Constant) continue;
    if (bindings_.count(v.id.value)) continue;
    if (v.shape.has_dynamic_dim())
      return Status::invalid_argument("cannot allocate intermediate with dynamic shape: " +
                                      v.name + " " + v.shape.to_string());
    auto t = std::make_unique<Tensor>(v.name, v.shape, v.dtype, v.device);
    if (v.device.type == DeviceType::HIP) {
      TRY(t->allocate_hip());
    } else if (v.device.type == DeviceType::CPU) {
      TRY(t->allocate_cpu());
    } else {
      return Status::unsupported("cannot allocate intermediate " + v.name + " on device " +
                                 v.device.to_string());
    }
    bindings_[v.id.value] = t.get();
    owned_.push_back(std::move(t));
  }
  return Status::make_ok();
}

Status RuntimeContext::advance_kv_cache_step() { return Status::make_ok(); }

// ---------------------------------------------------------------- executor
HipExecutor::HipExecutor(std::shared_ptr<Backend> backend, KernelRegistry& registry,
                         hipStream_t stream)
    : backend_(std::move(backend)), registry_(registry), stream_(stream) {}

Status HipExecutor::compile(const Graph& graph) {
  TRY(graph.validate());
  auto order = graph.topological_sort();
  if (!order) return order.error();
  for (const NodeId& nid : *order) {
    auto nd = graph.node(nid);
    if (!nd) return nd.error();
    const OpType op = (*nd)->op_type();
    if (op == OpType::Input || op == OpType::Constant || op == OpType::Output) continue;
    if (!backend_->supports(op))
      return Status::unsupported("backend " + std::string(backend_->name()) +
                                 " does not support op " + std::string(op_type_name(op)));
    if (!registry_.has(DeviceType::HIP, op))
      return Status::not_implemented("no HIP kernel registered for op " +
                                     std::string(op_type_name(op)));
  }
  graph_ = &graph;
  execution_order_ = std::move(*order);
  return Status::make_ok();
}

Status HipExecutor::run(RuntimeContext& ctx) {
  if (!graph_) return Status::runtime_error("executor not compiled");
  ctx.set_hip_stream(stream_);
  for (const NodeId& nid : execution_order_) {
    auto nd = graph_->node(nid);
    if (!nd) return nd.error();
    const OpType op = (*nd)->op_type();
    if (op == OpType::Input || op == OpType::Constant || op == OpType::Output) continue;
    auto kernel = registry_.find(DeviceType::HIP, op);
    if (!kernel) return kernel.error();
    const Status st = (*kernel)(**nd, ctx);
    if (!st.ok())
      return Status::runtime_error("HIP kernel " + std::string(op_type_name(op)) +
                                   " failed for node #" + std::to_string(nid.value) + " (" +
                                   std::string((*nd)->name()) + "): " + st.to_string());
  }
  const Status st = ctx.advance_kv_cache_step();
  if (!st.ok()) return Status::runtime_error("KV cache advance failed: " + st.to_string());
  return Status::make_ok();
}

}  // namespace minillm
