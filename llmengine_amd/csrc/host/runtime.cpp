// runtime.cpp -- registry, backends, runtime context, HIP executor
// (see include/minillm_hip/runtime.h).
#include "minillm_hip/runtime.h"

#include <algorithm>
#include <climits>
#include <map>
#include <unordered_map>
#include <unordered_set>

#include "fusion.hpp"
#include "mle_q8_0.h"

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
         op == OpType::SwiGLU || op == OpType::Output;
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

HipExecutor::~HipExecutor() { release_tiled_weights(); }

void HipExecutor::release_tiled_weights() {
  if (!tiled_bufs_.empty()) (void)hipStreamSynchronize(stream_);  // launches may still read them
  for (void* p : tiled_bufs_) (void)hipFree(p);
  tiled_bufs_.clear();
  tiled_.clear();
}

Status HipExecutor::tile_weights(RuntimeContext& ctx, bool release_raw) {
  if (!graph_) return Status::runtime_error("executor not compiled");
  // Overwritten weights get fresh copies: drop the old ones first.
  release_tiled_weights();
  in_place_ = 0;
  // Buffers read other than as a Linear weight, through any value bound to
  // them, keep their raw bytes: a MatMul operand cannot be read from tiles, and
  // an Embedding table (a tied lm_head) gathers twice as fast from raw bytes
  // (each row's quants share their 16-byte tile slots' cache lines with 15
  // other rows), which HBM capacity makes the better trade.  So does a buffer
  // that another tensor bound in `ctx` also views (the same bytes, or a range
  // overlapping them): freeing its raw bytes would leave that view dangling.
  std::unordered_set<const void*> other_use;
  struct Span {
    const Tensor* t;
    uintptr_t lo, hi;
  };
  std::vector<Span> spans;
  if (release_raw) {
    for (const Node& n : graph_->nodes())
      for (size_t i = 0; i < n.inputs().size(); ++i) {
        if (n.op_type() == OpType::Linear && i == 1) continue;
        if (const Tensor* t = ctx.get(n.inputs()[i]); t && t->data()) other_use.insert(t->data());
      }
    for (const Value& v : graph_->values())
      if (const Tensor* t = ctx.get(v.id); t && t->data() && t->allocated_bytes() > 0) {
        const uintptr_t lo = reinterpret_cast<uintptr_t>(t->data());
        spans.push_back(Span{t, lo, lo + t->allocated_bytes()});
      }
  }
  auto viewed_by_other = [&](const Tensor* w) {
    const uintptr_t lo = reinterpret_cast<uintptr_t>(w->data()), hi = lo + w->allocated_bytes();
    for (const Span& s : spans)
      if (s.t != w && s.lo < hi && lo < s.hi) return true;
    return false;
  };
  for (const Node& n : graph_->nodes()) {
    if (n.op_type() != OpType::Linear || n.inputs().size() < 2) continue;
    Tensor* w = ctx.get(n.inputs()[1]);
    if (!w || w->dtype() != DType::Q8_0 || w->device().type != DeviceType::HIP ||
        w->data() == nullptr || w->shape().rank() != 2)
      continue;  // not on this path: the node keeps its registered kernel and its checks
    if (w->storage_layout() != StorageLayout::Raw) continue;  // re-tiled in place already
    const int64_t N = w->shape().dim(0), K = w->shape().dim(1);
    if (N <= 0 || K <= 0 || K % 32 != 0 || N > INT32_MAX || K > INT32_MAX) continue;
    if (w->allocated_bytes() < q8_0_bytes(N * K)) continue;
    if (tiled_.count(w->data())) continue;  // shared by several nodes
    const size_t bytes = hip::q8_0_tiled_bytes(static_cast<int>(N), static_cast<int>(K));
    void* buf = nullptr;
    const hipError_t err = hipMalloc(&buf, bytes);
    if (err != hipSuccess) {
      release_tiled_weights();
      return Status::runtime_error(std::string("tiled weight allocation failed: ") +
                                   hipGetErrorString(err));
    }
    const bool in_place = release_raw && w->owns_hip_storage() && !other_use.count(w->data()) &&
                          !viewed_by_other(w);
    if (!in_place) tiled_bufs_.push_back(buf);
    Status st = hip::tile_q8_0(static_cast<const uint8_t*>(w->data()),
                               static_cast<uint8_t*>(buf), static_cast<int>(N),
                               static_cast<int>(K), stream_);
    if (in_place) {
      if (st.ok()) {
        // The tile kernel must be done with the raw bytes before they are freed.
        const hipError_t e = hipStreamSynchronize(stream_);
        st = e == hipSuccess ? w->adopt_hip_bytes(buf, bytes, StorageLayout::Q8_0Tiled)
                             : Status::runtime_error(std::string("hipStreamSynchronize failed: ") +
                                                     hipGetErrorString(e));
      }
      if (!st.ok()) {
        (void)hipStreamSynchronize(stream_);  // a launched tile kernel may still write buf
        (void)hipFree(buf);                   // not adopted: still this function's
      }
    }
    if (!st.ok()) {
      release_tiled_weights();
      return Status::runtime_error("tiling Linear weight of node #" + std::to_string(n.id().value) +
                                   " failed: " + st.to_string());
    }
    if (in_place) {
      ++in_place_;
      continue;
    }
    tiled_[w->data()] = detail::TiledCopy{static_cast<const uint8_t*>(buf), N, K, bytes};
  }
  return reserve_workspace(&ctx);
}

namespace {
// M, N, K of a Linear node from the tensors bound in ctx, else the graph's
// static value shapes (false when unknown or dynamic).
// M, N, K of a MatMul node: A [M, K] . B [K, N] (rank 2, static shapes).
bool matmul_dims(const Graph& g, const Node& n, const RuntimeContext* ctx, int64_t* M,
                 int64_t* N, int64_t* K) {
  if (n.op_type() != OpType::MatMul || n.inputs().size() < 2) return false;
  Shape as, bs;
  auto shape_of = [&](ValueId id, Shape* out) {
    if (ctx) {
      if (const Tensor* t = ctx->get(id)) {
        *out = t->shape();
        return !out->has_dynamic_dim();
      }
    }
    auto v = g.value(id);
    if (!v) return false;
    *out = (*v)->shape;
    return !out->has_dynamic_dim();
  };
  if (!shape_of(n.inputs()[0], &as) || !shape_of(n.inputs()[1], &bs)) return false;
  if (as.rank() != 2 || bs.rank() != 2) return false;
  *M = as.dim(0);
  *K = as.dim(1);
  *N = bs.dim(1);
  return *M > 0 && *N > 0 && *K > 0 && *M <= INT32_MAX && *N <= INT32_MAX && *K <= INT32_MAX &&
         *K % 32 == 0 && *N % 32 == 0;
}

bool linear_dims(const Graph& g, const Node& n, const RuntimeContext* ctx, int64_t* M,
                 int64_t* N, int64_t* K) {
  if (n.op_type() != OpType::Linear || n.inputs().size() < 2) return false;
  auto shape_of = [&](ValueId id, Shape* out) {
    if (ctx) {
      if (const Tensor* t = ctx->get(id)) {
        *out = t->shape();
        return !out->has_dynamic_dim();
      }
    }
    auto v = g.value(id);
    if (!v) return false;
    *out = (*v)->shape;
    return !out->has_dynamic_dim();
  };
  Shape xs, ws;
  if (!shape_of(n.inputs()[0], &xs) || !shape_of(n.inputs()[1], &ws)) return false;
  if (xs.rank() == 0 || ws.rank() != 2) return false;
  int64_t m = 1;
  for (size_t i = 0; i + 1 < xs.rank(); ++i) m *= xs.dim(i);
  *M = m;
  *K = xs.dim(xs.rank() - 1);
  *N = ws.dim(0);
  return *M > 0 && *N > 0 && *K > 0 && *M <= INT32_MAX && *N <= INT32_MAX && *K <= INT32_MAX &&
         *K % 32 == 0;
}
}  // namespace

Status HipExecutor::reserve_workspace(const RuntimeContext* ctx) {
  if (!graph_) return Status::runtime_error("executor not compiled");
  size_t bytes = 0, counters = 0;
  auto need = [&](int op, int M, int count, const int* N, int K) {
    for (int tiled = 0; tiled < 2; ++tiled) {
      size_t b = 0, c = 0;
      if (mle_q8_0_workspace_size(op, M, count, N, K, tiled, &b, &c) == MLE_OK) {
        bytes = std::max(bytes, b);
        counters = std::max(counters, c);
      }
    }
  };
  for (const Step& step : plan_) {
    std::vector<const Node*> nodes;
    for (const NodeId& nid : step.nodes) {
      auto nd = graph_->node(nid);
      if (nd) nodes.push_back(*nd);
    }
    // Every MatMul, and every Linear also on its own (a fused group that does
    // not fit its kernel runs node by node), then the fused launch of its group.
    std::vector<int> Ns;
    int64_t M0 = 0, K0 = 0;
    bool same = true;
    for (const Node* n : nodes) {
      int64_t M, N, K;
      if (matmul_dims(*graph_, *n, ctx, &M, &N, &K)) {
        const int n32 = static_cast<int>(N);
        need(MLE_OP_MATMUL, static_cast<int>(M), 1, &n32, static_cast<int>(K));
        continue;
      }
      if (!linear_dims(*graph_, *n, ctx, &M, &N, &K)) continue;
      const int n32 = static_cast<int>(N);
      need(MLE_OP_LINEAR, static_cast<int>(M), 1, &n32, static_cast<int>(K));
      if (Ns.empty()) M0 = M, K0 = K;
      same = same && M == M0 && K == K0;
      Ns.push_back(n32);
    }
    if (!same || Ns.size() < 2) continue;
    if (step.kind == Step::kSwiGLU && Ns.size() == 2 && Ns[0] == Ns[1])
      need(MLE_OP_LINEAR_SWIGLU, static_cast<int>(M0), 2, Ns.data(), static_cast<int>(K0));
    else if (step.kind == Step::kMulti && Ns.size() <= 3)
      need(MLE_OP_LINEAR_MULTI, static_cast<int>(M0), static_cast<int>(Ns.size()), Ns.data(),
           static_cast<int>(K0));
  }
  ws_bytes_ = std::max(ws_bytes_, bytes);
  ws_counters_ = std::max(ws_counters_, counters);
  if (ws_bytes_ == 0 && ws_counters_ == 0) {
    ws_pending_ = false;
    return Status::make_ok();
  }
  const int rc = mle_workspace_reserve(ws_bytes_, ws_counters_, stream_);
  if (rc != MLE_OK)
    return Status::runtime_error(std::string("workspace reservation failed: ") + mle_last_error());
  ws_pending_ = false;
  return Status::make_ok();
}

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

  // Fusion plan over the topological order.
  plan_.clear();
  std::unordered_map<size_t, int> uses;          // value -> consuming nodes
  std::unordered_map<size_t, size_t> producer;   // value -> node index
  for (const Node& n : graph.nodes()) {
    for (const ValueId& v : n.inputs()) ++uses[v.value];
    for (const ValueId& v : n.outputs()) producer[v.value] = n.id().value;
  }
  auto node_of = [&](size_t id) -> const Node* {
    auto nd = graph.node(NodeId{id});
    return nd ? *nd : nullptr;
  };
  auto value_kind = [&](ValueId v) {
    auto val = graph.value(v);
    return val ? (*val)->kind : ValueKind::Intermediate;
  };
  std::unordered_set<size_t> taken;
  std::unordered_map<size_t, std::vector<NodeId>> anchor;  // node -> fused group it starts
  std::unordered_map<size_t, Step::Kind> anchor_kind;
  if (fusion_) {
    for (const NodeId& nid : execution_order_) {
      const Node* sw = node_of(nid.value);
      if (!sw || sw->op_type() != OpType::SwiGLU || sw->inputs().size() != 2) continue;
      const ValueId g = sw->inputs()[0], u = sw->inputs()[1];
      if (!producer.count(g.value) || !producer.count(u.value)) continue;
      const Node* pg = node_of(producer[g.value]);
      const Node* pu = node_of(producer[u.value]);
      if (!pg || !pu || pg == pu || pg->op_type() != OpType::Linear ||
          pu->op_type() != OpType::Linear || pg->inputs().size() != 2 ||
          pu->inputs().size() != 2 || !(pg->inputs()[0] == pu->inputs()[0]))
        continue;
      if (uses[g.value] != 1 || uses[u.value] != 1 || value_kind(g) == ValueKind::Output ||
          value_kind(u) == ValueKind::Output)
        continue;
      if (taken.count(pg->id().value) || taken.count(pu->id().value)) continue;
      taken.insert({pg->id().value, pu->id().value, nid.value});
      anchor[nid.value] = {pg->id(), pu->id(), nid};
      anchor_kind[nid.value] = Step::kSwiGLU;
    }
    // Sibling Linears on one input whose other inputs are constants / inputs.
    std::map<size_t, std::vector<NodeId>> by_input;
    for (const NodeId& nid : execution_order_) {
      const Node* n = node_of(nid.value);
      if (!n || n->op_type() != OpType::Linear || taken.count(nid.value)) continue;
      bool ok = true;
      for (size_t i = 1; i < n->inputs().size(); ++i) {
        const ValueKind k = value_kind(n->inputs()[i]);
        ok = ok && (k == ValueKind::Constant || k == ValueKind::Input);
      }
      if (ok) by_input[n->inputs()[0].value].push_back(nid);
    }
    for (auto& [x, ids] : by_input) {
      (void)x;
      for (size_t i = 0; i + 1 < ids.size(); i += 3) {
        std::vector<NodeId> group(ids.begin() + i, ids.begin() + std::min(ids.size(), i + 3));
        for (const NodeId& m : group) taken.insert(m.value);
        anchor[group[0].value] = group;
        anchor_kind[group[0].value] = Step::kMulti;
      }
    }
  }
  for (const NodeId& nid : execution_order_) {
    auto a = anchor.find(nid.value);
    if (a != anchor.end()) {
      plan_.push_back(Step{anchor_kind[nid.value], a->second});
    } else if (!taken.count(nid.value)) {
      plan_.push_back(Step{Step::kNode, {nid}});
    }
  }
  // Workspace for the plan's largest launch, now when a HIP device is present;
  // on a host without one (graph-only use), at the first run.
  ws_bytes_ = ws_counters_ = 0;
  int devices = 0;
  if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
    ws_pending_ = true;
    return Status::make_ok();
  }
  return reserve_workspace(nullptr);
}

size_t HipExecutor::fused_groups() const {
  size_t n = 0;
  for (const Step& s : plan_) n += s.kind != Step::kNode;
  return n;
}

Status HipExecutor::run_nodes(const std::vector<NodeId>& ids, RuntimeContext& ctx) {
  for (const NodeId& nid : ids) {
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
  return Status::make_ok();
}

Status HipExecutor::run(RuntimeContext& ctx) {
  if (!graph_) return Status::runtime_error("executor not compiled");
  ctx.set_hip_stream(stream_);
  if (ws_pending_) TRY(reserve_workspace(&ctx));
  fused_launches_ = 0;
  tiled_launches_ = 0;
  const detail::TiledWeights* tiled = tiled_.empty() ? nullptr : &tiled_;
  for (const Step& step : plan_) {
    if (step.kind != Step::kNode) {
      std::vector<const Node*> nodes;
      for (const NodeId& nid : step.nodes) {
        auto nd = graph_->node(nid);
        if (!nd) return nd.error();
        nodes.push_back(*nd);
      }
      bool used_tiled = false;
      auto done = step.kind == Step::kSwiGLU
                      ? detail::run_fused_swiglu(*nodes[0], *nodes[1], *nodes[2], ctx, tiled,
                                                 &used_tiled)
                      : detail::run_fused_multi(nodes, ctx, tiled, &used_tiled);
      if (!done) {
        std::string ids;
        for (const Node* n : nodes)
          ids += (ids.empty() ? "#" : ", #") + std::to_string(n->id().value) + " (" +
                 std::string(n->name()) + ")";
        return Status::runtime_error(std::string("HIP fused ") +
                                     (step.kind == Step::kSwiGLU ? "Linear+Linear+SwiGLU"
                                                                 : "multi-output Linear") +
                                     " failed for nodes " + ids + ": " +
                                     done.error().to_string());
      }
      if (*done) {
        ++fused_launches_;
        tiled_launches_ += used_tiled;
        continue;
      }
    }
    if (step.kind == Step::kNode) {
      auto nd = graph_->node(step.nodes[0]);
      if (nd && (*nd)->op_type() == OpType::Linear) {
        auto done = detail::run_tiled_linear(**nd, ctx, tiled);
        if (!done)
          return Status::runtime_error("HIP kernel Linear failed for node #" +
                                       std::to_string(step.nodes[0].value) + " (" +
                                       std::string((*nd)->name()) + "): " +
                                       done.error().to_string());
        if (*done) {
          ++tiled_launches_;
          continue;
        }
      }
    }
    TRY(run_nodes(step.nodes, ctx));
  }
  const Status st = ctx.advance_kv_cache_step();
  if (!st.ok()) return Status::runtime_error("KV cache advance failed: " + st.to_string());
  return Status::make_ok();
}

}  // namespace minillm
