// graph.cpp -- graph IR and builder (see include/minillm_hip/graph.h).
#include "minillm_hip/graph.h"

#include <queue>

namespace minillm {

std::string_view op_type_name(OpType type) {
  switch (type) {
    case OpType::Input: return "Input";
    case OpType::Constant: return "Constant";
    case OpType::Embedding: return "Embedding";
    case OpType::MatMul: return "MatMul";
    case OpType::Linear: return "Linear";
    case OpType::Add: return "Add";
    case OpType::Mul: return "Mul";
    case OpType::RMSNorm: return "RMSNorm";
    case OpType::LayerNorm: return "LayerNorm";
    case OpType::SiLU: return "SiLU";
    case OpType::SwiGLU: return "SwiGLU";
    case OpType::RoPE: return "RoPE";
    case OpType::Attention: return "Attention";
    case OpType::QKNorm: return "QKNorm";
    case OpType::Softmax: return "Softmax";
    case OpType::Reshape: return "Reshape";
    case OpType::Transpose: return "Transpose";
    case OpType::View: return "View";
    case OpType::Contiguous: return "Contiguous";
    case OpType::Output: return "Output";
    case OpType::Custom: return "Custom";
  }
  return "Unknown";
}

// ---------------------------------------------------------------- Node
Node::Node(NodeId id, OpType op_type, std::string name, std::vector<ValueId> inputs,
           std::vector<ValueId> outputs)
    : id_(id), op_type_(op_type), name_(std::move(name)), inputs_(std::move(inputs)),
      outputs_(std::move(outputs)) {}

NodeId Node::id() const { return id_; }
OpType Node::op_type() const { return op_type_; }
std::string_view Node::name() const { return name_; }
const std::vector<ValueId>& Node::inputs() const { return inputs_; }
const std::vector<ValueId>& Node::outputs() const { return outputs_; }
void Node::set_attr(std::string key, AttributeValue value) { attrs_[std::move(key)] = std::move(value); }

std::optional<AttributeValue> Node::get_attr(std::string_view key) const {
  auto it = attrs_.find(std::string(key));
  if (it == attrs_.end()) return std::nullopt;
  return it->second;
}

const std::unordered_map<std::string, AttributeValue>& Node::attrs() const { return attrs_; }

// ---------------------------------------------------------------- Graph
expected<ValueId, Status> Graph::add_value(std::string name, Shape shape, DType dtype,
                                           Device device, ValueKind kind) {
  const ValueId id{values_.size()};
  values_.push_back(Value{id, std::move(name), std::move(shape), dtype, device, kind});
  return id;
}

expected<NodeId, Status> Graph::add_node(OpType op_type, std::string name,
                                         std::vector<ValueId> inputs,
                                         std::vector<ValueId> outputs) {
  const NodeId id{nodes_.size()};
  nodes_.emplace_back(id, op_type, std::move(name), std::move(inputs), std::move(outputs));
  return id;
}

expected<Value*, Status> Graph::mutable_value(ValueId id) {
  if (id.value >= values_.size())
    return unexpected(Status::out_of_range("ValueId %" + std::to_string(id.value) + " out of range"));
  return &values_[id.value];
}

expected<const Value*, Status> Graph::value(ValueId id) const {
  if (id.value >= values_.size())
    return unexpected(Status::out_of_range("ValueId %" + std::to_string(id.value) + " out of range"));
  return &values_[id.value];
}

expected<Node*, Status> Graph::mutable_node(NodeId id) {
  if (id.value >= nodes_.size())
    return unexpected(Status::out_of_range("NodeId #" + std::to_string(id.value) + " out of range"));
  return &nodes_[id.value];
}

expected<const Node*, Status> Graph::node(NodeId id) const {
  if (id.value >= nodes_.size())
    return unexpected(Status::out_of_range("NodeId #" + std::to_string(id.value) + " out of range"));
  return &nodes_[id.value];
}

const std::vector<Value>& Graph::values() const { return values_; }
const std::vector<Node>& Graph::nodes() const { return nodes_; }

Status Graph::validate() const {
  for (const Node& n : nodes_) {
    for (const auto* ids : {&n.inputs(), &n.outputs()}) {
      for (const ValueId& v : *ids) {
        if (v.value >= values_.size())
          return Status::invalid_argument(
              "Node #" + std::to_string(n.id().value) + " (" +
              std::string(op_type_name(n.op_type())) + ") references non-existent ValueId %" +
              std::to_string(v.value));
      }
    }
    if (n.op_type() == OpType::Output && n.inputs().empty())
      return Status::invalid_argument("Output node #" + std::to_string(n.id().value) +
                                      " must have at least one input");
  }
  return Status::make_ok();
}

// Kahn's algorithm over producer -> consumer edges, FIFO among ready nodes.
expected<std::vector<NodeId>, Status> Graph::topological_sort() const {
  const Status st = validate();
  if (!st.ok()) return unexpected(st);
  const size_t n = nodes_.size();
  std::unordered_map<size_t, size_t> producer;
  for (size_t i = 0; i < n; ++i)
    for (const ValueId& v : nodes_[i].outputs()) producer[v.value] = i;
  std::vector<std::vector<size_t>> consumers(n);
  std::vector<int> pending(n, 0);
  for (size_t i = 0; i < n; ++i) {
    for (const ValueId& v : nodes_[i].inputs()) {
      auto it = producer.find(v.value);
      if (it == producer.end()) continue;
      consumers[it->second].push_back(i);
      ++pending[i];
    }
  }
  std::queue<size_t> ready;
  for (size_t i = 0; i < n; ++i)
    if (pending[i] == 0) ready.push(i);
  std::vector<NodeId> order;
  order.reserve(n);
  while (!ready.empty()) {
    const size_t cur = ready.front();
    ready.pop();
    order.push_back(NodeId{cur});
    for (size_t c : consumers[cur])
      if (--pending[c] == 0) ready.push(c);
  }
  if (order.size() != n) return unexpected(Status::runtime_error("graph has cycles"));
  return order;
}

// ---------------------------------------------------------------- shape rules
expected<Shape, Status> infer_matmul_shape(const Shape& a, const Shape& b) {
  if (a.rank() != 2 || b.rank() != 2)
    return unexpected(Status::shape_mismatch("MatMul expects rank-2 inputs, got " +
                                             a.to_string() + " and " + b.to_string()));
  const int64_t ka = a.dim(1), kb = b.dim(0);
  if (ka >= 0 && kb >= 0 && ka != kb)
    return unexpected(Status::shape_mismatch("MatMul inner dims mismatch: " + a.to_string() +
                                             " x " + b.to_string()));
  return Shape({a.dim(0), b.dim(1)});
}

expected<Shape, Status> infer_linear_shape(const Shape& x, const Shape& weight) {
  if (weight.rank() != 2)
    return unexpected(Status::shape_mismatch("Linear weight must be rank 2, got " +
                                             weight.to_string()));
  if (x.rank() < 1)
    return unexpected(Status::shape_mismatch("Linear input must have rank >= 1, got " +
                                             x.to_string()));
  const int64_t in = x.dim(x.rank() - 1), w_in = weight.dim(1);
  if (in >= 0 && w_in >= 0 && in != w_in)
    return unexpected(Status::shape_mismatch("Linear in_features mismatch: x " + x.to_string() +
                                             " vs weight " + weight.to_string()));
  std::vector<int64_t> dims(x.dims().begin(), x.dims().end() - 1);
  dims.push_back(weight.dim(0));
  return Shape(std::move(dims));
}

expected<Shape, Status> infer_embedding_shape(const Shape& input_ids, const Shape& weight) {
  if (input_ids.rank() < 1 || weight.rank() != 2)
    return unexpected(Status::shape_mismatch(
        "Embedding expects input_ids rank>=1 and weight rank 2, got " + input_ids.to_string() +
        " and " + weight.to_string()));
  std::vector<int64_t> dims = input_ids.dims();
  dims.push_back(weight.dim(1));
  return Shape(std::move(dims));
}

// ---------------------------------------------------------------- builder
GraphBuilder::GraphBuilder(Graph& graph) : graph_(graph) {}

expected<ValueId, Status> GraphBuilder::make_intermediate(std::string name, Shape shape,
                                                          DType dtype, Device device) {
  return graph_.add_value(std::move(name), std::move(shape), dtype, device,
                          ValueKind::Intermediate);
}

expected<ValueId, Status> GraphBuilder::input(std::string name, Shape shape, DType dtype,
                                              Device device) {
  return graph_.add_value(std::move(name), std::move(shape), dtype, device, ValueKind::Input);
}

expected<ValueId, Status> GraphBuilder::constant(std::string name, Shape shape, DType dtype,
                                                 Device device) {
  return graph_.add_value(std::move(name), std::move(shape), dtype, device,
                          ValueKind::Constant);
}

expected<Shape, Status> infer_elementwise_shape(const Shape& a, const Shape& b) {
  if (a.rank() != b.rank())
    return unexpected(Status::shape_mismatch("Elementwise op requires same rank: " +
                                             a.to_string() + " vs " + b.to_string()));
  for (size_t i = 0; i < a.rank(); ++i) {
    const int64_t da = a.dim(i), db = b.dim(i);
    if (da >= 0 && db >= 0 && da != db)
      return unexpected(Status::shape_mismatch("Elementwise dim mismatch at axis " +
                                               std::to_string(i) + ": " + a.to_string() +
                                               " vs " + b.to_string()));
  }
  return a;
}

expected<ValueId, Status> GraphBuilder::swiglu(ValueId gate, ValueId up, std::string name) {
  auto gv = graph_.value(gate);
  if (!gv) return unexpected(gv.error());
  auto uv = graph_.value(up);
  if (!uv) return unexpected(uv.error());
  auto shape = infer_elementwise_shape((*gv)->shape, (*uv)->shape);
  if (!shape) return unexpected(shape.error());
  auto out = make_intermediate(name + ".out", std::move(*shape), (*gv)->dtype, (*gv)->device);
  if (!out) return out;
  auto nid = graph_.add_node(OpType::SwiGLU, std::move(name), {gate, up}, {*out});
  if (!nid) return unexpected(nid.error());
  return out;
}

expected<ValueId, Status> GraphBuilder::embedding(ValueId input_ids, ValueId weight,
                                                  std::string name) {
  auto iv = graph_.value(input_ids);
  if (!iv) return unexpected(iv.error());
  auto wv = graph_.value(weight);
  if (!wv) return unexpected(wv.error());
  auto shape = infer_embedding_shape((*iv)->shape, (*wv)->shape);
  if (!shape) return unexpected(shape.error());
  const DType dt = (*wv)->dtype;
  const Device dev = (*wv)->device;
  auto out = make_intermediate(name + ".out", std::move(*shape), dt, dev);
  if (!out) return out;
  auto nid = graph_.add_node(OpType::Embedding, std::move(name), {input_ids, weight}, {*out});
  if (!nid) return unexpected(nid.error());
  return out;
}

expected<ValueId, Status> GraphBuilder::matmul(ValueId a, ValueId b, std::string name) {
  auto av = graph_.value(a);
  if (!av) return unexpected(av.error());
  auto bv = graph_.value(b);
  if (!bv) return unexpected(bv.error());
  auto shape = infer_matmul_shape((*av)->shape, (*bv)->shape);
  if (!shape) return unexpected(shape.error());
  const DType dt = (*av)->dtype;
  const Device dev = (*av)->device;
  auto out = make_intermediate(name + ".out", std::move(*shape), dt, dev);
  if (!out) return out;
  auto nid = graph_.add_node(OpType::MatMul, std::move(name), {a, b}, {*out});
  if (!nid) return unexpected(nid.error());
  return out;
}

expected<ValueId, Status> GraphBuilder::linear(ValueId x, ValueId weight,
                                               std::optional<ValueId> bias, std::string name) {
  auto xv = graph_.value(x);
  if (!xv) return unexpected(xv.error());
  auto wv = graph_.value(weight);
  if (!wv) return unexpected(wv.error());
  auto shape = infer_linear_shape((*xv)->shape, (*wv)->shape);
  if (!shape) return unexpected(shape.error());
  if (bias) {
    auto bv = graph_.value(*bias);
    if (!bv) return unexpected(bv.error());
    if ((*bv)->shape.rank() != 1 || (*bv)->shape.dim(0) != (*wv)->shape.dim(0))
      return unexpected(Status::shape_mismatch(
          "Linear bias must have shape [" + std::to_string((*wv)->shape.dim(0)) + "], got " +
          (*bv)->shape.to_string()));
  }
  const DType dt = (*wv)->dtype;
  const Device dev = (*wv)->device;
  auto out = make_intermediate(name + ".out", std::move(*shape), dt, dev);
  if (!out) return out;
  std::vector<ValueId> inputs{x, weight};
  if (bias) inputs.push_back(*bias);
  auto nid = graph_.add_node(OpType::Linear, std::move(name), std::move(inputs), {*out});
  if (!nid) return unexpected(nid.error());
  return out;
}

// Marks `x` as a graph output (no node is added), as the reference does
// (src/graph/graph_builder.cpp:317-325).
expected<ValueId, Status> GraphBuilder::output(ValueId x, std::string name) {
  (void)name;
  auto v = graph_.mutable_value(x);
  if (!v) return unexpected(v.error());
  (*v)->kind = ValueKind::Output;
  return x;
}

}  // namespace minillm
