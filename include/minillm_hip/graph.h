// graph.h -- graph IR of the MiniLLMEngine host API (HIP backend restatement).
//
// Same names and semantics as the reference graph layer
// (include/minillm/graph/value.h:10-37, op_type.h:8-58, node.h:13-39,
// graph.h:11-40, graph_builder.h:14-89).  The builder here covers the ops of the
// Q8_0 path and the graph plumbing around them: input, constant, embedding,
// matmul, linear (optional bias) and output.  As in the reference, a weight
// Value is declared with its logical dtype (Float32) while the Tensor bound to
// it may be physically Q8_0, and an op's output Value takes the weight Value's
// dtype and device (reference src/graph/graph_builder.cpp:32-95).
#pragma once

#include <cstdint>
#include <optional>
#include <string>
#include <string_view>
#include <unordered_map>
#include <variant>
#include <vector>

#include "minillm_hip/core.h"

namespace minillm {

struct ValueId {
  size_t value{0};
  bool operator==(const ValueId& o) const { return value == o.value; }
};

struct NodeId {
  size_t value{0};
  bool operator==(const NodeId& o) const { return value == o.value; }
};

enum class ValueKind {
  Input,
  Constant,
  Intermediate,
  Output,
};

struct Value {
  ValueId id;
  std::string name;
  Shape shape;
  DType dtype{DType::Unknown};
  Device device{Device::cpu()};
  ValueKind kind{ValueKind::Intermediate};
};

// Full op set of the reference (op_type.h), so graphs that name other ops can be
// built; only Embedding, MatMul and Linear have HIP kernels here.
enum class OpType {
  Input,
  Constant,
  Embedding,
  MatMul,
  Linear,
  Add,
  Mul,
  RMSNorm,
  LayerNorm,
  SiLU,
  SwiGLU,
  RoPE,
  Attention,
  QKNorm,
  Softmax,
  Reshape,
  Transpose,
  View,
  Contiguous,
  Output,
  Custom,
};

std::string_view op_type_name(OpType type);

using AttributeValue =
    std::variant<int64_t, double, bool, std::string, Shape, std::vector<int64_t>>;

class Node {
 public:
  Node(NodeId id, OpType op_type, std::string name, std::vector<ValueId> inputs,
       std::vector<ValueId> outputs);

  NodeId id() const;
  OpType op_type() const;
  std::string_view name() const;
  const std::vector<ValueId>& inputs() const;
  const std::vector<ValueId>& outputs() const;
  void set_attr(std::string key, AttributeValue value);
  std::optional<AttributeValue> get_attr(std::string_view key) const;
  const std::unordered_map<std::string, AttributeValue>& attrs() const;

 private:
  NodeId id_;
  OpType op_type_;
  std::string name_;
  std::vector<ValueId> inputs_;
  std::vector<ValueId> outputs_;
  std::unordered_map<std::string, AttributeValue> attrs_;
};

class Graph {
 public:
  expected<ValueId, Status> add_value(std::string name, Shape shape, DType dtype,
                                      Device device, ValueKind kind);
  expected<NodeId, Status> add_node(OpType op_type, std::string name,
                                    std::vector<ValueId> inputs,
                                    std::vector<ValueId> outputs);

  expected<Value*, Status> mutable_value(ValueId id);
  expected<const Value*, Status> value(ValueId id) const;
  expected<Node*, Status> mutable_node(NodeId id);
  expected<const Node*, Status> node(NodeId id) const;

  const std::vector<Value>& values() const;
  const std::vector<Node>& nodes() const;

  Status validate() const;
  expected<std::vector<NodeId>, Status> topological_sort() const;

 private:
  std::vector<Value> values_;
  std::vector<Node> nodes_;
};

// Shape rules (reference src/graph/shape_infer.cpp:7-46,86-98).
expected<Shape, Status> infer_matmul_shape(const Shape& a, const Shape& b);
expected<Shape, Status> infer_linear_shape(const Shape& x, const Shape& weight);
expected<Shape, Status> infer_embedding_shape(const Shape& input_ids, const Shape& weight);
// Same rank, equal known dims (reference src/graph/shape_infer.cpp:48-63).
expected<Shape, Status> infer_elementwise_shape(const Shape& a, const Shape& b);

class GraphBuilder {
 public:
  explicit GraphBuilder(Graph& graph);

  expected<ValueId, Status> input(std::string name, Shape shape, DType dtype,
                                  Device device = Device::cpu());
  expected<ValueId, Status> constant(std::string name, Shape shape, DType dtype,
                                     Device device = Device::cpu());
  expected<ValueId, Status> embedding(ValueId input_ids, ValueId weight, std::string name);
  expected<ValueId, Status> matmul(ValueId a, ValueId b, std::string name);
  expected<ValueId, Status> linear(ValueId x, ValueId weight, std::optional<ValueId> bias,
                                   std::string name);
  // y = silu(gate) * up (reference src/graph/graph_builder.cpp:168-184).
  expected<ValueId, Status> swiglu(ValueId gate, ValueId up, std::string name);
  expected<ValueId, Status> output(ValueId x, std::string name);

 private:
  Graph& graph_;
  expected<ValueId, Status> make_intermediate(std::string name, Shape shape, DType dtype,
                                              Device device);
};

}  // namespace minillm
