// TensorIR types and the graph builder (semantics of the reference's
// src/tensor/TensorIR.cpp:1-175: dense strides, storage extent of a strided
// view, SSA value numbering, RMSNorm operand checks).
#include "TensorIR.hpp"

#include <cmath>
#include <limits>
#include <stdexcept>
#include <utility>

namespace tensor {
namespace {

constexpr std::size_t kMaxSize = std::numeric_limits<std::size_t>::max();

std::size_t checkedProduct(std::size_t a, std::size_t b, const char* what) {
  if (b != 0 && a > kMaxSize / b) throw std::overflow_error(what);
  return a * b;
}

// Row-major strides of `shape`, last dimension fastest.
std::vector<std::size_t> rowMajor(const std::vector<std::size_t>& shape) {
  std::vector<std::size_t> out(shape.size(), 1);
  std::size_t step = 1;
  for (std::size_t axis = shape.size(); axis-- > 0;) {
    out[axis] = step;
    step = checkedProduct(step, shape[axis], "Tensor strides exceed size_t capacity.");
  }
  return out;
}

}  // namespace

bool isFloatingDType(DType dtype) { return dtype != DType::Int32; }

std::size_t TensorType::elementCount() const {
  std::size_t count = 1;
  for (const std::size_t extent : shape) {
    if (extent == 0) throw std::invalid_argument("Tensor dimensions must be positive.");
    count = checkedProduct(count, extent, "Tensor element count exceeds size_t capacity.");
  }
  return count;
}

std::vector<std::size_t> TensorType::strides() const {
  (void)elementCount();  // validates the extents
  if (layout == Layout::Contiguous) {
    if (!explicitStrides.empty())
      throw std::invalid_argument("Contiguous tensors must not carry explicit strides.");
    return rowMajor(shape);
  }
  if (explicitStrides.size() != shape.size())
    throw std::invalid_argument("Strided tensors require one stride per dimension.");
  return explicitStrides;
}

std::size_t TensorType::storageElementCount() const {
  const std::vector<std::size_t> s = strides();
  std::size_t last = 0;  // offset of the last reachable element
  for (std::size_t axis = 0; axis < shape.size(); ++axis) {
    const std::size_t reach = checkedProduct(shape[axis] - 1, s[axis],
                                             "Tensor storage exceeds size_t capacity.");
    if (last > kMaxSize - reach) throw std::overflow_error("Tensor storage exceeds size_t capacity.");
    last += reach;
  }
  return last + 1;
}

bool TensorType::isContiguous() const {
  if (layout == Layout::Contiguous) return true;
  return strides() == rowMajor(shape);
}

const char* opName(OpType op) {
  switch (op) {
    case OpType::Add: return "Add";
    case OpType::Mul: return "Mul";
    case OpType::MatMul: return "MatMul";
    case OpType::RMSNorm: return "RMSNorm";
    case OpType::LayerNorm: return "LayerNorm";
    case OpType::ReLU: return "ReLU";
    case OpType::SiLU: return "SiLU";
    case OpType::Softmax: return "Softmax";
    case OpType::RoPE: return "RoPE";
    case OpType::ReduceSum: return "ReduceSum";
    case OpType::ReduceMean: return "ReduceMean";
    case OpType::Reshape: return "Reshape";
    case OpType::View: return "View";
    case OpType::Transpose: return "Transpose";
    case OpType::Contiguous: return "Contiguous";
    case OpType::MaskedFill: return "MaskedFill";
    case OpType::Slice: return "Slice";
    case OpType::Embedding: return "Embedding";
    case OpType::Gather: return "Gather";
  }
  return "Unknown";
}

bool isViewOp(OpType op) {
  return op == OpType::Reshape || op == OpType::View || op == OpType::Transpose;
}

ValueId TensorGraph::addInput(std::string name, TensorType type) {
  const ValueId id = values.size();
  values.push_back({std::move(name), std::move(type)});
  inputs.push_back(id);
  return id;
}

ValueId TensorGraph::addNode(OpType op, std::vector<ValueId> operands, OpAttributes attributes,
                             std::string name) {
  return addNodeResults(op, std::move(operands), {std::move(name)}, std::move(attributes)).front();
}

std::vector<ValueId> TensorGraph::addNodeResults(OpType op, std::vector<ValueId> operands,
                                                 std::vector<std::string> names,
                                                 OpAttributes attributes) {
  for (const ValueId operand : operands)
    if (operand >= values.size()) throw std::out_of_range("Operation operand is not a graph value.");
  if (names.empty()) throw std::invalid_argument("An operation needs at least one result.");
  Node node{op, std::move(operands), {}, std::move(attributes)};
  for (auto& name : names) {
    node.outputs.push_back(values.size());
    values.push_back({std::move(name), std::nullopt});
  }
  nodes.push_back(std::move(node));
  return nodes.back().outputs;
}

void RMSNormOp::validate() const {
  if (input.shape.empty()) throw std::invalid_argument("RMSNorm input must be ranked.");
  if (!isFloatingDType(input.dtype) || weight.dtype != input.dtype || output.dtype != input.dtype)
    throw std::invalid_argument("RMSNorm requires matching floating-point tensors.");
  if (output.shape != input.shape)
    throw std::invalid_argument("RMSNorm output shape must match input shape.");
  if (weight.shape.size() != 1 || weight.shape.front() != input.shape.back())
    throw std::invalid_argument("RMSNorm weight must match the last input dimension.");
  if (!std::isfinite(epsilon) || epsilon <= 0.0f)
    throw std::invalid_argument("RMSNorm epsilon must be finite and positive.");
}

}  // namespace tensor
