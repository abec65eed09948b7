#include "GraphExecutor.hpp"

#include "Benchmark.hpp"
#include "Tuning.hpp"
#include "tmc_hip.h"

#include <algorithm>
#include <cmath>
#include <limits>
#include <ostream>
#include <sstream>
#include <stdexcept>
#include <utility>

namespace tensor {

// ------------------------------------------------------------------ analysis
namespace analyzer {
namespace {

constexpr std::size_t kUndefined = std::numeric_limits<std::size_t>::max();

TensorType dense(std::vector<std::size_t> shape, DType dtype) {
  TensorType t;
  t.shape = std::move(shape);
  t.dtype = dtype;
  return t;
}

std::string valueLabel(const TensorGraph& g, ValueId v) {
  const std::string& name = g.values[v].name;
  return name.empty() ? "value " + std::to_string(v) : "'" + name + "'";
}

std::size_t axisIndex(std::int64_t axis, std::size_t rank, const char* op) {
  const std::int64_t r = static_cast<std::int64_t>(rank);
  const std::int64_t a = axis < 0 ? axis + r : axis;
  if (a < 0 || a >= r) throw std::invalid_argument(std::string(op) + " axis is out of range.");
  return static_cast<std::size_t>(a);
}

void needFloat(const TensorType& t, const char* op) {
  if (!isFloatingDType(t.dtype)) throw std::invalid_argument(std::string(op) + " requires a floating tensor.");
}

// Result type of node `n` (operand types known); views get their strides.
TensorType inferType(Node& n, const std::vector<TensorType>& types) {
  auto arity = [&](std::size_t k) {
    if (n.inputs.size() != k || n.outputs.size() != 1)
      throw std::invalid_argument(std::string(opName(n.op)) + " takes " + std::to_string(k) +
                                  " operand(s) and one result.");
  };
  switch (n.op) {
    case OpType::Add:
    case OpType::Mul: {
      arity(2);
      const TensorType& a = types[n.inputs[0]];
      const TensorType& b = types[n.inputs[1]];
      needFloat(a, opName(n.op));
      if (b.dtype != a.dtype) throw std::invalid_argument(std::string(opName(n.op)) + " operands must share a dtype.");
      if (a.shape != b.shape)
        throw std::invalid_argument(std::string(opName(n.op)) +
                                    " on the gfx950 graph path needs operands of one shape "
                                    "(no broadcasting).");
      return dense(a.shape, a.dtype);
    }
    case OpType::SiLU: {
      arity(1);
      needFloat(types[n.inputs[0]], "SiLU");
      return dense(types[n.inputs[0]].shape, types[n.inputs[0]].dtype);
    }
    case OpType::RMSNorm: {
      arity(2);
      if (std::holds_alternative<std::monostate>(n.attributes)) n.attributes = RMSNormAttributes{};
      const auto* at = std::get_if<RMSNormAttributes>(&n.attributes);
      if (!at) throw std::invalid_argument("RMSNorm takes RMSNormAttributes.");
      const TensorType& x = types[n.inputs[0]];
      if (x.shape.empty()) throw std::invalid_argument("RMSNorm input must be ranked.");
      if (axisIndex(at->axis, x.shape.size(), "RMSNorm") != x.shape.size() - 1)
        throw std::invalid_argument("RMSNorm normalizes the last axis only.");
      RMSNormOp op{x, types[n.inputs[1]], dense(x.shape, x.dtype), at->epsilon};
      op.input.layout = Layout::Contiguous;
      op.input.explicitStrides.clear();
      op.validate();
      return dense(x.shape, x.dtype);
    }
    case OpType::MatMul: {
      arity(2);
      const TensorType& a = types[n.inputs[0]];
      const TensorType& b = types[n.inputs[1]];
      needFloat(a, "MatMul");
      if (b.dtype != a.dtype) throw std::invalid_argument("MatMul operands must share a dtype.");
      if (a.shape.size() != 2 || b.shape.size() != 2 || a.shape[1] != b.shape[0])
        throw std::invalid_argument("MatMul on the gfx950 graph path takes [M, K] x [K, N].");
      return dense({a.shape[0], b.shape[1]}, a.dtype);
    }
    case OpType::Embedding: {
      arity(2);
      const TensorType& table = types[n.inputs[0]];
      const TensorType& ids = types[n.inputs[1]];
      if (table.shape.size() != 2 || !table.isContiguous() || !isFloatingDType(table.dtype) ||
          ids.dtype != DType::Int32)
        throw std::invalid_argument("Embedding requires a rank-2 table and int32 indices.");
      std::vector<std::size_t> shape = ids.shape;
      shape.push_back(table.shape[1]);
      return dense(std::move(shape), table.dtype);
    }
    case OpType::Reshape:
    case OpType::View: {
      arity(1);
      const auto* at = std::get_if<ReshapeAttributes>(&n.attributes);
      if (!at) throw std::invalid_argument(std::string(opName(n.op)) + " takes ReshapeAttributes.");
      const TensorType& a = types[n.inputs[0]];
      TensorType out = dense(at->shape, a.dtype);
      if (!a.isContiguous() || out.elementCount() != a.elementCount())
        throw std::invalid_argument("Reshape/View requires contiguous storage and equal element counts.");
      return out;
    }
    case OpType::Transpose: {
      arity(1);
      if (std::holds_alternative<std::monostate>(n.attributes)) n.attributes = TransposeAttributes{};
      auto* at = std::get_if<TransposeAttributes>(&n.attributes);
      if (!at) throw std::invalid_argument("Transpose takes TransposeAttributes.");
      const TensorType& a = types[n.inputs[0]];
      const std::size_t i = axisIndex(at->first, a.shape.size(), "Transpose");
      const std::size_t j = axisIndex(at->second, a.shape.size(), "Transpose");
      TensorType out = a;
      out.explicitStrides = a.strides();
      out.layout = Layout::Strided;
      std::swap(out.shape[i], out.shape[j]);
      std::swap(out.explicitStrides[i], out.explicitStrides[j]);
      at->first = static_cast<std::int64_t>(i);
      at->second = static_cast<std::int64_t>(j);
      return out;
    }
    default:
      throw std::invalid_argument(std::string("Operation ") + opName(n.op) +
                                  " is not in the gfx950 graph path's op set (Add, Mul, SiLU, "
                                  "RMSNorm, MatMul, Embedding, Reshape, View, Transpose).");
  }
}

}  // namespace

AnalyzedGraph analyze(const TensorGraph& graph) {
  AnalyzedGraph r;
  r.graph = graph;
  const std::size_t values = graph.values.size();
  r.types.resize(values);
  r.aliasOf.assign(values, std::nullopt);
  std::vector<bool> defined(values, false);
  for (const ValueId v : graph.inputs) {
    if (v >= values) throw std::invalid_argument("Graph input is not a graph value.");
    if (!graph.values[v].type)
      throw std::invalid_argument("Graph input " + valueLabel(graph, v) + " needs a type.");
    r.types[v] = *graph.values[v].type;
    (void)r.types[v].storageElementCount();  // validates shape and strides
    if (r.types[v].dtype == DType::BFloat16)
      throw std::invalid_argument("The gfx950 graph path stores fp16, fp32 and int32 tensors, not bf16.");
    defined[v] = true;
  }
  r.effects.assign(graph.nodes.size(), MemoryEffect::ReadOnly);
  for (std::size_t i = 0; i < graph.nodes.size(); ++i) {
    Node& n = r.graph.nodes[i];
    for (const ValueId v : n.inputs)
      if (v >= values || !defined[v])
        throw std::invalid_argument(std::string(opName(n.op)) + " (node " + std::to_string(i) +
                                    ") reads " + valueLabel(graph, v) + " before it is defined.");
    const TensorType type = inferType(n, r.types);
    const ValueId out = n.outputs.front();
    if (defined[out]) throw std::invalid_argument("Value " + valueLabel(graph, out) + " is defined twice.");
    r.types[out] = type;
    defined[out] = true;
    if (isViewOp(n.op)) {
      r.effects[i] = MemoryEffect::View;
      const ValueId base = n.inputs.front();
      r.aliasOf[out] = r.aliasOf[base] ? *r.aliasOf[base] : base;
    }
    r.order.push_back(i);
  }
  for (const ValueId v : graph.outputs)
    if (v >= values || !defined[v]) throw std::invalid_argument("A graph output is never defined.");
  return r;
}

const char* fusionName(FusionPattern pattern) {
  switch (pattern) {
    case FusionPattern::None: return "Unfused";
    case FusionPattern::AddRMSNorm: return "Add + RMSNorm";
    case FusionPattern::AddLayerNorm: return "Residual Add + LayerNorm";
    case FusionPattern::SiLUMul: return "SiLU + Mul";
    case FusionPattern::LinearReLU: return "Linear + ReLU";
  }
  return "Unknown";
}

std::vector<Region> formRegions(const AnalyzedGraph& a) {
  const TensorGraph& g = a.graph;
  std::vector<std::size_t> producer(g.values.size(), kUndefined);
  std::vector<std::vector<std::size_t>> users(g.values.size());
  for (std::size_t i = 0; i < g.nodes.size(); ++i) {
    for (const ValueId v : g.nodes[i].outputs) producer[v] = i;
    for (const ValueId v : g.nodes[i].inputs) users[v].push_back(i);
  }
  auto isOutput = [&](ValueId v) {
    return std::find(g.outputs.begin(), g.outputs.end(), v) != g.outputs.end();
  };
  // `v` flows only into node `to` and is neither a graph result nor a view.
  auto privateEdge = [&](ValueId v, std::size_t to) {
    return users[v].size() == 1 && users[v][0] == to && !isOutput(v) &&
           producer[v] != kUndefined && a.effects[producer[v]] == MemoryEffect::ReadOnly;
  };
  std::vector<bool> taken(g.nodes.size(), false);
  std::vector<Region> regions;
  for (const std::size_t first : a.order) {
    if (taken[first]) continue;
    Region region;
    region.id = regions.size();
    region.nodes = {first};
    const Node& n = g.nodes[first];
    const ValueId result = n.outputs.front();
    if (users[result].size() == 1) {
      const std::size_t next = users[result][0];
      const Node& m = g.nodes[next];
      if (!taken[next] && privateEdge(result, next)) {
        if (n.op == OpType::Add && m.op == OpType::RMSNorm && m.inputs.front() == result)
          region.fusion = FusionPattern::AddRMSNorm;
        else if (n.op == OpType::SiLU && m.op == OpType::Mul)
          region.fusion = FusionPattern::SiLUMul;
        if (region.fusion != FusionPattern::None) region.nodes.push_back(next);
      }
    }
    if (region.fusion != FusionPattern::None) {
      for (const std::size_t i : region.nodes)
        for (const ValueId v : g.nodes[i].inputs)
          if (!a.types[v].isContiguous()) {
            region.fusion = FusionPattern::None;
            region.nodes = {first};
          }
    }
    auto inside = [&](std::size_t node) {
      return std::find(region.nodes.begin(), region.nodes.end(), node) != region.nodes.end();
    };
    for (const std::size_t i : region.nodes) {
      taken[i] = true;
      for (const ValueId v : g.nodes[i].inputs)
        if ((producer[v] == kUndefined || !inside(producer[v])) &&
            std::find(region.inputs.begin(), region.inputs.end(), v) == region.inputs.end())
          region.inputs.push_back(v);
    }
    for (const std::size_t i : region.nodes)
      for (const ValueId v : g.nodes[i].outputs) {
        bool escapes = isOutput(v);
        for (const std::size_t u : users[v]) escapes = escapes || !inside(u);
        if (escapes) region.outputs.push_back(v);
      }
    if (region.outputs.empty()) region.outputs.push_back(g.nodes[region.nodes.back()].outputs.front());
    regions.push_back(std::move(region));
  }
  return regions;
}

}  // namespace analyzer

// ----------------------------------------------------------------- reference
namespace validation {
namespace {

// The value device storage of `dtype` holds for x (fp16: nearest, ties away
// from zero, through the runtime's own host conversion).
double stored(double x, DType dtype) {
  switch (dtype) {
    case DType::Float16: {
      const float f = static_cast<float>(x);
      std::uint16_t bits = 0;
      float back = 0.0f;
      if (tmc_host_encode(&f, 1, TMC_F16, &bits) != 0 || tmc_host_decode(&bits, 1, TMC_F16, &back) != 0)
        throw std::runtime_error(tmc_last_error());
      return back;
    }
    case DType::Float32: return static_cast<float>(x);
    case DType::Int32: return std::trunc(x);
    case DType::BFloat16: return x;
  }
  return x;
}

// Logical values of a view from its base's logical values.
std::vector<double> viewValues(const Node& n, const analyzer::AnalyzedGraph& a,
                               const std::vector<double>& base) {
  if (n.op != OpType::Transpose) return base;
  const TensorType& in = a.types[n.inputs.front()];
  const auto* at = std::get_if<TransposeAttributes>(&n.attributes);
  const std::size_t i = static_cast<std::size_t>(at->first), j = static_cast<std::size_t>(at->second);
  const TensorType& out = a.types[n.outputs.front()];
  TensorType denseIn = in;
  denseIn.layout = Layout::Contiguous;
  denseIn.explicitStrides.clear();
  const std::vector<std::size_t> inStrides = denseIn.strides();
  std::vector<double> result(out.elementCount());
  std::vector<std::size_t> index(out.shape.size(), 0);
  for (std::size_t linear = 0; linear < result.size(); ++linear) {
    std::size_t offset = 0;
    for (std::size_t d = 0; d < index.size(); ++d) {
      const std::size_t src = d == i ? j : d == j ? i : d;  // axis of the input
      offset += index[d] * inStrides[src];
    }
    result[linear] = base[offset];
    for (std::size_t d = index.size(); d-- > 0;) {
      if (++index[d] < out.shape[d]) break;
      index[d] = 0;
    }
  }
  return result;
}

}  // namespace

GraphReference evaluateGraph(const analyzer::AnalyzedGraph& a, const GraphInputs& inputs) {
  const TensorGraph& g = a.graph;
  GraphReference r;
  r.values.resize(g.values.size());
  for (const ValueId v : g.inputs) {
    const auto it = inputs.find(v);
    const std::size_t count = a.types[v].elementCount();
    if (it == inputs.end() || it->second.size() != count)
      throw std::invalid_argument("Graph input " + std::to_string(v) + " needs " + std::to_string(count) + " host values.");
    auto& out = r.values[v];
    out.resize(count);
    for (std::size_t k = 0; k < count; ++k) out[k] = stored(it->second[k], a.types[v].dtype);
  }
  for (const std::size_t index : a.order) {
    const Node& n = g.nodes[index];
    const ValueId o = n.outputs.front();
    const TensorType& type = a.types[o];
    if (isViewOp(n.op)) {
      r.values[o] = viewValues(n, a, r.values[n.inputs.front()]);
      continue;
    }
    const auto& x = r.values[n.inputs.front()];
    std::vector<double> y(type.elementCount());
    switch (n.op) {
      case OpType::Add:
      case OpType::Mul: {
        const auto& b = r.values[n.inputs[1]];
        for (std::size_t k = 0; k < y.size(); ++k) y[k] = n.op == OpType::Add ? x[k] + b[k] : x[k] * b[k];
        break;
      }
      case OpType::SiLU:
        for (std::size_t k = 0; k < y.size(); ++k) y[k] = x[k] / (1.0 + std::exp(-x[k]));
        break;
      case OpType::RMSNorm: {
        const auto& w = r.values[n.inputs[1]];
        const double eps = std::get<RMSNormAttributes>(n.attributes).epsilon;
        const std::size_t width = type.shape.back();
        for (std::size_t row = 0; row < y.size() / width; ++row) {
          double squares = 0.0;
          for (std::size_t c = 0; c < width; ++c) squares += x[row * width + c] * x[row * width + c];
          const double inverse = 1.0 / std::sqrt(squares / static_cast<double>(width) + eps);
          for (std::size_t c = 0; c < width; ++c)
            y[row * width + c] = x[row * width + c] * inverse * w[c];
        }
        break;
      }
      case OpType::MatMul: {
        const auto& b = r.values[n.inputs[1]];
        const std::size_t m = type.shape[0], cols = type.shape[1];
        const std::size_t k = a.types[n.inputs[0]].shape[1];
        // y[i][j] accumulates t = 0, 1, ... in order; the t loop runs
        // outside the j loop so that b is read row by row
        for (std::size_t i = 0; i < m; ++i) {
          double* row = y.data() + i * cols;
          for (std::size_t t = 0; t < k; ++t) {
            const double xv = x[i * k + t];
            const double* brow = b.data() + t * cols;
            for (std::size_t j = 0; j < cols; ++j) row[j] += xv * brow[j];
          }
        }
        break;
      }
      case OpType::Embedding: {
        const auto& ids = r.values[n.inputs[1]];
        const std::size_t width = type.shape.back();
        const std::size_t rows = a.types[n.inputs[0]].shape[0];
        for (std::size_t k = 0; k < y.size(); ++k) {
          const double id = ids[k / width];
          if (id < 0 || id >= static_cast<double>(rows))
            throw std::invalid_argument("Embedding index is out of range.");
          y[k] = x[static_cast<std::size_t>(id) * width + k % width];
        }
        break;
      }
      default:
        throw std::invalid_argument(std::string("No graph reference for ") + opName(n.op) + ".");
    }
    for (double& value : y) value = stored(value, type.dtype);
    r.values[o] = std::move(y);
  }
  for (const ValueId v : g.outputs) r.outputs.push_back(r.values[v]);
  return r;
}

}  // namespace validation

// ------------------------------------------------------------------ compile
namespace runtime {
namespace {

constexpr std::size_t kWarmup = planner::kTuningWarmup;
constexpr std::size_t kSamples = planner::kTuningSamples;
const std::vector<std::size_t> kRegionThreads = {64, 128, 256};

hip::ElementType elementOf(DType d) { return static_cast<hip::ElementType>(static_cast<int>(d)); }

const char* keyType(DType d) { return d == DType::Float16 ? "f16" : d == DType::Float32 ? "f32" : "i32"; }

std::string epsText(float eps) {
  std::ostringstream s;
  s.precision(9);
  s << eps;
  return s.str();
}

// Tolerances of a region or graph output check: fp16 storage 2e-3 absolute
// and relative, fp32 1e-5 absolute and 1e-4 relative.
std::pair<double, double> tolerance(DType d) {
  return d == DType::Float16 ? std::make_pair(2e-3, 2e-3) : std::make_pair(1e-5, 1e-4);
}

// Logical values of a buffer that stores `type` (a view reads its base).
std::vector<float> logicalRead(const hip::BufferHandle& buffer, const TensorType& type) {
  const std::vector<float> storage = buffer->read();
  if (type.isContiguous())
    return std::vector<float>(storage.begin(), storage.begin() + static_cast<long>(type.elementCount()));
  const std::vector<std::size_t> strides = type.strides();
  std::vector<float> out(type.elementCount());
  std::vector<std::size_t> index(type.shape.size(), 0);
  for (std::size_t linear = 0; linear < out.size(); ++linear) {
    std::size_t offset = 0;
    for (std::size_t d = 0; d < index.size(); ++d) offset += index[d] * strides[d];
    out[linear] = storage[offset];
    for (std::size_t d = index.size(); d-- > 0;) {
      if (++index[d] < type.shape[d]) break;
      index[d] = 0;
    }
  }
  return out;
}

// One kernel of a node: the resolved key, its operands (graph values) in
// the key's binding order, and extra buffers (fused region scratch).
struct KernelStep {
  std::size_t node = 0;
  hip::GeneratedKernel kernel;
  std::vector<ValueId> inputs;
  std::vector<ValueId> outputs;
  std::vector<hip::ElementType> inputTypes;
  std::vector<hip::ElementType> outputTypes;
  bool scratchSum = false;  // fused Add + RMSNorm: the sum goes to a scratch buffer
};

struct NodeTuning {
  std::size_t threads = 256;
  bool rmsBaseline = false;
};

KernelStep nodeKernel(const analyzer::AnalyzedGraph& a, std::size_t index, const NodeTuning& tune) {
  const Node& n = a.graph.nodes[index];
  const ValueId o = n.outputs.front();
  const TensorType& out = a.types[o];
  KernelStep k;
  k.node = index;
  k.outputs = {o};
  k.outputTypes = {elementOf(out.dtype)};
  auto needContiguous = [&](ValueId v) {
    if (!a.types[v].isContiguous())
      throw std::invalid_argument(std::string(opName(n.op)) +
                                  " on the gfx950 graph path reads contiguous operands.");
  };
  std::ostringstream key;
  switch (n.op) {
    case OpType::Add:
    case OpType::Mul:
    case OpType::SiLU: {
      for (const ValueId v : n.inputs) needContiguous(v);
      const char* name = n.op == OpType::Add ? "add" : n.op == OpType::Mul ? "mul" : "silu";
      key << name << "?count=" << out.elementCount() << "&dtype=" << keyType(out.dtype)
          << "&threads=" << tune.threads;
      k.kernel = {key.str(), name, (out.elementCount() + tune.threads - 1) / tune.threads, tune.threads};
      k.inputs = n.inputs;
      break;
    }
    case OpType::RMSNorm: {
      needContiguous(n.inputs[0]);
      RMSNormOp op{a.types[n.inputs[0]], a.types[n.inputs[1]], out,
                   std::get<RMSNormAttributes>(n.attributes).epsilon};
      k.kernel = tune.rmsBaseline ? hip::emitRMSNormBaseline(op) : hip::emitRMSNorm(op, tune.threads);
      k.inputs = n.inputs;
      break;
    }
    case OpType::MatMul: {
      // x [M, K] times the Transpose view of a contiguous [N, K] weight
      // (nn.Linear layout): the decode GEMV on the view's base storage.
      const TensorType& x = a.types[n.inputs[0]];
      const TensorType& w = a.types[n.inputs[1]];
      needContiguous(n.inputs[0]);
      const std::size_t m = x.shape[0], kin = x.shape[1], cols = w.shape[1];
      const std::vector<std::size_t> s = w.strides();
      if (w.isContiguous() || s[0] != 1 || s[1] != kin || !a.aliasOf[n.inputs[1]])
        throw std::invalid_argument(
            "MatMul on the gfx950 graph path takes its weight as the Transpose of a contiguous "
            "[N, K] tensor (nn.Linear layout).");
      if (x.dtype != DType::Float16)
        throw std::invalid_argument("MatMul on the gfx950 graph path runs on fp16 operands.");
      key << "decode_gemv?batch=" << m << "&in=" << kin << "&out=" << cols
          << "&dtype=f16&out_dtype=f16";
      k.kernel = {key.str(), "decode_gemv", (cols + 3) / 4, 256};
      k.inputs = {n.inputs[0], *a.aliasOf[n.inputs[1]]};
      break;
    }
    case OpType::Embedding: {
      const TensorType& table = a.types[n.inputs[0]];
      key << "embedding?rows=" << a.types[n.inputs[1]].elementCount() << "&hidden="
          << table.shape[1] << "&vocab=" << table.shape[0] << "&dtype=" << keyType(table.dtype);
      k.kernel = {key.str(), "embedding", a.types[n.inputs[1]].elementCount(), 256};
      needContiguous(n.inputs[1]);
      k.inputs = {n.inputs[1], n.inputs[0]};  // the kernel takes the ids first
      break;
    }
    default:
      throw std::invalid_argument(std::string("No gfx950 kernel for ") + opName(n.op) + ".");
  }
  for (const ValueId v : k.inputs) k.inputTypes.push_back(elementOf(a.types[v].dtype));
  return k;
}

// The fused kernel of a region at `threads`.
KernelStep fusedKernel(const analyzer::AnalyzedGraph& a, const analyzer::Region& region,
                       std::size_t threads) {
  const Node& first = a.graph.nodes[region.nodes[0]];
  const Node& second = a.graph.nodes[region.nodes[1]];
  const ValueId o = second.outputs.front();
  const TensorType& out = a.types[o];
  KernelStep k;
  k.node = region.nodes[0];
  std::ostringstream key;
  if (region.fusion == analyzer::FusionPattern::AddRMSNorm) {
    const std::size_t width = out.shape.back();
    key << "add_rmsnorm?rows=" << out.elementCount() / width << "&width=" << width
        << "&eps=" << epsText(std::get<RMSNormAttributes>(second.attributes).epsilon)
        << "&dtype=" << keyType(out.dtype) << "&threads=" << threads;
    k.kernel = {key.str(), "add_rmsnorm", out.elementCount() / width, threads};
    k.inputs = {first.inputs[0], first.inputs[1], second.inputs[1]};
    k.outputs = {first.outputs.front(), o};  // the sum goes to scratch storage
    k.scratchSum = true;
    k.outputTypes = {elementOf(out.dtype), elementOf(out.dtype)};
  } else {
    const ValueId activated = first.outputs.front();
    const ValueId other = second.inputs[0] == activated ? second.inputs[1] : second.inputs[0];
    key << "silu_mul?count=" << out.elementCount() << "&dtype=" << keyType(out.dtype)
        << "&threads=" << threads;
    k.kernel = {key.str(), "silu_mul", (out.elementCount() + threads - 1) / threads, threads};
    k.inputs = {first.inputs[0], other};
    k.outputs = {o};
    k.outputTypes = {elementOf(out.dtype)};
  }
  for (const ValueId v : k.inputs) k.inputTypes.push_back(elementOf(a.types[v].dtype));
  return k;
}

std::unique_ptr<hip::PreparedExecution> prepareStep(hip::HipRuntime& rt, const KernelStep& k,
                                                    const std::vector<hip::BufferHandle>& buffers,
                                                    const hip::BufferHandle& scratch,
                                                    std::string& error) {
  const auto pipeline = rt.createComputePipeline(k.kernel.source, k.kernel.functionName);
  if (!pipeline.pipelineCreationPassed) {
    error = pipeline.errorMessage;
    return nullptr;
  }
  error = hip::checkBufferInterface(pipeline, k.inputTypes, k.outputTypes);
  if (!error.empty()) return nullptr;
  std::vector<hip::BufferHandle> ins, outs;
  for (const ValueId v : k.inputs) ins.push_back(buffers[v]);
  for (std::size_t i = 0; i < k.outputs.size(); ++i)
    outs.push_back(k.scratchSum && i == 0 ? scratch : buffers[k.outputs[i]]);
  auto prepared = rt.prepareBuffers(ins, outs, {k.kernel.threadgroupCount, k.kernel.threadsPerThreadgroup});
  error = prepared.errorMessage;
  return std::move(prepared.execution);
}

std::unique_ptr<hip::PreparedSequence> sequenceOf(
    hip::HipRuntime& rt, const std::vector<std::unique_ptr<hip::PreparedExecution>>& steps,
    std::string& error) {
  std::vector<const hip::PreparedExecution*> raw;
  for (const auto& s : steps) raw.push_back(s.get());
  auto made = rt.prepareSequence(raw);
  error = made.errorMessage;
  return std::move(made.execution);
}

hip::BufferHandle newBuffer(hip::HipRuntime& rt, const TensorType& type, const std::vector<double>* init) {
  std::vector<float> data;
  if (init) data.assign(init->begin(), init->end());
  auto made = rt.createBuffer(init ? data.size() : type.storageElementCount(),
                              init ? data.data() : nullptr, elementOf(type.dtype));
  if (!made.buffer) throw std::runtime_error(made.errorMessage);
  return made.buffer;
}

std::vector<float> asFloats(const std::vector<double>& v) { return std::vector<float>(v.begin(), v.end()); }

struct RegionChoice {
  bool fused = false;
  std::size_t threads = 0;
};

// Region tuning: the unfused kernels must reproduce the reference; each
// fused candidate must too, and is admitted at >= 1.05x in two paired
// rounds (the lower speedup ranks it).
RegionChoice tuneRegion(hip::HipRuntime& rt, const analyzer::AnalyzedGraph& a,
                        const analyzer::Region& region, const std::vector<KernelStep>& baseline,
                        const validation::GraphReference& ref, std::ostream& log) {
  const std::string tag = "[graph] region " + std::to_string(region.id) + " (" +
                          analyzer::fusionName(region.fusion) + ")";
  const ValueId out = region.outputs.front();
  const TensorType& outType = a.types[out];
  // Region-local buffers: inputs hold their reference values (contiguous).
  std::vector<hip::BufferHandle> buffers(a.graph.values.size());
  for (const ValueId v : region.inputs) buffers[v] = newBuffer(rt, a.types[v], &ref.values[v]);
  for (const auto& k : baseline)
    for (const ValueId v : k.outputs) buffers[v] = newBuffer(rt, a.types[v], nullptr);
  std::vector<std::unique_ptr<hip::PreparedExecution>> steps;
  std::string error;
  for (const auto& k : baseline) {
    auto step = prepareStep(rt, k, buffers, nullptr, error);
    if (!step) throw std::runtime_error(tag + ": unfused kernel " + k.kernel.source + ": " + error);
    steps.push_back(std::move(step));
  }
  auto unfused = sequenceOf(rt, steps, error);
  if (!unfused) throw std::runtime_error(tag + ": unfused sequence: " + error);
  const auto run = unfused->execute();
  if (!run.executionPassed) throw std::runtime_error(tag + ": unfused run: " + run.errorMessage);
  const auto [atol, rtol] = tolerance(outType.dtype);
  const auto check = validation::compare(logicalRead(buffers[out], outType), ref.values[out], atol, rtol);
  if (!check.passed) throw std::runtime_error(tag + ": unfused kernels disagree with the reference: " + check.errorMessage);
  error = benchmark::warmup(benchmark::sampler(*unfused), kWarmup);
  if (!error.empty()) throw std::runtime_error(tag + ": unfused warmup: " + error);
  log << tag << ": unfused kernels match the reference\n";

  RegionChoice best;
  double bestSpeedup = 0.0;
  const auto hardware = rt.hardwareInfo();
  for (const std::size_t threads : kRegionThreads) {
    log << tag << ": fused at " << threads << " threads: ";
    if (threads > hardware.maxThreadsPerThreadgroup) {
      log << "over the workgroup limit\n";
      continue;
    }
    const KernelStep k = fusedKernel(a, region, threads);
    auto candidateBuffers = buffers;
    candidateBuffers[out] = newBuffer(rt, outType, nullptr);
    const hip::BufferHandle scratch = k.scratchSum ? newBuffer(rt, outType, nullptr) : nullptr;
    auto step = prepareStep(rt, k, candidateBuffers, scratch, error);
    if (!step) {
      log << "not prepared: " << error << '\n';
      continue;
    }
    std::vector<std::unique_ptr<hip::PreparedExecution>> one;
    one.push_back(std::move(step));
    auto fused = sequenceOf(rt, one, error);
    if (!fused) {
      log << "no sequence: " << error << '\n';
      continue;
    }
    const auto fusedRun = fused->execute();
    const auto fusedCheck = fusedRun.executionPassed
                                ? validation::compare(logicalRead(candidateBuffers[out], outType),
                                                      ref.values[out], atol, rtol)
                                : validation::ValidationResult{};
    if (!fusedRun.executionPassed || !fusedCheck.passed) {
      log << "rejected, output check: "
          << (fusedRun.executionPassed ? fusedCheck.errorMessage : fusedRun.errorMessage) << '\n';
      continue;
    }
    error = benchmark::warmup(benchmark::sampler(*fused), kWarmup);
    if (!error.empty()) {
      log << "warmup failed: " << error << '\n';
      continue;
    }
    const auto first = benchmark::measurePair(benchmark::sampler(*unfused), benchmark::sampler(*fused), kSamples);
    std::optional<benchmark::PairedResult> second;
    if (first.passed && first.speedup >= planner::kMinimumSpeedup)
      second = benchmark::measurePair(benchmark::sampler(*unfused), benchmark::sampler(*fused), kSamples);
    const auto decision = planner::admissionDecision(first, second);
    log << "output matches, unfused " << first.baseline.medianUs << " us, fused "
        << first.candidate.medianUs << " us, x" << decision.conservativeSpeedup
        << (decision.admitted ? " -> admitted\n" : " -> not admitted (" + decision.reason + ")\n");
    if (decision.admitted && decision.conservativeSpeedup > bestSpeedup) {
      bestSpeedup = decision.conservativeSpeedup;
      best = {true, threads};
    }
  }
  log << tag << ": " << (best.fused ? "fused kernel at " + std::to_string(best.threads) + " threads"
                                    : std::string("unfused kernels"))
      << '\n';
  return best;
}

}  // namespace

CompiledGraph::CompiledGraph(analyzer::AnalyzedGraph graph, std::vector<hip::BufferHandle> buffers,
                             std::vector<ExecutionUnit> units)
    : graph_(std::move(graph)), buffers_(std::move(buffers)), units_(std::move(units)) {}

std::vector<std::string> CompiledGraph::unitNames() const {
  std::vector<std::string> names;
  for (const auto& u : units_) names.push_back(u.name);
  return names;
}

GraphExecutionResult CompiledGraph::run() const {
  GraphExecutionResult result;
  double gpu = 0.0, cpu = 0.0;
  bool timed = true;
  for (const auto& unit : units_) {
    const auto r = unit.execution->execute();
    if (!r.executionPassed) {
      result.errorMessage = unit.name + ": " + r.errorMessage;
      return result;
    }
    if (r.gpuExecutionTimeUs) gpu += *r.gpuExecutionTimeUs;
    else timed = false;
    cpu += r.cpuSubmitToCompletionTimeUs;
  }
  for (const ValueId v : graph_.graph.outputs)
    result.outputs.push_back(logicalRead(buffers_[graph_.aliasOf[v] ? *graph_.aliasOf[v] : v], graph_.types[v]));
  if (timed) result.gpuExecutionTimeUs = gpu;
  result.cpuSubmitToCompletionTimeUs = cpu;
  result.passed = true;
  return result;
}

GraphCompilation compileGraph(hip::HipRuntime& rt, const TensorGraph& graph, const GraphInputs& inputs,
                              std::ostream& log) {
  GraphCompilation result;
  try {
    if (!rt.isAvailable()) throw std::runtime_error(rt.initializationError());
    analyzer::AnalyzedGraph a = analyzer::analyze(graph);
    const std::vector<analyzer::Region> regions = analyzer::formRegions(a);
    log << "[graph] analysis: " << graph.nodes.size() << " nodes, " << regions.size() << " regions\n";
    const validation::GraphReference ref = validation::evaluateGraph(a, inputs);

    // Kernel settings per node: every RMSNorm is tuned on its reference input.
    std::vector<NodeTuning> tuning(graph.nodes.size());
    for (const std::size_t i : a.order) {
      const Node& n = a.graph.nodes[i];
      if (n.op != OpType::RMSNorm) continue;
      RMSNormOp op{a.types[n.inputs[0]], a.types[n.inputs[1]], a.types[n.outputs[0]],
                   std::get<RMSNormAttributes>(n.attributes).epsilon};
      auto tuned = planner::tuneRMSNorm(rt, op, asFloats(ref.values[n.inputs[0]]),
                                        asFloats(ref.values[n.inputs[1]]), kRegionThreads, log);
      if (!tuned.success) throw std::runtime_error("RMSNorm node " + std::to_string(i) + ": " + tuned.errorMessage);
      tuning[i] = {tuned.selectedThreads, tuned.usedBaseline};
    }

    // Baseline kernels of each region and the fusion decisions.
    std::vector<std::vector<KernelStep>> baseline(regions.size());
    std::vector<RegionChoice> choices(regions.size());
    for (const auto& region : regions) {
      for (const std::size_t i : region.nodes)
        if (!isViewOp(a.graph.nodes[i].op)) baseline[region.id].push_back(nodeKernel(a, i, tuning[i]));
      if (region.fusion != analyzer::FusionPattern::None)
        choices[region.id] = tuneRegion(rt, a, region, baseline[region.id], ref, log);
    }

    // Graph storage: inputs with their host values, one buffer per other
    // materialized value, views sharing their base's buffer.
    std::vector<hip::BufferHandle> buffers(a.graph.values.size());
    for (const ValueId v : a.graph.inputs) buffers[v] = newBuffer(rt, a.types[v], nullptr);
    for (const ValueId v : a.graph.inputs) {
      const auto& host = inputs.at(v);
      if (!a.types[v].isContiguous() || host.size() != a.types[v].storageElementCount())
        throw std::invalid_argument("Graph inputs must be contiguous tensors with one host value per element.");
      const std::string err = rt.writeBuffer(buffers[v], host.data(), host.size());
      if (!err.empty()) throw std::runtime_error(err);
    }
    for (const std::size_t i : a.order) {
      const ValueId o = a.graph.nodes[i].outputs.front();
      if (!a.aliasOf[o]) buffers[o] = newBuffer(rt, a.types[o], nullptr);
    }
    for (ValueId v = 0; v < buffers.size(); ++v)
      if (a.aliasOf[v]) buffers[v] = buffers[*a.aliasOf[v]];

    std::vector<CompiledGraph::ExecutionUnit> units;
    for (const auto& region : regions) {
      if (baseline[region.id].empty()) continue;  // views only: no work
      CompiledGraph::ExecutionUnit unit;
      std::string error;
      if (choices[region.id].fused) {
        const KernelStep k = fusedKernel(a, region, choices[region.id].threads);
        const hip::BufferHandle scratch =
            k.scratchSum ? newBuffer(rt, a.types[region.outputs.front()], nullptr) : nullptr;
        auto step = prepareStep(rt, k, buffers, scratch, error);
        if (!step) throw std::runtime_error(k.kernel.source + ": " + error);
        unit.steps.push_back(std::move(step));
        unit.name = std::string(analyzer::fusionName(region.fusion)) + " (fused)";
      } else {
        for (const auto& k : baseline[region.id]) {
          auto step = prepareStep(rt, k, buffers, nullptr, error);
          if (!step) throw std::runtime_error(k.kernel.source + ": " + error);
          unit.steps.push_back(std::move(step));
        }
        unit.name = region.fusion == analyzer::FusionPattern::None
                        ? std::string(opName(a.graph.nodes[region.nodes.front()].op))
                        : std::string(analyzer::fusionName(region.fusion)) + " (unfused)";
      }
      unit.execution = sequenceOf(rt, unit.steps, error);
      if (!unit.execution) throw std::runtime_error(unit.name + ": " + error);
      units.push_back(std::move(unit));
    }
    for (const ValueId v : graph.outputs) result.outputTypes.push_back(a.types[v]);
    result.referenceOutputs = ref.outputs;
    result.executable = std::make_unique<CompiledGraph>(std::move(a), std::move(buffers), std::move(units));
    log << "[graph] compiled: " << result.executable->unitNames().size() << " execution units\n";
  } catch (const std::exception& e) {
    result.errorMessage = e.what();
  }
  return result;
}

}  // namespace runtime

}  // namespace tensor
