// The graph path on the gfx950 backend: compileGraph / CompiledGraph with
// the interface of the reference's src/runtime/GraphExecutor.hpp:9-47
// (GraphExecutor.cpp:346-430), over the TensorIR graph of TensorIR.hpp.
//
//   analyze       type inference and view aliasing (GraphAnalyzer.cpp), for
//                 the operations the gfx950 kernels implement: Add, Mul, SiLU,
//                 RMSNorm, MatMul, Embedding and the Reshape / View /
//                 Transpose views; any other operation is rejected by name.
//   formRegions   fusion regions (PatternAnalyzer.cpp:34-131): Add -> RMSNorm
//                 and SiLU -> Mul over exclusive, contiguous edges.
//   evaluateGraph the double-precision graph reference (GraphReference.cpp)
//                 that every tuned kernel is validated against.
//   compileGraph  tunes every RMSNorm kernel (tuneRMSNorm), admits each
//                 fusion region's fused kernel only when it matches the
//                 reference and is >= 1.05x faster than the unfused kernels in
//                 two paired rounds, then prepares one HIP-graph sequence per
//                 region over device buffers (views share their base's).
#pragma once

#include "HipRuntime.hpp"
#include "TensorIR.hpp"

#include <cstddef>
#include <iosfwd>
#include <memory>
#include <optional>
#include <string>
#include <vector>

namespace tensor {

namespace analyzer {

enum class MemoryEffect { ReadOnly, View };

struct AnalyzedGraph {
  TensorGraph graph;
  std::vector<TensorType> types;               // by ValueId
  std::vector<std::size_t> order;              // node execution order
  std::vector<MemoryEffect> effects;           // by node
  std::vector<std::optional<ValueId>> aliasOf;  // by ValueId: storage root of a view
};

// Throws std::invalid_argument naming the operation or value at fault.
[[nodiscard]] AnalyzedGraph analyze(const TensorGraph& graph);

enum class FusionPattern { None, AddRMSNorm, AddLayerNorm, SiLUMul, LinearReLU };
[[nodiscard]] const char* fusionName(FusionPattern pattern);

struct Region {
  std::size_t id = 0;
  std::vector<std::size_t> nodes;
  std::vector<ValueId> inputs;
  std::vector<ValueId> outputs;
  FusionPattern fusion = FusionPattern::None;
};

[[nodiscard]] std::vector<Region> formRegions(const AnalyzedGraph& graph);

}  // namespace analyzer

namespace validation {

// Logical (row-major over each value's shape) values of every graph value,
// each stored value rounded to its dtype as device storage holds it.
struct GraphReference {
  std::vector<std::vector<double>> values;
  std::vector<std::vector<double>> outputs;
};

[[nodiscard]] GraphReference evaluateGraph(const analyzer::AnalyzedGraph& graph,
                                           const GraphInputs& inputs);

}  // namespace validation

namespace runtime {

struct GraphExecutionResult {
  bool passed = false;
  std::vector<std::vector<float>> outputs;
  std::optional<double> gpuExecutionTimeUs;
  double cpuSubmitToCompletionTimeUs = 0.0;
  std::string errorMessage;
};

class CompiledGraph {
 public:
  struct ExecutionUnit {
    std::string name;
    // The kernels the sequence replays; declared first so that they outlive it.
    std::vector<std::unique_ptr<hip::PreparedExecution>> steps;
    std::unique_ptr<hip::PreparedSequence> execution;
  };

  CompiledGraph(analyzer::AnalyzedGraph graph, std::vector<hip::BufferHandle> buffers,
                std::vector<ExecutionUnit> units);
  // Runs every unit in order and reads the graph outputs.
  [[nodiscard]] GraphExecutionResult run() const;
  [[nodiscard]] std::vector<std::string> unitNames() const;

 private:
  analyzer::AnalyzedGraph graph_;
  std::vector<hip::BufferHandle> buffers_;
  std::vector<ExecutionUnit> units_;
};

struct GraphCompilation {
  std::unique_ptr<CompiledGraph> executable;
  std::vector<TensorType> outputTypes;
  std::vector<std::vector<double>> referenceOutputs;
  std::string errorMessage;
};

[[nodiscard]] GraphCompilation compileGraph(hip::HipRuntime& runtime, const TensorGraph& graph,
                                            const GraphInputs& inputs, std::ostream& log);

}  // namespace runtime

}  // namespace tensor
