// ref_driver.cpp — C entry points around the reference's own CPU oracle.
//
// TEST INFRASTRUCTURE ONLY.  Compiled (by oracle/Makefile, target `ref`)
// together with the reference sources that lie under /root/reference/src:
//   tensor/TensorIR.cpp, analyzer/GraphAnalyzer.cpp,
//   validation/GraphReference.cpp, validation/Validator.cpp
// into oracle/_ref/libtmc_ref.so.  Each function below builds a small
// TensorIR graph, runs tensor::validation::evaluateGraph
// (GraphReference.cpp:98-339) and returns its results, so that
// tests/golden/make_golden.py can record golden vectors that pin the
// clean-room restatement in oracle/tmc_oracle.c.  Nothing here is shipped.
#include "analyzer/GraphAnalyzer.hpp"
#include "validation/GraphReference.hpp"
#include "validation/Validator.hpp"

#include <cstring>
#include <exception>
#include <string>
#include <vector>

using namespace tensor;

namespace {

thread_local std::string g_error;

DType dtypeOf(int code) {
  switch (code) {
  case 0: return DType::Float16;
  case 2: return DType::BFloat16;
  case 3: return DType::Int32;
  default: return DType::Float32;
  }
}

std::vector<float> copy(const float *data, std::size_t count) {
  return std::vector<float>(data, data + count);
}

template <typename Fn> int guarded(Fn &&fn) {
  try {
    fn();
    return 0;
  } catch (const std::exception &error) {
    g_error = error.what();
    return 1;
  }
}

validation::GraphReference run(const TensorGraph &graph, const GraphInputs &inputs) {
  return validation::evaluateGraph(analyzer::analyze(graph), inputs);
}

void writeDoubles(const std::vector<double> &src, double *dst) {
  std::memcpy(dst, src.data(), src.size() * sizeof(double));
}

} // namespace

extern "C" {

const char *ref_last_error() { return g_error.c_str(); }

// Storage rounding of graph inputs (storeValue via evaluateGraph's input path).
int ref_store(const float *input, std::size_t count, int dtype, float *out) {
  return guarded([&] {
    TensorGraph graph;
    const auto x = graph.addInput("x", TensorType{{count}, dtypeOf(dtype)});
    graph.outputs = {graph.addNode(OpType::Reshape, {x}, ReshapeAttributes{{count}})};
    const auto result = run(graph, {{x, copy(input, count)}});
    std::memcpy(out, result.values[x].data(), count * sizeof(float));
  });
}

int ref_rmsnorm(const float *x, const float *w, std::size_t rows, std::size_t width, int dtype,
                float epsilon, double *out) {
  return guarded([&] {
    TensorGraph graph;
    const auto dt = dtypeOf(dtype);
    const auto xi = graph.addInput("x", TensorType{{rows, width}, dt});
    const auto wi = graph.addInput("w", TensorType{{width}, dt});
    graph.outputs = {graph.addNode(OpType::RMSNorm, {xi, wi}, RMSNormAttributes{epsilon, -1})};
    const auto result = run(graph, {{xi, copy(x, rows * width)}, {wi, copy(w, width)}});
    writeDoubles(result.outputs[0], out);
  });
}

int ref_add_rmsnorm(const float *x, const float *r, const float *w, std::size_t rows,
                    std::size_t width, int dtype, float epsilon, float *sum_stored,
                    double *out) {
  return guarded([&] {
    TensorGraph graph;
    const auto dt = dtypeOf(dtype);
    const auto xi = graph.addInput("x", TensorType{{rows, width}, dt});
    const auto ri = graph.addInput("r", TensorType{{rows, width}, dt});
    const auto wi = graph.addInput("w", TensorType{{width}, dt});
    const auto added = graph.addNode(OpType::Add, {xi, ri});
    graph.outputs = {graph.addNode(OpType::RMSNorm, {added, wi}, RMSNormAttributes{epsilon, -1})};
    const auto result = run(graph, {{xi, copy(x, rows * width)},
                                    {ri, copy(r, rows * width)},
                                    {wi, copy(w, width)}});
    std::memcpy(sum_stored, result.values[added].data(), rows * width * sizeof(float));
    writeDoubles(result.outputs[0], out);
  });
}

int ref_matmul(const float *a, const float *b, std::size_t m, std::size_t k, std::size_t n,
               int dtype, double *out) {
  return guarded([&] {
    TensorGraph graph;
    const auto dt = dtypeOf(dtype);
    const auto ai = graph.addInput("a", TensorType{{m, k}, dt});
    const auto bi = graph.addInput("b", TensorType{{k, n}, dt});
    graph.outputs = {graph.addNode(OpType::MatMul, {ai, bi})};
    const auto result = run(graph, {{ai, copy(a, m * k)}, {bi, copy(b, k * n)}});
    writeDoubles(result.outputs[0], out);
  });
}

int ref_silu_mul(const float *g, const float *u, std::size_t count, int dtype, double *out) {
  return guarded([&] {
    TensorGraph graph;
    const auto dt = dtypeOf(dtype);
    const auto gi = graph.addInput("g", TensorType{{count}, dt});
    const auto ui = graph.addInput("u", TensorType{{count}, dt});
    const auto activated = graph.addNode(OpType::SiLU, {gi});
    graph.outputs = {graph.addNode(OpType::Mul, {activated, ui})};
    const auto result = run(graph, {{gi, copy(g, count)}, {ui, copy(u, count)}});
    writeDoubles(result.outputs[0], out);
  });
}

// x [rows, heads, D] with per-row tables cos/sin [rows, 1, D/2] (fp32 graph).
int ref_rope(const float *x, const float *cosine, const float *sine, std::size_t rows,
             std::size_t heads, std::size_t head_dim, double *out) {
  return guarded([&] {
    TensorGraph graph;
    const auto xi = graph.addInput("x", TensorType{{rows, heads, head_dim}});
    const auto ci = graph.addInput("cos", TensorType{{rows, 1, head_dim / 2}});
    const auto si = graph.addInput("sin", TensorType{{rows, 1, head_dim / 2}});
    graph.outputs = {graph.addNode(OpType::RoPE, {xi, ci, si})};
    const auto tableCount = rows * (head_dim / 2);
    const auto result = run(graph, {{xi, copy(x, rows * heads * head_dim)},
                                    {ci, copy(cosine, tableCount)},
                                    {si, copy(sine, tableCount)}});
    writeDoubles(result.outputs[0], out);
  });
}

// softmax(q K^T * scale) V for `pairs` independent heads (fp32 graph):
// q [pairs,1,D], K and V [pairs,L,D], scale a scalar input.
int ref_attention(const float *q, const float *k, const float *v, std::size_t pairs,
                  std::size_t length, std::size_t head_dim, float scale, double *out) {
  return guarded([&] {
    TensorGraph graph;
    const auto qi = graph.addInput("q", TensorType{{pairs, 1, head_dim}});
    const auto ki = graph.addInput("k", TensorType{{pairs, length, head_dim}});
    const auto vi = graph.addInput("v", TensorType{{pairs, length, head_dim}});
    const auto si = graph.addInput("scale", TensorType{{}});
    const auto kt = graph.addNode(OpType::Transpose, {ki}, TransposeAttributes{1, 2});
    const auto scores = graph.addNode(OpType::MatMul, {qi, kt});
    const auto scaled = graph.addNode(OpType::Mul, {scores, si});
    const auto probabilities = graph.addNode(OpType::Softmax, {scaled}, SoftmaxAttributes{-1});
    graph.outputs = {graph.addNode(OpType::MatMul, {probabilities, vi})};
    const auto count = pairs * length * head_dim;
    const auto result = run(graph, {{qi, copy(q, pairs * head_dim)},
                                    {ki, copy(k, count)},
                                    {vi, copy(v, count)},
                                    {si, {scale}}});
    writeDoubles(result.outputs[0], out);
  });
}

// Gather rows of a [rows, width] table along axis 0 with int32 indices.
int ref_gather_rows(const float *table, std::size_t rows, std::size_t width,
                    const float *indices, std::size_t count, double *out) {
  return guarded([&] {
    TensorGraph graph;
    const auto ti = graph.addInput("table", TensorType{{rows, width}});
    const auto ii = graph.addInput("index", TensorType{{count}, DType::Int32});
    graph.outputs = {graph.addNode(OpType::Gather, {ti, ii}, GatherAttributes{0})};
    const auto result = run(graph, {{ti, copy(table, rows * width)}, {ii, copy(indices, count)}});
    writeDoubles(result.outputs[0], out);
  });
}

int ref_compare(const float *actual, const double *reference, std::size_t count, double atol,
                double rtol, double *max_abs, std::size_t *mismatches) {
  const auto result = validation::compare(std::vector<float>(actual, actual + count),
                                          std::vector<double>(reference, reference + count),
                                          atol, rtol);
  *max_abs = result.maxAbsoluteError;
  *mismatches = result.mismatchCount;
  return result.passed ? 1 : 0;
}

} // extern "C"
