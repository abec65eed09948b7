#include "Tuning.hpp"

#include "KernelRegistry.hpp"
#include "tmc_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <limits>
#include <ostream>
#include <sstream>
#include <stdexcept>
#include <utility>

namespace tensor {

namespace validation {

ValidationResult compare(const std::vector<float>& actual, const std::vector<double>& reference,
                         double absoluteTolerance, double relativeTolerance) {
  ValidationResult result;
  if (reference.empty() || actual.size() != reference.size()) {
    result.errorMessage = "Empty reference or unexpected output length.";
    return result;
  }
  for (std::size_t i = 0; i < reference.size(); ++i) {
    const double expected = reference[i];
    const double value = actual[i];
    const bool finite = std::isfinite(value) && std::isfinite(expected);
    const double error =
        finite ? std::abs(value - expected) : std::numeric_limits<double>::infinity();
    result.maxAbsoluteError = std::max(result.maxAbsoluteError, error);
    if (!finite || error > absoluteTolerance + relativeTolerance * std::abs(expected)) {
      if (result.mismatchCount == 0) {
        std::ostringstream message;
        message << "First mismatch at index " << i << ": expected=" << expected
                << ", actual=" << value;
        result.errorMessage = message.str();
      }
      ++result.mismatchCount;
    }
  }
  result.passed = result.mismatchCount == 0;
  return result;
}

std::vector<double> rmsNormReference(const RMSNormOp& op, const std::vector<float>& input,
                                     const std::vector<float>& weight) {
  op.validate();
  if (input.size() != op.input.elementCount() || weight.size() != op.weight.elementCount())
    throw std::invalid_argument("RMSNorm host inputs do not match TensorIR shapes.");
  const std::size_t width = op.input.shape.back();
  const std::size_t rows = input.size() / width;
  std::vector<double> out(input.size());
  for (std::size_t r = 0; r < rows; ++r) {
    double squares = 0.0;
    for (std::size_t c = 0; c < width; ++c) {
      const double x = input[r * width + c];
      squares += x * x;
    }
    const double inverse = 1.0 / std::sqrt(squares / static_cast<double>(width) + op.epsilon);
    for (std::size_t c = 0; c < width; ++c)
      out[r * width + c] =
          static_cast<double>(input[r * width + c]) * inverse * static_cast<double>(weight[c]);
  }
  return out;
}

}  // namespace validation

namespace hip {
namespace {

const char* keyDtype(ElementType type) {
  switch (type) {
  case ElementType::Float16: return "f16";
  case ElementType::Float32: return "f32";
  case ElementType::BFloat16: return "bf16";
  default: return "i32";
  }
}

ElementType elementTypeOf(DType dtype) {
  switch (dtype) {
  case DType::Float16: return ElementType::Float16;
  case DType::Float32: return ElementType::Float32;
  case DType::BFloat16: return ElementType::BFloat16;
  default: return ElementType::Int32;
  }
}

std::string epsilonText(float epsilon) {
  std::ostringstream s;
  s.precision(9);
  s << epsilon;
  return s.str();
}

}  // namespace

std::size_t decodeGEMVThreads(const DecodeGEMVConfig& c) {
  switch (c.algorithm) {
  case 2: return static_cast<std::size_t>(std::max(1, c.rowsPerWave * c.kSplit)) * 64;
  case 3: return static_cast<std::size_t>(std::max(1, c.kSplit)) * 64;
  case 4: return 128;
  default: return 256;
  }
}

std::size_t decodeGEMVLdsBytes(std::size_t batch, const DecodeGEMVConfig& c) {
  const std::size_t tile = 4 * 64 * sizeof(float);  // one 16x16 fp32 partial
  switch (c.algorithm) {
  case 2: {
    const std::size_t mt = std::min<std::size_t>(4, (std::min<std::size_t>(batch, 64) + 15) / 16);
    return static_cast<std::size_t>(c.rowsPerWave * c.kSplit) * (mt == 3 ? 4 : mt) * tile;
  }
  case 3: return static_cast<std::size_t>(c.kSplit * c.rowsPerWave) * tile;
  case 4: return 0;
  case 5: return (4 * 35 * static_cast<std::size_t>(c.rowsPerWave) + 128) * sizeof(float);
  default: return 4 * static_cast<std::size_t>(c.rowsPerWave) * 8 * sizeof(float);
  }
}

GeneratedKernel emitDecodeGEMV(std::size_t batch, std::size_t inputSize, std::size_t outputSize,
                               const DecodeGEMVConfig& config, const std::string& name,
                               ElementType elementType, ElementType outputType) {
  if (elementType != ElementType::Float16)
    throw std::invalid_argument("gfx950 decode GEMV stores fp16 weights and activations.");
  if (outputType != ElementType::Float16 && outputType != ElementType::Float32)
    throw std::invalid_argument("gfx950 decode GEMV writes fp16 or fp32 outputs.");
  std::ostringstream key;
  key << "decode_gemv?batch=" << batch << "&in=" << inputSize << "&out=" << outputSize
      << "&out_dtype=" << keyDtype(outputType);
  if (config.algorithm != 0)
    key << "&algorithm=" << config.algorithm << "&rows_per_wave=" << config.rowsPerWave
        << "&unroll=" << config.unroll << "&k_split=" << config.kSplit;
  return {key.str(), name, (outputSize + 3) / 4, decodeGEMVThreads(config)};
}

GeneratedKernel emitLinearBaseline(std::size_t batch, std::size_t inputSize,
                                   std::size_t outputSize, const std::string& name,
                                   ElementType elementType, ElementType outputType) {
  DecodeGEMVConfig baseline;
  baseline.algorithm = 4;
  auto kernel = emitDecodeGEMV(batch, inputSize, outputSize, baseline, name, elementType,
                               outputType);
  kernel.threadgroupCount = (batch * outputSize + 127) / 128;
  return kernel;
}

GeneratedKernel emitRMSNorm(const RMSNormOp& op, std::size_t threads) {
  op.validate();
  const std::size_t width = op.input.shape.back();
  const std::size_t rows = op.input.elementCount() / width;
  std::ostringstream key;
  key << "rmsnorm?rows=" << rows << "&width=" << width << "&eps=" << epsilonText(op.epsilon)
      << "&dtype=" << keyDtype(elementTypeOf(op.input.dtype)) << "&threads=" << threads;
  return {key.str(), "rmsnorm_" + std::to_string(threads), rows, threads};
}

GeneratedKernel emitRMSNormBaseline(const RMSNormOp& op) {
  auto kernel = emitRMSNorm(op, 256);
  kernel.source += "&variant=two_pass";
  kernel.functionName = "rmsnorm_baseline";
  return kernel;
}

}  // namespace hip

namespace planner {
namespace {

constexpr std::size_t kMaximumCpuReferenceOperations = 64u * 1024u * 1024u;
// Shapes validated against the baseline's GPU output are large: fewer samples.
constexpr std::size_t kLargeShapeSamples = 9;

// The value a float takes once uploaded as fp16 (the runtime's own upload
// conversion, ties away from zero), so the CPU reference sees the stored
// values.
float roundHalf(float value) {
  std::uint16_t bits = 0;
  tmc_host_encode(&value, 1, TMC_F16, &bits);
  float stored = 0.0f;
  tmc_host_decode(&bits, 1, TMC_F16, &stored);
  return stored;
}

// y[b, n] = sum_k x[b, k] W[n, k] in double over the stored (fp16) values.
std::vector<double> gemvReference(std::size_t batch, std::size_t in, std::size_t out,
                                  const std::vector<float>& x, const std::vector<float>& w) {
  std::vector<double> y(batch * out);
  std::vector<double> xs(x.size()), ws(w.size());
  std::transform(x.begin(), x.end(), xs.begin(), roundHalf);
  std::transform(w.begin(), w.end(), ws.begin(), roundHalf);
  for (std::size_t b = 0; b < batch; ++b)
    for (std::size_t n = 0; n < out; ++n) {
      double acc = 0.0;
      for (std::size_t k = 0; k < in; ++k) acc += xs[b * in + k] * ws[n * in + k];
      y[b * out + n] = acc;
    }
  return y;
}

std::string describe(const hip::DecodeGEMVConfig& c) {
  static const char* const names[] = {"default", "dot", "mfma", "mfma-rows", "linear",
                                      "persistent-dot"};
  std::ostringstream s;
  s << (c.algorithm >= 0 && c.algorithm <= 5 ? names[c.algorithm] : "?") << '(' << c.rowsPerWave
    << ',' << c.unroll << ',' << c.kSplit << ')';
  return s.str();
}

// ------------------------------------------------------------------ trials
// One entrant against the baseline: a paired round, a confirmation round
// only when the first reached the bar, and the admission rule over both.
struct Trial {
  benchmark::PairedResult first;
  std::optional<benchmark::PairedResult> confirmation;
  AdmissionDecision decision;
};

Trial runTrial(const benchmark::Sampler& baseline, const benchmark::Sampler& entrant,
               std::size_t samples) {
  Trial t;
  t.first = benchmark::measurePair(baseline, entrant, samples);
  if (t.first.passed && t.first.speedup >= kMinimumSpeedup)
    t.confirmation = benchmark::measurePair(baseline, entrant, samples);
  t.decision = admissionDecision(t.first, t.confirmation);
  return t;
}

std::string trialText(const Trial& t) {
  std::ostringstream s;
  if (!t.first.passed) return "timing failed (" + t.first.errorMessage + ")";
  s << "x" << t.first.speedup;
  if (t.confirmation && t.confirmation->passed) s << ", again x" << t.confirmation->speedup;
  s << (t.decision.admitted ? " -> admitted" : " -> not admitted: " + t.decision.reason);
  return s.str();
}

// ------------------------------------------------------------------ decode GEMV
// Builds one kernel over the tuning inputs, runs it once and checks its
// output; null with `why` set when it cannot be used.
using GemvBuilder = std::function<std::unique_ptr<hip::PreparedExecution>(
    const hip::GeneratedKernel& kernel, std::string& why)>;

// The sweep both tuneDecodeGEMV forms share: each candidate that passes the
// hardware filter is built and checked, warmed, and put through a trial
// against the baseline; the best conservative speedup is selected, else the
// linear baseline.
DecodeGEMVSelection sweepDecodeGEMV(hip::HipRuntime& runtime, std::size_t batch,
                                    std::size_t inputSize, std::size_t outputSize,
                                    const std::vector<hip::DecodeGEMVConfig>& candidates,
                                    hip::ElementType outputType,
                                    const benchmark::Sampler& baseline, const GemvBuilder& build,
                                    std::size_t samples, std::ostream& log) {
  DecodeGEMVSelection pick;
  const auto hardware = runtime.hardwareInfo();
  for (const auto& config : candidates) {
    log << "[decode-gemv] " << describe(config) << ": ";
    const std::string filtered =
        decodeGEMVHardwareFilter(config, batch, inputSize, outputSize, hardware);
    if (!filtered.empty()) {
      log << "Hardware Filter drops it (" << filtered << ")\n";
      continue;
    }
    std::string why;
    std::unique_ptr<hip::PreparedExecution> built;
    try {
      built = build(hip::emitDecodeGEMV(batch, inputSize, outputSize, config,
                                        "decode_gemv_candidate", hip::ElementType::Float16,
                                        outputType),
                    why);
    } catch (const std::exception& e) {
      why = e.what();
    }
    if (!built) {
      log << "unusable (" << why << ")\n";
      continue;
    }
    const auto sampler = benchmark::sampler(*built);
    const std::string cold = benchmark::warmup(sampler, kTuningWarmup);
    if (!cold.empty()) {
      log << "warmup failed (" << cold << ")\n";
      continue;
    }
    const Trial trial = runTrial(baseline, sampler, samples);
    log << trialText(trial) << '\n';
    if (trial.decision.admitted && trial.decision.conservativeSpeedup > pick.conservativeSpeedup) {
      pick.useBaseline = false;
      pick.config = config;
      pick.conservativeSpeedup = trial.decision.conservativeSpeedup;
    }
  }
  pick.success = true;
  if (pick.useBaseline) pick.config = hip::DecodeGEMVConfig{4, 1, 1, 1};
  log << "[decode-gemv] chosen: "
      << (pick.useBaseline ? std::string("linear baseline") : describe(pick.config))
      << " at x" << pick.conservativeSpeedup << '\n';
  return pick;
}

// Resolve `kernel`, prepare it over fresh fp16 buffers holding `input` and
// `weight`, run it once and compare with `expected` when given.
std::unique_ptr<hip::PreparedExecution> prepareGemv(hip::HipRuntime& runtime,
                                                    const hip::GeneratedKernel& kernel,
                                                    const std::vector<float>& input,
                                                    const std::vector<float>& weight,
                                                    std::size_t outputCount,
                                                    const std::vector<double>& expected,
                                                    std::string& why) {
  const auto fp16 = hip::ElementType::Float16;
  const auto pipeline = runtime.createComputePipeline(kernel.source, kernel.functionName);
  why = pipeline.pipelineCreationPassed ? hip::checkBufferInterface(pipeline, {fp16, fp16}, fp16)
                                        : pipeline.errorMessage;
  if (!why.empty()) return {};
  auto prepared =
      runtime.prepare({{input.data(), input.size(), fp16}, {weight.data(), weight.size(), fp16}},
                      outputCount, {kernel.threadgroupCount, kernel.threadsPerThreadgroup}, {},
                      fp16);
  if (!prepared.execution) {
    why = prepared.errorMessage;
    return {};
  }
  const auto run = prepared.execution->run();
  if (!run.executionPassed) {
    why = run.errorMessage;
    return {};
  }
  if (!expected.empty()) {
    const auto check = validation::compare(run.output, expected, 2e-2, 2e-2);
    if (!check.passed) {
      why = check.errorMessage;
      return {};
    }
  }
  return std::move(prepared.execution);
}

}  // namespace

AdmissionDecision admissionDecision(const benchmark::PairedResult& first,
                                    const std::optional<benchmark::PairedResult>& confirmation) {
  AdmissionDecision d;
  if (!first.passed) {
    d.reason = "Benchmark failed: " + first.errorMessage;
    return d;
  }
  d.conservativeSpeedup = first.speedup;
  if (first.speedup < kMinimumSpeedup) {
    d.reason = "Speedup is below 1.05x.";
    return d;
  }
  if (!confirmation) {
    d.reason = "No confirmation round.";
    return d;
  }
  if (!confirmation->passed) {
    d.reason = "Confirmation benchmark failed: " + confirmation->errorMessage;
    return d;
  }
  d.conservativeSpeedup = std::min(first.speedup, confirmation->speedup);
  if (d.conservativeSpeedup < kMinimumSpeedup) {
    d.reason = "Confirmation did not reach 1.05x.";
    return d;
  }
  d.admitted = true;
  return d;
}

std::vector<hip::DecodeGEMVConfig> decodeGEMVCandidates(std::size_t batch, bool prefill) {
  std::vector<hip::DecodeGEMVConfig> out;
  if (batch == 1 && !prefill) {
    for (int rpw : {1, 2})
      for (int unroll : {2, 4})
        for (int ks : {1, 2, 4}) out.push_back({1, rpw, unroll, ks});
    for (int rpw : {1, 2}) out.push_back({5, rpw, 1, 4});
    return out;
  }
  for (int tiles : {1, 2, 4})
    for (int unroll : {1, 2})
      for (int ks : {1, 2, 4, 8, 16}) out.push_back({3, tiles, unroll, ks});
  for (int ks : {2, 4, 8, 16}) out.push_back({2, 1, 2, ks});
  if (batch <= 8 && !prefill) out.push_back({1, 1, 2, 4});
  return out;
}

std::string decodeGEMVHardwareFilter(const hip::DecodeGEMVConfig& c, std::size_t batch,
                                     std::size_t inputSize, std::size_t outputSize,
                                     const hip::HardwareInfo& hardware) {
  const std::size_t threads = hip::decodeGEMVThreads(c);
  if (threads % 64 != 0 || threads > std::max<std::size_t>(hardware.maxThreadsPerThreadgroup, 64))
    return "workgroup is not a multiple of 64 lanes within the device limit";
  const std::size_t lds = hip::decodeGEMVLdsBytes(batch, c);
  if (lds > kLdsBytesPerLaunch || lds > kLdsBytesPerCU ||
      (hardware.maxThreadgroupMemoryLength && lds > hardware.maxThreadgroupMemoryLength))
    return "LDS budget exceeded";
  if (c.algorithm != 4 && inputSize % 8 != 0) return "input size is not a multiple of 8";
  if (c.algorithm == 1 && batch > 8) return "dot algorithm covers at most 8 batch rows per pass";
  if (c.algorithm == 3 && outputSize * inputSize * 2 >= 0xFFFFFFF0ull)
    return "weights exceed the 4 GiB buffer range";
  if (c.algorithm == 5 && (batch != 1 || inputSize > 16384 ||
                           (outputSize + 1) * inputSize * 2 >= 0xFFFFFFF0ull))
    return "the persistent dot takes batch 1, K <= 16384 and weights below 4 GiB";
  if (hardware.maxBufferLength &&
      (batch * inputSize * 2 > hardware.maxBufferLength ||
       outputSize * inputSize * 2 > hardware.maxBufferLength))
    return "buffer exceeds the device limit";
  return {};
}

DecodeGEMVSelection tuneDecodeGEMV(hip::HipRuntime& runtime, std::size_t batch,
                                   std::size_t inputSize, std::size_t outputSize,
                                   const std::vector<float>& input,
                                   const std::vector<float>& weight, std::ostream& log,
                                   DType storageDtype, bool prefill) {
  DecodeGEMVSelection fail;
  if (batch == 0 || inputSize == 0 || outputSize == 0 || input.size() != batch * inputSize ||
      weight.size() != outputSize * inputSize) {
    fail.errorMessage = "Decode GEMV tuning inputs do not match the shape.";
    return fail;
  }
  if (storageDtype != DType::Float16) {
    fail.errorMessage = "gfx950 decode GEMV tuning supports fp16 storage.";
    return fail;
  }
  // The CPU reference is affordable up to kMaximumCpuReferenceOperations
  // multiply-adds; above it the baseline's own GPU output is the reference.
  const bool cpuReference = inputSize <= kMaximumCpuReferenceOperations / outputSize &&
                            batch <= kMaximumCpuReferenceOperations / (inputSize * outputSize);
  std::vector<double> expected =
      cpuReference ? gemvReference(batch, inputSize, outputSize, input, weight)
                   : std::vector<double>{};
  const GemvBuilder build = [&](const hip::GeneratedKernel& kernel, std::string& why) {
    return prepareGemv(runtime, kernel, input, weight, batch * outputSize, expected, why);
  };
  std::string why;
  auto baseline = build(hip::emitLinearBaseline(batch, inputSize, outputSize,
                                                "decode_gemv_baseline", hip::ElementType::Float16,
                                                hip::ElementType::Float16),
                        why);
  if (!baseline) {
    fail.errorMessage = "Decode GEMV baseline failed: " + why;
    return fail;
  }
  if (!cpuReference) {
    const auto output = baseline->readOutputs().front();
    expected.assign(output.begin(), output.end());
  }
  const auto baselineSampler = benchmark::sampler(*baseline);
  const std::string cold = benchmark::warmup(baselineSampler, kTuningWarmup);
  if (!cold.empty()) {
    fail.errorMessage = "Decode GEMV baseline warmup failed: " + cold;
    return fail;
  }
  const std::size_t samples = cpuReference ? kTuningSamples : kLargeShapeSamples;
  log << "[decode-gemv] " << batch << "x" << inputSize << " -> " << outputSize << " fp16; "
      << (cpuReference ? "checked against the CPU double sums" : "checked against the baseline")
      << "; " << samples << " paired samples per round\n";
  return sweepDecodeGEMV(runtime, batch, inputSize, outputSize,
                         decodeGEMVCandidates(batch, prefill), hip::ElementType::Float16,
                         baselineSampler, build, samples, log);
}

DecodeGEMVSelection tuneDecodeGEMV(hip::HipRuntime& runtime, std::size_t batch,
                                   std::size_t inputSize, std::size_t outputSize,
                                   const hip::BufferHandle& input,
                                   const hip::BufferHandle& weight, std::ostream& log,
                                   hip::ElementType outputType) {
  DecodeGEMVSelection fail;
  const auto fp16 = hip::ElementType::Float16;
  if (!input || !weight || batch == 0 || inputSize == 0 || outputSize == 0 ||
      input->elementCount() < batch * inputSize ||
      weight->elementCount() < outputSize * inputSize || input->elementType() != fp16 ||
      weight->elementType() != fp16) {
    fail.errorMessage = "Decode GEMV tuning buffers do not match the shape (fp16 input, weight).";
    return fail;
  }
  auto output = runtime.createBuffer(batch * outputSize, nullptr, outputType);
  if (!output.buffer) {
    fail.errorMessage = output.errorMessage;
    return fail;
  }
  // Every candidate writes the same output buffer; the baseline's run is the
  // reference the others are checked against.
  const double tolerance = outputType == hip::ElementType::Float32 ? 2e-3 : 2e-2;
  std::vector<double> expected;
  const GemvBuilder build = [&](const hip::GeneratedKernel& kernel,
                                std::string& why) -> std::unique_ptr<hip::PreparedExecution> {
    const auto pipeline = runtime.createComputePipeline(kernel.source, kernel.functionName);
    if (!pipeline.pipelineCreationPassed) {
      why = pipeline.errorMessage;
      return {};
    }
    auto prepared = runtime.prepareBuffers({input, weight}, output.buffer,
                                           {kernel.threadgroupCount, kernel.threadsPerThreadgroup});
    if (!prepared.execution) {
      why = prepared.errorMessage;
      return {};
    }
    const auto run = prepared.execution->run();
    if (!run.executionPassed) {
      why = run.errorMessage;
      return {};
    }
    if (!expected.empty()) {
      const auto check = validation::compare(run.output, expected, tolerance, tolerance);
      if (!check.passed) {
        why = check.errorMessage;
        return {};
      }
    }
    return std::move(prepared.execution);
  };
  std::string why;
  auto baseline = build(hip::emitLinearBaseline(batch, inputSize, outputSize,
                                                "decode_gemv_baseline", fp16, outputType),
                        why);
  if (!baseline) {
    fail.errorMessage = "Decode GEMV baseline failed: " + why;
    return fail;
  }
  const auto first = baseline->readOutputs().front();
  expected.assign(first.begin(), first.end());
  if (!std::all_of(expected.begin(), expected.end(), [](double v) { return std::isfinite(v); })) {
    fail.errorMessage = "Decode GEMV tuning input produced non-finite outputs.";
    return fail;
  }
  const auto baselineSampler = benchmark::sampler(*baseline);
  const std::string cold = benchmark::warmup(baselineSampler, kTuningWarmup);
  if (!cold.empty()) {
    fail.errorMessage = "Decode GEMV baseline warmup failed: " + cold;
    return fail;
  }
  log << "[decode-gemv] " << batch << "x" << inputSize << " -> " << outputSize
      << " on resident buffers, checked against the baseline; " << kLargeShapeSamples
      << " paired samples per round\n";
  return sweepDecodeGEMV(runtime, batch, inputSize, outputSize, decodeGEMVCandidates(batch),
                         outputType, baselineSampler, build, kLargeShapeSamples, log);
}

std::string DecodeGEMVTuningCache::key(std::size_t batch, std::size_t inputSize,
                                       std::size_t outputSize, hip::ElementType outputType) {
  return "decode_gemv:b" + std::to_string(batch) + ":k" + std::to_string(inputSize) + ":n" +
         std::to_string(outputSize) + ":" + hip::elementTypeName(outputType);
}

std::optional<DecodeGEMVSelection> DecodeGEMVTuningCache::find(const std::string& key) const {
  const auto it = entries_.find(key);
  if (it == entries_.end()) return std::nullopt;
  return it->second;
}

void DecodeGEMVTuningCache::store(const std::string& key, const DecodeGEMVSelection& selection) {
  entries_[key] = selection;
}

DecodeGEMVTuningCache& decodeGEMVTuningCache() {
  static DecodeGEMVTuningCache cache;
  return cache;
}

DecodeGEMVSelection cachedDecodeGEMV(hip::HipRuntime& runtime, std::size_t batch,
                                     std::size_t inputSize, std::size_t outputSize,
                                     const hip::BufferHandle& input,
                                     const hip::BufferHandle& weight, std::ostream& log,
                                     hip::ElementType outputType) {
  auto& cache = decodeGEMVTuningCache();
  const auto key = DecodeGEMVTuningCache::key(batch, inputSize, outputSize, outputType);
  if (const auto hit = cache.find(key)) {
    log << "[decode-gemv] " << key << ": reusing " << describe(hit->config) << '\n';
    return *hit;
  }
  auto selection = tuneDecodeGEMV(runtime, batch, inputSize, outputSize, input, weight, log,
                                  outputType);
  if (selection.success) cache.store(key, selection);
  return selection;
}

std::vector<std::size_t> defaultRMSNormCandidates() { return {64, 128, 256, 512, 1024}; }

std::string rmsNormHardwareFilter(const RMSNormOp& op, std::size_t threads,
                                  const hip::HardwareInfo& hardware) {
  if (threads == 0 || threads % 64 != 0 || threads > 1024 ||
      (hardware.maxThreadsPerThreadgroup && threads > hardware.maxThreadsPerThreadgroup))
    return "Thread count must be a multiple of the 64-lane wave within the workgroup limit.";
  if (op.input.dtype != DType::Float16 && op.input.dtype != DType::Float32)
    return "gfx950 RMSNorm supports fp16 and fp32.";
  const std::size_t lds = threads / 64 * sizeof(float);
  if (hardware.maxThreadgroupMemoryLength && lds > hardware.maxThreadgroupMemoryLength)
    return "LDS budget exceeded.";
  return {};
}

namespace {

// ------------------------------------------------------------------ RMSNorm
// Where a kernel stopped on its way to being timed, and why.  The stage
// names make up the reports' outcome text ("<stage> FAIL").
struct Setback {
  std::string stage;
  std::string reason;
};

validation::ValidationResult checkRMSNorm(const hip::ExecutionResult& run,
                                          const std::vector<double>& reference, DType dtype) {
  if (!run.executionPassed) {
    validation::ValidationResult failed;
    failed.errorMessage = run.errorMessage;
    return failed;
  }
  const double tolerance = dtype == DType::Float16 ? 2e-3 : 1e-4;
  return validation::compare(run.output, reference, tolerance, tolerance);
}

// Filter, emit, resolve, check the binding interface, prepare over the
// inputs and validate one run; the setback says where it stopped.
std::unique_ptr<hip::PreparedExecution> buildRMSNorm(hip::HipRuntime& runtime, const RMSNormOp& op,
                                                     const std::vector<float>& input,
                                                     const std::vector<float>& weight,
                                                     const std::vector<double>& reference,
                                                     std::size_t threads, bool baseline,
                                                     Setback& setback, double& maxError) {
  const auto stop = [&](const char* stage, std::string reason) {
    setback = {stage, std::move(reason)};
    return std::unique_ptr<hip::PreparedExecution>{};
  };
  const std::string filtered = rmsNormHardwareFilter(op, threads, runtime.hardwareInfo());
  if (!filtered.empty()) return stop("Hardware Filter", filtered);
  hip::GeneratedKernel kernel;
  try {
    kernel = baseline ? hip::emitRMSNormBaseline(op) : hip::emitRMSNorm(op, threads);
  } catch (const std::exception& e) {
    return stop("Emit", e.what());
  }
  const auto pipeline = runtime.createComputePipeline(kernel.source, kernel.functionName);
  if (!pipeline.pipelineCreationPassed) return stop("Compile", pipeline.errorMessage);
  const auto type =
      op.input.dtype == DType::Float16 ? hip::ElementType::Float16 : hip::ElementType::Float32;
  const std::string mismatch = hip::checkBufferInterface(pipeline, {type, type}, type);
  if (!mismatch.empty()) return stop("Interface Check", mismatch);
  auto prepared =
      runtime.prepare({{input.data(), input.size(), type}, {weight.data(), weight.size(), type}},
                      op.output.elementCount(),
                      {kernel.threadgroupCount, kernel.threadsPerThreadgroup}, {}, type);
  if (!prepared.execution) return stop("Prepare", prepared.errorMessage);
  const auto check = checkRMSNorm(prepared.execution->run(), reference, op.output.dtype);
  if (!check.passed) return stop("Numerical Validate", check.errorMessage);
  maxError = check.maxAbsoluteError;
  return std::move(prepared.execution);
}

void summarize(const CandidateReport& r, std::ostream& log) {
  log << "[rmsnorm]   " << r.name << " (" << r.threads << " threads): " << r.outcome;
  if (!r.reason.empty()) log << " - " << r.reason;
  if (r.medianGpuUs) log << "; median " << *r.medianGpuUs << " us";
  if (r.pairedBaselineUs) log << " vs baseline " << *r.pairedBaselineUs << " us";
  if (r.speedup) log << ", x" << *r.speedup;
  log << '\n';
}

}  // namespace

TuningResult tuneRMSNorm(hip::HipRuntime& runtime, const RMSNormOp& op,
                         const std::vector<float>& input, const std::vector<float>& weight,
                         const std::vector<std::size_t>& candidateThreads, std::ostream& log) {
  TuningResult result;
  std::vector<double> reference;
  try {
    reference = validation::rmsNormReference(op, input, weight);
  } catch (const std::exception& e) {
    result.errorMessage = e.what();
    return result;
  }
  log << "[rmsnorm] " << candidateThreads.size() << " workgroup sizes against the 256-thread "
      << "two-pass kernel; outputs checked against the CPU double reference; a winner needs x"
      << kMinimumSpeedup << " in two paired rounds of " << kTuningSamples << " samples after "
      << kTuningWarmup << " warmup runs\n";
  const auto setBack = [&](CandidateReport& r, const Setback& s) {
    r.outcome = s.stage + " FAIL";
    r.reason = s.reason;
    log << "[rmsnorm] " << r.name << " stopped at " << s.stage << ": " << s.reason << '\n';
  };

  result.baseline.name = "baseline";
  result.baseline.threads = 256;
  Setback setback;
  double maxError = 0.0;
  auto baseline = buildRMSNorm(runtime, op, input, weight, reference, 256, true, setback, maxError);
  if (!baseline) {
    setBack(result.baseline, setback);
    result.errorMessage = "Baseline failed; no valid fallback: " + setback.reason;
    return result;
  }
  const auto baselineSampler = benchmark::sampler(*baseline);
  const std::string cold = benchmark::warmup(baselineSampler, kTuningWarmup);
  if (!cold.empty()) {
    setBack(result.baseline, {"Warmup", cold});
    result.errorMessage = "Baseline warmup failed; no valid fallback: " + cold;
    return result;
  }
  const auto alone = benchmark::measure(baselineSampler, kTuningSamples);
  result.baseline.outcome = alone.passed ? "Fallback ready" : "Performance unavailable";
  if (alone.passed) result.baseline.medianGpuUs = alone.stats.medianUs;
  else result.baseline.reason = alone.errorMessage;

  std::unique_ptr<hip::PreparedExecution> winner;
  std::size_t winnerIndex = 0;
  double bestSpeedup = 1.0;
  for (const std::size_t threads : candidateThreads) {
    result.candidates.push_back({});
    CandidateReport& report = result.candidates.back();
    report.name = "candidate_" + std::to_string(threads);
    report.threads = threads;
    auto candidate =
        buildRMSNorm(runtime, op, input, weight, reference, threads, false, setback, maxError);
    if (!candidate) {
      setBack(report, setback);
      continue;
    }
    log << "[rmsnorm] " << report.name << " matches the reference (max error " << maxError
        << ")\n";
    const auto sampler = benchmark::sampler(*candidate);
    const std::string warm = benchmark::warmup(sampler, kTuningWarmup);
    if (!warm.empty()) {
      setBack(report, {"Warmup", warm});
      continue;
    }
    if (!alone.passed) {
      report.outcome = "Not admitted";
      report.reason = "the baseline could not be timed, so nothing is compared";
      continue;
    }
    const Trial trial = runTrial(baselineSampler, sampler, kTuningSamples);
    if (trial.first.passed) {
      report.medianGpuUs = trial.first.candidate.medianUs;
      report.pairedBaselineUs = trial.first.baseline.medianUs;
      report.speedup = trial.decision.conservativeSpeedup;
    }
    if (!trial.decision.admitted) {
      setBack(report, {"Compare Baseline", trial.decision.reason});
      continue;
    }
    report.outcome = "Admitted";
    log << "[rmsnorm] " << report.name << " admitted at x" << trial.decision.conservativeSpeedup
        << '\n';
    if (trial.decision.conservativeSpeedup > bestSpeedup) {
      bestSpeedup = trial.decision.conservativeSpeedup;
      winnerIndex = result.candidates.size() - 1;
      winner = std::move(candidate);
    }
  }

  // The selection runs once more from fresh sentinel outputs with a
  // readback; a winner that fails there gives way to the baseline.
  const auto finalRun = [&](hip::PreparedExecution& execution) {
    result.finalExecution = execution.run();
    result.finalValidation = checkRMSNorm(result.finalExecution, reference, op.output.dtype);
    return result.finalValidation.passed;
  };
  if (winner && !finalRun(*winner)) {
    setBack(result.candidates[winnerIndex], {"Final execution", result.finalValidation.errorMessage});
    winner.reset();
  }
  if (!winner && !finalRun(*baseline)) {
    result.errorMessage =
        "Final baseline execution/validation failed: " + result.finalValidation.errorMessage;
    return result;
  }
  result.usedBaseline = !winner;
  result.selectedThreads = winner ? result.candidates[winnerIndex].threads : 256;
  result.selectedExecution = winner ? std::move(winner) : std::move(baseline);
  result.success = true;
  log << "[rmsnorm] summary (x = the lower speedup of the two rounds once confirmed):\n";
  summarize(result.baseline, log);
  for (const auto& report : result.candidates) summarize(report, log);
  log << "[rmsnorm] chosen: "
      << (result.usedBaseline ? std::string("the baseline") : result.candidates[winnerIndex].name)
      << " at " << result.selectedThreads << " threads\n";
  return result;
}

}  // namespace planner

namespace runtime {
namespace {

// The deterministic fusion test pattern: element i holds ((i mod 31) - 15) / 31.
std::vector<float> fusionTestPattern(std::size_t count) {
  std::vector<float> v(count);
  for (std::size_t i = 0; i < count; ++i)
    v[i] = static_cast<float>(static_cast<int>(i % 31) - 15) / 31.0f;
  return v;
}

std::unique_ptr<hip::PreparedSequence> sequenceOf(
    hip::HipRuntime& runtime, const std::vector<std::unique_ptr<hip::PreparedExecution>>& steps,
    std::size_t begin) {
  std::vector<const hip::PreparedExecution*> pointers;
  for (std::size_t i = begin; i < steps.size(); ++i) pointers.push_back(steps[i].get());
  auto prepared = runtime.prepareSequence(pointers);
  if (!prepared.execution) throw std::runtime_error(prepared.errorMessage);
  return std::move(prepared.execution);
}

// Run `sequence`; "" when every output agrees with its reference (2e-3 for
// fp32 outputs, 2e-2 for fp16/bf16), else the first disagreement.
std::string agrees(hip::PreparedSequence& sequence, const std::vector<hip::BufferHandle>& outputs,
                   const std::vector<std::vector<double>>& references) {
  const auto run = sequence.execute();
  if (!run.executionPassed) return run.errorMessage;
  for (std::size_t i = 0; i < outputs.size(); ++i) {
    const double tolerance = outputs[i]->elementType() == hip::ElementType::Float32 ? 2e-3 : 2e-2;
    const auto check = validation::compare(outputs[i]->read(), references[i], tolerance, tolerance);
    if (!check.passed) return check.errorMessage;
  }
  return {};
}

// The fused steps take the region's place at the end of `steps`.
void splice(std::vector<std::unique_ptr<hip::PreparedExecution>>& steps, std::size_t begin,
            std::vector<std::unique_ptr<hip::PreparedExecution>> fused) {
  steps.resize(begin);
  for (auto& step : fused) steps.push_back(std::move(step));
}

// Whether the fused steps stand in for steps[begin..]: the same outputs on
// the test pattern before and after timing, and the lower of two paired
// rounds; throws with the reason when the comparison cannot be made.
double fusionSpeedup(hip::HipRuntime& runtime, hip::PreparedSequence& unfused,
                     hip::PreparedSequence& fused, const std::vector<hip::BufferHandle>& testInputs,
                     const std::vector<hip::BufferHandle>& outputs) {
  for (const auto& input : testInputs) {
    const auto data = fusionTestPattern(input->elementCount());
    const auto error = runtime.writeBuffer(input, data.data(), data.size());
    if (!error.empty()) throw std::runtime_error(error);
  }
  const auto reference = unfused.execute();
  if (!reference.executionPassed) throw std::runtime_error(reference.errorMessage);
  std::vector<std::vector<double>> expected;
  for (const auto& output : outputs) {
    const auto values = output->read();
    expected.emplace_back(values.begin(), values.end());
  }
  if (auto why = agrees(fused, outputs, expected); !why.empty()) throw std::runtime_error(why);
  const auto before = benchmark::sampler(unfused);
  const auto after = benchmark::sampler(fused);
  for (const auto* s : {&before, &after})
    if (auto why = benchmark::warmup(*s, planner::kTuningWarmup); !why.empty())
      throw std::runtime_error(why);
  double slowest = std::numeric_limits<double>::infinity();
  for (int round = 0; round < 2; ++round) {
    const auto timing = benchmark::measurePair(before, after, planner::kTuningSamples);
    if (!timing.passed) throw std::runtime_error("Fusion benchmark failed.");
    slowest = std::min(slowest, timing.speedup);
  }
  if (auto why = agrees(fused, outputs, expected); !why.empty()) throw std::runtime_error(why);
  return slowest;
}

}  // namespace

bool admitFusion(hip::HipRuntime& runtime,
                 std::vector<std::unique_ptr<hip::PreparedExecution>>& steps, std::size_t begin,
                 const std::function<std::vector<std::unique_ptr<hip::PreparedExecution>>()>& build,
                 const std::vector<hip::BufferHandle>& testInputs,
                 const std::vector<hip::BufferHandle>& outputs, const std::string& name,
                 const std::string& decisionKey, FusionDecisionCache& decisions,
                 std::ostream& log) {
  if (const auto known = decisions.find(decisionKey); known != decisions.end()) {
    log << "Fusion " << name << ": cached decision, " << (known->second ? "fused" : "unfused")
        << '\n';
    if (!known->second) return false;
    try {
      splice(steps, begin, build());
      return true;
    } catch (const std::exception& e) {
      log << "Fusion " << name << ": rebuild error: " << e.what() << '\n';
      return false;
    }
  }
  bool admitted = false;
  try {
    if (begin > steps.size()) throw std::runtime_error("Fusion region starts past the steps.");
    auto fused = build();
    auto fusedSequence = sequenceOf(runtime, fused, 0);
    auto unfusedSequence = sequenceOf(runtime, steps, begin);
    const double speedup =
        fusionSpeedup(runtime, *unfusedSequence, *fusedSequence, testInputs, outputs);
    admitted = speedup >= planner::kMinimumSpeedup;
    log << "Fusion " << name << ": outputs agree, x" << speedup << " over the unfused steps -> "
        << (admitted ? "fused" : "unfused") << '\n';
    if (admitted) splice(steps, begin, std::move(fused));
  } catch (const std::exception& e) {
    log << "Fusion " << name << ": error: " << e.what() << " -> unfused\n";
    admitted = false;
  }
  decisions[decisionKey] = admitted;
  return admitted;
}

namespace {

constexpr std::size_t kGuardElements = 512;

std::vector<float> contractPattern(std::size_t count, std::size_t salt, float scale, float offset) {
  std::vector<float> v(count);
  for (std::size_t i = 0; i < count; ++i)
    v[i] = offset + scale * static_cast<float>(static_cast<int>((i * 7 + salt) % 29) - 14) / 14.0f;
  return v;
}

// One case of a region contract: its inputs, the sizes of the outputs and
// the template kernel key that writes the reference outputs.
struct ContractCase {
  std::vector<std::vector<float>> inputs;
  std::vector<std::size_t> outputCounts;
  std::string templateKey;
};

struct Contract {
  std::string pattern;       // registry name (decoder_...)
  std::string functionName;  // kernel key name a candidate must use
  hip::ElementType storage = hip::ElementType::Float16;
  std::vector<std::string> outputNames;
  std::vector<std::size_t> workgroupSizes;
  double tolerance = 2e-2;
  std::vector<ContractCase> cases;
};

Contract contractFor(const std::string& name) {
  Contract c;
  c.workgroupSizes = {64, 128, 256, 512, 1024};
  const bool norm = name == "RMSNorm" || name == "decoder_rmsnorm";
  const bool addNorm = name == "AddRMSNorm" || name == "decoder_residual_rmsnorm";
  if (norm || addNorm) {
    c.pattern = addNorm ? "decoder_residual_rmsnorm" : "decoder_rmsnorm";
    c.functionName = addNorm ? "add_rmsnorm" : "rmsnorm";
    c.outputNames = addNorm ? std::vector<std::string>{"sum", "norm"}
                            : std::vector<std::string>{"out"};
    for (const std::size_t rows : {std::size_t{1}, std::size_t{3}}) {
      const std::size_t width = 4096, n = rows * width;
      ContractCase k;
      k.inputs.push_back(contractPattern(n, 1, 1.0f, 0.0f));
      if (addNorm) k.inputs.push_back(contractPattern(n, 5, 1.0f, 0.0f));
      k.inputs.push_back(contractPattern(width, 3, 0.5f, 1.0f));
      k.outputCounts.assign(c.outputNames.size(), n);
      k.templateKey = c.functionName + "?rows=" + std::to_string(rows) +
                      "&width=" + std::to_string(width) + "&eps=1e-06&dtype=f16";
      c.cases.push_back(std::move(k));
    }
    return c;
  }
  if (name == "SiLUMul" || name == "decoder_silu_mul") {
    c.pattern = "decoder_silu_mul";
    c.functionName = "silu_mul";
    c.outputNames = {"out"};
    for (const std::size_t n : {std::size_t{11008}, std::size_t{8 * 11008}}) {
      ContractCase k;
      k.inputs = {contractPattern(n, 2, 4.0f, 0.0f), contractPattern(n, 9, 2.0f, 0.0f)};
      k.outputCounts = {n};
      k.templateKey = "silu_mul?count=" + std::to_string(n) + "&dtype=f16";
      c.cases.push_back(std::move(k));
    }
    return c;
  }
  throw std::invalid_argument("Unknown kernel contract pattern '" + name +
                              "' (RMSNorm, AddRMSNorm, SiLUMul).");
}

// The launch parameters a candidate key sets (threads, variant); the other
// cases of a contract run the same parameters on their own shapes.
std::string tuningOf(const std::string& key) {
  std::string tuning;
  const auto q = key.find('?');
  if (q == std::string::npos) return tuning;
  std::stringstream items(key.substr(q + 1));
  for (std::string item; std::getline(items, item, '&');) {
    const std::string field = item.substr(0, item.find('='));
    if (field == "threads" || field == "variant") tuning += "&" + item;
  }
  return tuning;
}

// A contract case prepared over its own buffers, as one-step sequence.
struct CaseRig {
  std::unique_ptr<hip::PreparedExecution> execution;
  std::unique_ptr<hip::PreparedSequence> sequence;
  std::vector<hip::BufferHandle> outputs;
};

// `guarded`: every buffer gets kGuardElements extra elements (inputs 1.0,
// outputs NaN) that a correct kernel never touches.
CaseRig rigCase(hip::HipRuntime& runtime, const Contract& contract, const ContractCase& data,
                const std::string& key, bool guarded) {
  const auto pipeline = runtime.createComputePipeline(key, contract.functionName);
  if (!pipeline.pipelineCreationPassed) throw std::runtime_error(pipeline.errorMessage);
  const std::size_t extra = guarded ? kGuardElements : 0;
  std::vector<hip::BufferHandle> inputs;
  for (auto values : data.inputs) {
    values.resize(values.size() + extra, 1.0f);
    auto made = runtime.createBuffer(values.size(), values.data(), contract.storage);
    if (!made.buffer) throw std::runtime_error(made.errorMessage);
    inputs.push_back(std::move(made.buffer));
  }
  CaseRig rig;
  for (const auto count : data.outputCounts) {
    auto made = runtime.createBuffer(count + extra, nullptr, contract.storage);
    if (!made.buffer) throw std::runtime_error(made.errorMessage);
    rig.outputs.push_back(std::move(made.buffer));
  }
  auto prepared = runtime.prepareBuffers(
      inputs, rig.outputs, {pipeline.threadgroupCount, pipeline.threadsPerThreadgroup});
  if (!prepared.execution) throw std::runtime_error(prepared.errorMessage);
  rig.execution = std::move(prepared.execution);
  auto sequence = runtime.prepareSequence({rig.execution.get()});
  if (!sequence.execution) throw std::runtime_error(sequence.errorMessage);
  rig.sequence = std::move(sequence.execution);
  return rig;
}

// Reset the outputs to NaN, run once and compare with the references;
// guard elements must still be NaN.  "" when correct.
std::string checkCase(hip::HipRuntime& runtime, CaseRig& rig, const Contract& contract,
                      const ContractCase& data, const std::vector<std::vector<double>>& expected,
                      bool guarded) {
  for (const auto& output : rig.outputs) {
    const std::vector<float> nan(output->elementCount(), std::numeric_limits<float>::quiet_NaN());
    if (auto why = runtime.writeBuffer(output, nan.data(), nan.size()); !why.empty()) return why;
  }
  const auto run = rig.sequence->execute();
  if (!run.executionPassed) return run.errorMessage;
  for (std::size_t i = 0; i < rig.outputs.size(); ++i) {
    const auto values = rig.outputs[i]->read();
    const std::size_t count = data.outputCounts[i];
    if (values.size() != count + (guarded ? kGuardElements : 0)) return "Output size mismatch.";
    const auto check = validation::compare({values.begin(), values.begin() + count}, expected[i],
                                           contract.tolerance, contract.tolerance);
    if (!check.passed) return contract.outputNames[i] + ": " + check.errorMessage;
    if (guarded && !std::all_of(values.begin() + count, values.end(),
                                [](float v) { return std::isnan(v); }))
      return "Output guard modified: " + contract.outputNames[i];
  }
  return {};
}

}  // namespace

std::string kernelContractText(const hip::HipRuntime& runtime, const std::string& pattern) {
  const auto contract = contractFor(pattern);
  const auto hw = runtime.hardwareInfo();
  std::ostringstream out;
  out << "{\"version\":1,\"pattern\":\"" << contract.pattern << "\",\"function_name\":\""
      << contract.functionName << "\",\"storage_dtype\":\"half\",\"accumulation_dtype\":\"float\""
      << ",\"target\":{\"backend\":\"hip\",\"arch\":\"gfx950\",\"device\":\""
      << jsonEscape(runtime.deviceName()) << "\",\"wave_size\":" << hw.waveSize
      << ",\"max_threads_per_workgroup\":" << hw.maxThreadsPerThreadgroup
      << ",\"max_lds_bytes\":" << hw.maxThreadgroupMemoryLength << "},\"outputs\":[";
  for (std::size_t i = 0; i < contract.outputNames.size(); ++i)
    out << (i ? "," : "") << '"' << contract.outputNames[i] << '"';
  out << "],\"workgroup_sizes\":[";
  for (std::size_t i = 0; i < contract.workgroupSizes.size(); ++i)
    out << (i ? "," : "") << contract.workgroupSizes[i];
  out << "],\"cases\":[";
  for (std::size_t i = 0; i < contract.cases.size(); ++i)
    out << (i ? "," : "") << '"' << contract.cases[i].templateKey << '"';
  out << "]}";
  return out.str();
}

std::string canonicalKernelPattern(const std::string& pattern) {
  return contractFor(pattern).pattern;
}

bool admitGeneratedKernel(hip::HipRuntime& runtime, const std::string& patternName,
                          const std::string& responsePath, const std::string& feedbackPath,
                          std::ostream& log, const std::string& artifactPath) {
  // Every exit writes the feedback file; only a fatal outcome returns false.
  const auto finish = [&](const AdmissionFeedback& f) {
    const std::string written = writeAdmissionFeedback(f, feedbackPath);
    log << "[admission] " << patternName << " " << f.stage << " -> " << f.status << ": "
        << f.message << '\n';
    if (!written.empty()) {
      log << "[admission] feedback not written: " << written << '\n';
      return false;
    }
    log << "[admission] " << patternName << " runs the "
        << (f.status == "admitted" ? "candidate" : "template") << " kernel\n";
    return f.status != "fatal";
  };
  Contract contract;
  std::vector<CaseRig> templates;
  std::vector<std::vector<std::vector<double>>> expected;
  try {
    contract = contractFor(patternName);
    for (const auto& data : contract.cases) {
      auto rig = rigCase(runtime, contract, data, data.templateKey, false);
      const auto run = rig.sequence->execute();
      if (!run.executionPassed) throw std::runtime_error(run.errorMessage);
      std::vector<std::vector<double>> outs;
      for (const auto& output : rig.outputs) {
        const auto values = output->read();
        outs.emplace_back(values.begin(), values.end());
      }
      expected.push_back(std::move(outs));
      if (auto why = benchmark::warmup(benchmark::sampler(*rig.sequence), planner::kTuningWarmup);
          !why.empty())
        throw std::runtime_error(why);
      log << "[admission] template " << data.templateKey << " ready\n";
      templates.push_back(std::move(rig));
    }
  } catch (const std::exception& e) {
    return finish({"fatal", "baseline_or_contract", e.what()});
  }

  AdmittedKernel candidate;
  {
    std::ifstream in(responsePath);
    if (!in) return finish({"retry", "response_parse", "Unable to read '" + responsePath + "'."});
    std::stringstream text;
    text << in.rdbuf();
    std::string workgroup;
    if (!jsonStringField(text.str(), "function_name", candidate.functionName) ||
        !jsonStringField(text.str(), "source", candidate.source) ||
        !jsonStringField(text.str(), "workgroup_size", workgroup))
      return finish({"retry", "response_parse",
                     "Response needs function_name, source and workgroup_size."});
    try {
      candidate.workgroupSize = static_cast<std::size_t>(std::stoul(workgroup));
    } catch (const std::exception&) {
      return finish({"retry", "response_parse", "workgroup_size is not an integer."});
    }
  }
  if (candidate.functionName != contract.functionName)
    return finish({"retry", "contract", "Expected function_name: " + contract.functionName});
  if (candidate.source.substr(0, candidate.source.find('?')) != contract.functionName)
    return finish({"retry", "contract", "The kernel key must name " + contract.functionName + "."});
  const bool legal = std::find(contract.workgroupSizes.begin(), contract.workgroupSizes.end(),
                               candidate.workgroupSize) != contract.workgroupSizes.end() &&
                     candidate.workgroupSize <= runtime.hardwareInfo().maxThreadsPerThreadgroup;
  if (!legal)
    return finish({"retry", "hardware_filter",
                   "workgroup_size is not legal for this contract/device."});

  std::string tuning = tuningOf(candidate.source);
  if (tuning.find("threads=") == std::string::npos)
    tuning += "&threads=" + std::to_string(candidate.workgroupSize);
  std::vector<CaseRig> rigs;
  for (std::size_t i = 0; i < contract.cases.size(); ++i) {
    const auto& data = contract.cases[i];
    const std::string key = data.templateKey + tuning;
    try {
      rigs.push_back(rigCase(runtime, contract, data, key, true));
    } catch (const std::exception& e) {
      return finish({"retry", i == 0 ? "compile" : "prepare", e.what()});
    }
    if (auto why = checkCase(runtime, rigs.back(), contract, data, expected[i], true); !why.empty())
      return finish({"retry", "numerical_validation", "case " + std::to_string(i) + ": " + why});
    log << "[admission] " << key << " matches the template outputs\n";
  }

  // Two paired rounds per case; the slowest round decides and is reported.
  std::optional<AdmissionFeedback> slowest;
  for (std::size_t i = 0; i < rigs.size(); ++i) {
    const auto base = benchmark::sampler(*templates[i].sequence);
    const auto cand = benchmark::sampler(*rigs[i].sequence);
    if (auto why = benchmark::warmup(cand, planner::kTuningWarmup); !why.empty())
      return finish({"retry", "warmup", why});
    for (int round = 1; round <= 2; ++round) {
      const auto t = benchmark::measurePair(base, cand, planner::kTuningSamples);
      if (!t.passed) return finish({"retry", "benchmark", t.errorMessage});
      log << "[admission] case " << i << " round " << round << ": template " << t.baseline.medianUs
          << " us, candidate " << t.candidate.medianUs << " us, x" << t.speedup << '\n';
      if (!slowest || t.speedup < *slowest->speedup) {
        const bool fast = t.speedup >= planner::kMinimumSpeedup;
        slowest = AdmissionFeedback{
            fast ? "admitted" : "retry", fast ? "admission" : "performance",
            fast ? "All cases passed correctness and two performance rounds."
                 : "case " + std::to_string(i) + " round " + std::to_string(round) +
                       " speedup is below 1.05x.",
            t.baseline.medianUs, t.candidate.medianUs, t.speedup};
      }
    }
    if (auto why = checkCase(runtime, rigs[i], contract, contract.cases[i], expected[i], true);
        !why.empty())
      return finish({"retry", "final_validation", why});
  }
  if (slowest->status == "admitted" && !artifactPath.empty()) {
    const std::string why = writeAdmittedKernel(runtime, contract.pattern, candidate, artifactPath);
    if (!why.empty()) return finish({"fatal", "artifact_write", why});
  }
  return finish(*slowest);
}

}  // namespace runtime

}  // namespace tensor
