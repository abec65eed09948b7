#include "Tuning.hpp"

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

std::size_t TensorType::elementCount() const {
  std::size_t count = 1;
  for (const auto d : shape) count *= d;
  return count;
}

void RMSNormOp::validate() const {
  if (input.shape.empty()) throw std::invalid_argument("RMSNorm input must be ranked.");
  const bool isFloat = input.dtype == DType::Float16 || input.dtype == DType::Float32 ||
                       input.dtype == DType::BFloat16;
  if (!isFloat || weight.dtype != input.dtype || output.dtype != input.dtype)
    throw std::invalid_argument("RMSNorm requires matching floating-point tensors.");
  if (output.shape != input.shape)
    throw std::invalid_argument("RMSNorm output shape must match input shape.");
  if (weight.shape.size() != 1 || weight.shape.front() != input.shape.back())
    throw std::invalid_argument("RMSNorm weight must match the last input dimension.");
  if (!std::isfinite(epsilon) || epsilon <= 0.0f)
    throw std::invalid_argument("RMSNorm epsilon must be finite and positive.");
}

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

std::vector<double> gemvReference(std::size_t batch, std::size_t in, std::size_t out,
                                  const std::vector<float>& x, const std::vector<float>& w) {
  std::vector<double> y(batch * out);
  std::vector<double> xs(x.size()), ws(w.size());
  for (std::size_t i = 0; i < x.size(); ++i) xs[i] = roundHalf(x[i]);
  for (std::size_t i = 0; i < w.size(); ++i) ws[i] = roundHalf(w[i]);
  for (std::size_t b = 0; b < batch; ++b)
    for (std::size_t n = 0; n < out; ++n) {
      double acc = 0.0;
      for (std::size_t k = 0; k < in; ++k) acc += xs[b * in + k] * ws[n * in + k];
      y[b * out + n] = acc;
    }
  return y;
}

std::string configText(const hip::DecodeGEMVConfig& c) {
  std::ostringstream s;
  s << "algorithm=" << c.algorithm << ", rows_per_wave=" << c.rowsPerWave
    << ", unroll=" << c.unroll << ", k_split=" << c.kSplit;
  return s.str();
}

// Resolve `kernel`, prepare it over fresh buffers holding `input` and
// `weight`, run it once and validate against `expected` when given.
std::unique_ptr<hip::PreparedExecution> prepareGemv(hip::HipRuntime& runtime,
                                                    const hip::GeneratedKernel& kernel,
                                                    const std::vector<float>& input,
                                                    const std::vector<float>& weight,
                                                    std::size_t outputCount,
                                                    const std::vector<double>& expected,
                                                    std::string& error) {
  const auto type = hip::ElementType::Float16;
  const auto pipeline = runtime.createComputePipeline(kernel.source, kernel.functionName);
  if (!pipeline.pipelineCreationPassed) {
    error = pipeline.errorMessage;
    return {};
  }
  error = hip::checkBufferInterface(pipeline, {type, type}, type);
  if (!error.empty()) return {};
  auto prepared = runtime.prepare({{input.data(), input.size(), type},
                                   {weight.data(), weight.size(), type}},
                                  outputCount,
                                  {kernel.threadgroupCount, kernel.threadsPerThreadgroup}, {},
                                  type);
  if (!prepared.execution) {
    error = prepared.errorMessage;
    return {};
  }
  const auto execution = prepared.execution->run();
  if (!execution.executionPassed) {
    error = execution.errorMessage;
    return {};
  }
  if (!expected.empty()) {
    const auto validation = validation::compare(execution.output, expected, 2e-2, 2e-2);
    if (!validation.passed) {
      error = validation.errorMessage;
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
  DecodeGEMVSelection result;
  if (batch == 0 || inputSize == 0 || outputSize == 0 || input.size() != batch * inputSize ||
      weight.size() != outputSize * inputSize) {
    result.errorMessage = "Decode GEMV tuning inputs do not match the shape.";
    return result;
  }
  if (storageDtype != DType::Float16) {
    result.errorMessage = "gfx950 decode GEMV tuning supports fp16 storage.";
    return result;
  }
  const bool useCpuReference =
      inputSize <= kMaximumCpuReferenceOperations / outputSize &&
      batch <= kMaximumCpuReferenceOperations / (inputSize * outputSize);
  const std::size_t samples = useCpuReference ? kTuningSamples : std::size_t{9};
  auto expected = useCpuReference ? gemvReference(batch, inputSize, outputSize, input, weight)
                                  : std::vector<double>{};
  std::string error;
  const auto baselineKernel =
      hip::emitLinearBaseline(batch, inputSize, outputSize, "decode_gemv_baseline",
                              hip::ElementType::Float16, hip::ElementType::Float16);
  auto baseline = prepareGemv(runtime, baselineKernel, input, weight, batch * outputSize,
                              expected, error);
  if (!baseline) {
    result.errorMessage = "Decode GEMV baseline failed: " + error;
    return result;
  }
  if (!useCpuReference) {
    const auto output = baseline->readOutputs().front();
    expected.assign(output.begin(), output.end());
    log << "Decode GEMV large-shape validation: baseline GPU output is the reference\n";
  }
  const auto baselineSampler = benchmark::sampler(*baseline);
  const auto warm = benchmark::warmup(baselineSampler, kTuningWarmup);
  if (!warm.empty()) {
    result.errorMessage = "Decode GEMV baseline warmup failed: " + warm;
    return result;
  }
  log << "Decode GEMV shape M=" << batch << ", K=" << inputSize << ", N=" << outputSize
      << ", dtype=fp16, samples=" << samples << " | baseline validation/warmup: PASS\n";

  const auto hardware = runtime.hardwareInfo();
  double best = 1.0;
  for (const auto& config : decodeGEMVCandidates(batch, prefill)) {
    log << "  candidate " << configText(config);
    const auto filter = decodeGEMVHardwareFilter(config, batch, inputSize, outputSize, hardware);
    if (!filter.empty()) {
      log << " | Hardware Filter: FAIL (" << filter << ")\n";
      continue;
    }
    hip::GeneratedKernel kernel;
    try {
      kernel = hip::emitDecodeGEMV(batch, inputSize, outputSize, config, "decode_gemv_candidate",
                                   hip::ElementType::Float16, hip::ElementType::Float16);
    } catch (const std::exception& e) {
      log << " | Emit: FAIL: " << e.what() << '\n';
      continue;
    }
    auto candidate = prepareGemv(runtime, kernel, input, weight, batch * outputSize, expected,
                                 error);
    if (!candidate) {
      log << " | Compile/interface/numerical: FAIL: " << error << '\n';
      continue;
    }
    const auto candidateSampler = benchmark::sampler(*candidate);
    const auto candidateWarm = benchmark::warmup(candidateSampler, kTuningWarmup);
    if (!candidateWarm.empty()) {
      log << " | Warmup: FAIL: " << candidateWarm << '\n';
      continue;
    }
    const auto first = benchmark::measurePair(baselineSampler, candidateSampler, samples);
    std::optional<benchmark::PairedResult> confirmation;
    if (first.passed && first.speedup >= kMinimumSpeedup)
      confirmation = benchmark::measurePair(baselineSampler, candidateSampler, samples);
    const auto decision = admissionDecision(first, confirmation);
    if (first.passed) log << " | validation: PASS, speedup=" << first.speedup << 'x';
    if (confirmation && confirmation->passed)
      log << ", confirmation=" << confirmation->speedup << 'x';
    if (!decision.admitted) {
      log << " -> fallback (" << decision.reason << ")\n";
      continue;
    }
    log << " -> admitted\n";
    if (decision.conservativeSpeedup > best) {
      best = decision.conservativeSpeedup;
      result.useBaseline = false;
      result.config = config;
      result.conservativeSpeedup = decision.conservativeSpeedup;
    }
  }
  result.success = true;
  if (result.useBaseline) {
    result.config = hip::DecodeGEMVConfig{4, 1, 1, 1};
    log << "Decode GEMV selected: linear baseline fallback\n";
  } else {
    log << "Decode GEMV selected: " << configText(result.config)
        << ", conservative speedup=" << result.conservativeSpeedup << "x\n";
  }
  return result;
}

DecodeGEMVSelection tuneDecodeGEMV(hip::HipRuntime& runtime, std::size_t batch,
                                   std::size_t inputSize, std::size_t outputSize,
                                   const hip::BufferHandle& input,
                                   const hip::BufferHandle& weight, std::ostream& log,
                                   hip::ElementType outputType) {
  DecodeGEMVSelection result;
  if (!input || !weight || batch == 0 || inputSize == 0 || outputSize == 0 ||
      input->elementCount() < batch * inputSize ||
      weight->elementCount() < outputSize * inputSize ||
      input->elementType() != hip::ElementType::Float16 ||
      weight->elementType() != hip::ElementType::Float16) {
    result.errorMessage = "Decode GEMV tuning buffers do not match the shape (fp16 input, weight).";
    return result;
  }
  const double tolerance = outputType == hip::ElementType::Float32 ? 2e-3 : 2e-2;
  const std::size_t samples = 9;
  auto output = runtime.createBuffer(batch * outputSize, nullptr, outputType);
  if (!output.buffer) {
    result.errorMessage = output.errorMessage;
    return result;
  }
  auto prepare = [&](const hip::GeneratedKernel& kernel,
                     std::string& error) -> std::unique_ptr<hip::PreparedExecution> {
    const auto pipeline = runtime.createComputePipeline(kernel.source, kernel.functionName);
    if (!pipeline.pipelineCreationPassed) {
      error = pipeline.errorMessage;
      return {};
    }
    auto prepared = runtime.prepareBuffers({input, weight}, output.buffer,
                                           {kernel.threadgroupCount, kernel.threadsPerThreadgroup});
    if (!prepared.execution) error = prepared.errorMessage;
    return std::move(prepared.execution);
  };
  std::string error;
  auto baseline = prepare(hip::emitLinearBaseline(batch, inputSize, outputSize, "decode_gemv_baseline",
                                                  hip::ElementType::Float16, outputType),
                          error);
  if (!baseline) {
    result.errorMessage = "Decode GEMV baseline failed: " + error;
    return result;
  }
  const auto baseRun = baseline->run();
  if (!baseRun.executionPassed) {
    result.errorMessage = "Decode GEMV baseline failed: " + baseRun.errorMessage;
    return result;
  }
  const std::vector<double> expected(baseRun.output.begin(), baseRun.output.end());
  for (const double v : expected)
    if (!std::isfinite(v)) {
      result.errorMessage = "Decode GEMV tuning input produced non-finite outputs.";
      return result;
    }
  const auto baselineSampler = benchmark::sampler(*baseline);
  const auto warm = benchmark::warmup(baselineSampler, kTuningWarmup);
  if (!warm.empty()) {
    result.errorMessage = "Decode GEMV baseline warmup failed: " + warm;
    return result;
  }
  log << "Decode GEMV shape M=" << batch << ", K=" << inputSize << ", N=" << outputSize
      << " (device buffers, baseline output as reference, samples=" << samples << ")\n";
  const auto hardware = runtime.hardwareInfo();
  double best = 1.0;
  for (const auto& config : decodeGEMVCandidates(batch)) {
    log << "  candidate " << configText(config);
    const auto filter = decodeGEMVHardwareFilter(config, batch, inputSize, outputSize, hardware);
    if (!filter.empty()) {
      log << " | Hardware Filter: FAIL (" << filter << ")\n";
      continue;
    }
    auto candidate = prepare(hip::emitDecodeGEMV(batch, inputSize, outputSize, config,
                                                 "decode_gemv_candidate", hip::ElementType::Float16,
                                                 outputType),
                             error);
    if (!candidate) {
      log << " | Compile/interface: FAIL: " << error << '\n';
      continue;
    }
    const auto run = candidate->run();
    const auto check = run.executionPassed
                           ? validation::compare(run.output, expected, tolerance, tolerance)
                           : validation::ValidationResult{};
    if (!check.passed) {
      log << " | numerical: FAIL: " << (run.executionPassed ? check.errorMessage : run.errorMessage)
          << '\n';
      continue;
    }
    const auto candidateSampler = benchmark::sampler(*candidate);
    const auto candidateWarm = benchmark::warmup(candidateSampler, kTuningWarmup);
    if (!candidateWarm.empty()) {
      log << " | Warmup: FAIL: " << candidateWarm << '\n';
      continue;
    }
    const auto first = benchmark::measurePair(baselineSampler, candidateSampler, samples);
    std::optional<benchmark::PairedResult> confirmation;
    if (first.passed && first.speedup >= kMinimumSpeedup)
      confirmation = benchmark::measurePair(baselineSampler, candidateSampler, samples);
    const auto decision = admissionDecision(first, confirmation);
    if (first.passed) log << " | speedup=" << first.speedup << 'x';
    if (!decision.admitted) {
      log << " -> fallback (" << decision.reason << ")\n";
      continue;
    }
    log << ", confirmed " << decision.conservativeSpeedup << "x -> admitted\n";
    if (decision.conservativeSpeedup > best) {
      best = decision.conservativeSpeedup;
      result.useBaseline = false;
      result.config = config;
      result.conservativeSpeedup = decision.conservativeSpeedup;
    }
  }
  result.success = true;
  if (result.useBaseline) result.config = hip::DecodeGEMVConfig{4, 1, 1, 1};
  log << "Decode GEMV selected: " << configText(result.config)
      << ", conservative speedup=" << result.conservativeSpeedup << "x\n";
  return result;
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
    log << "Decode GEMV " << key << ": cached " << configText(hit->config) << '\n';
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

void reject(CandidateReport& report, const std::string& stage, const std::string& reason,
            std::ostream& log) {
  report.outcome = stage + " FAIL";
  report.reason = reason;
  log << report.name << " | " << stage << ": FAIL: " << reason << '\n';
}

validation::ValidationResult validateExecution(const hip::ExecutionResult& execution,
                                               const std::vector<double>& reference,
                                               DType dtype) {
  if (!execution.executionPassed) {
    validation::ValidationResult r;
    r.errorMessage = execution.errorMessage;
    return r;
  }
  const double tolerance = dtype == DType::Float16 ? 2e-3 : 1e-4;
  return validation::compare(execution.output, reference, tolerance, tolerance);
}

std::unique_ptr<hip::PreparedExecution> buildRMSNorm(hip::HipRuntime& runtime,
                                                     const RMSNormOp& op,
                                                     const std::vector<float>& input,
                                                     const std::vector<float>& weight,
                                                     const std::vector<double>& reference,
                                                     bool baseline, CandidateReport& report,
                                                     std::ostream& log) {
  const auto hardware = runtime.hardwareInfo();
  const auto filter = rmsNormHardwareFilter(op, report.threads, hardware);
  if (!filter.empty()) {
    reject(report, "Hardware Filter", filter, log);
    return {};
  }
  hip::GeneratedKernel kernel;
  try {
    kernel = baseline ? hip::emitRMSNormBaseline(op) : hip::emitRMSNorm(op, report.threads);
  } catch (const std::exception& e) {
    reject(report, "Emit", e.what(), log);
    return {};
  }
  const auto pipeline = runtime.createComputePipeline(kernel.source, kernel.functionName);
  if (!pipeline.pipelineCreationPassed) {
    reject(report, "Compile", pipeline.errorMessage, log);
    return {};
  }
  const auto type = op.input.dtype == DType::Float16 ? hip::ElementType::Float16
                                                     : hip::ElementType::Float32;
  const auto interfaceError = hip::checkBufferInterface(pipeline, {type, type}, type);
  if (!interfaceError.empty()) {
    reject(report, "Interface Check", interfaceError, log);
    return {};
  }
  auto prepared = runtime.prepare({{input.data(), input.size(), type},
                                   {weight.data(), weight.size(), type}},
                                  op.output.elementCount(),
                                  {kernel.threadgroupCount, kernel.threadsPerThreadgroup}, {},
                                  type);
  if (!prepared.execution) {
    reject(report, "Prepare", prepared.errorMessage, log);
    return {};
  }
  const auto check = validateExecution(prepared.execution->run(), reference, op.output.dtype);
  if (!check.passed) {
    reject(report, "Numerical Validate", check.errorMessage, log);
    return {};
  }
  log << report.name << " | Numerical Validate: PASS, max absolute error="
      << check.maxAbsoluteError << '\n';
  report.outcome = "Correctness PASS";
  return std::move(prepared.execution);
}

void printReport(const CandidateReport& report, std::ostream& log) {
  log << "  " << report.name << " | threads=" << report.threads;
  if (report.medianGpuUs) log << " | GPU median(us)=" << *report.medianGpuUs;
  if (report.pairedBaselineUs) log << " | paired baseline(us)=" << *report.pairedBaselineUs;
  if (report.speedup) log << " | speedup=" << *report.speedup << 'x';
  log << " | " << report.outcome;
  if (!report.reason.empty()) log << " (" << report.reason << ')';
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
  log << "Enumerate: threads={";
  for (std::size_t i = 0; i < candidateThreads.size(); ++i)
    log << (i ? ", " : "") << candidateThreads[i];
  log << "}\nCPU correctness baseline: double-accumulation reference\n"
      << "GPU performance baseline: fixed 256-thread two-pass RMSNorm\n"
      << "Warmup=" << kTuningWarmup << ", samples=" << kTuningSamples
      << ", admission requires >= " << kMinimumSpeedup << "x in two paired rounds\n";

  result.baseline.name = "baseline";
  result.baseline.threads = 256;
  auto baseline = buildRMSNorm(runtime, op, input, weight, reference, true, result.baseline, log);
  if (!baseline) {
    result.errorMessage = "Baseline failed; no valid fallback: " + result.baseline.reason;
    return result;
  }
  const auto baselineSampler = benchmark::sampler(*baseline);
  const auto warm = benchmark::warmup(baselineSampler, kTuningWarmup);
  if (!warm.empty()) {
    reject(result.baseline, "Warmup", warm, log);
    result.errorMessage = "Baseline warmup failed; no valid fallback: " + warm;
    return result;
  }
  const auto baselineTiming = benchmark::measure(baselineSampler, kTuningSamples);
  if (baselineTiming.passed) {
    result.baseline.medianGpuUs = baselineTiming.stats.medianUs;
    result.baseline.outcome = "Fallback ready";
  } else {
    result.baseline.outcome = "Performance unavailable";
    result.baseline.reason = baselineTiming.errorMessage;
  }

  std::unique_ptr<hip::PreparedExecution> winner;
  std::size_t winnerIndex = 0;
  double best = 1.0;
  for (const std::size_t threads : candidateThreads) {
    CandidateReport report;
    report.name = "candidate_" + std::to_string(threads);
    report.threads = threads;
    result.candidates.push_back(std::move(report));
    auto& current = result.candidates.back();
    auto candidate = buildRMSNorm(runtime, op, input, weight, reference, false, current, log);
    if (!candidate) continue;
    const auto candidateSampler = benchmark::sampler(*candidate);
    const auto candidateWarm = benchmark::warmup(candidateSampler, kTuningWarmup);
    if (!candidateWarm.empty()) {
      reject(current, "Warmup", candidateWarm, log);
      continue;
    }
    if (!baselineTiming.passed) {
      current.outcome = "Not admitted";
      current.reason = "No usable baseline timing; performance comparison skipped.";
      continue;
    }
    const auto first = benchmark::measurePair(baselineSampler, candidateSampler, kTuningSamples);
    if (first.passed) {
      current.medianGpuUs = first.candidate.medianUs;
      current.pairedBaselineUs = first.baseline.medianUs;
      current.speedup = first.speedup;
    }
    std::optional<benchmark::PairedResult> confirmation;
    if (first.passed && first.speedup >= kMinimumSpeedup)
      confirmation = benchmark::measurePair(baselineSampler, candidateSampler, kTuningSamples);
    const auto decision = admissionDecision(first, confirmation);
    if (confirmation && confirmation->passed) current.speedup = decision.conservativeSpeedup;
    if (!decision.admitted) {
      reject(current, "Compare Baseline", decision.reason, log);
      continue;
    }
    current.outcome = "Admitted";
    log << current.name << " | Compare Baseline: PASS -> Admit\n";
    if (decision.conservativeSpeedup > best) {
      best = decision.conservativeSpeedup;
      winnerIndex = result.candidates.size() - 1;
      winner = std::move(candidate);
    }
  }

  // Run the selection once more with fresh sentinel outputs and readback.
  result.finalExecution = winner ? winner->run() : baseline->run();
  result.finalValidation = validateExecution(result.finalExecution, reference, op.output.dtype);
  if (!result.finalValidation.passed && winner) {
    reject(result.candidates[winnerIndex], "Final execution",
           result.finalValidation.errorMessage, log);
    winner.reset();
    result.finalExecution = baseline->run();
    result.finalValidation = validateExecution(result.finalExecution, reference, op.output.dtype);
  }
  if (!result.finalValidation.passed) {
    result.errorMessage =
        "Final baseline execution/validation failed: " + result.finalValidation.errorMessage;
    return result;
  }
  result.usedBaseline = !winner;
  result.selectedThreads = winner ? result.candidates[winnerIndex].threads : 256;
  result.selectedExecution = winner ? std::move(winner) : std::move(baseline);
  result.success = true;
  log << "Admission report (speedup is the lower of both rounds when confirmed):\n";
  printReport(result.baseline, log);
  for (const auto& report : result.candidates) printReport(report, log);
  log << "Selected: "
      << (result.usedBaseline ? std::string("baseline (fallback)")
                              : result.candidates[winnerIndex].name)
      << ", threads=" << result.selectedThreads << '\n';
  return result;
}

}  // namespace planner

namespace runtime {
namespace {

std::unique_ptr<hip::PreparedSequence> makeSequence(
    hip::HipRuntime& runtime, const std::vector<std::unique_ptr<hip::PreparedExecution>>& steps,
    std::size_t begin = 0) {
  std::vector<const hip::PreparedExecution*> pointers;
  for (std::size_t i = begin; i < steps.size(); ++i) pointers.push_back(steps[i].get());
  auto prepared = runtime.prepareSequence(pointers);
  if (!prepared.execution) throw std::runtime_error(prepared.errorMessage);
  return std::move(prepared.execution);
}

}  // namespace

bool admitFusion(hip::HipRuntime& runtime,
                 std::vector<std::unique_ptr<hip::PreparedExecution>>& steps, std::size_t begin,
                 const std::function<std::vector<std::unique_ptr<hip::PreparedExecution>>()>& build,
                 const std::vector<hip::BufferHandle>& testInputs,
                 const std::vector<hip::BufferHandle>& outputs, const std::string& name,
                 const std::string& decisionKey, FusionDecisionCache& decisions,
                 std::ostream& log) {
  try {
    const auto cached = decisions.find(decisionKey);
    if (cached != decisions.end()) {
      if (!cached->second) {
        log << "Fusion " << name << ": cached FALLBACK\n";
        return false;
      }
      auto fused = build();
      steps.resize(begin);
      for (auto& step : fused) steps.push_back(std::move(step));
      log << "Fusion " << name << ": cached ADMITTED\n";
      return true;
    }
    if (begin > steps.size()) throw std::runtime_error("Fusion region starts past the steps.");
    auto fused = build();
    auto candidate = makeSequence(runtime, fused);
    auto baseline = makeSequence(runtime, steps, begin);
    for (const auto& input : testInputs) {
      std::vector<float> data(input->elementCount());
      for (std::size_t i = 0; i < data.size(); ++i)
        data[i] = static_cast<float>(static_cast<int>(i % 31) - 15) / 31.0f;
      const auto error = runtime.writeBuffer(input, data.data(), data.size());
      if (!error.empty()) throw std::runtime_error(error);
    }
    const auto baseRun = baseline->execute();
    if (!baseRun.executionPassed) throw std::runtime_error(baseRun.errorMessage);
    std::vector<std::vector<double>> references;
    for (const auto& output : outputs) {
      const auto values = output->read();
      references.emplace_back(values.begin(), values.end());
    }
    auto validateCandidate = [&]() {
      const auto run = candidate->execute();
      if (!run.executionPassed) throw std::runtime_error(run.errorMessage);
      for (std::size_t i = 0; i < outputs.size(); ++i) {
        const double tolerance =
            outputs[i]->elementType() == hip::ElementType::Float32 ? 2e-3 : 2e-2;
        const auto comparison =
            validation::compare(outputs[i]->read(), references[i], tolerance, tolerance);
        if (!comparison.passed) throw std::runtime_error(comparison.errorMessage);
      }
    };
    validateCandidate();
    const auto baseSampler = benchmark::sampler(*baseline);
    const auto fusedSampler = benchmark::sampler(*candidate);
    for (const auto* sampler : {&baseSampler, &fusedSampler}) {
      const auto error = benchmark::warmup(*sampler, planner::kTuningWarmup);
      if (!error.empty()) throw std::runtime_error(error);
    }
    const auto first =
        benchmark::measurePair(baseSampler, fusedSampler, planner::kTuningSamples);
    const auto second =
        benchmark::measurePair(baseSampler, fusedSampler, planner::kTuningSamples);
    if (!first.passed || !second.passed) throw std::runtime_error("Fusion benchmark failed.");
    validateCandidate();
    const double speedup = std::min(first.speedup, second.speedup);
    const bool admitted = speedup >= planner::kMinimumSpeedup;
    log << "Fusion " << name << ": compile/interface/template-comparison PASS, speedup="
        << speedup << "x, " << (admitted ? "ADMITTED" : "FALLBACK") << '\n';
    if (admitted) {
      steps.resize(begin);
      for (auto& step : fused) steps.push_back(std::move(step));
    }
    decisions.emplace(decisionKey, admitted);
    return admitted;
  } catch (const std::exception& e) {
    decisions[decisionKey] = false;
    log << "Fusion " << name << ": FALLBACK: " << e.what() << '\n';
    return false;
  }
}

namespace {

constexpr std::size_t kGuardElements = 512;

struct Feedback {
  Feedback(std::string status_, std::string stage_, std::string message_,
           std::optional<double> baseline = std::nullopt,
           std::optional<double> candidate = std::nullopt,
           std::optional<double> ratio = std::nullopt)
      : status(std::move(status_)), stage(std::move(stage_)), message(std::move(message_)),
        baselineUs(baseline), candidateUs(candidate), speedup(ratio) {}
  std::string status;
  std::string stage;
  std::string message;
  std::optional<double> baselineUs;
  std::optional<double> candidateUs;
  std::optional<double> speedup;
};

std::string escapeJson(const std::string& text) {
  std::ostringstream out;
  const char hex[] = "0123456789abcdef";
  for (const unsigned char c : text) {
    switch (c) {
    case '"': out << "\\\""; break;
    case '\\': out << "\\\\"; break;
    case '\n': out << "\\n"; break;
    case '\r': out << "\\r"; break;
    case '\t': out << "\\t"; break;
    default:
      if (c < 0x20) out << "\\u00" << hex[c >> 4] << hex[c & 0xf];
      else out << static_cast<char>(c);
    }
  }
  return out.str();
}

std::string writeFeedback(const Feedback& f, const std::string& path) {
  std::ofstream out(path);
  if (!out) return "Unable to open generated-kernel feedback output '" + path + "'.";
  out << "{\n  \"version\":1,\n  \"status\":\"" << escapeJson(f.status) << "\",\n  \"stage\":\""
      << escapeJson(f.stage) << "\",\n  \"message\":\"" << escapeJson(f.message)
      << "\",\n  \"metrics\":";
  if (f.baselineUs && f.candidateUs && f.speedup)
    out << "{\"baseline_median_us\":" << *f.baselineUs
        << ",\"candidate_median_us\":" << *f.candidateUs << ",\"speedup\":" << *f.speedup << '}';
  else
    out << "null";
  out << "\n}\n";
  if (!out) return "Failed while writing generated-kernel feedback '" + path + "'.";
  return {};
}

// The few JSON fields a candidate response carries: flat object, string or
// integer values.
bool jsonField(const std::string& text, const std::string& key, std::string& value) {
  const auto at = text.find("\"" + key + "\"");
  if (at == std::string::npos) return false;
  auto pos = text.find(':', at + key.size() + 2);
  if (pos == std::string::npos) return false;
  ++pos;
  while (pos < text.size() && std::isspace(static_cast<unsigned char>(text[pos]))) ++pos;
  if (pos < text.size() && text[pos] == '"') {
    std::string out;
    for (++pos; pos < text.size() && text[pos] != '"'; ++pos) {
      if (text[pos] == '\\' && pos + 1 < text.size()) ++pos;
      out.push_back(text[pos]);
    }
    if (pos >= text.size()) return false;
    value = out;
    return true;
  }
  const auto end = text.find_first_of(",}\n", pos);
  value = text.substr(pos, end == std::string::npos ? std::string::npos : end - pos);
  while (!value.empty() && std::isspace(static_cast<unsigned char>(value.back()))) value.pop_back();
  return !value.empty();
}

// A contract case: named inputs (host floats) and the outputs the kernel
// writes, with the template kernel key that produces the reference outputs.
struct ContractCase {
  std::vector<std::vector<float>> inputs;
  std::vector<std::size_t> outputCounts;
  std::string templateKey;
};

struct Contract {
  std::string functionName;
  hip::ElementType storage = hip::ElementType::Float16;
  std::vector<std::string> outputNames;
  std::vector<std::size_t> workgroupSizes;
  double tolerance = 2e-2;
  std::vector<ContractCase> cases;
};

std::vector<float> pattern(std::size_t count, std::size_t salt, float scale, float offset) {
  std::vector<float> v(count);
  for (std::size_t i = 0; i < count; ++i)
    v[i] = offset + scale * static_cast<float>(static_cast<int>((i * 7 + salt) % 29) - 14) / 14.0f;
  return v;
}

Contract makeContract(const std::string& name) {
  Contract c;
  c.workgroupSizes = {64, 128, 256, 512, 1024};
  if (name == "RMSNorm" || name == "AddRMSNorm") {
    const bool add = name == "AddRMSNorm";
    c.functionName = add ? "add_rmsnorm" : "rmsnorm";
    c.outputNames = add ? std::vector<std::string>{"sum", "norm"} : std::vector<std::string>{"out"};
    for (const auto& shape : {std::pair<std::size_t, std::size_t>{1, 4096}, {3, 4096}}) {
      ContractCase k;
      const std::size_t n = shape.first * shape.second;
      k.inputs.push_back(pattern(n, 1, 1.0f, 0.0f));
      if (add) k.inputs.push_back(pattern(n, 5, 1.0f, 0.0f));
      k.inputs.push_back(pattern(shape.second, 3, 0.5f, 1.0f));
      k.outputCounts = add ? std::vector<std::size_t>{n, n} : std::vector<std::size_t>{n};
      k.templateKey = std::string(add ? "add_rmsnorm" : "rmsnorm") + "?rows=" +
                      std::to_string(shape.first) + "&width=" + std::to_string(shape.second) +
                      "&eps=1e-06&dtype=f16";
      c.cases.push_back(std::move(k));
    }
    return c;
  }
  if (name == "SiLUMul") {
    c.functionName = "silu_mul";
    c.outputNames = {"out"};
    for (const std::size_t n : {std::size_t{11008}, std::size_t{8 * 11008}}) {
      ContractCase k;
      k.inputs = {pattern(n, 2, 4.0f, 0.0f), pattern(n, 9, 2.0f, 0.0f)};
      k.outputCounts = {n};
      k.templateKey = "silu_mul?count=" + std::to_string(n) + "&dtype=f16";
      c.cases.push_back(std::move(k));
    }
    return c;
  }
  throw std::invalid_argument("Unknown kernel contract pattern '" + name +
                              "' (RMSNorm, AddRMSNorm, SiLUMul).");
}

// The candidate key must name the contract's function with the case's shape
// parameters; the response gives the key for the first case and the other
// cases reuse its tuning parameters.
std::string keyForCase(const std::string& responseKey, const ContractCase& data) {
  const auto q = responseKey.find('?');
  std::string tuning;
  if (q != std::string::npos) {
    std::stringstream items(responseKey.substr(q + 1));
    std::string item;
    while (std::getline(items, item, '&')) {
      const auto eq = item.find('=');
      const auto field = item.substr(0, eq);
      if (field == "threads" || field == "variant") tuning += "&" + item;
    }
  }
  return data.templateKey + tuning;
}

struct CaseRun {
  std::unique_ptr<hip::PreparedExecution> execution;
  std::unique_ptr<hip::PreparedSequence> sequence;
  std::vector<hip::BufferHandle> outputs;
};

CaseRun prepareCase(hip::HipRuntime& runtime, const Contract& contract, const ContractCase& data,
                    const std::string& key, const std::string& functionName, bool guarded) {
  const auto pipeline = runtime.createComputePipeline(key, functionName);
  if (!pipeline.pipelineCreationPassed) throw std::runtime_error(pipeline.errorMessage);
  CaseRun run;
  std::vector<hip::BufferHandle> inputs;
  for (const auto& values : data.inputs) {
    auto padded = values;
    if (guarded) padded.resize(padded.size() + kGuardElements, 1.0f);
    auto buffer = runtime.createBuffer(padded.size(), padded.data(), contract.storage);
    if (!buffer.buffer) throw std::runtime_error(buffer.errorMessage);
    inputs.push_back(std::move(buffer.buffer));
  }
  for (const auto count : data.outputCounts) {
    auto buffer =
        runtime.createBuffer(count + (guarded ? kGuardElements : 0), nullptr, contract.storage);
    if (!buffer.buffer) throw std::runtime_error(buffer.errorMessage);
    run.outputs.push_back(std::move(buffer.buffer));
  }
  auto prepared = runtime.prepareBuffers(
      inputs, run.outputs, {pipeline.threadgroupCount, pipeline.threadsPerThreadgroup});
  if (!prepared.execution) throw std::runtime_error(prepared.errorMessage);
  run.execution = std::move(prepared.execution);
  auto sequence = runtime.prepareSequence({run.execution.get()});
  if (!sequence.execution) throw std::runtime_error(sequence.errorMessage);
  run.sequence = std::move(sequence.execution);
  return run;
}

std::string validateCase(hip::HipRuntime& runtime, CaseRun& run, const Contract& contract,
                         const ContractCase& data,
                         const std::vector<std::vector<double>>& references, bool guarded) {
  for (const auto& output : run.outputs) {
    std::vector<float> sentinel(output->elementCount(), std::numeric_limits<float>::quiet_NaN());
    const auto error = runtime.writeBuffer(output, sentinel.data(), sentinel.size());
    if (!error.empty()) return error;
  }
  const auto result = run.sequence->execute();
  if (!result.executionPassed) return result.errorMessage;
  for (std::size_t i = 0; i < run.outputs.size(); ++i) {
    const auto values = run.outputs[i]->read();
    const auto count = data.outputCounts[i];
    if (values.size() != count + (guarded ? kGuardElements : 0)) return "Output size mismatch.";
    const std::vector<float> logical(values.begin(), values.begin() + count);
    const auto comparison =
        validation::compare(logical, references[i], contract.tolerance, contract.tolerance);
    if (!comparison.passed) return contract.outputNames[i] + ": " + comparison.errorMessage;
    if (guarded && !std::all_of(values.begin() + count, values.end(),
                                [](float v) { return std::isnan(v); }))
      return "Output guard modified: " + contract.outputNames[i];
  }
  return {};
}

}  // namespace

bool admitGeneratedKernel(hip::HipRuntime& runtime, const std::string& patternName,
                          const std::string& responsePath, const std::string& feedbackPath,
                          std::ostream& log, const std::string& artifactPath) {
  auto report = [&](const Feedback& feedback) -> bool {
    const auto error = writeFeedback(feedback, feedbackPath);
    log << "Generated candidate " << feedback.stage << ": "
        << (feedback.status == "admitted" ? "PASS" : "FAIL") << ": " << feedback.message << '\n';
    if (!error.empty()) {
      log << "Feedback error: " << error << '\n';
      return false;
    }
    log << "Generated kernel admission: "
        << (feedback.status == "admitted" ? "PASS"
                                          : feedback.status == "fatal" ? "FAIL" : "FALLBACK")
        << "\nSelected: " << (feedback.status == "admitted" ? "generated " : "template ")
        << patternName << '\n';
    return feedback.status != "fatal";
  };
  try {
    const auto contract = makeContract(patternName);
    // Template baselines and their reference outputs.
    std::vector<CaseRun> baselines;
    std::vector<std::vector<std::vector<double>>> references;
    for (std::size_t i = 0; i < contract.cases.size(); ++i) {
      const auto& data = contract.cases[i];
      auto base = prepareCase(runtime, contract, data, data.templateKey, contract.functionName,
                              false);
      const auto run = base.sequence->execute();
      if (!run.executionPassed) throw std::runtime_error(run.errorMessage);
      std::vector<std::vector<double>> outs;
      for (const auto& output : base.outputs) {
        const auto values = output->read();
        outs.emplace_back(values.begin(), values.end());
      }
      references.push_back(std::move(outs));
      const auto warm = benchmark::warmup(benchmark::sampler(*base.sequence), 5);
      if (!warm.empty()) throw std::runtime_error(warm);
      log << "Template baseline case " << i << ": " << data.templateKey << '\n';
      baselines.push_back(std::move(base));
    }
    std::ifstream in(responsePath);
    if (!in) return report({"retry", "response_parse", "Unable to read '" + responsePath + "'."});
    std::stringstream buffer;
    buffer << in.rdbuf();
    const std::string text = buffer.str();
    std::string functionName, source, workgroup;
    if (!jsonField(text, "function_name", functionName) || !jsonField(text, "source", source) ||
        !jsonField(text, "workgroup_size", workgroup))
      return report({"retry", "response_parse",
                     "Response needs function_name, source and workgroup_size."});
    if (functionName != contract.functionName)
      return report({"retry", "contract", "Expected function_name: " + contract.functionName});
    const auto qpos = source.find('?');
    if (source.substr(0, qpos) != contract.functionName)
      return report({"retry", "contract",
                     "The kernel key must name " + contract.functionName + "."});
    std::size_t workgroupSize = 0;
    try {
      workgroupSize = static_cast<std::size_t>(std::stoul(workgroup));
    } catch (const std::exception&) {
      return report({"retry", "response_parse", "workgroup_size is not an integer."});
    }
    const auto hardware = runtime.hardwareInfo();
    if (std::find(contract.workgroupSizes.begin(), contract.workgroupSizes.end(),
                  workgroupSize) == contract.workgroupSizes.end() ||
        workgroupSize > hardware.maxThreadsPerThreadgroup)
      return report({"retry", "hardware_filter",
                     "workgroup_size is not legal for this contract/device."});
    std::vector<CaseRun> candidates;
    for (std::size_t i = 0; i < contract.cases.size(); ++i) {
      const auto& data = contract.cases[i];
      std::string key = keyForCase(source, data);
      if (key.find("threads=") == std::string::npos)
        key += "&threads=" + std::to_string(workgroupSize);
      CaseRun run;
      try {
        run = prepareCase(runtime, contract, data, key, functionName, true);
      } catch (const std::exception& e) {
        return report({"retry", i == 0 ? "compile" : "prepare", e.what()});
      }
      const auto error = validateCase(runtime, run, contract, data, references[i], true);
      if (!error.empty())
        return report({"retry", "numerical_validation",
                       "case " + std::to_string(i) + ": " + error});
      log << "Generated candidate case " << i << " (" << key
          << ") all outputs numerical validation: PASS\n";
      candidates.push_back(std::move(run));
    }
    double worst = std::numeric_limits<double>::infinity();
    std::optional<Feedback> failure;
    Feedback accepted{"admitted", "admission",
                      "All cases passed correctness and two performance rounds."};
    for (std::size_t i = 0; i < candidates.size(); ++i) {
      const auto baseSampler = benchmark::sampler(*baselines[i].sequence);
      const auto candSampler = benchmark::sampler(*candidates[i].sequence);
      const auto warm = benchmark::warmup(candSampler, planner::kTuningWarmup);
      if (!warm.empty()) return report({"retry", "warmup", warm});
      for (int round = 0; round < 2; ++round) {
        const auto timing =
            benchmark::measurePair(baseSampler, candSampler, planner::kTuningSamples);
        if (!timing.passed) return report({"retry", "benchmark", timing.errorMessage});
        log << "Generated candidate case " << i << " round " << round + 1
            << ": baseline(us)=" << timing.baseline.medianUs
            << ", candidate(us)=" << timing.candidate.medianUs << ", speedup=" << timing.speedup
            << "x\n";
        if (timing.speedup < worst) {
          worst = timing.speedup;
          accepted.baselineUs = timing.baseline.medianUs;
          accepted.candidateUs = timing.candidate.medianUs;
          accepted.speedup = timing.speedup;
        }
        if (timing.speedup < planner::kMinimumSpeedup &&
            (!failure || timing.speedup < *failure->speedup))
          failure = Feedback{"retry", "performance",
                             "case " + std::to_string(i) + " round " + std::to_string(round + 1) +
                                 " speedup is below 1.05x.",
                             timing.baseline.medianUs, timing.candidate.medianUs, timing.speedup};
      }
      const auto finalError =
          validateCase(runtime, candidates[i], contract, contract.cases[i], references[i], true);
      if (!finalError.empty()) return report({"retry", "final_validation", finalError});
    }
    if (failure) return report(*failure);
    if (!artifactPath.empty()) {
      std::ofstream out(artifactPath);
      out << "{\"function_name\":\"" << escapeJson(functionName) << "\",\"source\":\""
          << escapeJson(source) << "\",\"workgroup_size\":" << workgroupSize << "}\n";
      if (!out) return report({"fatal", "artifact_write", "Unable to write " + artifactPath});
    }
    return report(accepted);
  } catch (const std::exception& e) {
    return report(Feedback("fatal", "baseline_or_contract", e.what()));
  }
}

}  // namespace runtime

}  // namespace tensor
