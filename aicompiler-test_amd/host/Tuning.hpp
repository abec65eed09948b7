// Kernel selection for the gfx950 decode path: the decode GEMV tuner, the
// RMSNorm tuner, fusion admission and kernel-candidate admission, with the
// interfaces and the admission rule of the reference:
//   tuneDecodeGEMV        src/planner/DecodeGEMVTuner.cpp:162-304
//   tuneRMSNorm           src/planner/RMSNormTuner.cpp:159-309
//   admitFusion           src/runtime/DecoderLLMExecutor.cpp:92-163
//   admitGeneratedKernel  src/runtime/GeneratedKernelAdmission.cpp:204-318
// A candidate is admitted only when it is correct against the reference (CPU
// double-precision reference where affordable, else the baseline's GPU
// output) and at least 1.05x faster than the baseline in two paired rounds
// (warmup 5, 31 samples each); the lower of the two speedups ranks it.
// Retargeting to gfx950: candidates are launch configurations of the HIP
// kernels (workgroups are multiples of the 64-lane wave, LDS within the 160
// KiB of a CU and the 64 KiB a launch here may ask for), and a "kernel
// source" is a kernel key resolved by the runtime.
#pragma once

#include "Benchmark.hpp"
#include "HipRuntime.hpp"
#include "KVCacheState.hpp"
#include "TensorIR.hpp"

#include <cstddef>
#include <functional>
#include <iosfwd>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <vector>

namespace tensor {

namespace validation {

// ValidationResult / compare (Validator.hpp:11-21, Validator.cpp:11-38):
// every element must satisfy |actual - expected| <= atol + rtol * |expected|
// and be finite.
struct ValidationResult {
  bool passed = false;
  double maxAbsoluteError = 0.0;
  std::size_t mismatchCount = 0;
  std::string errorMessage;
};

[[nodiscard]] ValidationResult compare(const std::vector<float>& actual,
                                       const std::vector<double>& reference,
                                       double absoluteTolerance, double relativeTolerance);

// rmsNormReference (Validator.cpp:40-66): double accumulation.
[[nodiscard]] std::vector<double> rmsNormReference(const RMSNormOp& op,
                                                   const std::vector<float>& input,
                                                   const std::vector<float>& weight);

}  // namespace validation

namespace hip {

// DecodeGEMVConfig (DecodeGEMVMetalEmitter.hpp:11-16) for gfx950: the fields
// of tmc_gemv_config (include/tmc_hip.h).  algorithm 0 = default for the
// shape, 1 = wave64 split-K dot, 2 = MFMA, 3 = MFMA row tiles, 4 = linear
// baseline.
struct DecodeGEMVConfig {
  int algorithm = 0;
  int rowsPerWave = 1;
  int unroll = 1;
  int kSplit = 1;
};

// GeneratedKernel (MetalEmitter.hpp:13-18): `source` is a gfx950 kernel key.
struct GeneratedKernel {
  std::string source;
  std::string functionName;
  std::size_t threadgroupCount = 0;
  std::size_t threadsPerThreadgroup = 0;
};

// emitDecodeGEMV (DecodeGEMVMetalEmitter.cpp:68-132) and emitLinearBaseline
// (:18-66) as kernel keys; elementType must be Float16, outputType Float16
// or Float32.
[[nodiscard]] GeneratedKernel emitDecodeGEMV(std::size_t batch, std::size_t inputSize,
                                             std::size_t outputSize,
                                             const DecodeGEMVConfig& config,
                                             const std::string& name, ElementType elementType,
                                             ElementType outputType);
[[nodiscard]] GeneratedKernel emitLinearBaseline(std::size_t batch, std::size_t inputSize,
                                                 std::size_t outputSize,
                                                 const std::string& name,
                                                 ElementType elementType,
                                                 ElementType outputType);
// emitRMSNorm(op, threads) (MetalEmitter.cpp:12-76) and emitRMSNormBaseline
// (RMSNormBaseline.cpp:13-72, fixed 256-thread two-pass kernel).
[[nodiscard]] GeneratedKernel emitRMSNorm(const RMSNormOp& op, std::size_t threads);
[[nodiscard]] GeneratedKernel emitRMSNormBaseline(const RMSNormOp& op);

// Workgroup size and LDS bytes one launch of `config` asks for.
[[nodiscard]] std::size_t decodeGEMVThreads(const DecodeGEMVConfig& config);
[[nodiscard]] std::size_t decodeGEMVLdsBytes(std::size_t batch, const DecodeGEMVConfig& config);

}  // namespace hip

namespace planner {

constexpr std::size_t kTuningWarmup = 5;
constexpr std::size_t kTuningSamples = 31;
constexpr double kMinimumSpeedup = 1.05;
// gfx950: LDS per compute unit, and what one launch here may allocate.
constexpr std::size_t kLdsBytesPerCU = 160 * 1024;
constexpr std::size_t kLdsBytesPerLaunch = 64 * 1024;

// The admission rule shared by every tuner: the first paired round must
// reach kMinimumSpeedup; the confirmation round is taken only then, and the
// candidate is admitted when the lower of the two speedups still reaches it.
struct AdmissionDecision {
  bool admitted = false;
  double conservativeSpeedup = 0.0;
  std::string reason;
};
[[nodiscard]] AdmissionDecision admissionDecision(
    const benchmark::PairedResult& first,
    const std::optional<benchmark::PairedResult>& confirmation);

struct DecodeGEMVSelection {
  bool success = false;
  bool useBaseline = true;
  hip::DecodeGEMVConfig config;
  double conservativeSpeedup = 1.0;
  std::string errorMessage;
};

// The gfx950 candidate list for a shape (decode: dot configurations at
// batch 1, MFMA configurations above), before the hardware filter.
[[nodiscard]] std::vector<hip::DecodeGEMVConfig> decodeGEMVCandidates(std::size_t batch,
                                                                      bool prefill = false);
// "" when `config` fits the device and the shape, else the reason.
[[nodiscard]] std::string decodeGEMVHardwareFilter(const hip::DecodeGEMVConfig& config,
                                                   std::size_t batch, std::size_t inputSize,
                                                   std::size_t outputSize,
                                                   const hip::HardwareInfo& hardware);

// tuneDecodeGEMV (DecodeGEMVTuner.cpp:162-304).  Weights are stored fp16
// (storageDtype must be Float16); the output is fp16 like the storage.  The
// baseline is the linear baseline (algorithm 4).
[[nodiscard]] DecodeGEMVSelection tuneDecodeGEMV(hip::HipRuntime& runtime, std::size_t batch,
                                                 std::size_t inputSize, std::size_t outputSize,
                                                 const std::vector<float>& input,
                                                 const std::vector<float>& weight,
                                                 std::ostream& log,
                                                 DType storageDtype = DType::Float16,
                                                 bool prefill = false);

// tuneDecodeGEMV over device buffers already resident (fp16 input
// [batch, in] and weight [out, in], finite values): no host copies of the
// weights; the linear baseline's output on the same buffers is the reference
// (the reference tuner's large-shape path, DecodeGEMVTuner.cpp:197-203).
[[nodiscard]] DecodeGEMVSelection tuneDecodeGEMV(hip::HipRuntime& runtime, std::size_t batch,
                                                 std::size_t inputSize, std::size_t outputSize,
                                                 const hip::BufferHandle& input,
                                                 const hip::BufferHandle& weight,
                                                 std::ostream& log,
                                                 hip::ElementType outputType =
                                                     hip::ElementType::Float16);

// Per-shape decode GEMV selections shared by every executor of the process.
// The reference tunes again for every compiled request (ServingRuntime.cpp
// :582-617); a shape is tuned once here.
class DecodeGEMVTuningCache {
 public:
  [[nodiscard]] static std::string key(std::size_t batch, std::size_t inputSize,
                                       std::size_t outputSize, hip::ElementType outputType);
  [[nodiscard]] std::optional<DecodeGEMVSelection> find(const std::string& key) const;
  void store(const std::string& key, const DecodeGEMVSelection& selection);
  [[nodiscard]] std::size_t size() const { return entries_.size(); }
  void clear() { entries_.clear(); }

 private:
  std::map<std::string, DecodeGEMVSelection> entries_;
};

[[nodiscard]] DecodeGEMVTuningCache& decodeGEMVTuningCache();

// The cached selection for the shape, tuning it on `input` / `weight` first
// when the cache has none.
[[nodiscard]] DecodeGEMVSelection cachedDecodeGEMV(hip::HipRuntime& runtime, std::size_t batch,
                                                   std::size_t inputSize, std::size_t outputSize,
                                                   const hip::BufferHandle& input,
                                                   const hip::BufferHandle& weight,
                                                   std::ostream& log,
                                                   hip::ElementType outputType =
                                                       hip::ElementType::Float16);

// CandidateReport / TuningResult (RMSNormTuner.hpp:12-38).
struct CandidateReport {
  std::string name;
  std::size_t threads = 0;
  std::string outcome;
  std::string reason;
  std::optional<double> medianGpuUs;
  std::optional<double> pairedBaselineUs;
  std::optional<double> speedup;
};

struct TuningResult {
  bool success = false;
  bool usedBaseline = true;
  std::size_t selectedThreads = 256;
  CandidateReport baseline;
  std::vector<CandidateReport> candidates;
  std::unique_ptr<hip::PreparedExecution> selectedExecution;
  hip::ExecutionResult finalExecution;
  validation::ValidationResult finalValidation;
  std::string errorMessage;
};

// Wave multiples up to the workgroup limit.
[[nodiscard]] std::vector<std::size_t> defaultRMSNormCandidates();
[[nodiscard]] std::string rmsNormHardwareFilter(const RMSNormOp& op, std::size_t threads,
                                                const hip::HardwareInfo& hardware);

// tuneRMSNorm (RMSNormTuner.cpp:159-309).
[[nodiscard]] TuningResult tuneRMSNorm(hip::HipRuntime& runtime, const RMSNormOp& op,
                                       const std::vector<float>& input,
                                       const std::vector<float>& weight,
                                       const std::vector<std::size_t>& candidateThreads,
                                       std::ostream& log);

}  // namespace planner

namespace runtime {

using FusionDecisionCache = std::map<std::string, bool>;

// admitFusion (DecoderLLMExecutor.cpp:92-163): replaces steps[begin, end)
// by the fused steps `build()` returns when, on deterministic test inputs
// (value i -> ((i % 31) - 15) / 31), the fused sequence reproduces the
// unfused outputs (tolerance 2e-3 for fp32 outputs, 2e-2 otherwise) and is
// >= 1.05x faster in two paired rounds.  Decisions are cached by key.
[[nodiscard]] bool admitFusion(
    hip::HipRuntime& runtime, std::vector<std::unique_ptr<hip::PreparedExecution>>& steps,
    std::size_t begin,
    const std::function<std::vector<std::unique_ptr<hip::PreparedExecution>>()>& build,
    const std::vector<hip::BufferHandle>& testInputs, const std::vector<hip::BufferHandle>& outputs,
    const std::string& name, const std::string& decisionKey, FusionDecisionCache& decisions,
    std::ostream& log);

// admitGeneratedKernel (GeneratedKernelAdmission.cpp:204-318) for gfx950.
// `pattern` names a region contract: "RMSNorm", "AddRMSNorm" or "SiLUMul"
// (or decoder_rmsnorm, decoder_residual_rmsnorm, decoder_silu_mul).  The
// response file is JSON with "function_name" (must equal the contract's),
// "source" (a gfx950 kernel key naming that function; its threads / variant
// parameters are applied to every contract case) and "workgroup_size" (a
// contract workgroup size within the device limit).  Every case is validated
// with guarded outputs (512 extra elements that must stay NaN) against the
// template kernel's result, then timed in two paired rounds against the
// template; the slowest round must reach 1.05x.  Feedback JSON goes to
// feedbackPath (see AdmissionFeedback).  Returns false only on a fatal
// outcome.  When admitted and artifactPath is given, the admitted-kernel
// artifact for the KernelRegistry is written there.
[[nodiscard]] bool admitGeneratedKernel(hip::HipRuntime& runtime, const std::string& pattern,
                                        const std::string& responsePath,
                                        const std::string& feedbackPath, std::ostream& log,
                                        const std::string& artifactPath = {});

}  // namespace runtime

}  // namespace tensor
