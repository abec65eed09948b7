// Timing helpers; see Benchmark.hpp.
#include "Benchmark.hpp"

#include <algorithm>
#include <cmath>

namespace tensor::benchmark {
namespace {

Statistics summarize(std::vector<double> values) {
  std::sort(values.begin(), values.end());
  const std::size_t n = values.size();
  Statistics s;
  s.samples = n;
  s.medianUs = n % 2 == 0 ? 0.5 * (values[n / 2 - 1] + values[n / 2]) : values[n / 2];
  const double position = 0.9 * static_cast<double>(n - 1);
  const auto lower = static_cast<std::size_t>(position);
  const auto upper = std::min(lower + 1, n - 1);
  const double weight = position - static_cast<double>(lower);
  s.p90Us = values[lower] * (1.0 - weight) + values[upper] * weight;
  s.minUs = values.front();
  s.maxUs = values.back();
  return s;
}

std::string take(const Sampler& run, std::vector<double>& values) {
  std::string error;
  const auto us = run(error);
  if (!error.empty()) return "GPU execution failed: " + error;
  if (!us || !std::isfinite(*us) || *us <= 0.0)
    return "GPU timestamps unavailable; no performance comparison is possible.";
  values.push_back(*us);
  return {};
}

template <typename Work>
Sampler makeSampler(const Work& work) {
  return [&work](std::string& error) -> std::optional<double> {
    const auto result = work.execute();
    if (!result.executionPassed) {
      error = result.errorMessage;
      return std::nullopt;
    }
    return result.gpuExecutionTimeUs;
  };
}

}  // namespace

std::optional<Statistics> summarizeTimings(const std::vector<double>& values) {
  if (values.empty()) return std::nullopt;
  return summarize(values);
}

std::string warmup(const Sampler& run, std::size_t iterations) {
  for (std::size_t i = 0; i < iterations; ++i) {
    std::string error;
    (void)run(error);
    if (!error.empty()) return error;
  }
  return {};
}

Result measure(const Sampler& run, std::size_t samples) {
  Result result;
  if (samples == 0) {
    result.errorMessage = "Benchmark requires at least one sample.";
    return result;
  }
  std::vector<double> values;
  for (std::size_t i = 0; i < samples; ++i) {
    result.errorMessage = take(run, values);
    if (!result.errorMessage.empty()) return result;
  }
  result.stats = summarize(values);
  result.passed = true;
  return result;
}

PairedResult measurePair(const Sampler& baseline, const Sampler& candidate, std::size_t samples) {
  PairedResult result;
  if (samples == 0) {
    result.errorMessage = "Benchmark requires at least one sample.";
    return result;
  }
  std::vector<double> base, cand;
  for (std::size_t i = 0; i < samples; ++i) {
    for (std::size_t slot = 0; slot < 2; ++slot) {
      const bool runBaseline = (i + slot) % 2 == 0;
      const auto error = take(runBaseline ? baseline : candidate, runBaseline ? base : cand);
      if (!error.empty()) {
        result.errorMessage = (runBaseline ? "Baseline: " : "Candidate: ") + error;
        return result;
      }
    }
  }
  result.baseline = summarize(base);
  result.candidate = summarize(cand);
  result.speedup = result.baseline.medianUs / result.candidate.medianUs;
  result.passed = true;
  return result;
}

Sampler sampler(const hip::PreparedExecution& execution) { return makeSampler(execution); }
Sampler sampler(const hip::PreparedSequence& sequence) { return makeSampler(sequence); }

}  // namespace tensor::benchmark
