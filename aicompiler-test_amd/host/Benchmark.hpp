// Timing helpers used by the tuners and the serving metrics, with the
// semantics of the reference's src/benchmark/Benchmark.hpp:10-56: statistics
// over GPU-timed samples (median, 90th percentile by linear interpolation,
// min, max) and paired measurements that alternate which candidate runs first.
#pragma once

#include "HipRuntime.hpp"

#include <cstddef>
#include <functional>
#include <optional>
#include <string>
#include <vector>

namespace tensor::benchmark {

struct Statistics {
  std::size_t samples = 0;
  double medianUs = 0.0;
  double p90Us = 0.0;
  double minUs = 0.0;
  double maxUs = 0.0;
};

struct Result {
  bool passed = false;
  Statistics stats;
  std::string errorMessage;
};

struct PairedResult {
  bool passed = false;
  Statistics baseline;
  Statistics candidate;
  double speedup = 0.0;  // baseline median / candidate median
  std::string errorMessage;
};

// One timed sample: returns the GPU time in microseconds or an error.
using Sampler = std::function<std::optional<double>(std::string& error)>;

[[nodiscard]] std::optional<Statistics> summarizeTimings(const std::vector<double>& values);

[[nodiscard]] std::string warmup(const Sampler& run, std::size_t iterations);
[[nodiscard]] Result measure(const Sampler& run, std::size_t samples);
[[nodiscard]] PairedResult measurePair(const Sampler& baseline, const Sampler& candidate,
                                       std::size_t samples);

// Samplers over prepared work (execute() with HIP-event timing).
[[nodiscard]] Sampler sampler(const hip::PreparedExecution& execution);
[[nodiscard]] Sampler sampler(const hip::PreparedSequence& sequence);

}  // namespace tensor::benchmark
