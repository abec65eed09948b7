// Timing helpers; see Benchmark.hpp.
#include "Benchmark.hpp"

#include <algorithm>
#include <cmath>

namespace tensor::benchmark {
namespace {

constexpr const char* kNoSamples = "Benchmark requires at least one sample.";

// Order statistics of a sample set: the value at fractional rank r of the
// sorted samples interpolates linearly between ranks floor(r) and
// floor(r) + 1.  The median is rank (n - 1) / 2 (the mean of the two middle
// samples when n is even), the 90th percentile rank 0.9 (n - 1).
Statistics describe(std::vector<double> us) {
  std::sort(us.begin(), us.end());
  const std::size_t last = us.size() - 1;
  const auto at = [&](double rank) {
    const std::size_t lo = static_cast<std::size_t>(rank);
    const std::size_t hi = std::min(lo + 1, last);
    const double t = rank - static_cast<double>(lo);
    return us[lo] + (us[hi] - us[lo]) * t;
  };
  Statistics s;
  s.samples = us.size();
  s.medianUs = at(0.5 * static_cast<double>(last));
  s.p90Us = at(0.9 * static_cast<double>(last));
  s.minUs = us.front();
  s.maxUs = us.back();
  return s;
}

// Run one timed sample and append its GPU time; "" or why it is unusable.
std::string record(const Sampler& run, std::vector<double>& us) {
  std::string failure;
  const std::optional<double> t = run(failure);
  if (!failure.empty()) return "GPU execution failed: " + failure;
  const bool usable = t.has_value() && std::isfinite(*t) && *t > 0.0;
  if (!usable) return "GPU timestamps unavailable; no performance comparison is possible.";
  us.push_back(*t);
  return {};
}

template <typename Work>
Sampler timed(const Work& work) {
  return [&work](std::string& failure) -> std::optional<double> {
    const auto r = work.execute();
    if (r.executionPassed) return r.gpuExecutionTimeUs;
    failure = r.errorMessage;
    return std::nullopt;
  };
}

}  // namespace

std::optional<Statistics> summarizeTimings(const std::vector<double>& values) {
  return values.empty() ? std::nullopt : std::optional<Statistics>(describe(values));
}

std::string warmup(const Sampler& run, std::size_t iterations) {
  std::string failure;
  for (std::size_t i = 0; i < iterations && failure.empty(); ++i) (void)run(failure);
  return failure;
}

Result measure(const Sampler& run, std::size_t samples) {
  Result out;
  if (samples == 0) {
    out.errorMessage = kNoSamples;
    return out;
  }
  std::vector<double> us;
  us.reserve(samples);
  while (us.size() < samples) {
    out.errorMessage = record(run, us);
    if (!out.errorMessage.empty()) return out;
  }
  out.stats = describe(std::move(us));
  out.passed = true;
  return out;
}

PairedResult measurePair(const Sampler& baseline, const Sampler& candidate, std::size_t samples) {
  PairedResult out;
  if (samples == 0) {
    out.errorMessage = kNoSamples;
    return out;
  }
  struct Arm {
    const Sampler* run;
    const char* label;
    std::vector<double> us;
  };
  Arm arms[2] = {{&baseline, "Baseline: ", {}}, {&candidate, "Candidate: ", {}}};
  for (std::size_t round = 0; round < samples; ++round) {
    // Each round times both; the one that goes first alternates, so neither
    // always meets the device right after the other.
    for (std::size_t k = 0; k < 2; ++k) {
      Arm& arm = arms[(round + k) % 2];
      const std::string failure = record(*arm.run, arm.us);
      if (!failure.empty()) {
        out.errorMessage = arm.label + failure;
        return out;
      }
    }
  }
  out.baseline = describe(std::move(arms[0].us));
  out.candidate = describe(std::move(arms[1].us));
  out.speedup = out.baseline.medianUs / out.candidate.medianUs;
  out.passed = true;
  return out;
}

Sampler sampler(const hip::PreparedExecution& execution) { return timed(execution); }
Sampler sampler(const hip::PreparedSequence& sequence) { return timed(sequence); }

}  // namespace tensor::benchmark
