// Admitted-kernel artifacts and the registry the decoder consults, with the
// interface of the reference's src/runtime/KernelRegistry.hpp:12-38
// (writeAdmittedKernel, KernelRegistry::load/find/track/completed/resetUsage/
// report).  On gfx950 an admitted kernel is a kernel key plus a workgroup
// size for one fused region of the decoder (decoder_rmsnorm,
// decoder_residual_rmsnorm, decoder_silu_mul), admitted by
// admitGeneratedKernel against the region's template kernel.
//
// Artifact (<library>/<pattern>/admitted.json):
//   {"version":1,"status":"admitted","contract":{...},"candidate":
//    {"function_name":"...","source":"<kernel key>","workgroup_size":N}}
// where "contract" is kernelContractText() for the pattern on the device that
// admitted it (arch gfx950, device name, wave size and workgroup / LDS
// limits).  load() takes an artifact only when its contract equals the
// current device's text exactly; anything else leaves the region on its
// template kernel, with the reason in the log.
#pragma once

#include "HipRuntime.hpp"

#include <cstddef>
#include <functional>
#include <iosfwd>
#include <map>
#include <optional>
#include <string>
#include <vector>

namespace tensor::runtime {

struct AdmittedKernel {
  std::string functionName;
  std::string source;  // gfx950 kernel key
  std::size_t workgroupSize = 0;
};

// The admission feedback file: {"version":1,"status","stage","message",
// "metrics":{"baseline_median_us","candidate_median_us","speedup"}|null};
// status "admitted" | "retry" | "fatal".
struct AdmissionFeedback {
  AdmissionFeedback(std::string status_, std::string stage_, std::string message_,
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
[[nodiscard]] std::string writeAdmissionFeedback(const AdmissionFeedback& feedback,
                                                 const std::string& path);

// Minimal JSON helpers for these flat records.
[[nodiscard]] std::string jsonEscape(const std::string& text);
// The value of "key" as text: a string's unescaped contents, a number's
// digits, or an object's raw text with its braces.  False when absent.
[[nodiscard]] bool jsonStringField(const std::string& text, const std::string& key,
                                   std::string& value);

// The region contract of `pattern` (RMSNorm / AddRMSNorm / SiLUMul or their
// decoder_* names) on this runtime's device, as compact JSON; throws
// std::invalid_argument for an unknown pattern.  Defined in Tuning.cpp.
[[nodiscard]] std::string kernelContractText(const hip::HipRuntime& runtime,
                                             const std::string& pattern);
// decoder_* name of a pattern (throws for an unknown one).
[[nodiscard]] std::string canonicalKernelPattern(const std::string& pattern);

// writeAdmittedKernel (KernelRegistry.mm:22-41): "" or the write error.
[[nodiscard]] std::string writeAdmittedKernel(const hip::HipRuntime& runtime,
                                              const std::string& pattern,
                                              const AdmittedKernel& kernel,
                                              const std::string& path);

struct KernelUsage {
  std::string node;
  std::string pattern;
  std::string implementation;  // "generated", "template" or "folded" (no launch)
  std::string functions;       // the kernel key it runs
  std::size_t dispatchesPerCall = 0;
  std::size_t completedCalls = 0;
};

class KernelRegistry {
 public:
  // KernelRegistry::load (KernelRegistry.mm:43-103): every decoder_*
  // directory under `directory` with an admitted.json whose contract matches
  // this device.  An empty directory name means template kernels only.
  void load(const hip::HipRuntime& runtime, const std::string& directory, std::ostream& log);
  // The same with the contract text supplied per pattern (host-only use).
  void load(const std::function<std::string(const std::string&)>& contractText,
            const std::string& directory, std::ostream& log);
  [[nodiscard]] const AdmittedKernel* find(const std::string& pattern) const;
  [[nodiscard]] std::size_t size() const noexcept { return entries_.size(); }
  // Usage audit: track() registers a region node and returns its index;
  // completed() counts one finished call of each listed index.
  std::size_t track(KernelUsage usage);
  void completed(const std::vector<std::size_t>& uses);
  void resetUsage() noexcept;
  void report(std::ostream& log) const;
  [[nodiscard]] const std::vector<KernelUsage>& usage() const noexcept { return usage_; }

 private:
  std::map<std::string, AdmittedKernel> entries_;
  std::vector<KernelUsage> usage_;
};

}  // namespace tensor::runtime
