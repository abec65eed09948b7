// Admitted-kernel artifacts and the kernel registry; see KernelRegistry.hpp.
#include "KernelRegistry.hpp"

#include <algorithm>
#include <cctype>
#include <filesystem>
#include <fstream>
#include <ostream>
#include <sstream>

namespace tensor::runtime {

std::string jsonEscape(const std::string& text) {
  std::string out;
  out.reserve(text.size());
  for (const unsigned char c : text) {
    if (c == '"' || c == '\\') {
      out += '\\';
      out += static_cast<char>(c);
    } else if (c == '\n') {
      out += "\\n";
    } else if (c == '\t') {
      out += "\\t";
    } else if (c < 0x20) {
      static const char digits[] = "0123456789abcdef";
      out += "\\u00";
      out += digits[c >> 4];
      out += digits[c & 15];
    } else {
      out += static_cast<char>(c);
    }
  }
  return out;
}

bool jsonStringField(const std::string& text, const std::string& key, std::string& value) {
  const std::string quoted = "\"" + key + "\"";
  std::size_t at = text.find(quoted);
  if (at == std::string::npos) return false;
  at = text.find(':', at + quoted.size());
  if (at == std::string::npos) return false;
  ++at;
  while (at < text.size() && std::isspace(static_cast<unsigned char>(text[at]))) ++at;
  if (at >= text.size()) return false;
  if (text[at] == '"') {  // string: unescape \" \\ \n \t
    std::string out;
    for (++at; at < text.size() && text[at] != '"'; ++at) {
      if (text[at] == '\\' && at + 1 < text.size()) {
        ++at;
        out += text[at] == 'n' ? '\n' : text[at] == 't' ? '\t' : text[at];
      } else {
        out += text[at];
      }
    }
    if (at >= text.size()) return false;
    value = out;
    return true;
  }
  if (text[at] == '{') {  // object: raw text up to the matching brace
    int depth = 0;
    bool inString = false;
    for (std::size_t i = at; i < text.size(); ++i) {
      const char c = text[i];
      if (inString) {
        if (c == '\\') ++i;
        else if (c == '"') inString = false;
      } else if (c == '"') {
        inString = true;
      } else if (c == '{') {
        ++depth;
      } else if (c == '}' && --depth == 0) {
        value = text.substr(at, i + 1 - at);
        return true;
      }
    }
    return false;
  }
  const std::size_t end = text.find_first_of(",}\n", at);
  value = text.substr(at, end == std::string::npos ? std::string::npos : end - at);
  while (!value.empty() && std::isspace(static_cast<unsigned char>(value.back()))) value.pop_back();
  return !value.empty();
}

std::string writeAdmissionFeedback(const AdmissionFeedback& f, const std::string& path) {
  std::ofstream out(path);
  if (!out) return "Unable to open generated-kernel feedback output '" + path + "'.";
  out << "{\n  \"version\":1,\n  \"status\":\"" << jsonEscape(f.status) << "\",\n  \"stage\":\""
      << jsonEscape(f.stage) << "\",\n  \"message\":\"" << jsonEscape(f.message)
      << "\",\n  \"metrics\":";
  if (f.baselineUs && f.candidateUs && f.speedup)
    out << "{\"baseline_median_us\":" << *f.baselineUs
        << ",\"candidate_median_us\":" << *f.candidateUs << ",\"speedup\":" << *f.speedup << '}';
  else
    out << "null";
  out << "\n}\n";
  return out ? std::string{} : "Failed while writing generated-kernel feedback '" + path + "'.";
}

std::string writeAdmittedKernel(const hip::HipRuntime& runtime, const std::string& pattern,
                                const AdmittedKernel& kernel, const std::string& path) {
  std::string contract;
  try {
    contract = kernelContractText(runtime, pattern);
  } catch (const std::exception& e) {
    return e.what();
  }
  const std::filesystem::path target(path);
  std::error_code ignored;
  if (target.has_parent_path()) std::filesystem::create_directories(target.parent_path(), ignored);
  // Written beside the target and renamed over it, so a reader never sees a
  // partial artifact.
  const std::string staging = path + ".partial";
  {
    std::ofstream out(staging);
    if (!out) return "Unable to write admitted kernel '" + path + "'.";
    out << "{\"version\":1,\"status\":\"admitted\",\"contract\":" << contract
        << ",\"candidate\":{\"function_name\":\"" << jsonEscape(kernel.functionName)
        << "\",\"source\":\"" << jsonEscape(kernel.source)
        << "\",\"workgroup_size\":" << kernel.workgroupSize << "}}\n";
    if (!out) return "Unable to write admitted kernel '" + path + "'.";
  }
  std::error_code error;
  std::filesystem::rename(staging, target, error);
  return error ? "Unable to write admitted kernel '" + path + "': " + error.message()
               : std::string{};
}

void KernelRegistry::load(const hip::HipRuntime& runtime, const std::string& directory,
                          std::ostream& log) {
  load([&runtime](const std::string& pattern) { return kernelContractText(runtime, pattern); },
       directory, log);
}

void KernelRegistry::load(const std::function<std::string(const std::string&)>& contractText,
                          const std::string& directory, std::ostream& log) {
  entries_.clear();
  usage_.clear();
  namespace fs = std::filesystem;
  if (directory.empty()) {
    log << "[registry] no kernel library: template kernels\n";
    return;
  }
  std::error_code error;
  if (!fs::is_directory(directory, error)) {
    log << "[registry] " << directory << " is not a directory: template kernels\n";
    return;
  }
  std::vector<std::string> patterns;
  for (const auto& entry : fs::directory_iterator(directory, error)) {
    const std::string name = entry.path().filename().string();
    if (entry.is_directory() && name.rfind("decoder_", 0) == 0) patterns.push_back(name);
  }
  std::sort(patterns.begin(), patterns.end());
  for (const auto& pattern : patterns) {
    const auto skip = [&](const std::string& why) {
      log << "[registry] " << pattern << ": " << why << "; template kernel\n";
    };
    std::ifstream in(fs::path(directory) / pattern / "admitted.json");
    if (!in) {
      skip("no admitted.json");
      continue;
    }
    std::stringstream buffer;
    buffer << in.rdbuf();
    const std::string text = buffer.str();
    std::string current;
    try {
      current = contractText(pattern);
    } catch (const std::exception& e) {
      skip(e.what());
      continue;
    }
    std::string version, status, contract, candidate;
    if (!jsonStringField(text, "version", version) || !jsonStringField(text, "status", status) ||
        !jsonStringField(text, "contract", contract) ||
        !jsonStringField(text, "candidate", candidate)) {
      skip("unreadable artifact");
      continue;
    }
    if (version != "1" || status != "admitted" || contract != current) {
      skip("artifact was admitted for another contract or device");
      continue;
    }
    AdmittedKernel kernel;
    std::string expectedFunction, workgroup;
    (void)jsonStringField(current, "function_name", expectedFunction);
    if (!jsonStringField(candidate, "function_name", kernel.functionName) ||
        !jsonStringField(candidate, "source", kernel.source) ||
        !jsonStringField(candidate, "workgroup_size", workgroup) ||
        kernel.functionName != expectedFunction ||
        kernel.source.substr(0, kernel.source.find('?')) != expectedFunction) {
      skip("invalid candidate");
      continue;
    }
    try {
      kernel.workgroupSize = static_cast<std::size_t>(std::stoul(workgroup));
    } catch (const std::exception&) {
      skip("invalid workgroup size");
      continue;
    }
    log << "[registry] " << pattern << ": admitted " << kernel.source << " loaded\n";
    entries_.emplace(pattern, std::move(kernel));
  }
}

const AdmittedKernel* KernelRegistry::find(const std::string& pattern) const {
  const auto it = entries_.find(pattern);
  return it == entries_.end() ? nullptr : &it->second;
}

std::size_t KernelRegistry::track(KernelUsage usage) {
  usage_.push_back(std::move(usage));
  return usage_.size() - 1;
}

void KernelRegistry::completed(const std::vector<std::size_t>& uses) {
  for (const std::size_t index : uses) ++usage_.at(index).completedCalls;
}

void KernelRegistry::resetUsage() noexcept {
  for (auto& use : usage_) use.completedCalls = 0;
}

void KernelRegistry::report(std::ostream& log) const {
  std::size_t generated = 0, templated = 0;
  log << "[registry] region usage:\n";
  for (const auto& use : usage_) {
    const std::size_t dispatches = use.completedCalls * use.dispatchesPerCall;
    (use.implementation == "generated" ? generated : templated) += dispatches;
    log << "[registry]   " << use.node << " (" << use.pattern << "): " << use.implementation
        << " " << use.functions << ", " << use.completedCalls << " calls, " << dispatches
        << " dispatches\n";
  }
  for (const auto& [pattern, kernel] : entries_) {
    const bool ran = std::any_of(usage_.begin(), usage_.end(), [&](const KernelUsage& u) {
      return u.pattern == pattern && u.implementation == "generated" && u.completedCalls > 0;
    });
    log << "[registry]   entry " << pattern << ": " << (ran ? "ran" : "loaded, never ran")
        << '\n';
  }
  log << "[registry] dispatches: generated " << generated << ", template " << templated << '\n';
}

}  // namespace tensor::runtime
