// `.tmc` manifest importers; see Importer.hpp.
#include "Importer.hpp"

#include <filesystem>
#include <fstream>
#include <iomanip>
#include <map>
#include <stdexcept>
#include <utility>

namespace tensor::importer {
namespace {

// Token reader over a manifest; every failure names what was being read and
// which manifest kind ("decoder-only", "KV cache") it belongs to.
class ManifestReader {
 public:
  ManifestReader(std::istream& input, std::string kind) : in_(input), kind_(std::move(kind)) {}

  void keyword(const char* expected) {
    std::string token;
    if (!(in_ >> token) || token != expected)
      throw std::runtime_error(std::string("Expected '") + expected + "' in " + kind_ +
                               " manifest.");
  }
  std::size_t size(const char* what) {
    std::size_t value = 0;
    if (!(in_ >> value)) fail(what);
    return value;
  }
  float real(const char* what) {
    float value = 0.0f;
    if (!(in_ >> value)) fail(what);
    return value;
  }
  std::string quoted(const char* what) {
    std::string value;
    if (!(in_ >> std::quoted(value))) fail(what);
    return value;
  }
  std::string word(const char* what) {
    std::string value;
    if (!(in_ >> value)) fail(what);
    return value;
  }
  bool atEnd() {
    std::string extra;
    return !(in_ >> extra);
  }

 private:
  [[noreturn]] void fail(const char* what) const {
    throw std::runtime_error(std::string("Invalid ") + what + " in " + kind_ + " manifest.");
  }
  std::istream& in_;
  std::string kind_;
};

// The whole float32 payload (the file's size must be a multiple of 4).
std::vector<float> loadPayload(const std::filesystem::path& path, const std::string& kind) {
  std::ifstream file(path, std::ios::binary | std::ios::ate);
  if (!file) throw std::runtime_error("Unable to open " + kind + " payload: " + path.string());
  const std::streamoff bytes = file.tellg();
  if (bytes < 0) throw std::runtime_error("Unable to determine " + kind + " payload size.");
  if (bytes % static_cast<std::streamoff>(sizeof(float)) != 0)
    throw std::runtime_error(kind + " payload is not float32-aligned.");
  std::vector<float> values(static_cast<std::size_t>(bytes) / sizeof(float));
  file.seekg(0);
  if (!values.empty() &&
      !file.read(reinterpret_cast<char*>(values.data()), static_cast<std::streamsize>(bytes)))
    throw std::runtime_error("Unable to read the complete " + kind + " payload.");
  return values;
}

std::filesystem::path besideManifest(const std::string& manifestPath, const std::string& name) {
  return std::filesystem::absolute(std::filesystem::path(manifestPath)).parent_path() / name;
}

struct Span {
  std::size_t offset = 0;
  std::size_t count = 0;
};

// Named float ranges of one payload.
class TensorTable {
 public:
  TensorTable(const std::vector<float>* payload, std::string kind)
      : payload_(payload), kind_(std::move(kind)) {}

  void read(ManifestReader& reader, std::size_t count) {
    for (std::size_t i = 0; i < count; ++i) {
      reader.keyword("TENSOR");
      const auto name = reader.quoted("tensor name");
      Span span;
      span.offset = reader.size("tensor offset");
      span.count = reader.size("tensor length");
      if (!spans_.emplace(name, span).second)
        throw std::runtime_error("Duplicate " + kind_ + " tensor '" + name + "'.");
    }
  }

  // The named tensor, which must hold exactly `expected` floats inside the payload.
  std::vector<float> take(const std::string& name, std::size_t expected) const {
    const auto it = spans_.find(name);
    if (it == spans_.end()) throw std::runtime_error("Missing " + kind_ + " tensor '" + name + "'.");
    if (it->second.count != expected)
      throw std::runtime_error("Invalid " + kind_ + " tensor range for '" + name + "'.");
    return slice(it->second, name);
  }

  std::vector<float> slice(const Span& span, const std::string& name) const {
    const auto& p = *payload_;
    if (span.offset > p.size() || span.count > p.size() - span.offset)
      throw std::runtime_error("Invalid " + kind_ + " tensor range for '" + name + "'.");
    return {p.begin() + static_cast<std::ptrdiff_t>(span.offset),
            p.begin() + static_cast<std::ptrdiff_t>(span.offset + span.count)};
  }

 private:
  const std::vector<float>* payload_;
  std::string kind_;
  std::map<std::string, Span> spans_;
};

std::vector<double> widen(const std::vector<float>& values) {
  return {values.begin(), values.end()};
}

DType dtypeToken(const std::string& token) {
  if (token == "F32") return DType::Float32;
  if (token == "F16") return DType::Float16;
  if (token == "BF16") return DType::BFloat16;
  throw std::runtime_error("Unsupported decoder-only dtype '" + token + "'.");
}

DecoderLLMReference readReference(const TensorTable& table, const std::string& prefix,
                                  const planner::DecoderLLMPlan& plan, std::size_t sequence,
                                  std::size_t cacheLength) {
  const auto& a = plan.attention;
  DecoderLLMReference r;
  r.tokenIds = table.take(prefix + ".tokens", a.batch * sequence);
  r.logits = widen(table.take(prefix + ".logits", a.batch * sequence * plan.vocabularySize));
  r.nextTokenIds = widen(table.take(prefix + ".next_tokens", a.batch));
  const std::size_t cache = a.batch * plan.kvHeads() * cacheLength * a.headDimension;
  for (std::size_t l = 0; l < plan.layerCount; ++l) {
    const auto layer = prefix + ".layer" + std::to_string(l);
    r.keyCaches.push_back(widen(table.take(layer + ".key_cache", cache)));
    r.valueCaches.push_back(widen(table.take(layer + ".value_cache", cache)));
  }
  return r;
}

}  // namespace

DecoderLLMImportResult importDecoderLLMWorkload(const std::string& manifestPath) {
  DecoderLLMImportResult result;
  const std::string kind = "decoder-only";
  try {
    std::ifstream file(manifestPath);
    if (!file) throw std::runtime_error("Unable to open decoder-only manifest: " + manifestPath);
    ManifestReader reader(file, kind);
    std::string magic;
    std::size_t version = 0;
    if (!(file >> magic >> version) || magic != "TMC_DECODER_LLM" || (version != 1 && version != 2))
      throw std::runtime_error("Invalid or unsupported decoder-only manifest header.");

    auto w = std::make_unique<DecoderLLMWorkload>();
    reader.keyword("MODEL");
    w->modelName = reader.quoted("model name");
    reader.keyword("PAYLOAD");
    const auto payloadName = reader.quoted("payload path");
    reader.keyword("CONFIG");
    auto& plan = w->plan;
    plan.attention.batch = reader.size("batch size");
    const std::size_t hidden = reader.size("hidden size");
    plan.attention.heads = reader.size("head count");
    if (plan.attention.heads == 0 || hidden % plan.attention.heads != 0)
      throw std::runtime_error("Decoder hidden size must be divisible by head count.");
    plan.attention.headDimension = hidden / plan.attention.heads;
    plan.intermediateSize = reader.size("intermediate size");
    plan.vocabularySize = reader.size("vocabulary size");
    plan.layerCount = reader.size("layer count");
    plan.attention.capacity = reader.size("cache capacity");
    plan.attention.prefillLength = reader.size("prefill length");
    w->decodeCount = reader.size("decode step count");
    plan.rmsNormEpsilon = reader.real("RMSNorm epsilon");

    // Version-1 manifests may go straight to TENSORS: fp32 storage.
    std::string section = reader.word("tensor section");
    w->requestedStorageDtype = DType::Float32;
    plan.attention.dtype = DType::Float32;
    if (section == "DTYPE") {
      w->requestedStorageDtype = dtypeToken(reader.word("dtype value"));
      plan.attention.dtype = version == 2 ? dtypeToken(reader.word("effective dtype value"))
                                          : w->requestedStorageDtype;
      section = reader.word("tensor section");
    }
    // Threads per threadgroup: 128, doubled until it covers the head
    // dimension (DecoderLLMImporter.cpp:220-224).
    plan.attention.threadsPerThreadgroup = 128;
    while (plan.attention.threadsPerThreadgroup < plan.attention.headDimension &&
           plan.attention.threadsPerThreadgroup < 1024)
      plan.attention.threadsPerThreadgroup *= 2;
    {
      auto check = plan;  // the structural rules; storage is fp16 on gfx950 whatever the manifest says
      check.attention.dtype = DType::Float16;
      check.validate();
    }
    if (w->decodeCount > plan.attention.capacity - plan.attention.prefillLength)
      throw std::runtime_error("Decoder decode steps exceed cache capacity.");
    if (section != "TENSORS") throw std::runtime_error("Expected 'TENSORS' in decoder-only manifest.");

    const std::size_t tensors = reader.size("named tensor count");
    const auto payload = loadPayload(besideManifest(manifestPath, payloadName), kind);
    TensorTable table(&payload, kind);
    table.read(reader, tensors);
    reader.keyword("END");
    if (!reader.atEnd()) throw std::runtime_error("Unexpected data after decoder-only END marker.");

    const std::size_t H = plan.hiddenSize(), I = plan.intermediateSize, V = plan.vocabularySize;
    w->embeddingWeight = table.take("embedding.weight", V * H);
    w->finalNormWeight = table.take("final_norm.weight", H);
    w->languageModelHeadWeight = table.take("lm_head.weight", V * H);
    const std::size_t rope = plan.attention.capacity * plan.attention.headDimension / 2;
    w->ropeCosine = table.take("rope.cosine", rope);
    w->ropeSine = table.take("rope.sine", rope);
    const std::size_t kv = plan.kvWidth() * H;
    for (std::size_t l = 0; l < plan.layerCount; ++l) {
      const auto p = "layer" + std::to_string(l) + ".";
      DecoderLLMLayerParameters layer;
      layer.inputNormWeight = table.take(p + "input_norm.weight", H);
      layer.queryWeight = table.take(p + "q.weight", H * H);
      layer.keyWeight = table.take(p + "k.weight", kv);
      layer.valueWeight = table.take(p + "v.weight", kv);
      layer.outputWeight = table.take(p + "o.weight", H * H);
      layer.postAttentionNormWeight = table.take(p + "post_norm.weight", H);
      layer.gateWeight = table.take(p + "gate.weight", I * H);
      layer.upWeight = table.take(p + "up.weight", I * H);
      layer.downWeight = table.take(p + "down.weight", H * I);
      w->layers.push_back(std::move(layer));
    }
    const std::size_t P = plan.attention.prefillLength;
    w->prefill = readReference(table, "prefill", plan, P, P);
    for (std::size_t s = 0; s < w->decodeCount; ++s)
      w->decodeSteps.push_back(readReference(table, "decode" + std::to_string(s), plan, 1, P + s + 1));
    result.workload = std::move(w);
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

KVCacheImportResult importKVCacheWorkload(const std::string& manifestPath) {
  KVCacheImportResult result;
  const std::string kind = "KV cache";
  try {
    std::ifstream file(manifestPath);
    if (!file) throw std::runtime_error("Unable to open KV cache manifest: " + manifestPath);
    ManifestReader reader(file, kind);
    std::string magic;
    std::size_t version = 0;
    if (!(file >> magic >> version) || magic != "TMC_KV_CACHE" || version != 1)
      throw std::runtime_error("Invalid or unsupported KV cache manifest header.");

    auto w = std::make_unique<ImportedKVCacheWorkload>();
    reader.keyword("MODEL");
    w->modelName = reader.quoted("model name");
    reader.keyword("PAYLOAD");
    const auto payload = loadPayload(besideManifest(manifestPath, reader.quoted("payload path")), kind);
    reader.keyword("CONFIG");
    auto& plan = w->plan;
    plan.batch = reader.size("batch");
    plan.heads = reader.size("head count");
    plan.headDimension = reader.size("head dimension");
    plan.capacity = reader.size("cache capacity");
    plan.prefillLength = reader.size("prefill length");
    const std::size_t decodeCount = reader.size("decode step count");
    plan.dtype = DType::Float32;
    plan.threadsPerThreadgroup = 128;
    plan.validate();
    if (decodeCount > plan.capacity - plan.prefillLength)
      throw std::runtime_error("Decode steps exceed the configured cache capacity.");

    reader.keyword("TENSORS");
    TensorTable table(&payload, kind);
    table.read(reader, reader.size("named tensor count"));
    const std::size_t D = plan.modelDimension();
    const std::size_t prefillCount = plan.inputElementCount(plan.prefillLength);
    w->queryWeight = table.take("query_weight", D * D);
    w->keyWeight = table.take("key_weight", D * D);
    w->valueWeight = table.take("value_weight", D * D);
    w->outputWeight = table.take("output_weight", D * D);
    w->prefill.query = table.take("prefill_query", prefillCount);
    w->prefill.key = table.take("prefill_key", prefillCount);
    w->prefill.value = table.take("prefill_value", prefillCount);
    w->prefill.output = widen(table.take("prefill_output", prefillCount));
    w->prefill.keyCache = widen(table.take("prefill_key_cache", prefillCount));
    w->prefill.valueCache = widen(table.take("prefill_value_cache", prefillCount));

    reader.keyword("STEPS");
    if (reader.size("declared decode step count") != decodeCount)
      throw std::runtime_error("KV cache CONFIG and STEPS counts disagree.");
    const std::size_t stepInput = plan.inputElementCount(1);
    for (std::size_t s = 0; s < decodeCount; ++s) {
      reader.keyword("STEP");
      if (reader.size("decode step index") != s)
        throw std::runtime_error("KV cache decode steps are out of order.");
      auto next = [&]() {
        Span span;
        span.offset = reader.size("step tensor offset");
        span.count = reader.size("step tensor length");
        return table.slice(span, "STEP " + std::to_string(s));
      };
      KVCacheReferenceStep step;
      step.query = next();
      step.key = next();
      step.value = next();
      step.output = widen(next());
      step.keyCache = widen(next());
      step.valueCache = widen(next());
      const std::size_t cache = plan.batch * plan.heads * (plan.prefillLength + s + 1) *
                                plan.headDimension;
      if (step.query.size() != stepInput || step.key.size() != stepInput ||
          step.value.size() != stepInput || step.output.size() != stepInput ||
          step.keyCache.size() != cache || step.valueCache.size() != cache)
        throw std::runtime_error("KV cache decode step tensor shape is inconsistent with CONFIG.");
      w->decodeSteps.push_back(std::move(step));
    }
    reader.keyword("END");
    if (!reader.atEnd()) throw std::runtime_error("Unexpected data after KV cache END marker.");
    result.workload = std::move(w);
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

}  // namespace tensor::importer
