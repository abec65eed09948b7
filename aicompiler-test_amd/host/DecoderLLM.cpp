// Decoder-LLM decode path on gfx950; see DecoderLLM.hpp.
#include "DecoderLLM.hpp"

#include "Tuning.hpp"
#include "tmc_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <mutex>
#include <ostream>
#include <sstream>
#include <stdexcept>
#include <utility>

namespace tensor {

// ---------------------------------------------------------------------- plan
namespace planner {

std::size_t DecoderLLMPlan::hiddenSize() const { return attention.modelDimension(); }

std::size_t DecoderLLMPlan::hiddenElementCount(std::size_t sequenceLength) const {
  return attention.inputElementCount(sequenceLength);
}

std::size_t DecoderLLMPlan::intermediateElementCount(std::size_t sequenceLength) const {
  return attention.batch * sequenceLength * intermediateSize;
}

std::size_t DecoderLLMPlan::logitsElementCount(std::size_t sequenceLength) const {
  return attention.batch * sequenceLength * vocabularySize;
}

void DecoderLLMPlan::validate() const {
  attention.validate();
  if (layerCount == 0 || intermediateSize == 0 || vocabularySize == 0)
    throw std::invalid_argument("Decoder-only dimensions must be nonzero.");
  if (attention.headDimension % 2 != 0)
    throw std::invalid_argument("Decoder-only RoPE requires an even head dimension.");
  if (!std::isfinite(rmsNormEpsilon) || rmsNormEpsilon <= 0.0f)
    throw std::invalid_argument("Decoder-only RMSNorm epsilon must be positive.");
  if (accumulationDtype != DType::Float32)
    throw std::invalid_argument("Decoder-only reductions currently require fp32 accumulation.");
  if (attention.heads % kvHeads() != 0)
    throw std::invalid_argument("Query heads must be a multiple of the key/value heads.");
  if (attention.dtype != DType::Float16)
    throw std::invalid_argument("The gfx950 decoder path stores activations and weights in fp16.");
  if (vocabularySize > static_cast<std::size_t>(std::numeric_limits<std::int32_t>::max()))
    throw std::invalid_argument("Vocabulary exceeds int32 token ids.");
}

KVCachePlan DecoderLLMPlan::kvPlan() const {
  KVCachePlan plan = attention;
  plan.batch = 1;
  plan.heads = kvHeads();
  plan.prefillLength = 1;
  return plan;
}

}  // namespace planner

void ropeTables(std::size_t capacity, std::size_t headDimension, double theta,
                std::vector<float>& cosine, std::vector<float>& sine) {
  const std::size_t pairs = headDimension / 2;
  cosine.assign(capacity * pairs, 0.0f);
  sine.assign(capacity * pairs, 0.0f);
  for (std::size_t i = 0; i < pairs; ++i) {
    const double frequency =
        std::exp(static_cast<double>(2 * i) * (-std::log(theta) / static_cast<double>(headDimension)));
    for (std::size_t position = 0; position < capacity; ++position) {
      const double angle = static_cast<double>(position) * frequency;
      cosine[position * pairs + i] = static_cast<float>(std::cos(angle));
      sine[position * pairs + i] = static_cast<float>(std::sin(angle));
    }
  }
}

namespace runtime {
namespace {

// Bring the device copy of a packed [layer][rows][pages] block-table array
// from `shadow` to `packed`.  A decode step usually changes one entry per
// layer for each request that entered a new page, spread across the whole
// array: those go as (index, value) pairs applied by a kernel (about 6 us on
// MI355X), where the one changed span would be a DMA copy of up to the whole
// array (512 KiB at batch 16 of a 7B model: about 80 us between two step
// graphs).  A short span, or many changes, goes as one copy.
std::string writeTableChanges(const hip::HipBuffer& tables, const std::vector<std::int32_t>& packed,
                              const std::vector<std::int32_t>& shadow) {
  constexpr std::size_t kDenseSpan = 4096;      // entries (16 KiB): copied whole
  constexpr std::size_t kSparsePairs = 16384;  // changed entries sent as pairs at most
  std::size_t first = 0, last = packed.size();
  while (first < last && packed[first] == shadow[first]) ++first;
  while (last > first && packed[last - 1] == shadow[last - 1]) --last;
  if (first == last) return {};
  if (last - first > kDenseSpan) {
    std::vector<std::int32_t> pairs;
    for (std::size_t i = first; i < last; ++i) {
      if (packed[i] == shadow[i]) continue;
      if (pairs.size() == 2 * kSparsePairs) break;
      pairs.push_back(static_cast<std::int32_t>(i));
      pairs.push_back(packed[i]);
    }
    if (pairs.size() < 2 * kSparsePairs || pairs[pairs.size() - 2] == static_cast<std::int32_t>(last - 1))
      return tables.writeSparseAsync(pairs);
  }
  return tables.writeRawAsync(packed.data() + first, last - first, first);
}

using hip::BufferHandle;
using hip::ElementType;

BufferHandle allocate(hip::HipRuntime& runtime, std::size_t count, const float* data,
                      ElementType type) {
  auto result = runtime.createBuffer(count, data, type);
  if (!result.buffer) throw std::runtime_error(result.errorMessage);
  return std::move(result.buffer);
}

BufferHandle view(hip::HipRuntime& runtime, const BufferHandle& base, std::size_t offset,
                  std::size_t count) {
  auto* bytes = static_cast<unsigned char*>(base->devicePointer()) +
                offset * hip::elementBytes(base->elementType());
  auto result = runtime.wrapBuffer(bytes, count, base->elementType());
  if (!result.buffer) throw std::runtime_error(result.errorMessage);
  return std::move(result.buffer);
}

void requireCount(const std::string& name, const std::vector<float>& values, std::size_t expected) {
  if (values.size() != expected)
    throw std::invalid_argument(name + " has " + std::to_string(values.size()) +
                                " elements; expected " + std::to_string(expected) + ".");
}

// validateWeights (DecoderLLMExecutor.cpp:169-204) with GQA key/value shapes.
void validateWeights(const DecoderLLMWorkload& workload) {
  const auto& plan = workload.plan;
  const std::size_t H = plan.hiddenSize(), KV = plan.kvWidth();
  if (workload.layers.size() != plan.layerCount)
    throw std::invalid_argument("Decoder workload layer count differs from the plan.");
  requireCount("embedding.weight", workload.embeddingWeight, plan.vocabularySize * H);
  requireCount("final_norm.weight", workload.finalNormWeight, H);
  requireCount("lm_head.weight", workload.languageModelHeadWeight, plan.vocabularySize * H);
  const std::size_t rope = plan.attention.capacity * plan.attention.headDimension / 2;
  requireCount("rope.cosine", workload.ropeCosine, rope);
  requireCount("rope.sine", workload.ropeSine, rope);
  for (std::size_t l = 0; l < workload.layers.size(); ++l) {
    const auto& layer = workload.layers[l];
    const std::string prefix = "layer" + std::to_string(l) + ".";
    requireCount(prefix + "input_norm.weight", layer.inputNormWeight, H);
    requireCount(prefix + "q.weight", layer.queryWeight, H * H);
    requireCount(prefix + "k.weight", layer.keyWeight, KV * H);
    requireCount(prefix + "v.weight", layer.valueWeight, KV * H);
    requireCount(prefix + "o.weight", layer.outputWeight, H * H);
    requireCount(prefix + "post_norm.weight", layer.postAttentionNormWeight, H);
    requireCount(prefix + "gate.weight", layer.gateWeight, plan.intermediateSize * H);
    requireCount(prefix + "up.weight", layer.upWeight, plan.intermediateSize * H);
    requireCount(prefix + "down.weight", layer.downWeight, H * plan.intermediateSize);
  }
}

void describe(DecoderLLMModelResources& r, const planner::DecoderLLMPlan& plan) {
  r.storageDtype = DType::Float16;
  r.plan = plan;
  r.hiddenSize = plan.hiddenSize();
  r.headCount = plan.attention.heads;
  r.kvHeadCount = plan.kvHeads();
  r.headDimension = plan.attention.headDimension;
  r.cacheCapacity = plan.attention.capacity;
  r.intermediateSize = plan.intermediateSize;
  r.vocabularySize = plan.vocabularySize;
  r.layerCount = plan.layerCount;
}

std::string fmt(double value) {
  std::ostringstream out;
  out.precision(9);
  out << value;
  return out.str();
}

}  // namespace

// ------------------------------------------------------------ model resources
ModelResourcesCreation createModelResources(hip::HipRuntime& runtime,
                                            const DecoderLLMWorkload& workload) {
  ModelResourcesCreation result;
  try {
    // weights are stored in fp16 whatever storage the workload's plan names
    // (an fp32 or bf16 manifest's host floats are rounded on upload)
    auto plan = workload.plan;
    plan.attention.dtype = DType::Float16;
    plan.validate();
    validateWeights(workload);
    auto r = std::make_shared<DecoderLLMModelResources>();
    describe(*r, plan);
    auto upload = [&](const std::vector<float>& values) {
      r->storageBytes += values.size() * 2;
      return allocate(runtime, values.size(), values.data(), ElementType::Float16);
    };
    r->embeddingWeight = upload(workload.embeddingWeight);
    r->finalNormWeight = upload(workload.finalNormWeight);
    r->languageModelHeadWeight = upload(workload.languageModelHeadWeight);
    r->ropeCosine = allocate(runtime, workload.ropeCosine.size(), workload.ropeCosine.data(),
                             ElementType::Float32);
    r->ropeSine = allocate(runtime, workload.ropeSine.size(), workload.ropeSine.data(),
                           ElementType::Float32);
    r->storageBytes += (workload.ropeCosine.size() + workload.ropeSine.size()) * 4;
    for (const auto& layer : workload.layers) {
      DecoderLLMModelLayerBuffers b;
      b.inputNormWeight = upload(layer.inputNormWeight);
      std::vector<float> qkv;
      qkv.reserve(layer.queryWeight.size() + 2 * layer.keyWeight.size());
      qkv.insert(qkv.end(), layer.queryWeight.begin(), layer.queryWeight.end());
      qkv.insert(qkv.end(), layer.keyWeight.begin(), layer.keyWeight.end());
      qkv.insert(qkv.end(), layer.valueWeight.begin(), layer.valueWeight.end());
      b.queryKeyValueWeight = upload(qkv);
      b.outputWeight = upload(layer.outputWeight);
      b.postAttentionNormWeight = upload(layer.postAttentionNormWeight);
      b.gateWeight = upload(layer.gateWeight);
      b.upWeight = upload(layer.upWeight);
      b.downWeight = upload(layer.downWeight);
      r->layers.push_back(std::move(b));
    }
    result.resources = std::move(r);
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

ModelResourcesCreation createSyntheticModelResources(hip::HipRuntime& runtime,
                                                     const planner::DecoderLLMPlan& plan,
                                                     std::uint64_t seed, float stddev,
                                                     double theta) {
  ModelResourcesCreation result;
  try {
    plan.validate();
    auto r = std::make_shared<DecoderLLMModelResources>();
    describe(*r, plan);
    const std::size_t H = plan.hiddenSize(), I = plan.intermediateSize, V = plan.vocabularySize;
    const std::size_t QKV = H + 2 * plan.kvWidth();
    std::uint64_t tensor = 0;
    auto random = [&](std::size_t count) {
      auto buffer = allocate(runtime, count, nullptr, ElementType::Float16);
      const auto error = runtime.fillNormal(buffer, seed + tensor++, 0.0f, stddev);
      if (!error.empty()) throw std::runtime_error(error);
      r->storageBytes += count * 2;
      return buffer;
    };
    const std::vector<float> ones(H, 1.0f);
    auto norm = [&]() {
      r->storageBytes += H * 2;
      return allocate(runtime, H, ones.data(), ElementType::Float16);
    };
    r->embeddingWeight = random(V * H);
    for (std::size_t l = 0; l < plan.layerCount; ++l) {
      DecoderLLMModelLayerBuffers b;
      b.inputNormWeight = norm();
      b.queryKeyValueWeight = random(QKV * H);
      b.outputWeight = random(H * H);
      b.postAttentionNormWeight = norm();
      b.gateWeight = random(I * H);
      b.upWeight = random(I * H);
      b.downWeight = random(H * I);
      r->layers.push_back(std::move(b));
    }
    r->finalNormWeight = norm();
    r->languageModelHeadWeight = random(V * H);
    std::vector<float> cosine, sine;
    ropeTables(plan.attention.capacity, plan.attention.headDimension, theta, cosine, sine);
    r->ropeCosine = allocate(runtime, cosine.size(), cosine.data(), ElementType::Float32);
    r->ropeSine = allocate(runtime, sine.size(), sine.data(), ElementType::Float32);
    r->storageBytes += (cosine.size() + sine.size()) * 4;
    const auto error = runtime.synchronize();
    if (!error.empty()) throw std::runtime_error(error);
    result.resources = std::move(r);
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

std::string ensurePackedWeights(hip::HipRuntime& runtime, DecoderLLMModelResources& model,
                                bool normScaled) {
  if (model.layers.empty()) return {};
  try {
    const auto& plan = model.plan;
    const std::size_t H = plan.hiddenSize(), I = plan.intermediateSize, V = plan.vocabularySize;
    const std::size_t QKV = H + 2 * plan.kvWidth();
    std::size_t bytes = 0;
    bool made = false;
    // fills `slot` once: W packed, with gamma folded in when given
    auto pack = [&](BufferHandle& slot, const BufferHandle& w, const BufferHandle* gamma,
                    std::size_t out, std::size_t in) {
      if (slot) return;
      const auto count = tmc_packed_weight_elements(static_cast<int64_t>(out),
                                                    static_cast<int64_t>(in));
      if (count <= 0) throw std::runtime_error("Packed weights: invalid matrix shape.");
      auto packed = allocate(runtime, static_cast<std::size_t>(count), nullptr,
                             ElementType::Float16);
      if (tmc_pack_weights_scaled_f16(w->devicePointer(),
                                      gamma ? (*gamma)->devicePointer() : nullptr,
                                      packed->devicePointer(), static_cast<int64_t>(out),
                                      static_cast<int64_t>(in), runtime.stream()) != 0)
        throw std::runtime_error(std::string("Packed weights: ") + tmc_last_error());
      bytes += static_cast<std::size_t>(count) * 2;
      slot = std::move(packed);
      made = true;
    };
    const std::size_t L = model.layers.size();
    auto packedLayers = model.packedLayers;
    auto scaledLayers = model.normScaledLayers;
    packedLayers.resize(L);
    if (normScaled) scaledLayers.resize(L);
    auto head = model.packedLanguageModelHead;
    auto scaledHead = model.normScaledLanguageModelHead;
    for (std::size_t l = 0; l < L; ++l) {
      const auto& w = model.layers[l];
      auto& b = packedLayers[l];
      pack(b.outputWeight, w.outputWeight, nullptr, H, H);
      pack(b.downWeight, w.downWeight, nullptr, H, I);
      if (normScaled) {
        auto& c = scaledLayers[l];
        pack(c.queryKeyValueWeight, w.queryKeyValueWeight, &w.inputNormWeight, QKV, H);
        pack(c.gateWeight, w.gateWeight, &w.postAttentionNormWeight, I, H);
        pack(c.upWeight, w.upWeight, &w.postAttentionNormWeight, I, H);
      } else {
        pack(b.queryKeyValueWeight, w.queryKeyValueWeight, nullptr, QKV, H);
        pack(b.gateWeight, w.gateWeight, nullptr, I, H);
        pack(b.upWeight, w.upWeight, nullptr, I, H);
      }
    }
    if (normScaled)
      pack(scaledHead, model.languageModelHeadWeight, &model.finalNormWeight, V, H);
    else
      pack(head, model.languageModelHeadWeight, nullptr, V, H);
    if (!made) return {};
    const auto error = runtime.synchronize();
    if (!error.empty()) throw std::runtime_error(error);
    model.packedLayers = std::move(packedLayers);
    model.normScaledLayers = std::move(scaledLayers);
    model.packedLanguageModelHead = std::move(head);
    model.normScaledLanguageModelHead = std::move(scaledHead);
    model.packedBytes += bytes;
  } catch (const std::exception& e) {
    return e.what();
  }
  return {};
}

// ------------------------------------------------------ BatchedDecodeExecutor
struct BatchedDecodeExecutor::Bucket {
  std::size_t rows = 0;
  std::vector<std::unique_ptr<hip::PreparedExecution>> steps;
  std::unique_ptr<hip::PreparedSequence> sequence;
  std::vector<std::size_t> uses;  // registry usage entries of this bucket
  // Token-only tail (partial + final argmax) and the sequence of the trunk
  // steps followed by it; null when the bucket has none.
  std::vector<std::unique_ptr<hip::PreparedExecution>> tokenSteps;
  std::unique_ptr<hip::PreparedSequence> tokenSequence;
  bool tokenChecked = false, tokenAdmitted = false;
  double tokenSpeedup = 0.0;
};

BatchedDecodeExecutor::~BatchedDecodeExecutor() = default;

std::vector<std::size_t> BatchedDecodeExecutor::buckets() const {
  std::vector<std::size_t> rows;
  for (const auto& b : buckets_) rows.push_back(b->rows);
  return rows;
}

std::size_t BatchedDecodeExecutor::dispatchesPerStep(std::size_t bucket) const {
  for (const auto& b : buckets_)
    if (b->rows == bucket) return b->steps.size();
  return 0;
}

void BatchedDecodeExecutor::build(std::ostream* log) {
  auto& rt = *runtime_;
  const auto& plan = model_->plan;
  const std::size_t M = maximumBatchSize_, L = plan.layerCount;
  const std::size_t H = plan.hiddenSize(), I = plan.intermediateSize, V = plan.vocabularySize;
  const std::size_t QH = plan.attention.heads, KVH = plan.kvHeads(), D = plan.attention.headDimension;
  const std::size_t QKV = H + 2 * plan.kvWidth();
  const std::size_t capacity = plan.attention.capacity;
  maxPages_ = (capacity + pageSize_ - 1) / pageSize_;

  // Metadata and block tables: one buffer each, per-layer views into the tables.
  std::vector<float> zeros(2 * M + 1, 0.0f);
  meta_ = allocate(rt, 2 * M + 1, zeros.data(), ElementType::Int32);
  tokensView_ = view(rt, meta_, 0, M);
  lengthsView_ = view(rt, meta_, M, M);
  activeView_ = view(rt, meta_, 2 * M, 1);
  const std::vector<float> none(L * M * maxPages_, -1.0f);
  tables_ = allocate(rt, none.size(), none.data(), ElementType::Int32);
  for (std::size_t l = 0; l < L; ++l)
    tableViews_.push_back(view(rt, tables_, l * M * maxPages_, M * maxPages_));
  metaShadow_.assign(2 * M + 1, 0);
  tableShadow_.assign(L * M * maxPages_, -1);

  auto act = [&](std::size_t count, ElementType type = ElementType::Float16) {
    activationBytes_ += count * hip::elementBytes(type);
    return allocate(rt, count, nullptr, type);
  };
  // normalized_ and gated_ (and, with the norms folded, residual_, after_
  // and context_) also hold the fragment-ordered activations of the batch > 1
  // buckets: whole 16-row passes.
  const std::size_t passRows = (M + 15) / 16 * 16;
  residual_ = act(std::max(M * H, passRows * ((H + 31) / 32 * 32)));
  after_ = act(std::max(M * H, passRows * ((H + 31) / 32 * 32)));
  normalized_ = act(std::max(M * H, passRows * ((H + 31) / 32 * 32)));
  qkv_ = act(M * QKV);
  query_ = act(M * H);
  context_ = act(std::max(M * H, passRows * ((H + 31) / 32 * 32)));
  projected_ = act(M * H);
  gated_ = act(std::max(M * I, passRows * ((I + 31) / 32 * 32)));
  mlp_ = act(M * H);
  logits_ = act(M * V, ElementType::Float32);
  nextTokens_ = act(M, ElementType::Int32);
  argmaxWorkspace_ = act(tmc_lm_head_argmax_workspace_bytes(static_cast<int64_t>(M),
                                                            static_cast<int64_t>(V)) / 4,
                         ElementType::Float32);

  std::vector<std::size_t> rows;
  for (std::size_t r = 1; r < M; r *= 2) rows.push_back(r);
  rows.push_back(M);
  if (M > 1) {
    // the batch > 1 buckets fold the norms under the same condition as the
    // bucket build below (foldPacked)
    const bool fuseRopeAll = H % 8 == 0 && D % 2 == 0;
    const bool scaled = foldNorms_ && fuseRopeAll && H % 32 == 0;
    const auto error = ensurePackedWeights(rt, *model_, scaled);
    if (!error.empty()) throw std::runtime_error(error);
  }

  // Tuned batch-1 GEMV configurations per shape (on finite scratch inputs and
  // layer 0's weights; a shape with no admitted candidate keeps its default).
  std::map<std::string, std::string> tunedSuffix;
  if (tuneKernels_) {
    std::ostringstream tuneLog;
    std::uint64_t seed = 9001;
    for (const auto& buffer : {normalized_, context_, gated_}) {
      const auto error = rt.fillNormal(buffer, seed++, 0.0f, 1.0f);
      if (!error.empty()) throw std::runtime_error(error);
    }
    const auto& w0 = model_->layers.front();
    struct Shape { std::size_t in, out; BufferHandle x, w; ElementType type; };
    const Shape shapes[] = {{H, QKV, normalized_, w0.queryKeyValueWeight, ElementType::Float16},
                            {H, H, context_, w0.outputWeight, ElementType::Float16},
                            {I, H, gated_, w0.downWeight, ElementType::Float16},
                            {H, V, normalized_, model_->languageModelHeadWeight,
                             ElementType::Float32}};
    for (const auto& shape : shapes) {
      const auto selection = planner::cachedDecodeGEMV(rt, 1, shape.in, shape.out, shape.x,
                                                       shape.w, tuneLog, shape.type);
      if (!selection.success) throw std::runtime_error("GEMV tuning: " + selection.errorMessage);
      if (selection.useBaseline) continue;
      const auto& c = selection.config;
      tunedSuffix[std::to_string(shape.in) + "x" + std::to_string(shape.out)] =
          "&algorithm=" + std::to_string(c.algorithm) + "&rows_per_wave=" +
          std::to_string(c.rowsPerWave) + "&unroll=" + std::to_string(c.unroll) +
          "&k_split=" + std::to_string(c.kSplit);
    }
    if (log) *log << tuneLog.str();
  }

  const std::string eps = fmt(plan.rmsNormEpsilon);
  for (const std::size_t m : rows) {
    auto bucket = std::make_unique<Bucket>();
    bucket->rows = m;
    const std::string B = std::to_string(m);
    auto add = [&](const std::string& key, const std::string& name,
                   const std::vector<BufferHandle>& inputs,
                   const std::vector<BufferHandle>& outputs) {
      const auto pipeline = rt.createComputePipeline(key, name);
      if (!pipeline.pipelineCreationPassed)
        throw std::runtime_error(name + ": " + pipeline.errorMessage);
      auto prepared = rt.prepareBuffers(
          inputs, outputs, {pipeline.threadgroupCount, pipeline.threadsPerThreadgroup});
      if (!prepared.execution) throw std::runtime_error(name + ": " + prepared.errorMessage);
      bucket->steps.push_back(std::move(prepared.execution));
    };
    // Batch 1 streams row-major weights with the dot GEMV; larger buckets run
    // the MFMA GEMM over the fragment-packed copies.
    // Above batch 1 the norms write the normalized rows, and the gated MLP
    // its output, in the GEMM's activation fragment order (x_layout=packed
    // for q.k.v, gate/up, down and the LM head; o reads the attention output
    // row-major).
    const bool packed = m > 1;
    auto gemv = [&](std::size_t in, std::size_t out, const char* outType, bool xPacked = true) {
      std::string tuned;
      if (!packed) {
        const auto it = tunedSuffix.find(std::to_string(in) + "x" + std::to_string(out));
        if (it != tunedSuffix.end()) tuned = it->second;
      }
      return std::string(packed ? "gemm_packed" : "decode_gemv") + "?batch=" + B +
             "&in=" + std::to_string(in) + "&out=" + std::to_string(out) + "&out_dtype=" + outType +
             (packed && xPacked ? "&x_layout=packed" : "") + tuned;
    };
    auto weights = [&](std::size_t l) -> const DecoderLLMModelLayerBuffers& {
      return packed ? model_->packedLayers[l] : model_->layers[l];
    };
    // Batch 1: 512 threads per row (one 16-byte chunk each at H = 4096) cut
    // the latency-bound norm by ~0.5 us after a GEMV against 256 (measured).
    const std::string normShape =
        "rows=" + B + "&width=" + std::to_string(H) + "&eps=" + eps + "&dtype=f16";
    // An admitted region kernel replaces the template's launch parameters
    // where its contract shape (one row of width 4096, row-major output)
    // matches; its threads / variant apply to every launch of the region.
    const auto regionKernel = [&](const char* pattern) -> std::string {
      const AdmittedKernel* entry = registry_ ? registry_->find(pattern) : nullptr;
      if (!entry || packed || m != 1 || H != 4096) return {};
      std::string tuning;
      std::stringstream items(entry->source.substr(std::min(entry->source.size(),
                                                            entry->source.find('?') + 1)));
      for (std::string item; std::getline(items, item, '&');) {
        const std::string field = item.substr(0, item.find('='));
        if (field == "threads" || field == "variant") tuning += "&" + item;
      }
      if (tuning.find("threads=") == std::string::npos)
        tuning += "&threads=" + std::to_string(entry->workgroupSize);
      return tuning;
    };
    const std::string generatedNorm = regionKernel("decoder_rmsnorm");
    const std::string generatedAddNorm = regionKernel("decoder_residual_rmsnorm");
    const std::string templateTuning =
        packed ? "&out_layout=packed" : H >= 4096 ? "&threads=512" : "";
    const std::string firstNorm =
        normShape + (generatedNorm.empty() ? templateTuning : generatedNorm);
    const std::string norm =
        normShape + (generatedAddNorm.empty() ? templateTuning : generatedAddNorm);
    const bool fuseRope = H % 8 == 0 && D % 2 == 0;
    // Batch 1 without admitted norm kernels: fold every norm into the
    // neighbouring GEMVs when the template norm holds one 16-byte chunk per
    // thread (512 threads at hidden 4096, 256 up to 2048), whose summation
    // order the GEMV prologue follows, so the step's results do not change.
    const std::size_t normThreads = H >= 4096 ? 512 : 256;
    const bool fold = foldNorms_ && !packed && fuseRope && generatedNorm.empty() &&
                      generatedAddNorm.empty() && H % 8 == 0 && H / 8 <= normThreads;
    // Batch > 1: the packed projections fold the norms too (q.k.v + RoPE,
    // gate/up and the LM head scale by the row's 1/rms; o and down add the
    // residual), with the residual stream in fragment order.  Not bit for
    // bit: the fp16 rounding falls on gamma * s rather than on the
    // normalized value (within the fp16 path tolerance).
    const bool foldPacked = foldNorms_ && packed && fuseRope && H % 32 == 0;
    // Paged attention + o projection + residual as one launch (opt-in; the
    // kernel's limits: head_dim 128, GQA group 1 or 2, pages of a multiple
    // of 16 positions, capacity <= 1024, pools below 4 GiB, an output width
    // its row slices divide).
    const std::string attentionOutputKey =
        "paged_attention_output?q_heads=" + std::to_string(QH) + "&kv_heads=" +
        std::to_string(KVH) + "&head_dim=" + std::to_string(D) + "&page_size=" +
        std::to_string(pageSize_) + "&max_pages=" + std::to_string(maxPages_) +
        "&out=" + std::to_string(H) + "&residual=1";
    bool fuseAttention = fold && fuseAttentionOutput_ && D == 128 && KVH > 0 && QH % KVH == 0 &&
                         QH / KVH <= 2 && pageSize_ % 16 == 0 && pageSize_ * maxPages_ <= 1024;
    for (std::size_t l = 0; fuseAttention && l < L; ++l)
      fuseAttention = pools_[l]->keyBuffer()->elementCount() * 2 < (std::size_t(1) << 32) - 16 &&
                      pools_[l]->valueBuffer()->elementCount() * 2 < (std::size_t(1) << 32) - 16;
    if (fuseAttention)
      fuseAttention = rt.createComputePipeline(attentionOutputKey, "attention_output_probe")
                          .pipelineCreationPassed;
    if (registry_) {
      const bool folded = fold || foldPacked;
      const auto track = [&](const char* node, const char* pattern, const std::string& tuning,
                             const std::string& key, std::size_t launches) {
        const char* implementation = folded ? "folded" : tuning.empty() ? "template" : "generated";
        bucket->uses.push_back(registry_->track(
            {"bucket " + B + " " + node, pattern, implementation, key, folded ? 0 : launches, 0}));
      };
      track("input norm", "decoder_rmsnorm", generatedNorm,
            fold ? "rmsnorm_qkv_rope_append" : "rmsnorm?" + firstNorm, 1);
      track("residual norms", "decoder_residual_rmsnorm", generatedAddNorm,
            fold ? "gemv_residual + rmsnorm_* prologues" : "add_rmsnorm?" + norm, 2 * L);
      if (fuseAttention)
        bucket->uses.push_back(registry_->track({"bucket " + B + " attention output",
                                                 "paged_attention_output_projection", "template",
                                                 attentionOutputKey, L, 0}));
    }
    const std::string embeddingKey =
        "embedding?rows=" + B + "&hidden=" + std::to_string(H) + "&vocab=" + std::to_string(V);
    if (foldPacked) {
      // the residual stream in fragment order from the start
      add(embeddingKey, "embedding", {tokensView_, model_->embeddingWeight}, {projected_});
      add("pack_activations?rows=" + B + "&cols=" + std::to_string(H), "embedding_pack",
          {projected_}, {residual_});
    } else {
      add(embeddingKey, "embedding", {tokensView_, model_->embeddingWeight}, {residual_});
    }
    if (!fold && !foldPacked)
      add("rmsnorm?" + firstNorm, "l0_input_norm", {residual_, model_->layers[0].inputNormWeight},
          {normalized_});
    const std::string ropeKey = "decode_rope_append?max_batch=" + B + "&q_heads=" + std::to_string(QH) +
                                "&kv_heads=" + std::to_string(KVH) + "&head_dim=" + std::to_string(D) +
                                "&capacity=" + std::to_string(capacity) +
                                "&page_size=" + std::to_string(pageSize_);
    const std::string ropeShape = "hidden=" + std::to_string(H) + "&q_heads=" + std::to_string(QH) +
                                  "&kv_heads=" + std::to_string(KVH) +
                                  "&head_dim=" + std::to_string(D) +
                                  "&capacity=" + std::to_string(capacity) +
                                  "&page_size=" + std::to_string(pageSize_);
    const std::string qkvRopeKey = packed ? "qkv_rope_append_packed?batch=" + B + "&" + ropeShape +
                                                "&x_layout=packed"
                                          : "qkv_rope_append?" + ropeShape;
    const std::string attentionKey =
        "paged_attention?max_batch=" + B + "&q_heads=" + std::to_string(QH) +
        "&kv_heads=" + std::to_string(KVH) + "&head_dim=" + std::to_string(D) +
        "&page_size=" + std::to_string(pageSize_) + "&max_pages=" + std::to_string(maxPages_);
    if (fold) {
      // residual_ -> [norm prologue] q.k.v + RoPE + append -> attention ->
      // o + residual -> after_ -> [norm prologue] gate/up -> down + residual
      // -> residual_; the LM head normalizes the last residual_.
      const std::string normKey = "&eps=" + eps;
      auto residualGemv = [&](std::size_t in, std::size_t out) {
        std::string key = "gemv_residual?in=" + std::to_string(in) + "&out=" + std::to_string(out);
        const auto it = tunedSuffix.find(std::to_string(in) + "x" + std::to_string(out));
        return it != tunedSuffix.end() ? key + it->second : key;
      };
      for (std::size_t l = 0; l < L; ++l) {
        const auto& w = model_->layers[l];
        const std::string p = "l" + std::to_string(l) + "_";
        add("rmsnorm_qkv_rope_append?" + ropeShape + normKey, p + "norm_qkv_rope_append",
            {residual_, w.inputNormWeight, w.queryKeyValueWeight, model_->ropeCosine,
             model_->ropeSine, lengthsView_, tableViews_[l], activeView_},
            {query_, pools_[l]->keyBuffer(), pools_[l]->valueBuffer()});
        if (fuseAttention) {
          add(attentionOutputKey, p + "attention_output",
              {query_, pools_[l]->keyBuffer(), pools_[l]->valueBuffer(), lengthsView_,
               tableViews_[l], activeView_, w.outputWeight, residual_},
              {after_});
        } else {
          add(attentionKey, p + "attention",
              {query_, pools_[l]->keyBuffer(), pools_[l]->valueBuffer(), lengthsView_,
               tableViews_[l], activeView_},
              {context_});
          add(residualGemv(H, H), p + "o_residual", {context_, w.outputWeight, residual_},
              {after_});
        }
        add("rmsnorm_gate_up_silu?in=" + std::to_string(H) + "&out=" + std::to_string(I) + normKey,
            p + "norm_gate_up_silu", {after_, w.postAttentionNormWeight, w.gateWeight, w.upWeight},
            {gated_});
        add(residualGemv(I, H), p + "down_residual", {gated_, w.downWeight, after_}, {residual_});
      }
      // the norm-fused LM head maps its waves to the norm's groups at k split
      // 4: a tuned dot configuration applies only with that split
      std::string head = "rmsnorm_gemv?in=" + std::to_string(H) + "&out=" + std::to_string(V) +
                         "&out_dtype=f32" + normKey;
      const auto it = tunedSuffix.find(std::to_string(H) + "x" + std::to_string(V));
      if (it != tunedSuffix.end() && it->second.find("&algorithm=1&") != std::string::npos &&
          it->second.find("&k_split=4") != std::string::npos)
        head += it->second;
      add(head, "norm_lm_head", {residual_, model_->finalNormWeight, model_->languageModelHeadWeight},
          {logits_});
    } else if (foldPacked) {
      // residual_ (packed) -> [norm] q.k.v + RoPE + append -> attention -> o
      // + residual -> after_ -> [norm] gate/up -> down + residual ->
      // residual_; the LM head folds the final norm.
      // gamma lives in the scaled packed weights (ensurePackedWeights)
      const std::string normKey = "&norm=1&eps=" + eps;
      const std::string hs = std::to_string(H), is = std::to_string(I);
      const bool packedContext = QH * D == H;
      for (std::size_t l = 0; l < L; ++l) {
        const auto& pw = weights(l);
        const auto& sw = model_->normScaledLayers[l];
        const std::string p = "l" + std::to_string(l) + "_";
        add(qkvRopeKey + normKey, p + "norm_qkv_rope_append",
            {residual_, sw.queryKeyValueWeight, model_->ropeCosine, model_->ropeSine,
             lengthsView_, tableViews_[l], activeView_},
            {query_, pools_[l]->keyBuffer(), pools_[l]->valueBuffer()});
        // the attention output in fragment order when its width is the o
        // projection's input width (q_heads * head_dim == hidden)
        add(attentionKey + (packedContext ? "&out_layout=packed" : ""), p + "attention",
            {query_, pools_[l]->keyBuffer(), pools_[l]->valueBuffer(), lengthsView_,
             tableViews_[l], activeView_},
            {context_});
        add("gemm_packed?batch=" + B + "&in=" + hs + "&out=" + hs + "&out_dtype=f16" +
                (packedContext ? "&x_layout=packed" : "") + "&y_layout=packed&residual=1",
            p + "o_residual", {context_, pw.outputWeight, residual_}, {after_});
        add("gate_up_silu_packed?batch=" + B + "&hidden=" + hs + "&inter=" + is +
                "&x_layout=packed&y_layout=packed" + normKey,
            p + "norm_gate_up_silu", {after_, sw.gateWeight, sw.upWeight}, {gated_});
        add("gemm_packed?batch=" + B + "&in=" + is + "&out=" + hs +
                "&out_dtype=f16&x_layout=packed&y_layout=packed&residual=1",
            p + "down_residual", {gated_, pw.downWeight, after_}, {residual_});
      }
      add("gemm_packed?batch=" + B + "&in=" + hs + "&out=" + std::to_string(V) +
              "&out_dtype=f32&x_layout=packed" + normKey,
          "norm_lm_head", {residual_, model_->normScaledLanguageModelHead}, {logits_});
    } else {
      for (std::size_t l = 0; l < L; ++l) {
        const auto& w = model_->layers[l];
        const std::string p = "l" + std::to_string(l) + "_";
        if (l > 0)
          add("add_rmsnorm?" + norm, p + "residual_input_norm", {after_, mlp_, w.inputNormWeight},
              {residual_, normalized_});
        const auto& pw = weights(l);
        if (fuseRope) {
          // RoPE and the K/V append run in the projection's epilogue (the dot
          // GEMV at batch 1, the packed GEMM above).
          add(qkvRopeKey, p + "qkv_rope_append",
              {normalized_, pw.queryKeyValueWeight, model_->ropeCosine, model_->ropeSine,
               lengthsView_, tableViews_[l], activeView_},
              {query_, pools_[l]->keyBuffer(), pools_[l]->valueBuffer()});
        } else {
          add(gemv(H, QKV, "f16"), p + "qkv", {normalized_, pw.queryKeyValueWeight}, {qkv_});
          add(ropeKey, p + "rope_append",
              {qkv_, model_->ropeCosine, model_->ropeSine, lengthsView_, tableViews_[l], activeView_},
              {query_, pools_[l]->keyBuffer(), pools_[l]->valueBuffer()});
        }
        add(attentionKey, p + "attention",
            {query_, pools_[l]->keyBuffer(), pools_[l]->valueBuffer(), lengthsView_, tableViews_[l],
             activeView_},
            {context_});
        add(gemv(H, H, "f16", false), p + "o", {context_, pw.outputWeight}, {projected_});
        add("add_rmsnorm?" + norm, p + "residual_post_norm",
            {residual_, projected_, w.postAttentionNormWeight}, {after_, normalized_});
        add(std::string(packed ? "gate_up_silu_packed" : "gate_up_silu") + "?batch=" + B +
                "&hidden=" + std::to_string(H) + "&inter=" + std::to_string(I) +
                (packed ? "&x_layout=packed&y_layout=packed" : ""),
            p + "gate_up_silu", {normalized_, pw.gateWeight, pw.upWeight}, {gated_});
        add(gemv(I, H, "f16"), p + "down", {gated_, pw.downWeight}, {mlp_});
      }
      add("add_rmsnorm?" + norm, "residual_final_norm", {after_, mlp_, model_->finalNormWeight},
          {residual_, normalized_});
      add(gemv(H, V, "f32"), "lm_head",
          {normalized_, packed ? model_->packedLanguageModelHead : model_->languageModelHeadWeight},
          {logits_});
    }
    add("argmax?rows=" + B + "&vocab=" + std::to_string(V), "argmax", {logits_}, {nextTokens_});
    std::vector<const hip::PreparedExecution*> pointers;
    for (const auto& step : bucket->steps) pointers.push_back(step.get());
    auto sequence = rt.prepareSequence(pointers);
    if (!sequence.execution) throw std::runtime_error(sequence.errorMessage);
    bucket->sequence = std::move(sequence.execution);
    if (fold || foldPacked) {
      // Token-only tail: the LM head with a partial argmax, then the final
      // argmax, after the same trunk (every step but the LM head and argmax).
      const std::size_t trunk = bucket->steps.size() - 2;
      const std::string vs = std::to_string(V), hs = std::to_string(H);
      if (fold)
        add("rmsnorm_lm_head_partial_argmax?in=" + hs + "&out=" + vs + "&eps=" + eps,
            "lm_head_partial_argmax",
            {residual_, model_->finalNormWeight, model_->languageModelHeadWeight},
            {argmaxWorkspace_});
      else
        add("lm_head_partial_argmax_packed?batch=" + B + "&in=" + hs + "&out=" + vs + "&eps=" +
                eps + "&x_layout=packed",
            "lm_head_partial_argmax", {residual_, model_->normScaledLanguageModelHead},
            {argmaxWorkspace_});
      add("lm_head_final_argmax?rows=" + B + "&vocab=" + vs, "lm_head_final_argmax",
          {argmaxWorkspace_}, {nextTokens_});
      for (std::size_t i = bucket->steps.size() - 2; i < bucket->steps.size(); ++i)
        bucket->tokenSteps.push_back(std::move(bucket->steps[i]));
      bucket->steps.resize(bucket->steps.size() - 2);
      std::vector<const hip::PreparedExecution*> tokenPointers(pointers.begin(),
                                                               pointers.begin() + trunk);
      for (const auto& step : bucket->tokenSteps) tokenPointers.push_back(step.get());
      auto tokens = rt.prepareSequence(tokenPointers);
      if (!tokens.execution) throw std::runtime_error(tokens.errorMessage);
      bucket->tokenSequence = std::move(tokens.execution);
    }
    if (log)
      *log << "Batched decode bucket rows=" << m << ": " << bucket->steps.size()
           << " dispatches captured\n";
    buckets_.push_back(std::move(bucket));
  }
}

BatchedDecodeExecutor::Creation createBatchedDecodeExecutor(
    hip::HipRuntime& runtime, std::shared_ptr<DecoderLLMModelResources> model,
    std::vector<std::shared_ptr<KVPagePool>> pools, std::size_t maximumBatchSize,
    std::ostream* log, bool tuneKernels, std::shared_ptr<KernelRegistry> registry,
    bool foldNorms, bool fuseAttentionOutput) {
  BatchedDecodeExecutor::Creation result;
  try {
    if (!model) throw std::invalid_argument("Batched decode needs model resources.");
    const auto& plan = model->plan;
    if (maximumBatchSize == 0 || maximumBatchSize > 4096)
      throw std::invalid_argument("Batched decode maximum batch must be in [1, 4096].");
    if (pools.size() != plan.layerCount)
      throw std::invalid_argument("Batched decode needs one KV page pool per layer.");
    const auto kv = plan.kvPlan();
    for (const auto& pool : pools) {
      if (!pool || !pool->hasStorage() || pool->pageSize() != pools.front()->pageSize() ||
          pool->plan().heads != kv.heads || pool->plan().headDimension != kv.headDimension ||
          pool->plan().dtype != DType::Float16 || pool->plan().batch != 1)
        throw std::invalid_argument("Batched decode KV pools do not match the model.");
    }
    std::unique_ptr<BatchedDecodeExecutor> executor(new BatchedDecodeExecutor());
    executor->runtime_ = &runtime;
    executor->model_ = std::move(model);
    executor->pools_ = std::move(pools);
    executor->maximumBatchSize_ = maximumBatchSize;
    executor->pageSize_ = executor->pools_.front()->pageSize();
    executor->tuneKernels_ = tuneKernels;
    executor->foldNorms_ = foldNorms;
    executor->fuseAttentionOutput_ = fuseAttentionOutput;
    executor->registry_ = std::move(registry);
    executor->build(log);
    result.executor = std::move(executor);
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

std::string BatchedDecodeExecutor::upload(const std::vector<std::int32_t>& tokens,
                                          const std::vector<std::int32_t>& lengths,
                                          const std::vector<std::vector<std::int32_t>>& tables,
                                          std::size_t rows, std::size_t bucket) {
  const std::size_t M = maximumBatchSize_;
  std::vector<std::int32_t> meta(2 * M + 1, 0);
  std::copy(tokens.begin(), tokens.end(), meta.begin());
  std::copy(lengths.begin(), lengths.end(), meta.begin() + static_cast<std::ptrdiff_t>(M));
  meta[2 * M] = static_cast<std::int32_t>(rows);
  (void)bucket;
  // Both uploads are queued on the runtime stream ahead of the step's
  // graph, with no host wait.
  if (meta != metaShadow_) {
    auto error = meta_->writeRawAsync(meta.data(), meta.size());
    if (!error.empty()) return error;
    metaShadow_ = std::move(meta);
  }
  return uploadTables(tables);
}

std::string BatchedDecodeExecutor::uploadTables(
    const std::vector<std::vector<std::int32_t>>& tables) {
  const std::size_t M = maximumBatchSize_;
  // Pack [layer][M][maxPages] and write what changed.
  std::vector<std::int32_t> packed(tableShadow_.size(), -1);
  for (std::size_t l = 0; l < tables.size(); ++l)
    std::copy(tables[l].begin(), tables[l].end(),
              packed.begin() + static_cast<std::ptrdiff_t>(l * M * maxPages_));
  auto error = writeTableChanges(*tables_, packed, tableShadow_);
  if (!error.empty()) return error;
  tableShadow_ = std::move(packed);
  return {};
}

BatchedDecodeRun BatchedDecodeExecutor::run(const std::vector<float>& tokenIds,
                                            const std::vector<float>& validLengths,
                                            const std::vector<std::vector<float>>& blockTables,
                                            bool readLogits) {
  std::vector<std::int32_t> tokens(tokenIds.begin(), tokenIds.end());
  std::vector<std::int32_t> lengths(validLengths.begin(), validLengths.end());
  std::vector<std::vector<std::int32_t>> tables;
  tables.reserve(blockTables.size());
  for (const auto& table : blockTables) tables.emplace_back(table.begin(), table.end());
  return run(tokens, lengths, tables, readLogits, true);
}

std::string BatchedDecodeExecutor::checkStep(
    const std::vector<std::int32_t>* tokenIds, const std::vector<std::int32_t>& validLengths,
    const std::vector<std::vector<std::int32_t>>& blockTables) const {
  const auto& plan = model_->plan;
  const std::size_t rows = validLengths.size();
  if (rows == 0 || rows > maximumBatchSize_ || (tokenIds && tokenIds->size() != rows) ||
      blockTables.size() != plan.layerCount)
    return "Batched decode metadata shape is invalid.";
  for (std::size_t l = 0; l < blockTables.size(); ++l)
    if (blockTables[l].size() != rows * maxPages_)
      return "Batched decode block-table shape is invalid.";
  // Host checks that keep every device access inside its buffer: token ids in
  // the vocabulary, lengths in [1, capacity], pages allocated in their pool
  // and present for every attended position.
  for (std::size_t r = 0; r < rows; ++r) {
    if (tokenIds &&
        ((*tokenIds)[r] < 0 || static_cast<std::size_t>((*tokenIds)[r]) >= plan.vocabularySize))
      return "Batched decode token id is outside the vocabulary.";
    if (validLengths[r] <= 0 || static_cast<std::size_t>(validLengths[r]) > plan.attention.capacity)
      return "KV cache valid length is outside the configured capacity.";
    const std::size_t needed = (static_cast<std::size_t>(validLengths[r]) + pageSize_ - 1) / pageSize_;
    for (std::size_t l = 0; l < blockTables.size(); ++l) {
      for (std::size_t p = 0; p < maxPages_; ++p) {
        const std::int32_t page = blockTables[l][r * maxPages_ + p];
        if ((p < needed && !pools_[l]->isAllocated(page)) || (page >= 0 && !pools_[l]->isAllocated(page)))
          return "Batched decode block table names a page that is not allocated in its layer's "
                 "pool.";
      }
    }
  }
  return {};
}

std::string BatchedDecodeExecutor::reserveHistory(std::size_t steps) {
  if (steps == 0) return "Chained decode needs at least one history step.";
  if (steps <= historySteps_) return {};
  try {
    history_ = allocate(*runtime_, steps * maximumBatchSize_, nullptr, ElementType::Int32);
  } catch (const std::exception& error) {
    return error.what();
  }
  historySteps_ = steps;
  return {};
}

std::string BatchedDecodeExecutor::launchChained(
    const std::vector<std::int32_t>& tokenIds, const std::vector<std::int32_t>& validLengths,
    const std::vector<std::vector<std::int32_t>>& blockTables, std::size_t historyStep) {
  const std::size_t rows = validLengths.size();
  if (historyStep >= historySteps_) return "Chained decode history step is out of range.";
  if (tokenIds.empty() && rows != chainedRows_)
    return "Chained decode without tokens needs the previous step's row count.";
  auto error = checkStep(tokenIds.empty() ? nullptr : &tokenIds, validLengths, blockTables);
  if (!error.empty()) return error;
  std::size_t index = 0;
  while (buckets_[index]->rows < rows) ++index;
  auto& bucket = *buckets_[index];
  // After a chained step the device holds that step's tokens in the token
  // slots and its lengths advanced by one (tmc_decode_chain below).  The
  // metadata goes up in full for the first step; later steps send only the
  // lengths, and only when they do not follow the previous step's by one.
  const std::size_t M = maximumBatchSize_;
  std::fill(metaShadow_.begin(), metaShadow_.end(), std::numeric_limits<std::int32_t>::min());
  if (!tokenIds.empty()) {
    error = upload(tokenIds, validLengths, blockTables, rows, bucket.rows);
  } else {
    bool follows = chainedLengths_.size() == rows;
    for (std::size_t r = 0; follows && r < rows; ++r)
      follows = validLengths[r] == chainedLengths_[r] + 1;
    if (!follows) {
      std::vector<std::int32_t> lengths(M + 1, 0);
      std::copy(validLengths.begin(), validLengths.end(), lengths.begin());
      lengths[M] = static_cast<std::int32_t>(rows);
      error = meta_->writeRawAsync(lengths.data(), lengths.size(), M);
    }
    if (error.empty()) error = uploadTables(blockTables);
  }
  hip::PreparedSequence* sequence = nullptr;
  if (error.empty()) error = stepSequence(bucket, false, sequence);
  if (error.empty()) error = sequence->launch();
  if (error.empty() && registry_) registry_->completed(bucket.uses);
  if (error.empty() &&
      tmc_decode_chain(static_cast<const std::int32_t*>(nextTokens_->devicePointer()),
                       static_cast<std::int32_t*>(tokensView_->devicePointer()),
                       static_cast<std::int32_t*>(lengthsView_->devicePointer()),
                       static_cast<std::int32_t*>(history_->devicePointer()) + historyStep * M,
                       static_cast<std::int64_t>(rows), runtime_->stream()) != 0)
    error = std::string("Chained decode: ") + tmc_last_error();
  std::fill(metaShadow_.begin(), metaShadow_.end(), std::numeric_limits<std::int32_t>::min());
  chainedRows_ = error.empty() ? rows : 0;
  if (error.empty())
    chainedLengths_ = validLengths;
  else
    chainedLengths_.clear();
  return error;
}

std::string BatchedDecodeExecutor::readHistory(std::size_t steps,
                                               std::vector<std::int32_t>& out) const {
  if (steps == 0 || steps > historySteps_) return "Chained decode history range is invalid.";
  out.assign(steps * maximumBatchSize_, 0);
  return history_->readRaw(out.data(), out.size());  // waits for the stream
}

namespace {
// Token-only admissions per process: key = model dimensions, bucket rows and
// fold form; value = (admitted, measured speedup, 0 when untimed).
std::mutex g_token_mutex;
std::map<std::string, std::pair<bool, double>> g_token_decisions;
}  // namespace

std::string BatchedDecodeExecutor::tokenOnlyKey(const Bucket& bucket) const {
  const auto& plan = model_->plan;
  std::ostringstream key;
  key << "H" << plan.hiddenSize() << "_I" << plan.intermediateSize << "_V"
      << plan.vocabularySize << "_L" << plan.layerCount << "_QH" << plan.attention.heads << "_KVH"
      << plan.kvHeads() << "_D" << plan.attention.headDimension << "_cap"
      << plan.attention.capacity << "_page" << pageSize_ << "_rows" << bucket.rows
      << (bucket.rows > 1 ? "_packed" : "_dot");
  return key.str();
}

std::string BatchedDecodeExecutor::checkTokenOnly(Bucket& bucket) {
  bucket.tokenChecked = true;
  bucket.tokenAdmitted = false;
  if (!bucket.tokenSequence || tokenPolicy_ == TokenOnlyPolicy::Never) return {};
  const std::string key = tokenOnlyKey(bucket);
  if (tokenPolicy_ != TokenOnlyPolicy::Always) {
    std::lock_guard<std::mutex> lock(g_token_mutex);
    const auto known = g_token_decisions.find(key);
    if (known != g_token_decisions.end()) {
      bucket.tokenAdmitted = known->second.first;
      bucket.tokenSpeedup = known->second.second;
      return {};
    }
  }
  if (tokenPolicy_ == TokenOnlyPolicy::CachedOnly) {
    bucket.tokenChecked = false;  // decided by a later admission, if any
    return {};
  }
  // Both sequences write the same staged K/V slots and read the same
  // uploaded metadata, so replaying the step is safe and appends nothing.
  const std::size_t rows = bucket.rows;
  std::vector<std::int32_t> expected(rows), actual(rows);
  auto baseline = bucket.sequence->execute();
  if (!baseline.executionPassed) return baseline.errorMessage;
  auto error = nextTokens_->readRaw(expected.data(), rows);
  if (!error.empty()) return error;
  auto candidate = bucket.tokenSequence->execute();
  if (!candidate.executionPassed) return candidate.errorMessage;
  error = nextTokens_->readRaw(actual.data(), rows);
  if (!error.empty()) return error;
  if (actual != expected) {  // tokens disagree: keep the logits tail
    std::lock_guard<std::mutex> lock(g_token_mutex);
    g_token_decisions[key] = {false, 0.0};
    return {};
  }
  if (tokenPolicy_ == TokenOnlyPolicy::Always) {
    bucket.tokenAdmitted = true;
    return {};
  }
  const auto base = benchmark::sampler(*bucket.sequence);
  const auto cand = benchmark::sampler(*bucket.tokenSequence);
  error = benchmark::warmup(cand, 5);
  if (!error.empty()) return error;
  const auto first = benchmark::measurePair(base, cand, 31);
  const auto second = benchmark::measurePair(base, cand, 31);
  if (first.passed && second.passed) {
    bucket.tokenSpeedup = std::min(first.speedup, second.speedup);
    bucket.tokenAdmitted = bucket.tokenSpeedup >= planner::kMinimumSpeedup;
  }
  std::lock_guard<std::mutex> lock(g_token_mutex);
  g_token_decisions[key] = {bucket.tokenAdmitted, bucket.tokenSpeedup};
  // the last replay was the token sequence: its tokens equal the logits tail's
  return {};
}

std::string BatchedDecodeExecutor::stepSequence(Bucket& bucket, bool readLogits,
                                                hip::PreparedSequence*& sequence) {
  sequence = bucket.sequence.get();
  if (readLogits || !bucket.tokenSequence || tokenPolicy_ == TokenOnlyPolicy::Never) return {};
  if (!bucket.tokenChecked) {
    const auto error = checkTokenOnly(bucket);
    if (!error.empty()) return error;
  }
  if (bucket.tokenAdmitted) sequence = bucket.tokenSequence.get();
  return {};
}

std::string BatchedDecodeExecutor::admitTokenOnly(
    const std::vector<std::int32_t>& tokenIds, const std::vector<std::int32_t>& validLengths,
    const std::vector<std::vector<std::int32_t>>& blockTables) {
  const std::size_t rows = tokenIds.size();
  auto error = checkStep(&tokenIds, validLengths, blockTables);
  if (!error.empty()) return error;
  std::size_t index = 0;
  while (buckets_[index]->rows < rows) ++index;
  auto& bucket = *buckets_[index];
  if (bucket.tokenChecked || !bucket.tokenSequence) return {};
  error = upload(tokenIds, validLengths, blockTables, rows, bucket.rows);
  if (!error.empty()) return error;
  return checkTokenOnly(bucket);
}

BatchedDecodeExecutor::TokenOnlyStatus BatchedDecodeExecutor::tokenOnlyStatus(
    std::size_t rows) const {
  TokenOnlyStatus status;
  for (const auto& b : buckets_)
    if (b->rows >= rows) {  // the bucket a step of `rows` rows runs
      status.available = b->tokenSequence != nullptr;
      status.checked = b->tokenChecked;
      status.admitted = b->tokenAdmitted;
      status.speedup = b->tokenSpeedup;
      break;
    }
  return status;
}

BatchedDecodeRun BatchedDecodeExecutor::run(const std::vector<std::int32_t>& tokenIds,
                                            const std::vector<std::int32_t>& validLengths,
                                            const std::vector<std::vector<std::int32_t>>& blockTables,
                                            bool readLogits, bool timeGpu) {
  BatchedDecodeRun result;
  const auto& plan = model_->plan;
  const std::size_t rows = tokenIds.size();
  result.errorMessage = checkStep(&tokenIds, validLengths, blockTables);
  if (!result.errorMessage.empty()) return result;
  std::size_t index = 0;
  while (buckets_[index]->rows < rows) ++index;
  auto& bucket = *buckets_[index];
  auto error = upload(tokenIds, validLengths, blockTables, rows, bucket.rows);
  if (!error.empty()) {
    result.errorMessage = error;
    return result;
  }
  hip::PreparedSequence* sequence = nullptr;
  error = stepSequence(bucket, readLogits, sequence);
  if (!error.empty()) {
    result.errorMessage = error;
    return result;
  }
  if (timeGpu) {
    const auto execution = sequence->execute();
    if (!execution.executionPassed) {
      result.errorMessage = execution.errorMessage;
      return result;
    }
    result.gpuExecutionTimeUs = execution.gpuExecutionTimeUs;
    result.cpuSubmitToCompletionTimeUs = execution.cpuSubmitToCompletionTimeUs;
  } else {
    error = sequence->launch();
    if (!error.empty()) {
      result.errorMessage = error;
      return result;
    }
  }
  if (registry_) registry_->completed(bucket.uses);
  std::vector<std::int32_t> next(rows);
  error = nextTokens_->readRaw(next.data(), rows);  // waits for the stream
  if (!error.empty()) {
    result.errorMessage = error;
    return result;
  }
  result.nextTokenIds.assign(next.begin(), next.end());
  if (readLogits) {
    result.logits.resize(rows * plan.vocabularySize);
    error = logits_->readRaw(result.logits.data(), result.logits.size());
    if (!error.empty()) {
      result.errorMessage = error;
      return result;
    }
  }
  result.passed = true;
  return result;
}

// ----------------------------------------------------- ChunkedPrefillExecutor
struct ChunkedPrefillExecutor::Stage {
  std::size_t rows = 0;
  std::vector<std::unique_ptr<hip::PreparedExecution>> steps;
  std::unique_ptr<hip::PreparedSequence> sequence;
};

ChunkedPrefillExecutor::~ChunkedPrefillExecutor() = default;

std::vector<std::size_t> ChunkedPrefillExecutor::buckets() const {
  std::vector<std::size_t> rows;
  for (const auto& stage : stages_) rows.push_back(stage->rows);
  return rows;
}

std::size_t ChunkedPrefillExecutor::dispatchesPerChunk(std::size_t bucket) const {
  for (const auto& stage : stages_)
    if (stage->rows == bucket) return stage->steps.size();
  return 0;
}

void ChunkedPrefillExecutor::build(std::ostream* log) {
  auto& rt = *runtime_;
  const auto& plan = model_->plan;
  const std::size_t S = chunkSize_, L = plan.layerCount;
  const std::size_t H = plan.hiddenSize(), I = plan.intermediateSize, V = plan.vocabularySize;
  const std::size_t QH = plan.attention.heads, KVH = plan.kvHeads(), D = plan.attention.headDimension;
  const std::size_t QKV = H + 2 * plan.kvWidth();
  const std::size_t capacity = plan.attention.capacity;
  maxPages_ = (capacity + pageSize_ - 1) / pageSize_;

  const std::size_t R = maxRequests_, T = R * maxPages_;  // table entries per layer
  std::vector<float> zeros(3 * S + 1, 0.0f);
  meta_ = allocate(rt, 3 * S + 1, zeros.data(), ElementType::Int32);
  tokensView_ = view(rt, meta_, 0, S);
  lengthsView_ = view(rt, meta_, S, S);
  rowTableView_ = view(rt, meta_, 2 * S, S);
  activeView_ = view(rt, meta_, 3 * S, 1);
  const std::vector<float> none(L * T, -1.0f);
  tables_ = allocate(rt, none.size(), none.data(), ElementType::Int32);
  for (std::size_t l = 0; l < L; ++l) tableViews_.push_back(view(rt, tables_, l * T, T));
  metaShadow_.assign(3 * S + 1, 0);
  tableShadow_.assign(L * T, -1);

  auto act = [&](std::size_t count, ElementType type = ElementType::Float16) {
    activationBytes_ += count * hip::elementBytes(type);
    return allocate(rt, count, nullptr, type);
  };
  residual_ = act(S * H);
  after_ = act(S * H);
  normalized_ = act(S * H);
  qkv_ = act(S * QKV);
  query_ = act(S * H);
  context_ = act(S * H);
  projected_ = act(S * H);
  gate_ = act(S * I);
  up_ = act(S * I);
  gated_ = act(S * I);
  mlp_ = act(S * H);
  logits_ = act(S * V, ElementType::Float32);
  nextTokens_ = act(S, ElementType::Int32);
  workspace_ = act(tmc_gemm_rows_workspace_bytes() / 4, ElementType::Int32);

  std::vector<std::size_t> rows;
  for (std::size_t r = 16; r < S; r *= 2) rows.push_back(r);
  rows.push_back(S);

  const std::string eps = fmt(plan.rmsNormEpsilon);
  for (const std::size_t m : rows) {
    auto stage = std::make_unique<Stage>();
    stage->rows = m;
    const std::string B = std::to_string(m);
    auto add = [&](const std::string& key, const std::string& name,
                   const std::vector<BufferHandle>& inputs,
                   const std::vector<BufferHandle>& outputs) {
      const auto pipeline = rt.createComputePipeline(key, name);
      if (!pipeline.pipelineCreationPassed)
        throw std::runtime_error(name + ": " + pipeline.errorMessage);
      auto prepared = rt.prepareBuffers(
          inputs, outputs, {pipeline.threadgroupCount, pipeline.threadsPerThreadgroup});
      if (!prepared.execution) throw std::runtime_error(name + ": " + prepared.errorMessage);
      stage->steps.push_back(std::move(prepared.execution));
    };
    auto gemm = [&](std::size_t in, std::size_t out, const char* outType) {
      return "gemm_rows?m=" + B + "&in=" + std::to_string(in) + "&out=" + std::to_string(out) +
             "&out_dtype=" + outType + "&workspace=1";
    };
    const std::string norm = "rows=" + B + "&width=" + std::to_string(H) + "&eps=" + eps + "&dtype=f16";
    const std::string heads = "&q_heads=" + std::to_string(QH) + "&kv_heads=" + std::to_string(KVH) +
                              "&head_dim=" + std::to_string(D) +
                              "&page_size=" + std::to_string(pageSize_);
    // Several requests per chunk: R table rows and the per-row table index.
    const std::string multi = R > 1 ? "&tables=" + std::to_string(R) : "";
    const std::string ropeKey =
        "prefill_rope_append?rows=" + B + heads + "&capacity=" + std::to_string(capacity) + multi;
    const std::string attentionKey =
        "prefill_attention?rows=" + B + heads + "&max_pages=" + std::to_string(maxPages_) + multi;
    auto tableInputs = [&](std::size_t l) {
      std::vector<BufferHandle> in{lengthsView_, tableViews_[l]};
      if (R > 1) in.push_back(rowTableView_);
      in.push_back(activeView_);
      return in;
    };
    add("embedding?rows=" + B + "&hidden=" + std::to_string(H) + "&vocab=" + std::to_string(V),
        "embedding", {tokensView_, model_->embeddingWeight}, {residual_});
    add("rmsnorm?" + norm, "l0_input_norm", {residual_, model_->layers[0].inputNormWeight},
        {normalized_});
    for (std::size_t l = 0; l < L; ++l) {
      const auto& w = model_->layers[l];
      const std::string p = "l" + std::to_string(l) + "_";
      if (l > 0)
        add("add_rmsnorm?" + norm, p + "residual_input_norm", {after_, mlp_, w.inputNormWeight},
            {residual_, normalized_});
      add(gemm(H, QKV, "f16"), p + "qkv", {normalized_, w.queryKeyValueWeight, workspace_}, {qkv_});
      {
        std::vector<BufferHandle> in{qkv_, model_->ropeCosine, model_->ropeSine};
        const auto t = tableInputs(l);
        in.insert(in.end(), t.begin(), t.end());
        add(ropeKey, p + "rope_append", in,
            {query_, pools_[l]->keyBuffer(), pools_[l]->valueBuffer()});
      }
      {
        std::vector<BufferHandle> in{query_, pools_[l]->keyBuffer(), pools_[l]->valueBuffer()};
        const auto t = tableInputs(l);
        in.insert(in.end(), t.begin(), t.end());
        add(attentionKey, p + "attention", in, {context_});
      }
      add(gemm(H, H, "f16"), p + "o", {context_, w.outputWeight, workspace_}, {projected_});
      add("add_rmsnorm?" + norm, p + "residual_post_norm",
          {residual_, projected_, w.postAttentionNormWeight}, {after_, normalized_});
      add(gemm(H, I, "f16"), p + "gate", {normalized_, w.gateWeight, workspace_}, {gate_});
      add(gemm(H, I, "f16"), p + "up", {normalized_, w.upWeight, workspace_}, {up_});
      add("silu_mul?count=" + std::to_string(m * I) + "&dtype=f16", p + "silu_mul", {gate_, up_},
          {gated_});
      add(gemm(I, H, "f16"), p + "down", {gated_, w.downWeight, workspace_}, {mlp_});
    }
    add("add_rmsnorm?" + norm, "residual_final_norm", {after_, mlp_, model_->finalNormWeight},
        {residual_, normalized_});
    add(gemm(H, V, "f32"), "lm_head", {normalized_, model_->languageModelHeadWeight, workspace_},
        {logits_});
    add("argmax?rows=" + B + "&vocab=" + std::to_string(V), "argmax", {logits_}, {nextTokens_});
    std::vector<const hip::PreparedExecution*> pointers;
    for (const auto& step : stage->steps) pointers.push_back(step.get());
    auto sequence = rt.prepareSequence(pointers);
    if (!sequence.execution) throw std::runtime_error(sequence.errorMessage);
    stage->sequence = std::move(sequence.execution);
    if (log)
      *log << "Chunked prefill stage rows=" << m << ": " << stage->steps.size()
           << " dispatches (eager)\n";
    stages_.push_back(std::move(stage));
  }
}

ChunkedPrefillExecutor::Creation createChunkedPrefillExecutor(
    hip::HipRuntime& runtime, std::shared_ptr<DecoderLLMModelResources> model,
    std::vector<std::shared_ptr<KVPagePool>> pools, std::size_t chunkSize, std::ostream* log,
    std::size_t maximumRequests) {
  ChunkedPrefillExecutor::Creation result;
  try {
    if (!model) throw std::invalid_argument("Chunked prefill needs model resources.");
    const auto& plan = model->plan;
    if (chunkSize == 0 || chunkSize > 8192)
      throw std::invalid_argument("Chunked prefill chunk size must be in [1, 8192].");
    if (pools.size() != plan.layerCount)
      throw std::invalid_argument("Chunked prefill needs one KV page pool per layer.");
    const auto kv = plan.kvPlan();
    for (const auto& pool : pools) {
      if (!pool || !pool->hasStorage() || pool->pageSize() != pools.front()->pageSize() ||
          pool->plan().heads != kv.heads || pool->plan().headDimension != kv.headDimension ||
          pool->plan().dtype != DType::Float16 || pool->plan().batch != 1)
        throw std::invalid_argument("Chunked prefill KV pools do not match the model.");
    }
    const std::size_t D = plan.attention.headDimension;
    const std::size_t group = plan.attention.heads / plan.kvHeads();
    if ((D != 64 && D != 128) || 64 % group != 0)
      throw std::invalid_argument(
          "Chunked prefill attention needs head_dim 64 or 128 and heads / kv_heads dividing 64.");
    if (maximumRequests == 0 || maximumRequests > 1024)
      throw std::invalid_argument("Chunked prefill requests per chunk must be in [1, 1024].");
    std::unique_ptr<ChunkedPrefillExecutor> executor(new ChunkedPrefillExecutor());
    executor->runtime_ = &runtime;
    executor->model_ = std::move(model);
    executor->pools_ = std::move(pools);
    executor->chunkSize_ = chunkSize;
    executor->maxRequests_ = maximumRequests;
    executor->tileRows_ = 64 / group;  // tokens per query tile of tmc_prefill_attention_f16
    executor->pageSize_ = executor->pools_.front()->pageSize();
    executor->build(log);
    result.executor = std::move(executor);
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

std::size_t ChunkedPrefillExecutor::packedRows(const std::vector<std::size_t>& counts) const noexcept {
  std::size_t rows = 0;
  for (std::size_t i = 0; i < counts.size(); ++i)
    rows = i + 1 < counts.size() ? (rows + counts[i] + tileRows_ - 1) / tileRows_ * tileRows_
                                 : rows + counts[i];
  return rows;
}

std::string ChunkedPrefillExecutor::validate(const PrefillSegment& segment) const {
  const auto& plan = model_->plan;
  const std::size_t rows = segment.tokenIds.size();
  if (rows == 0 || segment.blockTables.size() != plan.layerCount)
    return "Chunked prefill input shape is invalid.";
  if (segment.start + rows > plan.attention.capacity)
    return "KV cache valid length is outside the configured capacity.";
  for (const auto token : segment.tokenIds)
    if (token < 0 || static_cast<std::size_t>(token) >= plan.vocabularySize)
      return "Chunked prefill token id is outside the vocabulary.";
  // Every page the segment writes or attends is allocated in its layer's
  // pool; entries past them are absent or allocated.
  const std::size_t needed = (segment.start + rows + pageSize_ - 1) / pageSize_;
  for (std::size_t l = 0; l < segment.blockTables.size(); ++l) {
    if (segment.blockTables[l].size() != maxPages_) return "Chunked prefill block-table shape is invalid.";
    for (std::size_t p = 0; p < maxPages_; ++p) {
      const std::int32_t page = segment.blockTables[l][p];
      if ((p < needed || page >= 0) && !pools_[l]->isAllocated(page))
        return "Chunked prefill block table names a page that is not allocated in its layer's pool.";
    }
  }
  return {};
}

BatchedDecodeRun ChunkedPrefillExecutor::run(const std::vector<std::int32_t>& tokenIds,
                                             std::size_t start,
                                             const std::vector<std::vector<std::int32_t>>& blockTables,
                                             bool readLogits, bool timeGpu) {
  PrefillSegment segment{tokenIds, start, blockTables};
  auto result = runBatch({segment}, false, timeGpu);
  if (!result.passed || !readLogits) return result;
  // All rows' logits of the one segment (rows 0 .. n-1 of the chunk).
  result.logits.resize(tokenIds.size() * model_->plan.vocabularySize);
  const auto error = logits_->readRaw(result.logits.data(), result.logits.size());
  if (!error.empty()) {
    result.passed = false;
    result.errorMessage = error;
  }
  return result;
}

BatchedDecodeRun ChunkedPrefillExecutor::runBatch(const std::vector<PrefillSegment>& segments,
                                                  bool readLogits, bool timeGpu) {
  BatchedDecodeRun result;
  const auto& plan = model_->plan;
  const std::size_t S = chunkSize_, L = plan.layerCount, V = plan.vocabularySize;
  if (segments.empty() || segments.size() > maxRequests_) {
    result.errorMessage = "Chunked prefill needs 1 to maximumRequests() segments.";
    return result;
  }
  std::vector<std::size_t> counts;
  for (const auto& segment : segments) {
    auto error = validate(segment);
    if (!error.empty()) {
      result.errorMessage = error;
      return result;
    }
    counts.push_back(segment.tokenIds.size());
  }
  const std::size_t rows = packedRows(counts);
  if (rows > S) {
    result.errorMessage = "Chunked prefill segments do not fit the chunk.";
    return result;
  }
  // Pack: segment i's rows from a tile boundary; padding rows have length 0
  // (skipped by the kernels) and row table -1.
  std::vector<std::int32_t> meta(3 * S + 1, 0);
  std::vector<std::size_t> first(segments.size());
  std::fill(meta.begin() + static_cast<std::ptrdiff_t>(2 * S),
            meta.begin() + static_cast<std::ptrdiff_t>(3 * S), -1);
  for (std::size_t i = 0, row = 0; i < segments.size(); ++i) {
    first[i] = row;
    for (std::size_t r = 0; r < counts[i]; ++r) {
      meta[row + r] = segments[i].tokenIds[r];
      meta[S + row + r] = static_cast<std::int32_t>(segments[i].start + r + 1);
      meta[2 * S + row + r] = static_cast<std::int32_t>(i);
    }
    row = (row + counts[i] + tileRows_ - 1) / tileRows_ * tileRows_;
  }
  meta[3 * S] = static_cast<std::int32_t>(rows);
  std::string error;
  if (meta != metaShadow_) {
    error = meta_->writeRawAsync(meta.data(), meta.size());
    if (!error.empty()) {
      result.errorMessage = error;
      return result;
    }
    metaShadow_ = std::move(meta);
  }
  const std::size_t T = maxRequests_ * maxPages_;
  std::vector<std::int32_t> packed(tableShadow_.size(), -1);
  for (std::size_t l = 0; l < L; ++l)
    for (std::size_t i = 0; i < segments.size(); ++i)
      std::copy(segments[i].blockTables[l].begin(), segments[i].blockTables[l].end(),
                packed.begin() + static_cast<std::ptrdiff_t>(l * T + i * maxPages_));
  error = writeTableChanges(*tables_, packed, tableShadow_);
  if (!error.empty()) {
    result.errorMessage = error;
    return result;
  }
  tableShadow_ = std::move(packed);
  std::size_t index = 0;
  while (stages_[index]->rows < rows) ++index;
  auto& stage = *stages_[index];
  if (timeGpu) {
    const auto execution = stage.sequence->execute();
    if (!execution.executionPassed) {
      result.errorMessage = execution.errorMessage;
      return result;
    }
    result.gpuExecutionTimeUs = execution.gpuExecutionTimeUs;
    result.cpuSubmitToCompletionTimeUs = execution.cpuSubmitToCompletionTimeUs;
  } else {
    error = stage.sequence->launch();
    if (!error.empty()) {
      result.errorMessage = error;
      return result;
    }
  }
  std::vector<std::int32_t> next(rows);
  error = nextTokens_->readRaw(next.data(), rows);  // waits for the stream
  if (!error.empty()) {
    result.errorMessage = error;
    return result;
  }
  for (std::size_t i = 0; i < segments.size(); ++i)
    for (std::size_t r = 0; r < counts[i]; ++r)
      result.nextTokenIds.push_back(static_cast<float>(next[first[i] + r]));
  if (readLogits) {
    result.logits.resize(segments.size() * V);
    for (std::size_t i = 0; i < segments.size(); ++i) {
      error = logits_->readRaw(result.logits.data() + i * V, V, (first[i] + counts[i] - 1) * V);
      if (!error.empty()) {
        result.errorMessage = error;
        return result;
      }
    }
  }
  result.passed = true;
  return result;
}

// --------------------------------------------------------- CompiledDecoderLLM
class CompiledDecoderLLM::Impl {
 public:
  hip::HipRuntime* runtime = nullptr;
  planner::DecoderLLMPlan plan;
  std::shared_ptr<DecoderLLMModelResources> model;
  std::vector<std::shared_ptr<KVPagePool>> pools;
  std::vector<std::unique_ptr<KVCacheState>> states;
  std::unique_ptr<BatchedDecodeExecutor> executor;
  std::unique_ptr<ChunkedPrefillExecutor> prefillExecutor;
  std::shared_ptr<KernelRegistry> registry = std::make_shared<KernelRegistry>();
  std::size_t requestedPageSize = 0;
  std::size_t kvBytes = 0;

  [[nodiscard]] std::size_t currentLength() const noexcept {
    return states.empty() ? 0 : states.front()->currentLength();
  }

  std::vector<std::vector<std::int32_t>> tables() const {
    std::vector<std::vector<std::int32_t>> out;
    out.reserve(states.size());
    for (const auto& state : states) {
      auto table = state->pageTable();
      table.resize(executor->maxPages(), -1);
      out.push_back(std::move(table));
    }
    return out;
  }

  std::string stage(std::size_t length) {
    const std::size_t previous = currentLength();
    for (auto& state : states) {
      const auto error = state->stageLength(*runtime, length);
      if (!error.empty()) {
        for (auto& staged : states) (void)staged->rollbackLength(*runtime, previous);
        return error;
      }
    }
    return {};
  }

  DecoderLLMRunResult step(float token, bool readLogits) {
    DecoderLLMRunResult result;
    const std::size_t previous = currentLength();
    const std::size_t next = previous + 1;
    if (next > plan.attention.capacity) {
      result.errorMessage = "Decoder KV cache capacity has been reached.";
      return result;
    }
    auto error = stage(next);
    if (!error.empty()) {
      result.errorMessage = error;
      return result;
    }
    const auto run = executor->run({static_cast<std::int32_t>(token)},
                                   {static_cast<std::int32_t>(next)}, tables(), readLogits, true);
    if (!run.passed) {
      for (auto& state : states) (void)state->rollbackLength(*runtime, previous);
      result.errorMessage = run.errorMessage;
      return result;
    }
    for (auto& state : states) state->commitLength(next);
    result.passed = true;
    result.logits = run.logits;
    result.nextTokenIds = run.nextTokenIds;
    result.gpuExecutionTimeUs = run.gpuExecutionTimeUs;
    result.cpuSubmitToCompletionTimeUs = run.cpuSubmitToCompletionTimeUs;
    return result;
  }
};

CompiledDecoderLLM::CompiledDecoderLLM(std::unique_ptr<Impl> impl) : impl_(std::move(impl)) {}
CompiledDecoderLLM::~CompiledDecoderLLM() = default;

std::string CompiledDecoderLLM::reset() {
  for (auto& state : impl_->states) {
    const auto error = state->reset(*impl_->runtime);
    if (!error.empty()) return error;
  }
  return {};
}

DecoderLLMRunResult CompiledDecoderLLM::prefill(const std::vector<float>& tokenIds,
                                                bool readLogits) {
  DecoderLLMRunResult result;
  if (currentLength() != 0) {
    result.errorMessage = "Decoder prefill requires an empty cache; call reset first.";
    return result;
  }
  if (tokenIds.empty() || tokenIds.size() > impl_->plan.attention.capacity) {
    result.errorMessage = "Decoder prefill length is outside the cache capacity.";
    return result;
  }
  double gpu = 0.0;
  bool timed = true;
  for (std::size_t i = 0; i < tokenIds.size(); ++i) {
    auto step = impl_->step(tokenIds[i], readLogits);
    if (!step.passed) {
      (void)reset();
      return step;
    }
    if (readLogits)
      result.logits.insert(result.logits.end(), step.logits.begin(), step.logits.end());
    result.nextTokenIds = step.nextTokenIds;
    result.cpuSubmitToCompletionTimeUs += step.cpuSubmitToCompletionTimeUs;
    if (step.gpuExecutionTimeUs) gpu += *step.gpuExecutionTimeUs; else timed = false;
  }
  if (timed) result.gpuExecutionTimeUs = gpu;
  result.passed = true;
  return result;
}

DecoderLLMRunResult CompiledDecoderLLM::prefillChunked(const std::vector<float>& tokenIds,
                                                       bool readLogits) {
  DecoderLLMRunResult result;
  if (currentLength() != 0) {
    result.errorMessage = "Chunked decoder prefill requires an empty cache; call reset first.";
    return result;
  }
  if (!impl_->prefillExecutor) {
    result.errorMessage = "Chunked decoder prefill was not compiled.";
    return result;
  }
  if (tokenIds.empty() || tokenIds.size() > impl_->plan.attention.capacity) {
    result.errorMessage = "Decoder prefill length is outside the cache capacity.";
    return result;
  }
  auto& executor = *impl_->prefillExecutor;
  const std::size_t chunk = executor.chunkSize();
  double gpu = 0.0;
  bool timed = true;
  for (std::size_t offset = 0; offset < tokenIds.size();) {
    const std::size_t count = std::min(chunk, tokenIds.size() - offset);
    const std::size_t start = currentLength();
    auto error = impl_->stage(start + count);
    if (!error.empty()) {
      (void)reset();
      result.errorMessage = error;
      return result;
    }
    std::vector<std::int32_t> tokens(count);
    for (std::size_t i = 0; i < count; ++i)
      tokens[i] = static_cast<std::int32_t>(tokenIds[offset + i]);
    std::vector<std::vector<std::int32_t>> tables;
    for (const auto& state : impl_->states) {
      auto table = state->pageTable();
      table.resize(executor.maxPages(), -1);
      tables.push_back(std::move(table));
    }
    const auto run = executor.run(tokens, start, tables, readLogits, true);
    if (!run.passed) {
      (void)reset();
      result.errorMessage = run.errorMessage;
      return result;
    }
    for (auto& state : impl_->states) state->commitLength(start + count);
    if (readLogits) result.logits.insert(result.logits.end(), run.logits.begin(), run.logits.end());
    result.nextTokenIds = run.nextTokenIds;
    result.cpuSubmitToCompletionTimeUs += run.cpuSubmitToCompletionTimeUs;
    if (run.gpuExecutionTimeUs) gpu += *run.gpuExecutionTimeUs; else timed = false;
    offset += count;
  }
  if (timed) result.gpuExecutionTimeUs = gpu;
  result.passed = true;
  return result;
}

std::size_t CompiledDecoderLLM::prefillChunkSize() const noexcept {
  return impl_->prefillExecutor ? impl_->prefillExecutor->chunkSize() : 0;
}

DecoderLLMRunResult CompiledDecoderLLM::decode(const std::vector<float>& tokenIds,
                                               bool readLogits) {
  DecoderLLMRunResult result;
  if (currentLength() == 0) {
    result.errorMessage = "Decoder decode requires a completed prefill.";
    return result;
  }
  if (currentLength() >= impl_->plan.attention.capacity) {
    result.errorMessage = "Decoder KV cache capacity has been reached.";
    return result;
  }
  if (tokenIds.size() != 1) {
    result.errorMessage = "Decoder token input shape does not match the compiled stage.";
    return result;
  }
  return impl_->step(tokenIds.front(), readLogits);
}

std::size_t CompiledDecoderLLM::currentLength() const noexcept { return impl_->currentLength(); }

std::vector<float> CompiledDecoderLLM::readKeyPrefix(std::size_t layer) const {
  if (layer >= impl_->states.size()) throw std::out_of_range("Decoder layer index is out of range.");
  return impl_->states[layer]->readKeyPrefix();
}

std::vector<float> CompiledDecoderLLM::readValuePrefix(std::size_t layer) const {
  if (layer >= impl_->states.size()) throw std::out_of_range("Decoder layer index is out of range.");
  return impl_->states[layer]->readValuePrefix();
}

bool CompiledDecoderLLM::cacheStorageReused() const noexcept {
  for (const auto& state : impl_->states)
    if (!state->storageReused()) return false;
  return true;
}

bool CompiledDecoderLLM::usesPagedKVCache() const noexcept { return impl_->requestedPageSize != 0; }

std::size_t CompiledDecoderLLM::kvPageSize() const noexcept { return impl_->requestedPageSize; }

std::size_t CompiledDecoderLLM::allocatedKVPageCount() const noexcept {
  return usesPagedKVCache() && !impl_->states.empty() ? impl_->states.front()->allocatedPageCount()
                                                      : 0;
}

std::size_t CompiledDecoderLLM::modelStorageBytes() const noexcept {
  return impl_->model->storageBytes;
}

std::size_t CompiledDecoderLLM::kvStorageBytes() const noexcept { return impl_->kvBytes; }

std::size_t CompiledDecoderLLM::activationStorageBytes() const noexcept {
  return impl_->executor->activationStorageBytes() +
         (impl_->prefillExecutor ? impl_->prefillExecutor->activationStorageBytes() : 0);
}

std::string CompiledDecoderLLM::kernelUsageReport(bool reset) const {
  std::ostringstream out;
  impl_->registry->report(out);
  if (reset) impl_->registry->resetUsage();
  return out.str();
}

std::shared_ptr<DecoderLLMModelResources> CompiledDecoderLLM::sharedModelResources()
    const noexcept {
  return impl_->model;
}

std::vector<std::int32_t> CompiledDecoderLLM::kvBlockTable(std::size_t layer) const {
  if (layer >= impl_->states.size()) throw std::out_of_range("Decoder layer index is out of range.");
  return impl_->states[layer]->pageTable();
}

DecoderKVSnapshot CompiledDecoderLLM::snapshotKVCache() const {
  DecoderKVSnapshot snapshot;
  snapshot.length = currentLength();
  for (const auto& state : impl_->states) {
    snapshot.keyCaches.push_back(state->readKeyPrefix());
    snapshot.valueCaches.push_back(state->readValuePrefix());
  }
  return snapshot;
}

std::string CompiledDecoderLLM::releaseKVCache() { return reset(); }

std::string CompiledDecoderLLM::restoreKVCache(const DecoderKVSnapshot& snapshot) {
  if (currentLength() != 0) return "Decoder KV restore requires an empty cache.";
  if (snapshot.length == 0 || snapshot.keyCaches.size() != impl_->states.size() ||
      snapshot.valueCaches.size() != impl_->states.size())
    return "Decoder KV snapshot does not match the compiled model.";
  for (std::size_t l = 0; l < impl_->states.size(); ++l) {
    const auto error = impl_->states[l]->restore(*impl_->runtime, snapshot.length,
                                                 snapshot.keyCaches[l], snapshot.valueCaches[l]);
    if (!error.empty()) {
      for (auto& state : impl_->states) (void)state->reset(*impl_->runtime);
      return error;
    }
  }
  return {};
}

std::string CompiledDecoderLLM::stageKVLength(std::size_t length) { return impl_->stage(length); }

void CompiledDecoderLLM::commitKVLength(std::size_t length) {
  for (auto& state : impl_->states) state->commitLength(length);
}

std::string CompiledDecoderLLM::rollbackKVLength(std::size_t length) {
  std::string first;
  for (auto& state : impl_->states) {
    const auto error = state->rollbackLength(*impl_->runtime, length);
    if (first.empty()) first = error;
  }
  return first;
}

DecoderLLMCompilation compileDecoderLLM(hip::HipRuntime& runtime,
                                        const DecoderLLMWorkload& workload, std::ostream& log,
                                        const DecoderLLMCompileOptions& options) {
  DecoderLLMCompilation result;
  try {
    if (!runtime.isAvailable()) throw std::runtime_error(runtime.initializationError());
    if (options.storageDtype != DType::Float16)
      throw std::invalid_argument("The gfx950 decoder path stores weights and caches in fp16.");
    auto impl = std::make_unique<CompiledDecoderLLM::Impl>();
    impl->runtime = &runtime;
    impl->plan = workload.plan;
    impl->plan.attention.dtype = DType::Float16;
    impl->plan.validate();
    if (impl->plan.attention.batch != 1)
      throw std::invalid_argument("CompiledDecoderLLM runs one request; use the batched executor.");
    if (options.sharedModelResources) {
      const auto& shared = options.sharedModelResources;
      if (shared->layerCount != impl->plan.layerCount || shared->hiddenSize != impl->plan.hiddenSize() ||
          shared->headCount != impl->plan.attention.heads ||
          shared->kvHeadCount != impl->plan.kvHeads() ||
          shared->headDimension != impl->plan.attention.headDimension ||
          shared->cacheCapacity != impl->plan.attention.capacity ||
          shared->intermediateSize != impl->plan.intermediateSize ||
          shared->vocabularySize != impl->plan.vocabularySize)
        throw std::invalid_argument("Shared model resources do not match the decoder plan.");
      impl->model = shared;
    } else {
      auto created = createModelResources(runtime, workload);
      if (!created.resources) throw std::runtime_error(created.errorMessage);
      impl->model = std::move(created.resources);
    }
    const auto kvPlan = impl->plan.kvPlan();
    impl->requestedPageSize = options.kvPageSize;
    if (!options.sharedKVPools.empty()) {
      if (options.kvPageSize == 0 || options.sharedKVPools.size() != impl->plan.layerCount)
        throw std::invalid_argument("Shared KV pools need a page size and one pool per layer.");
      for (const auto& pool : options.sharedKVPools)
        if (!pool || pool->pageSize() != options.kvPageSize)
          throw std::invalid_argument("Shared KV pool page size differs from the options.");
      impl->pools = options.sharedKVPools;
    } else {
      // kvPageSize 0: one page of `capacity` tokens, which is the contiguous
      // [heads][capacity][D] layout of the reference's unpaged cache.
      const std::size_t pageSize = options.kvPageSize ? options.kvPageSize : kvPlan.capacity;
      const std::size_t pages = (kvPlan.capacity + pageSize - 1) / pageSize;
      for (std::size_t l = 0; l < impl->plan.layerCount; ++l) {
        auto pool = createKVPagePool(runtime, kvPlan, pageSize, pages);
        if (!pool.pool) throw std::runtime_error(pool.errorMessage);
        impl->kvBytes += 2 * pool.pool->keyBuffer()->storageBytes();
        impl->pools.push_back(std::move(pool.pool));
      }
    }
    for (const auto& pool : impl->pools) {
      auto state = createKVCacheState(runtime, kvPlan, pool, false);
      if (!state.state) throw std::runtime_error(state.errorMessage);
      impl->states.push_back(std::move(state.state));
    }
    impl->registry->load(runtime, options.kernelLibrary, log);
    auto executor =
        createBatchedDecodeExecutor(runtime, impl->model, impl->pools, 1, &log, false, impl->registry);
    if (!executor.executor) throw std::runtime_error(executor.errorMessage);
    impl->executor = std::move(executor.executor);
    if (options.prefillChunkSize != 0) {
      auto prefill = createChunkedPrefillExecutor(runtime, impl->model, impl->pools,
                                                  options.prefillChunkSize, &log);
      if (!prefill.executor) throw std::runtime_error(prefill.errorMessage);
      impl->prefillExecutor = std::move(prefill.executor);
    }
    log << "Decoder compile: layers=" << impl->plan.layerCount
        << ", kv_page_size=" << options.kvPageSize << ", dispatches/token="
        << impl->executor->dispatchesPerStep(1) << '\n';
    result.executable.reset(new CompiledDecoderLLM(std::move(impl)));
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

}  // namespace runtime
}  // namespace tensor
