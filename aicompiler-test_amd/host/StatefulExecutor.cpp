// KV-cache attention module executor; see StatefulExecutor.hpp.
#include "StatefulExecutor.hpp"

#include <ostream>
#include <stdexcept>
#include <utility>

namespace tensor::runtime {
namespace {

using hip::BufferHandle;
using hip::ElementType;

// Row counts up to this run the projections on the decode GEMV; larger
// prompts on the prompt GEMM.
constexpr std::size_t kGemvRows = 16;

BufferHandle makeBuffer(hip::HipRuntime& runtime, std::size_t count, const float* data,
                        ElementType type) {
  auto made = runtime.createBuffer(count, data, type);
  if (!made.buffer) throw std::runtime_error(made.errorMessage);
  return std::move(made.buffer);
}

// One invocation shape (S rows per tensor batch) prepared as a sequence.
struct Stage {
  std::size_t rows = 0;  // batch * S
  BufferHandle query, key, value;                 // inputs [rows, dim]
  BufferHandle queryRows, keyRows, valueRows;     // projections [rows, dim]
  BufferHandle context, output;                   // [rows, dim]
  BufferHandle rowLengths, rowTables, rowCount;   // S > 1 attention metadata
  std::vector<std::unique_ptr<hip::PreparedExecution>> steps;
  std::unique_ptr<hip::PreparedSequence> sequence;
};

Stage buildStage(hip::HipRuntime& runtime, const planner::KVCachePlan& plan, std::size_t S,
                 const BufferHandle& wq, const BufferHandle& wk, const BufferHandle& wv,
                 const BufferHandle& wo, KVCacheState& state, std::ostream& log) {
  const std::size_t B = plan.batch, H = plan.heads, D = plan.headDimension;
  const std::size_t dim = H * D, cap = plan.capacity;
  Stage st;
  st.rows = B * S;
  const auto fp16 = ElementType::Float16;
  for (BufferHandle* b : {&st.query, &st.key, &st.value, &st.queryRows, &st.keyRows, &st.valueRows,
                          &st.context, &st.output})
    *b = makeBuffer(runtime, st.rows * dim, nullptr, fp16);
  const auto add = [&](const std::string& key, const std::vector<BufferHandle>& inputs,
                       const std::vector<BufferHandle>& outputs) {
    const auto pipeline = runtime.createComputePipeline(key, key.substr(0, key.find('?')));
    if (!pipeline.pipelineCreationPassed) throw std::runtime_error(key + ": " + pipeline.errorMessage);
    auto prepared = runtime.prepareBuffers(
        inputs, outputs, {pipeline.threadgroupCount, pipeline.threadsPerThreadgroup});
    if (!prepared.execution) throw std::runtime_error(key + ": " + prepared.errorMessage);
    st.steps.push_back(std::move(prepared.execution));
  };
  const std::string d = std::to_string(dim);
  const std::string gemm = st.rows <= kGemvRows
                               ? "decode_gemv?batch=" + std::to_string(st.rows) + "&in=" + d +
                                     "&out=" + d + "&out_dtype=f16"
                               : "gemm_rows?m=" + std::to_string(st.rows) + "&in=" + d +
                                     "&out=" + d + "&out_dtype=f16";
  const std::string append = "kv_append?batch=" + std::to_string(B) + "&seq=" +
                             std::to_string(S) + "&heads=" + std::to_string(H) +
                             "&head_dim=" + std::to_string(D) + "&capacity=" +
                             std::to_string(cap) + "&head_major=0&dtype=f16";
  add(gemm, {st.query, wq}, {st.queryRows});
  add(gemm, {st.key, wk}, {st.keyRows});
  add(append, {st.keyRows, state.lengthBuffer()}, {state.keyBuffer()});
  add(gemm, {st.value, wv}, {st.valueRows});
  add(append, {st.valueRows, state.lengthBuffer()}, {state.valueBuffer()});
  if (S == 1) {
    add("decode_attention?batch=" + std::to_string(B) + "&q_heads=" + std::to_string(H) +
            "&kv_heads=" + std::to_string(H) + "&head_dim=" + std::to_string(D) + "&capacity=" +
            std::to_string(cap) + "&dtype=f16",
        {st.queryRows, state.keyBuffer(), state.valueBuffer(), state.lengthBuffer()},
        {st.context});
  } else {
    // Every row (b, s) attends all of batch b's cached positions: the cache
    // of batch b is page b of a one-page-per-request pool, and every row's
    // length is the valid length after this call (written per call).
    std::vector<float> tables(st.rows);
    for (std::size_t r = 0; r < st.rows; ++r) tables[r] = static_cast<float>(r / S);
    const float rows = static_cast<float>(st.rows);
    st.rowLengths = makeBuffer(runtime, st.rows, nullptr, ElementType::Int32);
    st.rowTables = makeBuffer(runtime, st.rows, tables.data(), ElementType::Int32);
    st.rowCount = makeBuffer(runtime, 1, &rows, ElementType::Int32);
    add("paged_attention?max_batch=" + std::to_string(st.rows) + "&q_heads=" + std::to_string(H) +
            "&kv_heads=" + std::to_string(H) + "&head_dim=" + std::to_string(D) +
            "&page_size=" + std::to_string(cap) + "&max_pages=1&page_stride=" +
            std::to_string(H * cap * D) + "&head_stride=" + std::to_string(cap * D) + "&dtype=f16",
        {st.queryRows, state.keyBuffer(), state.valueBuffer(), st.rowLengths, st.rowTables,
         st.rowCount},
        {st.context});
  }
  add(gemm, {st.context, wo}, {st.output});
  std::vector<const hip::PreparedExecution*> pointers;
  for (const auto& step : st.steps) pointers.push_back(step.get());
  auto sequence = runtime.prepareSequence(pointers);
  if (!sequence.execution) throw std::runtime_error(sequence.errorMessage);
  st.sequence = std::move(sequence.execution);
  log << "KV attention stage of " << S << " row(s) per batch: " << st.steps.size()
      << " launches (" << gemm.substr(0, gemm.find('?')) << " projections)\n";
  return st;
}

}  // namespace

class CompiledKVCacheAttention::Impl {
 public:
  hip::HipRuntime* runtime = nullptr;
  planner::KVCachePlan plan;
  std::unique_ptr<KVCacheState> state;
  BufferHandle wq, wk, wv, wo;
  Stage prefill, decode;

  // Stage the next length, run the stage and commit; on a failed run the
  // state goes back to its previous length (its pages or rows unchanged).
  KVCacheRunResult run(Stage& st, std::size_t nextLength, const std::vector<float>& q,
                       const std::vector<float>& k, const std::vector<float>& v) {
    KVCacheRunResult out;
    const std::size_t count = st.query->elementCount();
    if (q.size() != count || k.size() != count || v.size() != count) {
      out.errorMessage = "KV cache invocation input shape does not match its compiled plan.";
      return out;
    }
    for (const auto& [buffer, data] : {std::pair{&st.query, &q}, {&st.key, &k}, {&st.value, &v}}) {
      out.errorMessage = runtime->writeBuffer(*buffer, data->data(), data->size());
      if (!out.errorMessage.empty()) return out;
    }
    if (st.rowLengths) {
      const std::vector<float> lengths(st.rows, static_cast<float>(nextLength));
      out.errorMessage = runtime->writeBuffer(st.rowLengths, lengths.data(), lengths.size());
      if (!out.errorMessage.empty()) return out;
    }
    const std::size_t previous = state->currentLength();
    out.errorMessage = state->stageLength(*runtime, nextLength);
    if (!out.errorMessage.empty()) return out;
    const auto execution = st.sequence->execute();
    if (!execution.executionPassed) {
      (void)state->rollbackLength(*runtime, previous);
      out.errorMessage = execution.errorMessage;
      return out;
    }
    state->commitLength(nextLength);
    out.output = st.output->read();
    out.gpuExecutionTimeUs = execution.gpuExecutionTimeUs;
    out.cpuSubmitToCompletionTimeUs = execution.cpuSubmitToCompletionTimeUs;
    out.passed = true;
    return out;
  }
};

CompiledKVCacheAttention::CompiledKVCacheAttention(std::unique_ptr<Impl> impl)
    : impl_(std::move(impl)) {}
CompiledKVCacheAttention::~CompiledKVCacheAttention() = default;

std::string CompiledKVCacheAttention::reset() { return impl_->state->reset(*impl_->runtime); }

KVCacheRunResult CompiledKVCacheAttention::prefill(const std::vector<float>& query,
                                                   const std::vector<float>& key,
                                                   const std::vector<float>& value) {
  if (impl_->state->currentLength() != 0) {
    KVCacheRunResult refused;
    refused.errorMessage = "Prefill requires an empty KV cache; call reset first.";
    return refused;
  }
  return impl_->run(impl_->prefill, impl_->plan.prefillLength, query, key, value);
}

KVCacheRunResult CompiledKVCacheAttention::decode(const std::vector<float>& query,
                                                  const std::vector<float>& key,
                                                  const std::vector<float>& value) {
  const std::size_t current = impl_->state->currentLength();
  KVCacheRunResult refused;
  if (current == 0) refused.errorMessage = "Decode requires a completed prefill.";
  else if (current >= impl_->plan.capacity) refused.errorMessage = "KV cache capacity has been reached.";
  if (!refused.errorMessage.empty()) return refused;
  return impl_->run(impl_->decode, current + 1, query, key, value);
}

std::size_t CompiledKVCacheAttention::currentLength() const noexcept {
  return impl_->state->currentLength();
}
std::vector<float> CompiledKVCacheAttention::readKeyPrefix() const {
  return impl_->state->readKeyPrefix();
}
std::vector<float> CompiledKVCacheAttention::readValuePrefix() const {
  return impl_->state->readValuePrefix();
}
bool CompiledKVCacheAttention::cacheStorageReused() const noexcept {
  return impl_->state->storageReused();
}

KVCacheCompilation compileKVCacheAttention(hip::HipRuntime& runtime,
                                           const planner::KVCachePlan& plan,
                                           const std::vector<float>& queryWeight,
                                           const std::vector<float>& keyWeight,
                                           const std::vector<float>& valueWeight,
                                           const std::vector<float>& outputWeight,
                                           std::ostream& log) {
  KVCacheCompilation result;
  try {
    plan.validate();
    if (!runtime.isAvailable()) throw std::runtime_error(runtime.initializationError());
    if (plan.dtype == DType::BFloat16)
      throw std::invalid_argument("The gfx950 KV attention module stores fp16 (or fp32 plans as fp16).");
    const std::size_t weights = plan.modelDimension() * plan.modelDimension();
    for (const auto* w : {&queryWeight, &keyWeight, &valueWeight, &outputWeight})
      if (w->size() != weights)
        throw std::invalid_argument("KV cache projection weight shape is invalid.");
    auto impl = std::make_unique<CompiledKVCacheAttention::Impl>();
    impl->runtime = &runtime;
    impl->plan = plan;
    impl->plan.dtype = DType::Float16;
    auto state = createKVCacheState(runtime, impl->plan);
    if (!state.state) throw std::runtime_error(state.errorMessage);
    impl->state = std::move(state.state);
    const auto fp16 = ElementType::Float16;
    impl->wq = makeBuffer(runtime, weights, queryWeight.data(), fp16);
    impl->wk = makeBuffer(runtime, weights, keyWeight.data(), fp16);
    impl->wv = makeBuffer(runtime, weights, valueWeight.data(), fp16);
    impl->wo = makeBuffer(runtime, weights, outputWeight.data(), fp16);
    impl->prefill = buildStage(runtime, impl->plan, impl->plan.prefillLength, impl->wq, impl->wk,
                               impl->wv, impl->wo, *impl->state, log);
    impl->decode = buildStage(runtime, impl->plan, 1, impl->wq, impl->wk, impl->wv, impl->wo,
                              *impl->state, log);
    result.executable.reset(new CompiledKVCacheAttention(std::move(impl)));
    log << "KV attention module compiled: heads=" << plan.heads << ", head_dim="
        << plan.headDimension << ", capacity=" << plan.capacity << ", prefill="
        << plan.prefillLength << " (fp16 cache)\n";
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

}  // namespace tensor::runtime
