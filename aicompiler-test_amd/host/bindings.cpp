// Python module _tmc_host: the C++ host layer (HipRuntime, KV pools and
// states, the decoder executors and the serving loop) for tests and the
// benchmark.  Names follow the C++ classes; weights and logits cross as numpy
// float32 arrays.
#include <pybind11/functional.h>
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <sstream>

#include "Benchmark.hpp"
#include "DecoderLLM.hpp"
#include "GraphExecutor.hpp"
#include "Importer.hpp"
#include "KVCacheState.hpp"
#include "ServingRuntime.hpp"
#include "StatefulExecutor.hpp"
#include "Tuning.hpp"

namespace py = pybind11;
using namespace tensor;
using namespace tensor::runtime;

namespace {

using FloatArray = py::array_t<float, py::array::c_style | py::array::forcecast>;

std::vector<float> toVector(const FloatArray& a) {
  return std::vector<float>(a.data(), a.data() + a.size());
}

py::array_t<float> toArray(const std::vector<float>& v) {
  py::array_t<float> out(static_cast<py::ssize_t>(v.size()));
  std::copy(v.begin(), v.end(), out.mutable_data());
  return out;
}

py::array_t<double> toArray(const std::vector<double>& v) {
  py::array_t<double> out(static_cast<py::ssize_t>(v.size()));
  std::copy(v.begin(), v.end(), out.mutable_data());
  return out;
}

py::list toArrays(const std::vector<std::vector<double>>& vs) {
  py::list out;
  for (const auto& v : vs) out.append(toArray(v));
  return out;
}

template <typename T, typename Field>
void weightProperty(py::class_<T>& cls, const char* name, Field T::*field) {
  cls.def_property(
      name, [field](const T& self) { return toArray(self.*field); },
      [field](T& self, const FloatArray& a) { self.*field = toVector(a); });
}

py::dict runToDict(const BatchedDecodeRun& run) {
  py::dict d;
  d["passed"] = run.passed;
  d["logits"] = toArray(run.logits);
  d["next_token_ids"] = run.nextTokenIds;
  d["gpu_us"] = run.gpuExecutionTimeUs ? py::cast(*run.gpuExecutionTimeUs) : py::none();
  d["cpu_us"] = run.cpuSubmitToCompletionTimeUs;
  d["error"] = run.errorMessage;
  return d;
}

py::dict resultToDict(const DecoderLLMRunResult& run) {
  py::dict d;
  d["passed"] = run.passed;
  d["logits"] = toArray(run.logits);
  d["next_token_ids"] = run.nextTokenIds;
  d["gpu_us"] = run.gpuExecutionTimeUs ? py::cast(*run.gpuExecutionTimeUs) : py::none();
  d["cpu_us"] = run.cpuSubmitToCompletionTimeUs;
  d["error"] = run.errorMessage;
  return d;
}

py::dict statsToDict(const benchmark::Statistics& s) {
  py::dict d;
  d["samples"] = s.samples;
  d["median_us"] = s.medianUs;
  d["p90_us"] = s.p90Us;
  d["min_us"] = s.minUs;
  d["max_us"] = s.maxUs;
  return d;
}

py::dict servingToDict(const ServingExecutionResult& r) {
  py::dict d;
  d["passed"] = r.passed;
  d["error"] = r.errorMessage;
  py::list requests;
  for (const auto& out : r.requests) {
    py::dict q;
    q["id"] = out.id;
    q["prefill_logits"] = toArray(out.prefillLogits);
    py::list logits;
    for (const auto& l : out.decodeLogits) logits.append(toArray(l));
    q["decode_logits"] = logits;
    q["generated_token_ids"] = out.generatedTokenIds;
    q["ttft_us"] = out.timeToFirstTokenUs;
    requests.append(q);
  }
  d["requests"] = requests;
  const auto& m = r.metrics;
  py::dict metrics;
  metrics["decode_gpu"] = statsToDict(m.decodeGpu);
  metrics["decode_end_to_end"] = statsToDict(m.decodeEndToEnd);
  metrics["total_time_us"] = m.totalTimeUs;
  metrics["tokens_per_second"] = m.tokensPerSecond;
  metrics["decode_phase_tokens_per_second"] = m.decodePhaseTokensPerSecond;
  metrics["scheduler_overhead_us"] = m.schedulerOverheadUs;
  metrics["kv_management_overhead_us"] = m.kvManagementOverheadUs;
  metrics["preemption_overhead_us"] = m.preemptionOverheadUs;
  metrics["average_active_batch_size"] = m.averageActiveBatchSize;
  metrics["maximum_active_batch_size"] = m.maximumActiveBatchSize;
  metrics["preemption_count"] = m.preemptionCount;
  metrics["spilled_bytes"] = m.spilledBytes;
  metrics["resume_count"] = m.resumeCount;
  metrics["peak_pages_per_layer"] = m.peakPagesPerLayer;
  metrics["page_allocation_count"] = m.pageAllocationCount;
  metrics["page_release_count"] = m.pageReleaseCount;
  metrics["decode_command_submissions"] = m.decodeCommandSubmissions;
  metrics["prefill_chunk_submissions"] = m.prefillChunkSubmissions;
  metrics["decoded_tokens"] = m.decodedTokens;
  metrics["prompt_tokens"] = m.promptTokens;
  metrics["model_storage_bytes"] = m.modelStorageBytes;
  metrics["kv_pool_storage_bytes"] = m.kvPoolStorageBytes;
  metrics["batched_activation_storage_bytes"] = m.batchedActivationStorageBytes;
  d["metrics"] = metrics;
  return d;
}

OpAttributes toAttributes(const py::object& o) {
  if (o.is_none()) return std::monostate{};
  if (py::isinstance<RMSNormAttributes>(o)) return o.cast<RMSNormAttributes>();
  if (py::isinstance<ReshapeAttributes>(o)) return o.cast<ReshapeAttributes>();
  if (py::isinstance<TransposeAttributes>(o)) return o.cast<TransposeAttributes>();
  if (py::isinstance<SoftmaxAttributes>(o)) return o.cast<SoftmaxAttributes>();
  throw std::invalid_argument("Unsupported attribute object.");
}

GraphInputs toGraphInputs(const py::dict& d) {
  GraphInputs in;
  for (const auto& item : d) {
    const auto values = py::array_t<float, py::array::c_style | py::array::forcecast>::ensure(item.second);
    if (!values) throw std::invalid_argument("Graph input values must be a float sequence.");
    in[item.first.cast<ValueId>()] = std::vector<float>(values.data(), values.data() + values.size());
  }
  return in;
}

py::dict graphResultDict(const runtime::GraphExecutionResult& r) {
  py::dict d;
  d["passed"] = r.passed;
  d["outputs"] = r.outputs;
  d["gpu_us"] = r.gpuExecutionTimeUs ? py::cast(*r.gpuExecutionTimeUs) : py::none();
  d["error"] = r.errorMessage;
  return d;
}

}  // namespace

PYBIND11_MODULE(_tmc_host, m) {
  m.doc() = "C++ host layer of the gfx950 decode backend.";

  py::enum_<DType>(m, "DType")
      .value("Float16", DType::Float16)
      .value("Float32", DType::Float32)
      .value("BFloat16", DType::BFloat16)
      .value("Int32", DType::Int32);

  py::class_<hip::HipRuntime>(m, "HipRuntime")
      .def(py::init<>())
      .def("is_available", &hip::HipRuntime::isAvailable)
      .def("device_name", &hip::HipRuntime::deviceName)
      .def("initialization_error", &hip::HipRuntime::initializationError)
      .def("hardware_info",
           [](const hip::HipRuntime& rt) {
             const auto h = rt.hardwareInfo();
             py::dict d;
             d["max_threads_per_threadgroup"] = h.maxThreadsPerThreadgroup;
             d["max_threadgroup_memory_length"] = h.maxThreadgroupMemoryLength;
             d["max_buffer_length"] = h.maxBufferLength;
             d["supports_bfloat16"] = h.supportsBFloat16;
             d["compute_units"] = h.computeUnits;
             d["wave_size"] = h.waveSize;
             return d;
           })
      .def("synchronize", &hip::HipRuntime::synchronize)
      .def("fail_next", &hip::HipRuntime::failNext)
      .def("stream", [](const hip::HipRuntime& rt) {
        return reinterpret_cast<std::uintptr_t>(rt.stream());
      });

  py::class_<planner::KVCachePlan>(m, "KVCachePlan")
      .def(py::init<>())
      .def_readwrite("batch", &planner::KVCachePlan::batch)
      .def_readwrite("heads", &planner::KVCachePlan::heads)
      .def_readwrite("head_dimension", &planner::KVCachePlan::headDimension)
      .def_readwrite("capacity", &planner::KVCachePlan::capacity)
      .def_readwrite("prefill_length", &planner::KVCachePlan::prefillLength)
      .def_readwrite("dtype", &planner::KVCachePlan::dtype)
      .def_readwrite("threads_per_threadgroup", &planner::KVCachePlan::threadsPerThreadgroup)
      .def("validate", &planner::KVCachePlan::validate);

  py::class_<planner::DecoderLLMPlan>(m, "DecoderLLMPlan")
      .def(py::init<>())
      .def_readwrite("attention", &planner::DecoderLLMPlan::attention)
      .def_readwrite("layer_count", &planner::DecoderLLMPlan::layerCount)
      .def_readwrite("intermediate_size", &planner::DecoderLLMPlan::intermediateSize)
      .def_readwrite("vocabulary_size", &planner::DecoderLLMPlan::vocabularySize)
      .def_readwrite("rms_norm_epsilon", &planner::DecoderLLMPlan::rmsNormEpsilon)
      .def_readwrite("key_value_heads", &planner::DecoderLLMPlan::keyValueHeads)
      .def("hidden_size", &planner::DecoderLLMPlan::hiddenSize)
      .def("kv_heads", &planner::DecoderLLMPlan::kvHeads)
      .def("validate", &planner::DecoderLLMPlan::validate)
      .def("kv_plan", &planner::DecoderLLMPlan::kvPlan);

  py::class_<KVPagePool, std::shared_ptr<KVPagePool>>(m, "KVPagePool")
      .def("page_size", &KVPagePool::pageSize)
      .def("capacity_pages", &KVPagePool::capacityPages)
      .def("used_pages", &KVPagePool::usedPages)
      .def("available_pages", &KVPagePool::availablePages)
      .def("peak_used_pages", &KVPagePool::peakUsedPages)
      .def("allocation_count", &KVPagePool::allocationCount)
      .def("release_count", &KVPagePool::releaseCount)
      .def("has_storage", &KVPagePool::hasStorage)
      .def("page_elements", &KVPagePool::pageElements)
      .def("key_pointer",
           [](const KVPagePool& p) {
             return p.keyBuffer() ? reinterpret_cast<std::uintptr_t>(p.keyBuffer()->devicePointer())
                                  : std::uintptr_t{0};
           })
      .def("value_pointer", [](const KVPagePool& p) {
        return p.valueBuffer() ? reinterpret_cast<std::uintptr_t>(p.valueBuffer()->devicePointer())
                               : std::uintptr_t{0};
      });

  m.def("create_kv_page_pool",
        [](hip::HipRuntime& rt, const planner::KVCachePlan& plan, std::size_t pageSize,
           std::size_t pages) -> py::object {
          auto r = createKVPagePool(rt, plan, pageSize, pages);
          if (!r.pool) throw std::runtime_error(r.errorMessage);
          return py::cast(r.pool);
        });
  m.def("create_host_kv_page_pool",
        [](const planner::KVCachePlan& plan, std::size_t pageSize, std::size_t pages) {
          auto r = createHostKVPagePool(plan, pageSize, pages);
          if (!r.pool) throw std::runtime_error(r.errorMessage);
          return r.pool;
        });

  py::class_<KVPageSpill>(m, "KVPageSpill")
      .def_readonly("length", &KVPageSpill::length)
      .def_readonly("pages", &KVPageSpill::pages)
      .def_readonly("page_bytes", &KVPageSpill::pageBytes)
      .def("bytes", &KVPageSpill::bytes);

  py::class_<KVCacheState>(m, "KVCacheState")
      .def("spill_pages",
           [](const KVCacheState& s, hip::HipRuntime& rt) {
             KVPageSpill spill;
             const auto error = s.spillPages(rt, spill);
             if (!error.empty()) throw std::runtime_error(error);
             return spill;
           })
      .def("restore_pages", &KVCacheState::restorePages)
      .def("current_length", &KVCacheState::currentLength)
      .def("capacity", &KVCacheState::capacity)
      .def("reset", &KVCacheState::reset)
      .def("stage_length", &KVCacheState::stageLength)
      .def("rollback_length", &KVCacheState::rollbackLength)
      .def("restore",
           [](KVCacheState& s, hip::HipRuntime& rt, std::size_t length, const FloatArray& k,
              const FloatArray& v) { return s.restore(rt, length, toVector(k), toVector(v)); })
      .def("commit_length", &KVCacheState::commitLength)
      .def("read_key_prefix", [](const KVCacheState& s) { return toArray(s.readKeyPrefix()); })
      .def("read_value_prefix", [](const KVCacheState& s) { return toArray(s.readValuePrefix()); })
      .def("storage_reused", &KVCacheState::storageReused)
      .def("is_paged", &KVCacheState::isPaged)
      .def("page_size", &KVCacheState::pageSize)
      .def("allocated_page_count", &KVCacheState::allocatedPageCount)
      .def("page_table", &KVCacheState::pageTable)
      .def("has_device_mirror", [](const KVCacheState& s) { return s.blockTableBuffer() != nullptr; })
      .def("read_device_table",
           [](const KVCacheState& s) {
             std::vector<std::int32_t> out;
             if (!s.blockTableBuffer()) return out;
             out.resize(s.blockTableBuffer()->elementCount());
             const auto error = s.blockTableBuffer()->readRaw(out.data(), out.size());
             if (!error.empty()) throw std::runtime_error(error);
             return out;
           })
      .def("read_device_length", [](const KVCacheState& s) {
        std::int32_t value = -1;
        if (!s.lengthBuffer()) return value;
        const auto error = s.lengthBuffer()->readRaw(&value, 1);
        if (!error.empty()) throw std::runtime_error(error);
        return value;
      });

  m.def("create_kv_cache_state",
        [](hip::HipRuntime& rt, const planner::KVCachePlan& plan, std::shared_ptr<KVPagePool> pool,
           bool mirror) {
          auto r = createKVCacheState(rt, plan, std::move(pool), mirror);
          if (!r.state) throw std::runtime_error(r.errorMessage);
          return std::move(r.state);
        },
        py::arg("runtime"), py::arg("plan"), py::arg("pool"), py::arg("device_mirror") = true);
  m.def("create_private_kv_cache_state",
        [](hip::HipRuntime& rt, const planner::KVCachePlan& plan, std::size_t pageSize) {
          auto r = createKVCacheState(rt, plan, pageSize);
          if (!r.state) throw std::runtime_error(r.errorMessage);
          return std::move(r.state);
        });

  py::class_<DecoderLLMLayerParameters> layer(m, "DecoderLLMLayerParameters");
  layer.def(py::init<>());
  weightProperty(layer, "input_norm_weight", &DecoderLLMLayerParameters::inputNormWeight);
  weightProperty(layer, "query_weight", &DecoderLLMLayerParameters::queryWeight);
  weightProperty(layer, "key_weight", &DecoderLLMLayerParameters::keyWeight);
  weightProperty(layer, "value_weight", &DecoderLLMLayerParameters::valueWeight);
  weightProperty(layer, "output_weight", &DecoderLLMLayerParameters::outputWeight);
  weightProperty(layer, "post_attention_norm_weight",
                 &DecoderLLMLayerParameters::postAttentionNormWeight);
  weightProperty(layer, "gate_weight", &DecoderLLMLayerParameters::gateWeight);
  weightProperty(layer, "up_weight", &DecoderLLMLayerParameters::upWeight);
  weightProperty(layer, "down_weight", &DecoderLLMLayerParameters::downWeight);

  py::class_<DecoderLLMWorkload> workload(m, "DecoderLLMWorkload");
  workload.def(py::init<>())
      .def_readwrite("model_name", &DecoderLLMWorkload::modelName)
      .def_readwrite("plan", &DecoderLLMWorkload::plan)
      .def_readwrite("decode_count", &DecoderLLMWorkload::decodeCount)
      .def_readwrite("layers", &DecoderLLMWorkload::layers);
  weightProperty(workload, "embedding_weight", &DecoderLLMWorkload::embeddingWeight);
  weightProperty(workload, "final_norm_weight", &DecoderLLMWorkload::finalNormWeight);
  weightProperty(workload, "language_model_head_weight", &DecoderLLMWorkload::languageModelHeadWeight);
  weightProperty(workload, "rope_cosine", &DecoderLLMWorkload::ropeCosine);
  weightProperty(workload, "rope_sine", &DecoderLLMWorkload::ropeSine);
  workload.def_readwrite("requested_storage_dtype", &DecoderLLMWorkload::requestedStorageDtype)
      .def_readonly("prefill", &DecoderLLMWorkload::prefill)
      .def_readonly("decode_steps", &DecoderLLMWorkload::decodeSteps);

  py::class_<DecoderLLMReference>(m, "DecoderLLMReference")
      .def_property_readonly("token_ids", [](const DecoderLLMReference& r) { return toArray(r.tokenIds); })
      .def_property_readonly("logits", [](const DecoderLLMReference& r) { return toArray(r.logits); })
      .def_property_readonly("next_token_ids",
                             [](const DecoderLLMReference& r) { return toArray(r.nextTokenIds); })
      .def_property_readonly("key_caches", [](const DecoderLLMReference& r) { return toArrays(r.keyCaches); })
      .def_property_readonly("value_caches",
                             [](const DecoderLLMReference& r) { return toArrays(r.valueCaches); });

  // importDecoderLLMWorkload / importKVCacheWorkload: (workload or None, error).
  m.def("import_decoder_llm_workload", [](const std::string& path) {
    auto r = importer::importDecoderLLMWorkload(path);
    return py::make_tuple(r.workload ? py::cast(std::move(r.workload)) : py::none(), r.errorMessage);
  });
  py::class_<importer::KVCacheReferenceStep>(m, "KVCacheReferenceStep")
      .def_property_readonly("query", [](const importer::KVCacheReferenceStep& s) { return toArray(s.query); })
      .def_property_readonly("key", [](const importer::KVCacheReferenceStep& s) { return toArray(s.key); })
      .def_property_readonly("value", [](const importer::KVCacheReferenceStep& s) { return toArray(s.value); })
      .def_property_readonly("output", [](const importer::KVCacheReferenceStep& s) { return toArray(s.output); })
      .def_property_readonly("key_cache",
                             [](const importer::KVCacheReferenceStep& s) { return toArray(s.keyCache); })
      .def_property_readonly("value_cache",
                             [](const importer::KVCacheReferenceStep& s) { return toArray(s.valueCache); });
  py::class_<importer::ImportedKVCacheWorkload>(m, "ImportedKVCacheWorkload")
      .def_readonly("model_name", &importer::ImportedKVCacheWorkload::modelName)
      .def_readonly("plan", &importer::ImportedKVCacheWorkload::plan)
      .def_property_readonly("query_weight",
                             [](const importer::ImportedKVCacheWorkload& w) { return toArray(w.queryWeight); })
      .def_property_readonly("key_weight",
                             [](const importer::ImportedKVCacheWorkload& w) { return toArray(w.keyWeight); })
      .def_property_readonly("value_weight",
                             [](const importer::ImportedKVCacheWorkload& w) { return toArray(w.valueWeight); })
      .def_property_readonly("output_weight",
                             [](const importer::ImportedKVCacheWorkload& w) { return toArray(w.outputWeight); })
      .def_readonly("prefill", &importer::ImportedKVCacheWorkload::prefill)
      .def_readonly("decode_steps", &importer::ImportedKVCacheWorkload::decodeSteps);
  m.def("import_kv_cache_workload", [](const std::string& path) {
    auto r = importer::importKVCacheWorkload(path);
    return py::make_tuple(r.workload ? py::cast(std::move(r.workload)) : py::none(), r.errorMessage);
  });

  m.def("rope_tables", [](std::size_t capacity, std::size_t headDimension, double theta) {
    std::vector<float> c, s;
    ropeTables(capacity, headDimension, theta, c, s);
    return py::make_tuple(toArray(c), toArray(s));
  });

  py::class_<DecoderLLMModelResources, std::shared_ptr<DecoderLLMModelResources>>(
      m, "DecoderLLMModelResources")
      .def_readonly("storage_bytes", &DecoderLLMModelResources::storageBytes)
      .def_readonly("layer_count", &DecoderLLMModelResources::layerCount)
      .def_readonly("hidden_size", &DecoderLLMModelResources::hiddenSize)
      .def_readonly("vocabulary_size", &DecoderLLMModelResources::vocabularySize)
      .def_readonly("plan", &DecoderLLMModelResources::plan);

  m.def("create_model_resources", [](hip::HipRuntime& rt, const DecoderLLMWorkload& w) {
    auto r = createModelResources(rt, w);
    if (!r.resources) throw std::runtime_error(r.errorMessage);
    return r.resources;
  });
  m.def("create_synthetic_model_resources",
        [](hip::HipRuntime& rt, const planner::DecoderLLMPlan& plan, std::uint64_t seed,
           float stddev, double theta) {
          auto r = createSyntheticModelResources(rt, plan, seed, stddev, theta);
          if (!r.resources) throw std::runtime_error(r.errorMessage);
          return r.resources;
        },
        py::arg("runtime"), py::arg("plan"), py::arg("seed"), py::arg("stddev") = 0.02f,
        py::arg("theta") = 10000.0);

  py::class_<BatchedDecodeExecutor>(m, "BatchedDecodeExecutor")
      .def("run",
           [](BatchedDecodeExecutor& e, const std::vector<std::int32_t>& tokens,
              const std::vector<std::int32_t>& lengths,
              const std::vector<std::vector<std::int32_t>>& tables, bool readLogits, bool timeGpu) {
             BatchedDecodeRun run;
             {
               py::gil_scoped_release release;
               run = e.run(tokens, lengths, tables, readLogits, timeGpu);
             }
             return runToDict(run);
           },
           py::arg("tokens"), py::arg("valid_lengths"), py::arg("tables"),
           py::arg("read_logits") = true, py::arg("time_gpu") = false)
      .def("maximum_batch_size", &BatchedDecodeExecutor::maximumBatchSize)
      .def("max_pages", &BatchedDecodeExecutor::maxPages)
      .def("buckets", &BatchedDecodeExecutor::buckets)
      .def("dispatches_per_step", &BatchedDecodeExecutor::dispatchesPerStep)
      .def("activation_storage_bytes", &BatchedDecodeExecutor::activationStorageBytes)
      .def("set_token_only_policy",
           [](BatchedDecodeExecutor& e, const std::string& policy) {
             using P = BatchedDecodeExecutor::TokenOnlyPolicy;
             if (policy == "admission") e.setTokenOnlyPolicy(P::Admission);
             else if (policy == "always") e.setTokenOnlyPolicy(P::Always);
             else if (policy == "never") e.setTokenOnlyPolicy(P::Never);
             else if (policy == "cached_only") e.setTokenOnlyPolicy(P::CachedOnly);
             else throw std::invalid_argument("policy: admission | always | never | cached_only");
           })
      .def("admit_token_only",
           [](BatchedDecodeExecutor& e, const std::vector<std::int32_t>& tokens,
              const std::vector<std::int32_t>& lengths,
              const std::vector<std::vector<std::int32_t>>& tables) {
             std::string error;
             {
               py::gil_scoped_release release;
               error = e.admitTokenOnly(tokens, lengths, tables);
             }
             if (!error.empty()) throw std::runtime_error(error);
           })
      .def("token_only_status", [](const BatchedDecodeExecutor& e, std::size_t rows) {
        const auto st = e.tokenOnlyStatus(rows);
        py::dict d;
        d["available"] = st.available;
        d["checked"] = st.checked;
        d["admitted"] = st.admitted;
        d["speedup"] = st.speedup;
        return d;
      })
      .def("reserve_history",
           [](BatchedDecodeExecutor& e, std::size_t steps) {
             const auto error = e.reserveHistory(steps);
             if (!error.empty()) throw std::runtime_error(error);
           })
      .def("launch_chained",
           [](BatchedDecodeExecutor& e, const std::vector<std::int32_t>& tokens,
              const std::vector<std::int32_t>& lengths,
              const std::vector<std::vector<std::int32_t>>& tables, std::size_t step) {
             std::string error;
             {
               py::gil_scoped_release release;
               error = e.launchChained(tokens, lengths, tables, step);
             }
             if (!error.empty()) throw std::runtime_error(error);
           })
      .def("read_history", [](const BatchedDecodeExecutor& e, std::size_t steps) {
        std::vector<std::int32_t> out;
        const auto error = e.readHistory(steps, out);
        if (!error.empty()) throw std::runtime_error(error);
        return out;
      });

  m.def("create_batched_decode_executor",
        [](hip::HipRuntime& rt, std::shared_ptr<DecoderLLMModelResources> model,
           std::vector<std::shared_ptr<KVPagePool>> pools, std::size_t maxBatch, bool tune,
           bool foldNorms, bool fuseAttentionOutput) {
          std::ostringstream log;
          auto r = createBatchedDecodeExecutor(rt, std::move(model), std::move(pools), maxBatch,
                                               &log, tune, nullptr, foldNorms,
                                               fuseAttentionOutput);
          if (!r.executor) throw std::runtime_error(r.errorMessage + "\n" + log.str());
          return std::move(r.executor);
        },
        py::arg("runtime"), py::arg("model"), py::arg("pools"), py::arg("maximum_batch_size"),
        py::arg("tune_kernels") = false, py::arg("fold_norms") = true,
        py::arg("fuse_attention_output") = false);
  py::class_<ChunkedPrefillExecutor>(m, "ChunkedPrefillExecutor")
      .def("run",
           [](ChunkedPrefillExecutor& e, const std::vector<std::int32_t>& tokens, std::size_t start,
              const std::vector<std::vector<std::int32_t>>& tables, bool readLogits, bool timeGpu) {
             BatchedDecodeRun run;
             {
               py::gil_scoped_release release;
               run = e.run(tokens, start, tables, readLogits, timeGpu);
             }
             return runToDict(run);
           },
           py::arg("tokens"), py::arg("start"), py::arg("tables"), py::arg("read_logits") = true,
           py::arg("time_gpu") = false)
      .def("run_batch",
           [](ChunkedPrefillExecutor& e, const std::vector<py::tuple>& segments, bool readLogits,
              bool timeGpu) {
             std::vector<PrefillSegment> segs;
             for (const auto& t : segments)
               segs.push_back(PrefillSegment{t[0].cast<std::vector<std::int32_t>>(),
                                             t[1].cast<std::size_t>(),
                                             t[2].cast<std::vector<std::vector<std::int32_t>>>()});
             BatchedDecodeRun run;
             {
               py::gil_scoped_release release;
               run = e.runBatch(segs, readLogits, timeGpu);
             }
             return runToDict(run);
           },
           py::arg("segments"), py::arg("read_logits") = false, py::arg("time_gpu") = false)
      .def("maximum_requests", &ChunkedPrefillExecutor::maximumRequests)
      .def("tile_rows", &ChunkedPrefillExecutor::tileRows)
      .def("packed_rows", &ChunkedPrefillExecutor::packedRows)
      .def("chunk_size", &ChunkedPrefillExecutor::chunkSize)
      .def("max_pages", &ChunkedPrefillExecutor::maxPages)
      .def("buckets", &ChunkedPrefillExecutor::buckets)
      .def("dispatches_per_chunk", &ChunkedPrefillExecutor::dispatchesPerChunk)
      .def("activation_storage_bytes", &ChunkedPrefillExecutor::activationStorageBytes);

  m.def("create_chunked_prefill_executor",
        [](hip::HipRuntime& rt, std::shared_ptr<DecoderLLMModelResources> model,
           std::vector<std::shared_ptr<KVPagePool>> pools, std::size_t chunkSize,
           std::size_t maxRequests) {
          std::ostringstream log;
          auto r = createChunkedPrefillExecutor(rt, std::move(model), std::move(pools), chunkSize,
                                                &log, maxRequests);
          if (!r.executor) throw std::runtime_error(r.errorMessage + "\n" + log.str());
          return std::move(r.executor);
        },
        py::arg("runtime"), py::arg("model"), py::arg("pools"), py::arg("chunk_size"),
        py::arg("maximum_requests") = 1);
  m.def("decode_gemv_cache_size", []() { return planner::decodeGEMVTuningCache().size(); });
  m.def("clear_decode_gemv_cache", []() { planner::decodeGEMVTuningCache().clear(); });

  // Statistics and paired timing over Python samplers (host logic only): a
  // sampler returns microseconds, None (no timestamp) or a str (a failure).
  m.def("summarize_timings", [](const std::vector<double>& values) -> py::object {
    const auto s = benchmark::summarizeTimings(values);
    return s ? py::object(statsToDict(*s)) : py::object(py::none());
  });
  m.def("measure_pair", [](py::function baseline, py::function candidate, std::size_t samples) {
    const auto wrap = [](py::function f) -> benchmark::Sampler {
      return [f](std::string& failure) -> std::optional<double> {
        const py::object r = f();
        if (r.is_none()) return std::nullopt;
        if (py::isinstance<py::str>(r)) {
          failure = r.cast<std::string>();
          return std::nullopt;
        }
        return r.cast<double>();
      };
    };
    const auto r = benchmark::measurePair(wrap(baseline), wrap(candidate), samples);
    py::dict d;
    d["passed"] = r.passed;
    d["error"] = r.errorMessage;
    d["baseline"] = statsToDict(r.baseline);
    d["candidate"] = statsToDict(r.candidate);
    d["speedup"] = r.speedup;
    return d;
  });

  py::class_<DecoderLLMCompileOptions>(m, "DecoderLLMCompileOptions")
      .def(py::init<>())
      .def_readwrite("kv_page_size", &DecoderLLMCompileOptions::kvPageSize)
      .def_readwrite("prefill_chunk_size", &DecoderLLMCompileOptions::prefillChunkSize)
      .def_readwrite("shared_kv_pools", &DecoderLLMCompileOptions::sharedKVPools)
      .def_readwrite("storage_dtype", &DecoderLLMCompileOptions::storageDtype)
      .def_readwrite("shared_model_resources", &DecoderLLMCompileOptions::sharedModelResources)
      .def_readwrite("kernel_library", &DecoderLLMCompileOptions::kernelLibrary);

  py::class_<DecoderKVSnapshot>(m, "DecoderKVSnapshot")
      .def_readonly("length", &DecoderKVSnapshot::length)
      .def("key_cache", [](const DecoderKVSnapshot& s, std::size_t l) { return toArray(s.keyCaches.at(l)); })
      .def("value_cache",
           [](const DecoderKVSnapshot& s, std::size_t l) { return toArray(s.valueCaches.at(l)); });

  py::class_<CompiledDecoderLLM>(m, "CompiledDecoderLLM")
      .def("reset", &CompiledDecoderLLM::reset)
      .def("prefill",
           [](CompiledDecoderLLM& d, const std::vector<float>& tokens, bool readLogits) {
             return resultToDict(d.prefill(tokens, readLogits));
           },
           py::arg("token_ids"), py::arg("read_logits") = true)
      .def("prefill_chunked",
           [](CompiledDecoderLLM& d, const std::vector<float>& tokens, bool readLogits) {
             DecoderLLMRunResult r;
             {
               py::gil_scoped_release release;
               r = d.prefillChunked(tokens, readLogits);
             }
             return resultToDict(r);
           },
           py::arg("token_ids"), py::arg("read_logits") = true)
      .def("prefill_chunk_size", &CompiledDecoderLLM::prefillChunkSize)
      .def("decode",
           [](CompiledDecoderLLM& d, const std::vector<float>& tokens, bool readLogits) {
             return resultToDict(d.decode(tokens, readLogits));
           },
           py::arg("token_ids"), py::arg("read_logits") = true)
      .def("current_length", &CompiledDecoderLLM::currentLength)
      .def("read_key_prefix", [](const CompiledDecoderLLM& d, std::size_t l) { return toArray(d.readKeyPrefix(l)); })
      .def("read_value_prefix",
           [](const CompiledDecoderLLM& d, std::size_t l) { return toArray(d.readValuePrefix(l)); })
      .def("cache_storage_reused", &CompiledDecoderLLM::cacheStorageReused)
      .def("uses_paged_kv_cache", &CompiledDecoderLLM::usesPagedKVCache)
      .def("kv_page_size", &CompiledDecoderLLM::kvPageSize)
      .def("kernel_usage_report", &CompiledDecoderLLM::kernelUsageReport,
           py::arg("reset") = false)
      .def("allocated_kv_page_count", &CompiledDecoderLLM::allocatedKVPageCount)
      .def("model_storage_bytes", &CompiledDecoderLLM::modelStorageBytes)
      .def("kv_storage_bytes", &CompiledDecoderLLM::kvStorageBytes)
      .def("activation_storage_bytes", &CompiledDecoderLLM::activationStorageBytes)
      .def("shared_model_resources", &CompiledDecoderLLM::sharedModelResources)
      .def("kv_block_table", &CompiledDecoderLLM::kvBlockTable)
      .def("snapshot_kv_cache", &CompiledDecoderLLM::snapshotKVCache)
      .def("release_kv_cache", &CompiledDecoderLLM::releaseKVCache)
      .def("restore_kv_cache", &CompiledDecoderLLM::restoreKVCache)
      .def("stage_kv_length", &CompiledDecoderLLM::stageKVLength)
      .def("commit_kv_length", &CompiledDecoderLLM::commitKVLength)
      .def("rollback_kv_length", &CompiledDecoderLLM::rollbackKVLength);

  m.def("compile_decoder_llm",
        [](hip::HipRuntime& rt, const DecoderLLMWorkload& w, const DecoderLLMCompileOptions& o) {
          std::ostringstream log;
          auto r = compileDecoderLLM(rt, w, log, o);
          if (!r.executable) throw std::runtime_error(r.errorMessage);
          return py::make_tuple(py::cast(std::move(r.executable)), log.str());
        });

  const auto kvRun = [](const KVCacheRunResult& r) {
    py::dict d;
    d["passed"] = r.passed;
    d["output"] = toArray(r.output);
    d["gpu_us"] = r.gpuExecutionTimeUs ? py::cast(*r.gpuExecutionTimeUs) : py::none();
    d["error"] = r.errorMessage;
    return d;
  };
  py::class_<CompiledKVCacheAttention>(m, "CompiledKVCacheAttention")
      .def("reset", &CompiledKVCacheAttention::reset)
      .def("prefill",
           [kvRun](CompiledKVCacheAttention& e, const std::vector<float>& q,
                   const std::vector<float>& k, const std::vector<float>& v) {
             return kvRun(e.prefill(q, k, v));
           })
      .def("decode",
           [kvRun](CompiledKVCacheAttention& e, const std::vector<float>& q,
                   const std::vector<float>& k, const std::vector<float>& v) {
             return kvRun(e.decode(q, k, v));
           })
      .def("current_length", &CompiledKVCacheAttention::currentLength)
      .def("read_key_prefix",
           [](const CompiledKVCacheAttention& e) { return toArray(e.readKeyPrefix()); })
      .def("read_value_prefix",
           [](const CompiledKVCacheAttention& e) { return toArray(e.readValuePrefix()); })
      .def("cache_storage_reused", &CompiledKVCacheAttention::cacheStorageReused);
  m.def("compile_kv_cache_attention",
        [](hip::HipRuntime& rt, const planner::KVCachePlan& plan, FloatArray wq, FloatArray wk,
           FloatArray wv, FloatArray wo) {
          const auto vec = [](const FloatArray& a) {
            return std::vector<float>(a.data(), a.data() + a.size());
          };
          std::ostringstream log;
          auto r = compileKVCacheAttention(rt, plan, vec(wq), vec(wk), vec(wv), vec(wo), log);
          if (!r.executable) throw std::runtime_error(r.errorMessage);
          return py::make_tuple(py::cast(std::move(r.executable)), log.str());
        });

  py::class_<ServingRequestSpec>(m, "ServingRequestSpec")
      .def(py::init<>())
      .def_readwrite("id", &ServingRequestSpec::id)
      .def_readwrite("prompt_token_ids", &ServingRequestSpec::promptTokenIds)
      .def_readwrite("decode_token_count", &ServingRequestSpec::decodeTokenCount)
      .def_readwrite("arrival_step", &ServingRequestSpec::arrivalStep);

  py::class_<ServingConfig>(m, "ServingConfig")
      .def(py::init<>())
      .def_readwrite("page_size", &ServingConfig::pageSize)
      .def_readwrite("physical_pages_per_layer", &ServingConfig::physicalPagesPerLayer)
      .def_readwrite("maximum_batch_size", &ServingConfig::maximumBatchSize)
      .def_readwrite("record_decode_logits", &ServingConfig::recordDecodeLogits)
      .def_readwrite("record_prefill_logits", &ServingConfig::recordPrefillLogits)
      .def_readwrite("tune_kernels", &ServingConfig::tuneKernels)
      .def_readwrite("prefill_chunk_size", &ServingConfig::prefillChunkSize)
      .def_readwrite("prefill_requests_per_chunk", &ServingConfig::prefillRequestsPerChunk);

  m.def("run_continuous_batch",
        [](hip::HipRuntime& rt, std::shared_ptr<DecoderLLMModelResources> model,
           const std::vector<ServingRequestSpec>& specs, const ServingConfig& config) {
          std::ostringstream log;
          ServingExecutionResult r;
          {
            py::gil_scoped_release release;
            r = runContinuousBatch(rt, std::move(model), specs, config, log);
          }
          auto d = servingToDict(r);
          d["log"] = log.str();
          return d;
        });

  m.def("measure_decode_throughput",
        [](hip::HipRuntime& rt, std::shared_ptr<DecoderLLMModelResources> model,
           const std::vector<std::vector<std::int32_t>>& prompts, std::size_t decodeTokens,
           std::size_t pageSize, bool timeGpu, bool tune, std::size_t prefillChunk) {
          DecodeThroughput r;
          {
            py::gil_scoped_release release;
            r = measureDecodeThroughput(rt, std::move(model), prompts, decodeTokens, pageSize,
                                        timeGpu, tune, prefillChunk);
          }
          py::dict d;
          d["passed"] = r.passed;
          d["error"] = r.errorMessage;
          d["rows"] = r.rows;
          d["decode_steps"] = r.decodeSteps;
          d["prompt_phase_us"] = r.promptPhaseUs;
          d["prompt_tokens_per_second"] = r.promptTokensPerSecond;
          d["prefill_chunk_size"] = r.prefillChunkSize;
          d["decode_phase_us"] = r.decodePhaseUs;
          d["tokens_per_second"] = r.tokensPerSecond;
          d["step_gpu"] = statsToDict(r.stepGpu);
          d["step_host"] = statsToDict(r.stepHost);
          d["generated_token_ids"] = r.generatedTokenIds;
          d["kv_bytes_read"] = r.kvBytesRead;
          d["token_only_available"] = r.tokenOnlyAvailable;
          d["token_only_admitted"] = r.tokenOnlyAdmitted;
          d["token_only_speedup"] = r.tokenOnlySpeedup;
          return d;
        },
        py::arg("runtime"), py::arg("model"), py::arg("prompts"), py::arg("decode_tokens"),
        py::arg("page_size") = 16, py::arg("time_gpu") = false, py::arg("tune_kernels") = false,
        py::arg("prefill_chunk_size") = 0);

  // The scheduler over host-only pools and a Python step (CPU tests):
  // step(tokens, valid_lengths, tables, read_logits) -> (next_tokens, logits).
  m.def("run_continuous_batch_with",
        [](hip::HipRuntime& rt, const planner::DecoderLLMPlan& plan,
           const std::vector<std::shared_ptr<KVPagePool>>& pools, std::size_t maxBatch,
           std::size_t maxPages, py::function step, const std::vector<ServingRequestSpec>& specs,
           const ServingConfig& config, py::object prefillStep, std::size_t tileRows,
           std::size_t maxRequests) {
          // prefill([(tokens, start, tables), ...], read_logits) ->
          //   (next tokens of every segment row, last-row logits per segment)
          PrefillStep prefill;
          PrefillPacking packing;
          if (!prefillStep.is_none()) {
            prefill = [prefillStep](const std::vector<PrefillSegment>& segments, bool readLogits) {
              BatchedDecodeRun run;
              py::list arg;
              std::size_t rows = 0;
              for (const auto& s : segments) {
                arg.append(py::make_tuple(s.tokenIds, s.start, s.blockTables));
                rows += s.tokenIds.size();
              }
              py::tuple out = prefillStep(arg, readLogits);
              run.nextTokenIds = out[0].cast<std::vector<float>>();
              if (readLogits) run.logits = toVector(out[1].cast<FloatArray>());
              run.passed = run.nextTokenIds.size() == rows;
              if (!run.passed) run.errorMessage = "prefill returned the wrong number of tokens";
              return run;
            };
            packing.chunkRows = config.prefillChunkSize;
            packing.tileRows = tileRows;
            packing.maxRequests = maxRequests;
          }
          BatchedStep wrapped = [&step](const std::vector<std::int32_t>& tokens,
                                        const std::vector<std::int32_t>& lengths,
                                        const std::vector<std::vector<std::int32_t>>& tables,
                                        bool readLogits) {
            BatchedDecodeRun run;
            py::tuple out = step(tokens, lengths, tables, readLogits);
            run.nextTokenIds = out[0].cast<std::vector<float>>();
            if (readLogits) run.logits = toVector(out[1].cast<FloatArray>());
            run.passed = run.nextTokenIds.size() == tokens.size();
            if (!run.passed) run.errorMessage = "step returned the wrong number of tokens";
            return run;
          };
          std::ostringstream log;
          auto r = runContinuousBatch(rt, plan, pools, maxBatch, maxPages, wrapped, specs, config,
                                      log, prefill, packing);
          auto d = servingToDict(r);
          d["log"] = log.str();
          return d;
        },
        py::arg("runtime"), py::arg("plan"), py::arg("pools"), py::arg("maximum_batch_size"),
        py::arg("max_pages"), py::arg("step"), py::arg("specs"), py::arg("config"),
        py::arg("prefill") = py::none(), py::arg("prefill_tile_rows") = 1,
        py::arg("prefill_max_requests") = 1);
  // Kernel selection (tuners and admission).
  py::class_<hip::DecodeGEMVConfig>(m, "DecodeGEMVConfig")
      .def(py::init<>())
      .def(py::init([](int a, int r, int u, int k) { return hip::DecodeGEMVConfig{a, r, u, k}; }))
      .def_readwrite("algorithm", &hip::DecodeGEMVConfig::algorithm)
      .def_readwrite("rows_per_wave", &hip::DecodeGEMVConfig::rowsPerWave)
      .def_readwrite("unroll", &hip::DecodeGEMVConfig::unroll)
      .def_readwrite("k_split", &hip::DecodeGEMVConfig::kSplit)
      .def("astuple", [](const hip::DecodeGEMVConfig& c) {
        return py::make_tuple(c.algorithm, c.rowsPerWave, c.unroll, c.kSplit);
      });
  m.def("decode_gemv_candidates", &planner::decodeGEMVCandidates, py::arg("batch"),
        py::arg("prefill") = false);
  m.def("decode_gemv_hardware_filter",
        [](const hip::DecodeGEMVConfig& c, std::size_t batch, std::size_t in, std::size_t out,
           std::size_t maxThreads, std::size_t lds, std::size_t maxBuffer) {
          hip::HardwareInfo h;
          h.maxThreadsPerThreadgroup = maxThreads;
          h.maxThreadgroupMemoryLength = lds;
          h.maxBufferLength = maxBuffer;
          return planner::decodeGEMVHardwareFilter(c, batch, in, out, h);
        });
  m.def("decode_gemv_lds_bytes", &hip::decodeGEMVLdsBytes);
  m.def("decode_gemv_threads", &hip::decodeGEMVThreads);
  m.def("emit_decode_gemv_key",
        [](std::size_t batch, std::size_t in, std::size_t out, const hip::DecodeGEMVConfig& c,
           bool f32) {
          return hip::emitDecodeGEMV(batch, in, out, c, "decode_gemv", hip::ElementType::Float16,
                                     f32 ? hip::ElementType::Float32 : hip::ElementType::Float16)
              .source;
        });
  m.def("admission_decision",
        [](bool firstPassed, double firstSpeedup, py::object second) {
          benchmark::PairedResult first;
          first.passed = firstPassed;
          first.speedup = firstSpeedup;
          std::optional<benchmark::PairedResult> confirmation;
          if (!second.is_none()) {
            benchmark::PairedResult c;
            c.passed = true;
            c.speedup = second.cast<double>();
            confirmation = c;
          }
          const auto d = planner::admissionDecision(first, confirmation);
          return py::make_tuple(d.admitted, d.conservativeSpeedup, d.reason);
        });
  m.def("tune_decode_gemv",
        [](hip::HipRuntime& rt, std::size_t batch, std::size_t in, std::size_t out,
           const FloatArray& input, const FloatArray& weight) {
          std::ostringstream log;
          const auto r = planner::tuneDecodeGEMV(rt, batch, in, out, toVector(input),
                                                 toVector(weight), log);
          py::dict d;
          d["success"] = r.success;
          d["use_baseline"] = r.useBaseline;
          d["config"] = py::make_tuple(r.config.algorithm, r.config.rowsPerWave, r.config.unroll,
                                       r.config.kSplit);
          d["speedup"] = r.conservativeSpeedup;
          d["error"] = r.errorMessage;
          d["log"] = log.str();
          return d;
        });
  m.def("rms_norm_hardware_filter",
        [](std::size_t rows, std::size_t width, bool f16, std::size_t threads) {
          RMSNormOp op;
          const DType t = f16 ? DType::Float16 : DType::Float32;
          op.input = {{rows, width}, t, Layout::Contiguous, {}};
          op.weight = {{width}, t, Layout::Contiguous, {}};
          op.output = {{rows, width}, t, Layout::Contiguous, {}};
          hip::HardwareInfo h;
          h.maxThreadsPerThreadgroup = 1024;
          h.maxThreadgroupMemoryLength = 160 * 1024;
          return planner::rmsNormHardwareFilter(op, threads, h);
        });
  m.def("rms_norm_reference",
        [](std::size_t rows, std::size_t width, float eps, const FloatArray& input,
           const FloatArray& weight) {
          RMSNormOp op;
          op.input = {{rows, width}, DType::Float32, Layout::Contiguous, {}};
          op.weight = {{width}, DType::Float32, Layout::Contiguous, {}};
          op.output = {{rows, width}, DType::Float32, Layout::Contiguous, {}};
          op.epsilon = eps;
          const auto ref = validation::rmsNormReference(op, toVector(input), toVector(weight));
          return std::vector<double>(ref.begin(), ref.end());
        });
  m.def("tune_rms_norm",
        [](hip::HipRuntime& rt, std::size_t rows, std::size_t width, float eps, bool f16,
           const FloatArray& input, const FloatArray& weight, std::vector<std::size_t> threads) {
          RMSNormOp op;
          const DType t = f16 ? DType::Float16 : DType::Float32;
          op.input = {{rows, width}, t, Layout::Contiguous, {}};
          op.weight = {{width}, t, Layout::Contiguous, {}};
          op.output = {{rows, width}, t, Layout::Contiguous, {}};
          op.epsilon = eps;
          if (threads.empty()) threads = planner::defaultRMSNormCandidates();
          std::ostringstream log;
          auto r = planner::tuneRMSNorm(rt, op, toVector(input), toVector(weight), threads, log);
          py::dict d;
          d["success"] = r.success;
          d["used_baseline"] = r.usedBaseline;
          d["selected_threads"] = r.selectedThreads;
          d["output"] = toArray(r.finalExecution.output);
          d["max_abs_error"] = r.finalValidation.maxAbsoluteError;
          py::list cands;
          for (const auto& c : r.candidates) {
            py::dict cd;
            cd["name"] = c.name;
            cd["threads"] = c.threads;
            cd["outcome"] = c.outcome;
            cd["reason"] = c.reason;
            cd["speedup"] = c.speedup ? py::cast(*c.speedup) : py::none();
            cands.append(cd);
          }
          d["candidates"] = cands;
          d["error"] = r.errorMessage;
          d["log"] = log.str();
          return d;
        },
        py::arg("runtime"), py::arg("rows"), py::arg("width"), py::arg("eps"), py::arg("f16"),
        py::arg("input"), py::arg("weight"), py::arg("threads") = std::vector<std::size_t>{});
  // admitFusion over Add+RMSNorm: the unfused region (add, then rmsnorm over
  // the sum) against the fused add_rmsnorm kernel, both over the same buffers.
  m.def("admit_add_rmsnorm_fusion",
        [](hip::HipRuntime& rt, std::size_t rows, std::size_t width, bool f16) {
          const auto t = f16 ? hip::ElementType::Float16 : hip::ElementType::Float32;
          const std::string dt = f16 ? "f16" : "f32";
          const std::size_t n = rows * width;
          auto make = [&](std::size_t count) {
            auto b = rt.createBuffer(count, nullptr, t);
            if (!b.buffer) throw std::runtime_error(b.errorMessage);
            return b.buffer;
          };
          auto residual = make(n), update = make(n), gamma = make(width), sum = make(n),
               norm = make(n);
          std::vector<float> g(width);
          for (std::size_t i = 0; i < width; ++i) g[i] = 0.5f + static_cast<float>(i % 11) / 10.0f;
          if (auto e = rt.writeBuffer(gamma, g.data(), g.size()); !e.empty())
            throw std::runtime_error(e);
          auto prepare = [&](const std::string& key, std::vector<hip::BufferHandle> in,
                             std::vector<hip::BufferHandle> out) {
            const auto p = rt.createComputePipeline(key, "fusion_step");
            if (!p.pipelineCreationPassed) throw std::runtime_error(p.errorMessage);
            auto prepared =
                rt.prepareBuffers(in, out, {p.threadgroupCount, p.threadsPerThreadgroup});
            if (!prepared.execution) throw std::runtime_error(prepared.errorMessage);
            return std::move(prepared.execution);
          };
          const std::string shape = "rows=" + std::to_string(rows) + "&width=" +
                                    std::to_string(width) + "&eps=1e-06&dtype=" + dt;
          std::vector<std::unique_ptr<hip::PreparedExecution>> steps;
          steps.push_back(prepare("add?count=" + std::to_string(n) + "&dtype=" + dt,
                                  {residual, update}, {sum}));
          steps.push_back(prepare("rmsnorm?" + shape, {sum, gamma}, {norm}));
          runtime::FusionDecisionCache cache;
          std::ostringstream log;
          const bool admitted = runtime::admitFusion(
              rt, steps, 0,
              [&]() {
                std::vector<std::unique_ptr<hip::PreparedExecution>> fused;
                fused.push_back(prepare("add_rmsnorm?" + shape, {residual, update, gamma},
                                        {sum, norm}));
                return fused;
              },
              {residual, update}, {sum, norm}, "AddRMSNorm", "add_rmsnorm:" + shape, cache, log);
          const bool cachedAgain = runtime::admitFusion(
              rt, steps, 0, [&]() {
                std::vector<std::unique_ptr<hip::PreparedExecution>> fused;
                fused.push_back(prepare("add_rmsnorm?" + shape, {residual, update, gamma},
                                        {sum, norm}));
                return fused;
              },
              {residual, update}, {sum, norm}, "AddRMSNorm", "add_rmsnorm:" + shape, cache, log);
          py::dict d;
          d["admitted"] = admitted;
          d["cached_admitted"] = cachedAgain;
          d["steps"] = steps.size();
          d["sum"] = toArray(sum->read());
          d["norm"] = toArray(norm->read());
          d["log"] = log.str();
          return d;
        });
  m.def("admit_generated_kernel",
        [](hip::HipRuntime& rt, const std::string& pattern, const std::string& response,
           const std::string& feedback, const std::string& artifact) {
          std::ostringstream log;
          const bool ok = runtime::admitGeneratedKernel(rt, pattern, response, feedback, log,
                                                        artifact);
          return py::make_tuple(ok, log.str());
        },
        py::arg("runtime"), py::arg("pattern"), py::arg("response"), py::arg("feedback"),
        py::arg("artifact") = std::string());

  m.def("write_admitted_kernel",
        [](const hip::HipRuntime& rt, const std::string& pattern, const std::string& function,
           const std::string& source, std::size_t workgroup, const std::string& path) {
          return runtime::writeAdmittedKernel(rt, runtime::canonicalKernelPattern(pattern),
                                              {function, source, workgroup}, path);
        });
  m.def("kernel_contract_text", [](const hip::HipRuntime& rt, const std::string& pattern) {
    return runtime::kernelContractText(rt, pattern);
  });
  py::class_<runtime::KernelRegistry, std::shared_ptr<runtime::KernelRegistry>>(m, "KernelRegistry")
      .def(py::init<>())
      .def("load",
           [](runtime::KernelRegistry& r, const hip::HipRuntime& rt, const std::string& dir) {
             std::ostringstream log;
             r.load(rt, dir, log);
             return log.str();
           })
      .def("find",
           [](const runtime::KernelRegistry& r, const std::string& pattern) -> py::object {
             const auto* k = r.find(pattern);
             if (!k) return py::none();
             py::dict d;
             d["function_name"] = k->functionName;
             d["source"] = k->source;
             d["workgroup_size"] = k->workgroupSize;
             return d;
           })
      .def("size", &runtime::KernelRegistry::size)
      .def("track",
           [](runtime::KernelRegistry& r, const std::string& node, const std::string& pattern,
              const std::string& implementation, const std::string& functions,
              std::size_t dispatches) {
             return r.track({node, pattern, implementation, functions, dispatches, 0});
           })
      .def("completed", &runtime::KernelRegistry::completed)
      .def("reset_usage", &runtime::KernelRegistry::resetUsage)
      .def("report", [](const runtime::KernelRegistry& r) {
        std::ostringstream log;
        r.report(log);
        return log.str();
      });

  // ---------------------------------------------------------------- graph path
  py::enum_<Layout>(m, "Layout").value("Contiguous", Layout::Contiguous).value("Strided", Layout::Strided);
  py::enum_<OpType>(m, "OpType")
      .value("Add", OpType::Add).value("Mul", OpType::Mul).value("MatMul", OpType::MatMul)
      .value("RMSNorm", OpType::RMSNorm).value("LayerNorm", OpType::LayerNorm)
      .value("ReLU", OpType::ReLU).value("SiLU", OpType::SiLU).value("Softmax", OpType::Softmax)
      .value("RoPE", OpType::RoPE).value("ReduceSum", OpType::ReduceSum)
      .value("ReduceMean", OpType::ReduceMean).value("Reshape", OpType::Reshape)
      .value("View", OpType::View).value("Transpose", OpType::Transpose)
      .value("Contiguous", OpType::Contiguous).value("MaskedFill", OpType::MaskedFill)
      .value("Slice", OpType::Slice).value("Embedding", OpType::Embedding)
      .value("Gather", OpType::Gather);
  py::class_<TensorType>(m, "TensorType")
      .def(py::init([](std::vector<std::size_t> shape, DType dtype) {
             TensorType t;
             t.shape = std::move(shape);
             t.dtype = dtype;
             return t;
           }),
           py::arg("shape"), py::arg("dtype") = DType::Float32)
      .def_readwrite("shape", &TensorType::shape)
      .def_readwrite("dtype", &TensorType::dtype)
      .def_readwrite("layout", &TensorType::layout)
      .def_readwrite("explicit_strides", &TensorType::explicitStrides)
      .def("element_count", &TensorType::elementCount)
      .def("storage_element_count", &TensorType::storageElementCount)
      .def("strides", &TensorType::strides)
      .def("is_contiguous", &TensorType::isContiguous);
  py::class_<RMSNormAttributes>(m, "RMSNormAttributes")
      .def(py::init([](float eps, std::int64_t axis) { return RMSNormAttributes{eps, axis}; }),
           py::arg("epsilon") = 1e-5f, py::arg("axis") = -1);
  py::class_<ReshapeAttributes>(m, "ReshapeAttributes")
      .def(py::init([](std::vector<std::size_t> shape) { return ReshapeAttributes{std::move(shape)}; }));
  py::class_<TransposeAttributes>(m, "TransposeAttributes")
      .def(py::init([](std::int64_t a, std::int64_t b) { return TransposeAttributes{a, b}; }),
           py::arg("first") = 0, py::arg("second") = 1);
  py::class_<SoftmaxAttributes>(m, "SoftmaxAttributes")
      .def(py::init([](std::int64_t axis) { return SoftmaxAttributes{axis}; }), py::arg("axis") = -1);
  py::class_<TensorGraph>(m, "TensorGraph")
      .def(py::init<>())
      .def("add_input", &TensorGraph::addInput)
      .def("add_node",
           [](TensorGraph& g, OpType op, std::vector<ValueId> operands, py::object attributes,
              std::string name) { return g.addNode(op, std::move(operands), toAttributes(attributes), std::move(name)); },
           py::arg("op"), py::arg("operands"), py::arg("attributes") = py::none(), py::arg("name") = "")
      .def_readwrite("outputs", &TensorGraph::outputs)
      .def_readonly("inputs", &TensorGraph::inputs)
      .def("value_count", [](const TensorGraph& g) { return g.values.size(); });
  m.def("analyze_graph", [](const TensorGraph& g) {
    const auto a = analyzer::analyze(g);
    py::dict d;
    d["types"] = a.types;
    std::vector<py::object> alias;
    for (const auto& x : a.aliasOf) alias.push_back(x ? py::cast(*x) : py::none());
    d["alias_of"] = alias;
    return d;
  });
  m.def("graph_regions", [](const TensorGraph& g) {
    py::list out;
    for (const auto& r : analyzer::formRegions(analyzer::analyze(g))) {
      py::dict d;
      d["fusion"] = analyzer::fusionName(r.fusion);
      d["nodes"] = r.nodes;
      d["inputs"] = r.inputs;
      d["outputs"] = r.outputs;
      out.append(d);
    }
    return out;
  });
  m.def("evaluate_graph", [](const TensorGraph& g, const py::dict& inputs) {
    const auto ref = validation::evaluateGraph(analyzer::analyze(g), toGraphInputs(inputs));
    py::dict d;
    d["values"] = ref.values;
    d["outputs"] = ref.outputs;
    return d;
  });
  py::class_<runtime::CompiledGraph, std::shared_ptr<runtime::CompiledGraph>>(m, "CompiledGraph")
      .def("run", [](const runtime::CompiledGraph& c) {
        runtime::GraphExecutionResult r;
        {
          py::gil_scoped_release release;
          r = c.run();
        }
        return graphResultDict(r);
      })
      .def("unit_names", &runtime::CompiledGraph::unitNames);
  m.def("compile_graph", [](hip::HipRuntime& rt, const TensorGraph& g, const py::dict& inputs) {
    const GraphInputs in = toGraphInputs(inputs);
    std::ostringstream log;
    runtime::GraphCompilation c;
    {
      py::gil_scoped_release release;
      c = runtime::compileGraph(rt, g, in, log);
    }
    py::dict d;
    d["error"] = c.errorMessage;
    d["log"] = log.str();
    d["output_types"] = c.outputTypes;
    d["reference_outputs"] = c.referenceOutputs;
    d["graph"] = c.executable ? py::cast(std::shared_ptr<runtime::CompiledGraph>(std::move(c.executable)))
                              : py::none();
    return d;
  });
}
