// Continuous-batching serving loop; see ServingRuntime.hpp.
#include "ServingRuntime.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <limits>
#include <optional>
#include <ostream>
#include <stdexcept>

namespace tensor::runtime {
namespace {

using Clock = std::chrono::steady_clock;

double elapsedUs(Clock::time_point start, Clock::time_point end) {
  return std::chrono::duration<double, std::micro>(end - start).count();
}

std::size_t pagesFor(std::size_t tokens, std::size_t pageSize) {
  return tokens == 0 ? 0 : (tokens + pageSize - 1) / pageSize;
}

enum class RequestState { Waiting, Active, Preempted, Finished };

// A preempted request's KV state: raw pages in pinned host memory per layer
// for device pools, float prefixes for the host-only pools of the CPU tests.
struct Snapshot {
  std::size_t length = 0;
  std::vector<KVPageSpill> spills;
  std::vector<std::vector<float>> keys, values;
};

struct Request {
  ServingRequestSpec spec;
  std::vector<std::int32_t> prompt;
  RequestState state = RequestState::Waiting;
  ServingRequestOutput output;
  std::vector<std::unique_ptr<KVCacheState>> states;  // one per layer
  std::size_t consumed = 0;                            // prompt tokens in the cache
  std::int32_t lastToken = -1;
  std::size_t decoded = 0;
  std::optional<Snapshot> snapshot;
  std::optional<Clock::time_point> arrivalTime;

  [[nodiscard]] std::size_t length() const { return states.front()->currentLength(); }
  [[nodiscard]] std::size_t pages() const { return states.front()->allocatedPageCount(); }
  // Pages the rest of the prompt will still allocate.
  [[nodiscard]] std::size_t outstandingPromptPages(std::size_t pageSize) const {
    if (state != RequestState::Active || consumed >= prompt.size()) return 0;
    return pagesFor(prompt.size(), pageSize) - pagesFor(length(), pageSize);
  }
};

std::size_t availablePages(const std::vector<std::shared_ptr<KVPagePool>>& pools) {
  std::size_t available = std::numeric_limits<std::size_t>::max();
  for (const auto& pool : pools) available = std::min(available, pool->availablePages());
  return pools.empty() ? 0 : available;
}

std::size_t promisedPages(const std::vector<Request>& requests, std::size_t pageSize) {
  std::size_t pages = 0;
  for (const auto& r : requests) pages += r.outstandingPromptPages(pageSize);
  return pages;
}

std::size_t activeCount(const std::vector<Request>& requests) {
  return static_cast<std::size_t>(std::count_if(requests.begin(), requests.end(), [](const Request& r) {
    return r.state == RequestState::Active;
  }));
}

// The check of auditPageIsolation (ServingRuntime.cpp:436-452): no physical
// page of a layer's pool appears twice among the active requests' page
// tables.  One mark per page of the pool (`seen`, reused across layers and
// cleared through the pages it marked); a page id outside the pool is
// reported as such.
bool auditPageIsolation(const std::vector<Request>& requests,
                        const std::vector<std::shared_ptr<KVPagePool>>& pools,
                        std::string& error) {
  std::vector<std::uint8_t> seen;
  std::vector<std::int32_t> marked;
  for (std::size_t l = 0; l < pools.size(); ++l) {
    const std::size_t capacity = pools[l]->capacityPages();
    if (seen.size() < capacity) seen.resize(capacity, 0);
    bool clash = false, outside = false;
    for (const auto& r : requests) {
      if (r.state != RequestState::Active) continue;
      for (const auto page : r.states[l]->pageTable()) {
        if (page < 0 || static_cast<std::size_t>(page) >= capacity) {
          outside = true;
        } else if (seen[static_cast<std::size_t>(page)]) {
          clash = true;
        } else {
          seen[static_cast<std::size_t>(page)] = 1;
          marked.push_back(page);
        }
      }
    }
    for (const auto page : marked) seen[static_cast<std::size_t>(page)] = 0;
    marked.clear();
    if (clash) {
      error = "Two active requests own the same physical KV page in layer " + std::to_string(l) +
              ".";
      return false;
    }
    if (outside) {
      error = "An active request holds a page id outside the pool in layer " + std::to_string(l) +
              ".";
      return false;
    }
  }
  return true;
}

std::string releaseAll(hip::HipRuntime& runtime, Request& r) {
  for (auto& state : r.states) {
    const auto error = state->reset(runtime);
    if (!error.empty()) return error;
  }
  return {};
}

}  // namespace

ServingExecutionResult runContinuousBatch(hip::HipRuntime& runtime,
                                          const planner::DecoderLLMPlan& plan,
                                          const std::vector<std::shared_ptr<KVPagePool>>& pools,
                                          std::size_t maximumBatchSize, std::size_t maxPages,
                                          const BatchedStep& step,
                                          const std::vector<ServingRequestSpec>& specs,
                                          const ServingConfig& config, std::ostream& log,
                                          const PrefillStep& prefill,
                                          const PrefillPacking& packing) {
  ServingExecutionResult result;
  auto& metrics = result.metrics;
  try {
    if (specs.empty() || config.pageSize == 0 || config.physicalPagesPerLayer == 0)
      throw std::invalid_argument("Serving configuration and requests must be nonempty.");
    if (config.prefillChunkSize != 0 &&
        (!prefill || packing.chunkRows == 0 || packing.tileRows == 0 || packing.maxRequests == 0))
      throw std::invalid_argument("Chunked serving prefill needs a prefill step and its packing.");
    if (pools.size() != plan.layerCount || maximumBatchSize == 0)
      throw std::invalid_argument("Serving needs one page pool per layer and a batch size.");
    const std::size_t capacity = plan.attention.capacity, P = config.pageSize;
    const auto kvPlan = plan.kvPlan();
    std::size_t largest = 0;
    std::vector<Request> requests;
    requests.reserve(specs.size());
    for (const auto& spec : specs) {
      if (spec.id.empty() || spec.promptTokenIds.size() < 2 ||
          spec.promptTokenIds.size() >= capacity ||
          spec.decodeTokenCount > capacity - spec.promptTokenIds.size())
        throw std::invalid_argument("Serving request dimensions are invalid.");
      Request r;
      r.spec = spec;
      for (const float token : spec.promptTokenIds) {
        if (!(token >= 0.0f) || token != std::floor(token) ||
            token >= static_cast<float>(plan.vocabularySize))
          throw std::invalid_argument("Serving request " + spec.id + " has an invalid token id.");
        r.prompt.push_back(static_cast<std::int32_t>(token));
      }
      r.output.id = spec.id;
      largest = std::max(largest, pagesFor(spec.promptTokenIds.size() + spec.decodeTokenCount, P));
      requests.push_back(std::move(r));
    }
    if (config.physicalPagesPerLayer < largest || pools.front()->capacityPages() < largest)
      throw std::invalid_argument("Shared KV pool cannot hold the largest configured request.");
    for (auto& r : requests) {
      for (const auto& pool : pools) {
        auto state = createKVCacheState(runtime, kvPlan, pool, false);
        if (!state.state) throw std::runtime_error(state.errorMessage);
        r.states.push_back(std::move(state.state));
      }
      log << "Serving request " << r.spec.id << ": prompt=" << r.prompt.size()
          << ", decode=" << r.spec.decodeTokenCount << ", arrival_step=" << r.spec.arrivalStep
          << '\n';
    }

    std::vector<double> gpuTimes, hostTimes;
    std::size_t completed = 0, tick = 0, batchSamples = 0, batchSum = 0;
    std::size_t decodeRows = 0;
    double decodeOnlyUs = 0.0;
    const auto start = Clock::now();
    auto finish = [&](Request& r) {
      const auto kvStart = Clock::now();
      const auto error = releaseAll(runtime, r);
      metrics.kvManagementOverheadUs += elapsedUs(kvStart, Clock::now());
      if (!error.empty()) throw std::runtime_error(error);
      r.state = RequestState::Finished;
      ++completed;
      log << "Serving request " << r.spec.id << ": finished\n";
    };

    while (completed < requests.size()) {
      if (tick > 10000000) throw std::runtime_error("Serving scheduler exceeded its progress limit.");
      bool progress = false;

      // Resume preempted requests whose snapshot fits.
      for (auto& r : requests) {
        const auto t0 = Clock::now();
        const bool fits = r.state == RequestState::Preempted && r.snapshot &&
                          activeCount(requests) < maximumBatchSize &&
                          availablePages(pools) >= promisedPages(requests, P) &&
                          availablePages(pools) - promisedPages(requests, P) >=
                              pagesFor(r.snapshot->length, P);
        metrics.schedulerOverheadUs += elapsedUs(t0, Clock::now());
        if (!fits) continue;
        const auto restoreStart = Clock::now();
        for (std::size_t l = 0; l < r.states.size(); ++l) {
          const auto error =
              l < r.snapshot->spills.size()
                  ? r.states[l]->restorePages(runtime, r.snapshot->spills[l])
                  : r.states[l]->restore(runtime, r.snapshot->length, r.snapshot->keys[l],
                                         r.snapshot->values[l]);
          if (!error.empty())
            throw std::runtime_error("Request " + r.spec.id + " resume failed: " + error);
        }
        metrics.preemptionOverheadUs += elapsedUs(restoreStart, Clock::now());
        r.snapshot.reset();
        r.state = RequestState::Active;
        ++metrics.resumeCount;
        log << "Serving request " << r.spec.id << ": resumed at length=" << r.length() << '\n';
        progress = true;
      }

      // Admit arrived requests whose prompt pages fit.
      for (auto& r : requests) {
        const auto t0 = Clock::now();
        const bool eligible = r.state == RequestState::Waiting && r.spec.arrivalStep <= tick;
        if (eligible && !r.arrivalTime) r.arrivalTime = Clock::now();
        const std::size_t promised = promisedPages(requests, P), available = availablePages(pools);
        const bool fits = eligible && activeCount(requests) < maximumBatchSize &&
                          available >= promised &&
                          available - promised >= pagesFor(r.prompt.size(), P);
        metrics.schedulerOverheadUs += elapsedUs(t0, Clock::now());
        if (!fits) continue;
        r.state = RequestState::Active;
        progress = true;
      }

      // Chunked prefill of the prompts admitted above (their pages were
      // counted at admission), several requests per chunk when the packing
      // allows: each request's rows start at a tile boundary.  The last row
      // of a request's last segment is its first generated token.
      while (config.prefillChunkSize != 0) {
        std::vector<std::size_t> who, starts;
        std::vector<PrefillSegment> segments;
        std::size_t row = 0;
        const auto kvStart = Clock::now();
        auto rollback = [&]() {
          for (std::size_t k = 0; k < who.size(); ++k)
            for (auto& s : requests[who[k]].states) (void)s->rollbackLength(runtime, starts[k]);
        };
        for (std::size_t i = 0; i < requests.size(); ++i) {
          auto& r = requests[i];
          if (r.state != RequestState::Active || r.consumed >= r.prompt.size()) continue;
          if (segments.size() == packing.maxRequests || row >= packing.chunkRows) break;
          const std::size_t start = r.consumed;
          const std::size_t count = std::min(r.prompt.size() - start, packing.chunkRows - row);
          PrefillSegment segment;
          segment.start = start;
          segment.tokenIds.assign(r.prompt.begin() + static_cast<std::ptrdiff_t>(start),
                                  r.prompt.begin() + static_cast<std::ptrdiff_t>(start + count));
          for (auto& state : r.states) {
            const auto error = state->stageLength(runtime, start + count);
            if (!error.empty()) {
              for (auto& s : r.states) (void)s->rollbackLength(runtime, start);
              rollback();
              throw std::runtime_error("Request " + r.spec.id + " KV stage failed: " + error);
            }
            auto table = state->pageTable();
            table.resize(maxPages, -1);
            segment.blockTables.push_back(std::move(table));
          }
          who.push_back(i);
          starts.push_back(start);
          segments.push_back(std::move(segment));
          row = (row + count + packing.tileRows - 1) / packing.tileRows * packing.tileRows;
        }
        metrics.kvManagementOverheadUs += elapsedUs(kvStart, Clock::now());
        if (segments.empty()) break;
        const auto out = prefill(segments, config.recordPrefillLogits);
        ++metrics.prefillChunkSubmissions;
        std::size_t rowsOut = 0;
        for (const auto& segment : segments) rowsOut += segment.tokenIds.size();
        if (!out.passed || out.nextTokenIds.size() != rowsOut) {
          rollback();
          throw std::runtime_error("Chunked prefill failed: " + out.errorMessage);
        }
        std::size_t offset = 0;
        for (std::size_t k = 0; k < who.size(); ++k) {
          auto& r = requests[who[k]];
          const std::size_t count = segments[k].tokenIds.size();
          for (auto& state : r.states) state->commitLength(starts[k] + count);
          r.consumed += count;
          metrics.promptTokens += count;
          offset += count;
          if (r.consumed < r.prompt.size()) continue;
          const auto next = static_cast<std::int32_t>(out.nextTokenIds[offset - 1]);
          r.output.generatedTokenIds.push_back(static_cast<float>(next));
          r.lastToken = next;
          r.output.timeToFirstTokenUs = elapsedUs(*r.arrivalTime, Clock::now());
          if (config.recordPrefillLogits && out.logits.size() == segments.size() * plan.vocabularySize) {
            const auto V = static_cast<std::ptrdiff_t>(plan.vocabularySize);
            r.output.prefillLogits.assign(out.logits.begin() + static_cast<std::ptrdiff_t>(k) * V,
                                          out.logits.begin() + static_cast<std::ptrdiff_t>(k + 1) * V);
          }
          log << "Serving request " << r.spec.id << ": prompt complete (chunked), pages="
              << r.pages() << ", ttft(us)=" << r.output.timeToFirstTokenUs << '\n';
          if (r.spec.decodeTokenCount == 0) finish(r);
        }
        progress = true;
      }

      // Pages for every active row's next token; preempt the largest owner
      // while they are missing (selectPreemptionVictim, ServingRuntime.cpp:454-467).
      auto active = [&]() {
        std::vector<std::size_t> rows;
        for (std::size_t i = 0; i < requests.size(); ++i)
          if (requests[i].state == RequestState::Active) rows.push_back(i);
        return rows;
      };
      auto rows = active();
      auto required = [&]() {
        std::size_t pages = 0;
        for (const auto i : rows)
          pages += pagesFor(requests[i].length() + 1, P) - pagesFor(requests[i].length(), P);
        return pages;
      };
      while (!rows.empty() && availablePages(pools) < required()) {
        std::optional<std::size_t> victim;
        for (const auto i : rows)
          if (!victim || requests[i].pages() > requests[*victim].pages()) victim = i;
        auto& v = requests[*victim];
        const auto t0 = Clock::now();
        if (v.length() == 0) {
          v.state = RequestState::Waiting;
        } else {
          Snapshot snap;
          snap.length = v.length();
          for (const auto& state : v.states) {
            if (state->keyBuffer()) {
              KVPageSpill spill;
              const auto error = state->spillPages(runtime, spill);
              if (!error.empty())
                throw std::runtime_error("Request " + v.spec.id + " spill failed: " + error);
              metrics.spilledBytes += spill.bytes();
              snap.spills.push_back(std::move(spill));
            } else {
              snap.keys.push_back(state->readKeyPrefix());
              snap.values.push_back(state->readValuePrefix());
            }
          }
          const auto error = releaseAll(runtime, v);
          if (!error.empty())
            throw std::runtime_error("Request " + v.spec.id + " preemption failed: " + error);
          v.snapshot = std::move(snap);
          v.state = RequestState::Preempted;
          ++metrics.preemptionCount;
        }
        metrics.preemptionOverheadUs += elapsedUs(t0, Clock::now());
        log << "Serving request " << v.spec.id << ": preempted for page pressure\n";
        progress = true;
        rows = active();
      }

      if (!rows.empty()) {
        const auto stageStart = Clock::now();
        std::vector<std::size_t> previous;
        for (const auto i : rows) {
          auto& r = requests[i];
          previous.push_back(r.length());
          for (auto& state : r.states) {
            const auto error = state->stageLength(runtime, r.length() + 1);
            if (!error.empty()) {
              for (std::size_t k = 0; k < previous.size(); ++k)
                for (auto& s : requests[rows[k]].states) (void)s->rollbackLength(runtime, previous[k]);
              throw std::runtime_error("Request " + r.spec.id + " KV stage failed: " + error);
            }
          }
        }
        metrics.kvManagementOverheadUs += elapsedUs(stageStart, Clock::now());

        const auto packStart = Clock::now();
        std::vector<std::int32_t> tokens, lengths;
        std::vector<std::vector<std::int32_t>> tables(plan.layerCount);
        bool readLogits = false, promptRows = false;
        for (std::size_t k = 0; k < rows.size(); ++k) {
          const auto& r = requests[rows[k]];
          const bool inPrompt = r.consumed < r.prompt.size();
          promptRows = promptRows || inPrompt;
          tokens.push_back(inPrompt ? r.prompt[r.consumed] : r.lastToken);
          lengths.push_back(static_cast<std::int32_t>(previous[k] + 1));
          readLogits = readLogits || (inPrompt && r.consumed + 1 == r.prompt.size() &&
                                      config.recordPrefillLogits) ||
                       (!inPrompt && config.recordDecodeLogits);
          for (std::size_t l = 0; l < plan.layerCount; ++l) {
            auto table = r.states[l]->pageTable();
            table.resize(maxPages, -1);
            tables[l].insert(tables[l].end(), table.begin(), table.end());
          }
        }
        metrics.schedulerOverheadUs += elapsedUs(packStart, Clock::now());

        const auto stepStart = Clock::now();
        const auto out = step(tokens, lengths, tables, readLogits);
        const double stepUs = elapsedUs(stepStart, Clock::now());
        hostTimes.push_back(stepUs);
        ++metrics.decodeCommandSubmissions;
        if (!out.passed) {
          for (std::size_t k = 0; k < rows.size(); ++k)
            for (auto& s : requests[rows[k]].states) (void)s->rollbackLength(runtime, previous[k]);
          throw std::runtime_error("Batched decode failed: " + out.errorMessage);
        }
        if (out.gpuExecutionTimeUs) gpuTimes.push_back(*out.gpuExecutionTimeUs);

        const auto commitStart = Clock::now();
        std::size_t stepDecodeRows = 0;
        for (std::size_t k = 0; k < rows.size(); ++k) {
          auto& r = requests[rows[k]];
          for (auto& state : r.states) state->commitLength(previous[k] + 1);
          const auto next = static_cast<std::int32_t>(out.nextTokenIds[k]);
          auto logitsOf = [&]() {
            const auto V = static_cast<std::ptrdiff_t>(plan.vocabularySize);
            return std::vector<float>(out.logits.begin() + static_cast<std::ptrdiff_t>(k) * V,
                                      out.logits.begin() + static_cast<std::ptrdiff_t>(k + 1) * V);
          };
          if (r.consumed < r.prompt.size()) {
            ++r.consumed;
            ++metrics.promptTokens;
            if (r.consumed == r.prompt.size()) {
              r.output.generatedTokenIds.push_back(static_cast<float>(next));
              r.lastToken = next;
              r.output.timeToFirstTokenUs = elapsedUs(*r.arrivalTime, Clock::now());
              if (config.recordPrefillLogits && !out.logits.empty()) r.output.prefillLogits = logitsOf();
              log << "Serving request " << r.spec.id << ": prompt complete, pages=" << r.pages()
                  << ", ttft(us)=" << r.output.timeToFirstTokenUs << '\n';
              if (r.spec.decodeTokenCount == 0) finish(r);
            }
          } else {
            r.output.generatedTokenIds.push_back(static_cast<float>(next));
            if (config.recordDecodeLogits && !out.logits.empty()) r.output.decodeLogits.push_back(logitsOf());
            r.lastToken = next;
            ++r.decoded;
            ++metrics.decodedTokens;
            ++stepDecodeRows;
            if (r.decoded == r.spec.decodeTokenCount) finish(r);
          }
        }
        metrics.kvManagementOverheadUs += elapsedUs(commitStart, Clock::now());
        if (!promptRows) {
          decodeRows += stepDecodeRows;
          decodeOnlyUs += stepUs;
        }
        progress = true;
        ++batchSamples;
        batchSum += rows.size();
        metrics.maximumActiveBatchSize = std::max(metrics.maximumActiveBatchSize, rows.size());
      }

      std::string isolation;
      if (!auditPageIsolation(requests, pools, isolation))
        throw std::runtime_error(isolation);
      if (!progress) {
        const bool future = std::any_of(requests.begin(), requests.end(), [&](const Request& r) {
          return r.state == RequestState::Waiting && r.spec.arrivalStep > tick;
        });
        if (!future) throw std::runtime_error("Serving scheduler made no progress.");
      }
      ++tick;
    }

    metrics.totalTimeUs = elapsedUs(start, Clock::now());
    if (metrics.totalTimeUs > 0.0)
      metrics.tokensPerSecond = static_cast<double>(metrics.decodedTokens) * 1e6 / metrics.totalTimeUs;
    if (decodeOnlyUs > 0.0)
      metrics.decodePhaseTokensPerSecond = static_cast<double>(decodeRows) * 1e6 / decodeOnlyUs;
    if (batchSamples)
      metrics.averageActiveBatchSize = static_cast<double>(batchSum) / static_cast<double>(batchSamples);
    if (const auto s = benchmark::summarizeTimings(gpuTimes)) metrics.decodeGpu = *s;
    if (const auto s = benchmark::summarizeTimings(hostTimes)) metrics.decodeEndToEnd = *s;
    metrics.peakPagesPerLayer = pools.front()->peakUsedPages();
    metrics.pageAllocationCount = pools.front()->allocationCount();
    metrics.pageReleaseCount = pools.front()->releaseCount();
    for (const auto& pool : pools) {
      if (pool->usedPages() != 0) throw std::runtime_error("Serving completed with unreleased KV pages.");
      if (pool->allocationCount() != metrics.pageAllocationCount ||
          pool->releaseCount() != metrics.pageReleaseCount)
        throw std::runtime_error("Per-layer KV page-pool lifecycle counts diverged.");
    }
    for (auto& r : requests) result.requests.push_back(std::move(r.output));
    result.passed = true;
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

ServingExecutionResult runContinuousBatch(hip::HipRuntime& runtime,
                                          std::shared_ptr<DecoderLLMModelResources> model,
                                          const std::vector<ServingRequestSpec>& requests,
                                          const ServingConfig& config, std::ostream& log) {
  ServingExecutionResult result;
  try {
    if (!model) throw std::invalid_argument("Serving needs model resources.");
    const auto& plan = model->plan;
    const std::size_t M = config.maximumBatchSize ? config.maximumBatchSize : requests.size();
    std::vector<std::shared_ptr<KVPagePool>> pools;
    for (std::size_t l = 0; l < plan.layerCount; ++l) {
      auto pool = createKVPagePool(runtime, plan.kvPlan(), config.pageSize, config.physicalPagesPerLayer);
      if (!pool.pool) throw std::runtime_error(pool.errorMessage);
      pools.push_back(std::move(pool.pool));
    }
    auto created = createBatchedDecodeExecutor(runtime, model, pools, M, &log, config.tuneKernels);
    if (!created.executor) throw std::runtime_error(created.errorMessage);
    auto& executor = *created.executor;
    // ticks that read no logits take the token-only tail where an earlier
    // admission of this shape admitted it; no candidate is timed mid-run
    executor.setTokenOnlyPolicy(BatchedDecodeExecutor::TokenOnlyPolicy::CachedOnly);
    BatchedStep step = [&executor](const std::vector<std::int32_t>& tokens,
                                   const std::vector<std::int32_t>& lengths,
                                   const std::vector<std::vector<std::int32_t>>& tables,
                                   bool readLogits) {
      return executor.run(tokens, lengths, tables, readLogits, true);
    };
    std::unique_ptr<ChunkedPrefillExecutor> prefillExecutor;
    PrefillStep prefill;
    PrefillPacking packing;
    if (config.prefillChunkSize != 0) {
      auto made = createChunkedPrefillExecutor(runtime, model, pools, config.prefillChunkSize, &log,
                                               std::max<std::size_t>(1, config.prefillRequestsPerChunk));
      if (!made.executor) throw std::runtime_error(made.errorMessage);
      prefillExecutor = std::move(made.executor);
      prefill = [&prefillExecutor](const std::vector<PrefillSegment>& segments, bool readLogits) {
        return prefillExecutor->runBatch(segments, readLogits, false);
      };
      packing.chunkRows = prefillExecutor->chunkSize();
      packing.tileRows = prefillExecutor->tileRows();
      packing.maxRequests = prefillExecutor->maximumRequests();
    }
    result = runContinuousBatch(runtime, plan, pools, M, executor.maxPages(), step, requests,
                                config, log, prefill, packing);
    result.metrics.modelStorageBytes = model->storageBytes;
    result.metrics.kvPoolStorageBytes = 2 * plan.layerCount * pools.front()->keyBuffer()->storageBytes();
    result.metrics.batchedActivationStorageBytes =
        executor.activationStorageBytes() +
        (prefillExecutor ? prefillExecutor->activationStorageBytes() : 0);
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

DecodeThroughput measureDecodeThroughput(hip::HipRuntime& runtime,
                                         std::shared_ptr<DecoderLLMModelResources> model,
                                         const std::vector<std::vector<std::int32_t>>& prompts,
                                         std::size_t decodeTokens, std::size_t pageSize,
                                         bool timeGpu, bool tuneKernels,
                                         std::size_t prefillChunkSize) {
  DecodeThroughput result;
  try {
    if (!model || prompts.empty() || pageSize == 0)
      throw std::invalid_argument("Decode measurement needs a model, prompts and a page size.");
    const auto& plan = model->plan;
    const std::size_t B = prompts.size(), L = plan.layerCount;
    std::size_t pagesNeeded = 0, longest = 0;
    for (const auto& prompt : prompts) {
      if (prompt.empty() || prompt.size() + decodeTokens > plan.attention.capacity)
        throw std::invalid_argument("Prompt plus decode tokens exceed the cache capacity.");
      for (const auto token : prompt)
        if (token < 0 || static_cast<std::size_t>(token) >= plan.vocabularySize)
          throw std::invalid_argument("Prompt token outside the vocabulary.");
      pagesNeeded += pagesFor(prompt.size() + decodeTokens, pageSize);
      longest = std::max(longest, prompt.size());
    }
    const std::size_t poolPages = std::max(pagesNeeded, pagesFor(plan.attention.capacity, pageSize));
    std::vector<std::shared_ptr<KVPagePool>> pools;
    for (std::size_t l = 0; l < L; ++l) {
      auto pool = createKVPagePool(runtime, plan.kvPlan(), pageSize, poolPages);
      if (!pool.pool) throw std::runtime_error(pool.errorMessage);
      pools.push_back(std::move(pool.pool));
    }
    auto created = createBatchedDecodeExecutor(runtime, model, pools, B, nullptr, tuneKernels);
    if (!created.executor) throw std::runtime_error(created.errorMessage);
    auto& executor = *created.executor;
    std::vector<std::vector<std::unique_ptr<KVCacheState>>> states(B);
    for (auto& row : states)
      for (const auto& pool : pools) {
        auto state = createKVCacheState(runtime, plan.kvPlan(), pool, false);
        if (!state.state) throw std::runtime_error(state.errorMessage);
        row.push_back(std::move(state.state));
      }
    result.rows = B;
    result.generatedTokenIds.assign(B, {});
    std::vector<std::int32_t> last(B, -1);

    // The next lengths and block tables of `rows` (pages staged as needed).
    std::vector<double> gpuTimes, hostTimes;
    auto stage = [&](const std::vector<std::size_t>& rows, std::vector<std::int32_t>& lengths,
                     std::vector<std::vector<std::int32_t>>& tables) {
      lengths.clear();
      tables.assign(L, {});
      for (const auto r : rows) {
        const std::size_t next = states[r].front()->currentLength() + 1;
        lengths.push_back(static_cast<std::int32_t>(next));
        for (std::size_t l = 0; l < L; ++l) {
          const auto error = states[r][l]->stageLength(runtime, next);
          if (!error.empty()) throw std::runtime_error(error);
          auto table = states[r][l]->pageTable();
          table.resize(executor.maxPages(), -1);
          tables[l].insert(tables[l].end(), table.begin(), table.end());
        }
      }
    };
    auto commit = [&](const std::vector<std::size_t>& rows, const std::vector<std::int32_t>& lengths) {
      for (std::size_t k = 0; k < rows.size(); ++k)
        for (auto& state : states[rows[k]]) state->commitLength(static_cast<std::size_t>(lengths[k]));
    };
    // One batched step over `rows`; commits the new lengths.
    auto step = [&](const std::vector<std::size_t>& rows, const std::vector<std::int32_t>& tokens,
                    bool record) {
      std::vector<std::int32_t> lengths;
      std::vector<std::vector<std::int32_t>> tables;
      stage(rows, lengths, tables);
      const auto t0 = Clock::now();
      const auto out = executor.run(tokens, lengths, tables, false, timeGpu);
      const double us = elapsedUs(t0, Clock::now());
      if (!out.passed) throw std::runtime_error(out.errorMessage);
      if (record) {
        hostTimes.push_back(us);
        if (out.gpuExecutionTimeUs) gpuTimes.push_back(*out.gpuExecutionTimeUs);
      }
      commit(rows, lengths);
      return out.nextTokenIds;
    };

    std::unique_ptr<ChunkedPrefillExecutor> prefill;
    if (prefillChunkSize != 0) {
      auto made = createChunkedPrefillExecutor(runtime, model, pools,
                                               std::min(prefillChunkSize, plan.attention.capacity),
                                               nullptr, B);
      if (!made.executor) throw std::runtime_error(made.errorMessage);
      prefill = std::move(made.executor);
      // One chunk per stage on row 0's states, then released: the prompt
      // GEMMs pick their library algorithms here, outside the timed phase.
      for (const auto rows : prefill->buckets()) {
        std::vector<std::vector<std::int32_t>> tables;
        for (auto& state : states[0]) {
          const auto error = state->stageLength(runtime, rows);
          if (!error.empty()) throw std::runtime_error(error);
          auto table = state->pageTable();
          table.resize(prefill->maxPages(), -1);
          tables.push_back(std::move(table));
        }
        const auto out = prefill->run(std::vector<std::int32_t>(rows, 0), 0, tables, false, false);
        if (!out.passed) throw std::runtime_error(out.errorMessage);
        for (auto& state : states[0]) {
          const auto error = state->reset(runtime);
          if (!error.empty()) throw std::runtime_error(error);
        }
      }
      result.prefillChunkSize = prefill->chunkSize();
    }

    const auto promptStart = Clock::now();
    if (prefill) {
      // Prompts packed into chunks, several requests per chunk (each from a
      // tile boundary); a request's last row gives its first generated token.
      std::vector<std::size_t> consumed(B, 0);
      for (std::size_t next = 0; next < B;) {
        std::vector<std::size_t> who;
        std::vector<PrefillSegment> segments;
        std::size_t row = 0;
        for (std::size_t r = next; r < B && row < prefill->chunkSize(); ++r) {
          const auto& prompt = prompts[r];
          const std::size_t start = consumed[r];
          const std::size_t count = std::min(prompt.size() - start, prefill->chunkSize() - row);
          PrefillSegment segment;
          segment.start = start;
          segment.tokenIds.assign(prompt.begin() + static_cast<std::ptrdiff_t>(start),
                                  prompt.begin() + static_cast<std::ptrdiff_t>(start + count));
          for (auto& state : states[r]) {
            const auto error = state->stageLength(runtime, start + count);
            if (!error.empty()) throw std::runtime_error(error);
            auto table = state->pageTable();
            table.resize(prefill->maxPages(), -1);
            segment.blockTables.push_back(std::move(table));
          }
          who.push_back(r);
          segments.push_back(std::move(segment));
          row = (row + count + prefill->tileRows() - 1) / prefill->tileRows() * prefill->tileRows();
        }
        const auto out = prefill->runBatch(segments, false, false);
        if (!out.passed) throw std::runtime_error(out.errorMessage);
        std::size_t offset = 0;
        for (std::size_t k = 0; k < who.size(); ++k) {
          const std::size_t r = who[k], count = segments[k].tokenIds.size();
          for (auto& state : states[r]) state->commitLength(consumed[r] + count);
          consumed[r] += count;
          offset += count;
          if (consumed[r] == prompts[r].size()) {
            last[r] = static_cast<std::int32_t>(out.nextTokenIds[offset - 1]);
            result.generatedTokenIds[r].push_back(out.nextTokenIds[offset - 1]);
            next = std::max(next, r + 1);
          }
        }
      }
    }
    for (std::size_t t = 0; !prefill && t < longest; ++t) {
      std::vector<std::size_t> rows;
      std::vector<std::int32_t> tokens;
      for (std::size_t r = 0; r < B; ++r)
        if (t < prompts[r].size()) {
          rows.push_back(r);
          tokens.push_back(prompts[r][t]);
        }
      const auto next = step(rows, tokens, false);
      for (std::size_t k = 0; k < rows.size(); ++k)
        if (t + 1 == prompts[rows[k]].size()) {
          last[rows[k]] = static_cast<std::int32_t>(next[k]);
          result.generatedTokenIds[rows[k]].push_back(next[k]);
        }
    }
    result.promptPhaseUs = elapsedUs(promptStart, Clock::now());
    std::size_t promptTokens = 0;
    for (const auto& prompt : prompts) promptTokens += prompt.size();
    if (result.promptPhaseUs > 0.0)
      result.promptTokensPerSecond = static_cast<double>(promptTokens) * 1e6 / result.promptPhaseUs;

    std::vector<std::size_t> all(B);
    for (std::size_t r = 0; r < B; ++r) all[r] = r;
    std::size_t kvTokens = 0;
    for (std::size_t r = 0; r < B; ++r)
      for (std::size_t s = 0; s < decodeTokens; ++s) kvTokens += prompts[r].size() + 1 + s;
    result.kvBytesRead = kvTokens * L * 2 * plan.kvWidth() * 2;
    if (decodeTokens > 0) {
      if (!timeGpu) {
        const auto error = executor.reserveHistory(decodeTokens);
        if (!error.empty()) throw std::runtime_error(error);
      }
      // The token-only admission of the decode bucket (both tails replay the
      // first decode step at its staged length), outside the timed phase.
      std::vector<std::int32_t> lengths;
      std::vector<std::vector<std::int32_t>> tables;
      stage(all, lengths, tables);
      const auto error = executor.admitTokenOnly(last, lengths, tables);
      if (!error.empty()) throw std::runtime_error(error);
      const auto status = executor.tokenOnlyStatus(B);
      result.tokenOnlyAvailable = status.available;
      result.tokenOnlyAdmitted = status.admitted;
      result.tokenOnlySpeedup = status.speedup;
    }
    const auto decodeStart = Clock::now();
    if (timeGpu) {
      for (std::size_t s = 0; s < decodeTokens; ++s) {
        const auto next = step(all, last, true);
        for (std::size_t r = 0; r < B; ++r) {
          last[r] = static_cast<std::int32_t>(next[r]);
          result.generatedTokenIds[r].push_back(next[r]);
        }
      }
    } else if (decodeTokens > 0) {
      // Greedy tokens stay on the device from step to step (chained steps,
      // no host wait); they are read back once at the end, so the host's
      // staging and graph launches overlap the GPU's work.
      std::vector<std::int32_t> lengths;
      std::vector<std::vector<std::int32_t>> tables;
      for (std::size_t s = 0; s < decodeTokens; ++s) {
        stage(all, lengths, tables);
        const auto t0 = Clock::now();
        const auto error =
            executor.launchChained(s == 0 ? last : std::vector<std::int32_t>{}, lengths, tables, s);
        if (!error.empty()) throw std::runtime_error(error);
        hostTimes.push_back(elapsedUs(t0, Clock::now()));
        commit(all, lengths);
      }
      std::vector<std::int32_t> history;
      const auto error = executor.readHistory(decodeTokens, history);
      if (!error.empty()) throw std::runtime_error(error);
      const std::size_t M = executor.maximumBatchSize();
      for (std::size_t s = 0; s < decodeTokens; ++s)
        for (std::size_t r = 0; r < B; ++r) {
          last[r] = history[s * M + r];
          result.generatedTokenIds[r].push_back(static_cast<float>(last[r]));
        }
    }
    result.decodePhaseUs = elapsedUs(decodeStart, Clock::now());
    result.decodeSteps = decodeTokens;
    if (result.decodePhaseUs > 0.0)
      result.tokensPerSecond = static_cast<double>(B * decodeTokens) * 1e6 / result.decodePhaseUs;
    if (const auto st = benchmark::summarizeTimings(gpuTimes)) result.stepGpu = *st;
    if (const auto st = benchmark::summarizeTimings(hostTimes)) result.stepHost = *st;
    result.passed = true;
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

}  // namespace tensor::runtime
