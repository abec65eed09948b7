// Continuous-batching serving loop for the gfx950 decode path, with the
// interface of the reference's src/runtime/ServingRuntime.hpp:13-74 and the
// scheduling rules of ServingRuntime.cpp:426-930:
//  * per-layer page pools shared by all requests (LIFO free lists);
//  * a request is admitted when its arrival step has come and the pools hold
//    pages for its prompt; preempted requests are resumed first, when the
//    pools hold pages for their snapshot;
//  * before every batched step the pages the active rows need for their next
//    token are counted; while they are missing, the active request owning the
//    most pages is preempted (its KV pages copied raw into pinned host memory,
//    pages released);
//  * after every step page isolation between active requests is audited and
//    finished requests release their pages; at the end every pool must be
//    empty with equal allocation/release counts across layers.
// Prompts run through the batched decode graph one token per tick (prefill
// by decode): a request's row carries its next prompt token until the prompt
// is consumed, then its last generated token, so prompt and decode rows share
// one batched step.  The tick that consumes the last prompt token yields the
// first generated token (the reference's prefill output); each later tick is
// one decode step.  With ServingConfig::prefillChunkSize > 0 an admitted
// request's prompt instead runs at admission through the chunked prefill
// executor (the reference's prefillChunked per request,
// ServingRuntime.cpp:682-700), and the request joins the decode ticks with
// its first token.
#pragma once

#include "Benchmark.hpp"
#include "DecoderLLM.hpp"

#include <cstddef>
#include <functional>
#include <iosfwd>
#include <string>
#include <vector>

namespace tensor::runtime {

struct ServingRequestSpec {
  std::string id;
  std::vector<float> promptTokenIds;
  std::size_t decodeTokenCount = 0;
  std::size_t arrivalStep = 0;
};

struct ServingConfig {
  std::size_t pageSize = 16;
  std::size_t physicalPagesPerLayer = 8;
  // Rows per batched step; 0 = the number of requests.
  std::size_t maximumBatchSize = 0;
  // Keep every decode step's logits per request (vocabulary floats each).
  bool recordDecodeLogits = false;
  // Keep the logits of the last prompt position.
  bool recordPrefillLogits = true;
  // Batch-1 GEMVs with the decode GEMV tuner's cached per-shape selection.
  bool tuneKernels = false;
  // > 0: prompts run at admission in chunks of this many tokens through the
  // chunked prefill executor; 0: prefill by decode in the batched ticks.
  std::size_t prefillChunkSize = 0;
  // Requests whose prompts may share one chunk (1: one request per chunk,
  // as the reference's per-request prefillChunked).
  std::size_t prefillRequestsPerChunk = 1;
};

struct ServingRequestOutput {
  std::string id;
  std::vector<float> prefillLogits;
  std::vector<std::vector<float>> decodeLogits;
  std::vector<float> generatedTokenIds;
  double timeToFirstTokenUs = 0.0;
};

struct ServingMetrics {
  benchmark::Statistics decodeGpu;        // per batched step, GPU time
  benchmark::Statistics decodeEndToEnd;   // per batched step, host time
  double totalTimeUs = 0.0;
  double tokensPerSecond = 0.0;           // decodedTokens / totalTime
  double decodePhaseTokensPerSecond = 0.0;  // decode rows / time of steps with no prompt rows
  double schedulerOverheadUs = 0.0;
  double kvManagementOverheadUs = 0.0;
  double preemptionOverheadUs = 0.0;
  double averageActiveBatchSize = 0.0;
  std::size_t maximumActiveBatchSize = 0;
  std::size_t preemptionCount = 0;
  std::size_t spilledBytes = 0;           // KV pages copied to pinned host memory
  std::size_t resumeCount = 0;
  std::size_t peakPagesPerLayer = 0;
  std::size_t pageAllocationCount = 0;
  std::size_t pageReleaseCount = 0;
  std::size_t decodeCommandSubmissions = 0;
  std::size_t prefillChunkSubmissions = 0;  // chunked prefill stages run
  std::size_t decodedTokens = 0;
  std::size_t promptTokens = 0;
  std::size_t modelStorageBytes = 0;
  std::size_t kvPoolStorageBytes = 0;
  std::size_t batchedActivationStorageBytes = 0;
};

struct ServingExecutionResult {
  bool passed = false;
  std::vector<ServingRequestOutput> requests;
  ServingMetrics metrics;
  std::string errorMessage;
};

// One batched step as the scheduler sees it: tokens, valid lengths and
// per-layer tables in, next tokens (and logits when asked) out.
using BatchedStep = std::function<BatchedDecodeRun(
    const std::vector<std::int32_t>& tokens, const std::vector<std::int32_t>& validLengths,
    const std::vector<std::vector<std::int32_t>>& tables, bool readLogits)>;

// One prefill chunk: segments of up to `maxRequests` requests, each from a
// multiple of `tileRows` rows, at most `chunkRows` rows in all
// (ChunkedPrefillExecutor::runBatch).  Out: next tokens per segment row and,
// when asked, each segment's last-row logits.
using PrefillStep = std::function<BatchedDecodeRun(const std::vector<PrefillSegment>& segments,
                                                   bool readLogits)>;
struct PrefillPacking {
  std::size_t chunkRows = 0;
  std::size_t tileRows = 1;
  std::size_t maxRequests = 1;
};

// The scheduler over existing pools and any step function (the CPU tests
// drive it with host-only pools and a host step).  `prefill` is used when
// config.prefillChunkSize > 0.
[[nodiscard]] ServingExecutionResult runContinuousBatch(
    hip::HipRuntime& runtime, const planner::DecoderLLMPlan& plan,
    const std::vector<std::shared_ptr<KVPagePool>>& pools, std::size_t maximumBatchSize,
    std::size_t maxPages, const BatchedStep& step,
    const std::vector<ServingRequestSpec>& requests, const ServingConfig& config,
    std::ostream& log, const PrefillStep& prefill = {}, const PrefillPacking& packing = {});

// runContinuousBatch (ServingRuntime.cpp:513-930) on the GPU: creates the
// per-layer pools and the batched decode executor over `model`.
[[nodiscard]] ServingExecutionResult runContinuousBatch(
    hip::HipRuntime& runtime, std::shared_ptr<DecoderLLMModelResources> model,
    const std::vector<ServingRequestSpec>& requests, const ServingConfig& config,
    std::ostream& log);

// Steady-state decode throughput of `prompts.size()` requests decoding
// together: every prompt is first run through batched steps (prefill by
// decode, rows leave the batch when their prompt ends) or, with
// prefillChunkSize > 0, request by request through the chunked prefill
// executor (its library GEMM algorithms are chosen before the prompt phase
// starts); then all rows decode `decodeTokens` greedy tokens in lock-step.
// Both phases are timed on the host clock.
struct DecodeThroughput {
  bool passed = false;
  std::size_t rows = 0;
  std::size_t decodeSteps = 0;
  double promptPhaseUs = 0.0;
  double promptTokensPerSecond = 0.0;  // prompt tokens / promptPhaseUs
  std::size_t prefillChunkSize = 0;    // 0: prompts ran one token per batched step
  double decodePhaseUs = 0.0;      // host wall time of the timed steps
  double tokensPerSecond = 0.0;    // rows * decodeSteps / decodePhaseUs
  benchmark::Statistics stepGpu;   // per timed step, HIP-event time (timeGpu only)
  // per timed step, host wall time: the whole step with timeGpu, else the
  // enqueue time of a chained step (the GPU runs behind the host)
  benchmark::Statistics stepHost;
  std::vector<std::vector<float>> generatedTokenIds;  // per row
  std::size_t kvBytesRead = 0;     // K/V bytes the timed attention steps read
  // token-only tail of the decode bucket (BatchedDecodeExecutor::admitTokenOnly)
  bool tokenOnlyAvailable = false;
  bool tokenOnlyAdmitted = false;
  double tokenOnlySpeedup = 0.0;
  std::string errorMessage;
};

[[nodiscard]] DecodeThroughput measureDecodeThroughput(
    hip::HipRuntime& runtime, std::shared_ptr<DecoderLLMModelResources> model,
    const std::vector<std::vector<std::int32_t>>& prompts, std::size_t decodeTokens,
    std::size_t pageSize, bool timeGpu, bool tuneKernels = false,
    std::size_t prefillChunkSize = 0);

}  // namespace tensor::runtime
