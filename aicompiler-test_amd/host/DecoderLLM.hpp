// Decoder-LLM decode path on gfx950: model resources, the batched decode
// executor and the single-request CompiledDecoderLLM.
//
// Interfaces follow the reference:
//   planner::DecoderLLMPlan           src/planner/DecoderLLMPlan.hpp:9-23
//   DecoderLLMWorkload / parameters   src/tensor/DecoderLLM.hpp:10-44
//   DecoderLLMModelResources          src/runtime/DecoderLLMModelResources.hpp:10-41
//   CompiledDecoderLLM / compile      src/runtime/DecoderLLMExecutor.hpp:16-102
//   BatchedDecodeExecutor             src/runtime/ServingRuntime.cpp:119-407
//
// One decode step for m rows (rows >= active count are padding and leave the
// caches alone) runs, per layer l, as gfx950 kernels:
//   l == 0: embedding, RMSNorm                    -> x, n
//   l  > 0: Add+RMSNorm(after, mlp)               -> x = h(after + mlp), n
//   fused q|k|v GEMV [(QH+2KVH)*D, H]             -> qkv
//   RoPE(q, k) + paged append of k and v          -> q, pools
//   paged decode attention over [0, valid)        -> ctx
//   o GEMV, Add+RMSNorm(x, o)                     -> after = h(x + o), n
//   gate/up GEMV + SiLU*Mul, down GEMV            -> mlp
// then Add+RMSNorm with the final norm, the LM-head GEMV (fp32 logits) and
// argmax.  Every kernel output is stored in the storage dtype (fp16) before
// the next kernel reads it, as in DecoderLLMExecutor.cpp:322-849.  The whole
// step for one bucket of rows is captured once into a HIP graph.
#pragma once

#include "HipRuntime.hpp"
#include "KVCacheState.hpp"
#include "KernelRegistry.hpp"

#include <cstddef>
#include <cstdint>
#include <iosfwd>
#include <memory>
#include <optional>
#include <string>
#include <vector>

namespace tensor {

namespace planner {

struct DecoderLLMPlan {
  KVCachePlan attention;  // heads = query heads; batch = rows per step
  std::size_t layerCount = 1;
  std::size_t intermediateSize = 1;
  std::size_t vocabularySize = 1;
  float rmsNormEpsilon = 1e-5f;
  DType accumulationDtype = DType::Float32;
  // Grouped-query attention (an extension of the reference plan): key/value
  // heads, 0 = attention.heads.  attention.heads must be a multiple of it.
  std::size_t keyValueHeads = 0;

  [[nodiscard]] std::size_t hiddenSize() const;
  [[nodiscard]] std::size_t kvHeads() const noexcept {
    return keyValueHeads ? keyValueHeads : attention.heads;
  }
  [[nodiscard]] std::size_t kvWidth() const noexcept { return kvHeads() * attention.headDimension; }
  [[nodiscard]] std::size_t hiddenElementCount(std::size_t sequenceLength) const;
  [[nodiscard]] std::size_t intermediateElementCount(std::size_t sequenceLength) const;
  [[nodiscard]] std::size_t logitsElementCount(std::size_t sequenceLength) const;
  // DecoderLLMPlan.cpp:40-58 plus the GQA and fp16-storage rules of this
  // backend; throws std::invalid_argument.
  void validate() const;
  // KV plan of one layer's pool: one request, kvHeads heads.
  [[nodiscard]] KVCachePlan kvPlan() const;
};

}  // namespace planner

// Host weights as floats (values representable in the storage dtype), nn.Linear
// layout [out, in].  key/value weights are [kvHeads*D, hidden].
struct DecoderLLMLayerParameters {
  std::vector<float> inputNormWeight;
  std::vector<float> queryWeight;
  std::vector<float> keyWeight;
  std::vector<float> valueWeight;
  std::vector<float> outputWeight;
  std::vector<float> postAttentionNormWeight;
  std::vector<float> gateWeight;
  std::vector<float> upWeight;
  std::vector<float> downWeight;
};

// A step's reference results (src/tensor/DecoderLLM.hpp:22-28): tokens
// [batch, seq], logits [batch, seq, vocabulary], next tokens [batch], K/V
// caches per layer [batch, heads, length, D].
struct DecoderLLMReference {
  std::vector<float> tokenIds;
  std::vector<double> logits;
  std::vector<double> nextTokenIds;
  std::vector<std::vector<double>> keyCaches;
  std::vector<std::vector<double>> valueCaches;
};

struct DecoderLLMWorkload {
  std::string modelName;
  planner::DecoderLLMPlan plan;
  DType requestedStorageDtype = DType::Float32;
  std::size_t decodeCount = 0;
  std::vector<float> embeddingWeight;
  std::vector<float> finalNormWeight;
  std::vector<float> languageModelHeadWeight;
  std::vector<float> ropeCosine;  // [capacity, head_dim/2]
  std::vector<float> ropeSine;
  std::vector<DecoderLLMLayerParameters> layers;
  DecoderLLMReference prefill;  // filled by the .tmc importer
  std::vector<DecoderLLMReference> decodeSteps;
};

// RoPE tables as in workloads/pytorch/decoder_llm.py:48-55 (angle =
// position * theta^(-2i/D), evaluated in double, stored as fp32).
void ropeTables(std::size_t capacity, std::size_t headDimension, double theta,
                std::vector<float>& cosine, std::vector<float>& sine);

namespace runtime {

struct DecoderLLMModelLayerBuffers {
  hip::BufferHandle inputNormWeight;
  hip::BufferHandle queryKeyValueWeight;  // rows: q (QH*D) | k (KVH*D) | v (KVH*D)
  hip::BufferHandle outputWeight;
  hip::BufferHandle postAttentionNormWeight;
  hip::BufferHandle gateWeight;
  hip::BufferHandle upWeight;
  hip::BufferHandle downWeight;
};

// Immutable device model shared by every executor of one runtime.
struct DecoderLLMModelResources {
  DType storageDtype = DType::Float16;
  planner::DecoderLLMPlan plan;
  std::size_t hiddenSize = 0;
  std::size_t headCount = 0;
  std::size_t kvHeadCount = 0;
  std::size_t headDimension = 0;
  std::size_t cacheCapacity = 0;
  std::size_t intermediateSize = 0;
  std::size_t vocabularySize = 0;
  std::size_t layerCount = 0;
  std::size_t storageBytes = 0;
  hip::BufferHandle embeddingWeight;
  hip::BufferHandle finalNormWeight;
  hip::BufferHandle languageModelHeadWeight;
  hip::BufferHandle ropeCosine;
  hip::BufferHandle ropeSine;
  std::vector<DecoderLLMModelLayerBuffers> layers;
  // Fragment-packed copies of the matrices for the batch > 1 skinny GEMM
  // (tmc_pack_weights_f16), created by ensurePackedWeights as the buckets
  // need them.  Batch 1 keeps streaming the row-major weights, which the dot
  // GEMV reads faster.  packedLayers: o and down always; q.k.v, gate and up
  // (and packedLanguageModelHead) for buckets that run the norm kernels.
  // normScaledLayers: q.k.v (x input norm gamma), gate and up (x post-
  // attention norm gamma) and normScaledLanguageModelHead (x final norm
  // gamma), packed with tmc_pack_weights_scaled_f16 for buckets that fold
  // the norms into the projections.
  std::vector<DecoderLLMModelLayerBuffers> packedLayers;
  hip::BufferHandle packedLanguageModelHead;
  std::vector<DecoderLLMModelLayerBuffers> normScaledLayers;
  hip::BufferHandle normScaledLanguageModelHead;
  std::size_t packedBytes = 0;
};

// Create the packed copies a batch > 1 bucket needs, once per model
// (idempotent; "" on success): normScaled selects the gamma-scaled q.k.v,
// gate/up and LM head copies of the folded-norm buckets instead of the
// plain ones.
[[nodiscard]] std::string ensurePackedWeights(hip::HipRuntime& runtime,
                                              DecoderLLMModelResources& model,
                                              bool normScaled = false);

struct ModelResourcesCreation {
  std::shared_ptr<DecoderLLMModelResources> resources;
  std::string errorMessage;
};

// Upload a workload's weights (fp16 storage; q, k, v fused row-wise).
[[nodiscard]] ModelResourcesCreation createModelResources(hip::HipRuntime& runtime,
                                                          const DecoderLLMWorkload& workload);
// Random-init weights on the device: every matrix and the embedding
// ~ N(0, stddev) from seed + tensor index, norm weights 1, RoPE tables with
// `theta`.  No host copy of the weights is made.
[[nodiscard]] ModelResourcesCreation createSyntheticModelResources(
    hip::HipRuntime& runtime, const planner::DecoderLLMPlan& plan, std::uint64_t seed,
    float stddev = 0.02f, double theta = 10000.0);

struct BatchedDecodeRun {
  bool passed = false;
  std::vector<float> logits;        // [rows, vocabulary] when requested
  std::vector<float> nextTokenIds;  // [rows]
  std::optional<double> gpuExecutionTimeUs;
  double cpuSubmitToCompletionTimeUs = 0.0;
  std::string errorMessage;
};

// Decode steps for up to maximumBatchSize rows over per-layer page pools.
// Graphs are captured for row buckets 1, 2, 4, ... and maximumBatchSize; a
// step runs the smallest bucket that holds its rows.
class BatchedDecodeExecutor {
 public:
  struct Creation;
  ~BatchedDecodeExecutor();
  BatchedDecodeExecutor(const BatchedDecodeExecutor&) = delete;
  BatchedDecodeExecutor& operator=(const BatchedDecodeExecutor&) = delete;

  // ServingRuntime.cpp:155-226: tokens and valid lengths per row, block
  // tables per layer as [rows * maxPages()] (-1 = no page).  The new token of
  // row r lands at position validLengths[r] - 1.
  [[nodiscard]] BatchedDecodeRun run(const std::vector<float>& tokenIds,
                                     const std::vector<float>& validLengths,
                                     const std::vector<std::vector<float>>& blockTables,
                                     bool readLogits = true);
  [[nodiscard]] BatchedDecodeRun run(const std::vector<std::int32_t>& tokenIds,
                                     const std::vector<std::int32_t>& validLengths,
                                     const std::vector<std::vector<std::int32_t>>& blockTables,
                                     bool readLogits = true, bool timeGpu = false);

  // Chained decode: steps queued back to back with no host wait.  A step
  // with empty `tokenIds` takes the previous step's greedy tokens on the
  // device (same row count); every step's next tokens also go to history
  // slot `historyStep` (reserveHistory first).  readHistory waits for
  // the stream and returns [steps][maximumBatchSize()] token ids.  Same
  // checks and results as run(); the loop of measureDecodeThroughput.
  [[nodiscard]] std::string reserveHistory(std::size_t steps);
  [[nodiscard]] std::string launchChained(const std::vector<std::int32_t>& tokenIds,
                                          const std::vector<std::int32_t>& validLengths,
                                          const std::vector<std::vector<std::int32_t>>& blockTables,
                                          std::size_t historyStep);
  [[nodiscard]] std::string readHistory(std::size_t steps, std::vector<std::int32_t>& out) const;

  // Token-only steps (DecoderLLMExecutor.cpp:837-845,906-931): the folded
  // buckets (batch 1 with the norms folded, batch > 1 on packed weights)
  // also hold a second sequence whose tail is the LM head with a partial
  // argmax and a final argmax instead of the fp32 logits and the argmax.  A
  // step that reads no logits (run with readLogits false, every chained
  // step) uses it once admitted: at the bucket's first such step both
  // sequences replay the staged step (they append the same K/V), the tokens
  // must agree, and the token sequence must time >= 1.05x faster in two
  // paired rounds of 31 samples.  admitTokenOnly runs that check for the
  // bucket of these rows now (uploading their metadata), outside a timed
  // phase.  Decisions are kept per process and shape (model dimensions,
  // bucket rows, fold form), so a later executor of the same shape reuses
  // them.  TokenOnlyPolicy::Always skips the timing (tokens must still
  // agree), Never keeps the logits tail, CachedOnly uses the token tail only
  // where an earlier admission of this shape admitted it and never times
  // during steps (the serving loop's policy: no admission inside its ticks).
  enum class TokenOnlyPolicy { Admission, Always, Never, CachedOnly };
  void setTokenOnlyPolicy(TokenOnlyPolicy policy) noexcept { tokenPolicy_ = policy; }
  [[nodiscard]] std::string admitTokenOnly(const std::vector<std::int32_t>& tokenIds,
                                           const std::vector<std::int32_t>& validLengths,
                                           const std::vector<std::vector<std::int32_t>>& blockTables);
  struct TokenOnlyStatus {
    bool available = false;  // the bucket has a token-only sequence
    bool checked = false;
    bool admitted = false;
    double speedup = 0.0;    // min of the two paired rounds (0 when not timed)
  };
  // status of the bucket that runs steps of `rows` rows
  [[nodiscard]] TokenOnlyStatus tokenOnlyStatus(std::size_t rows) const;

  [[nodiscard]] std::size_t maximumBatchSize() const noexcept { return maximumBatchSize_; }
  [[nodiscard]] std::size_t maxPages() const noexcept { return maxPages_; }
  [[nodiscard]] std::size_t activationStorageBytes() const noexcept { return activationBytes_; }
  [[nodiscard]] std::vector<std::size_t> buckets() const;
  [[nodiscard]] std::size_t dispatchesPerStep(std::size_t bucket) const;
  [[nodiscard]] const std::vector<std::shared_ptr<KVPagePool>>& pools() const noexcept {
    return pools_;
  }

 private:
  friend struct Creation;
  friend Creation createBatchedDecodeExecutor(hip::HipRuntime&,
                                              std::shared_ptr<DecoderLLMModelResources>,
                                              std::vector<std::shared_ptr<KVPagePool>>,
                                              std::size_t, std::ostream*, bool,
                                              std::shared_ptr<KernelRegistry>, bool, bool);
  BatchedDecodeExecutor() = default;
  void build(std::ostream* log);
  [[nodiscard]] std::string upload(const std::vector<std::int32_t>& tokens,
                                   const std::vector<std::int32_t>& lengths,
                                   const std::vector<std::vector<std::int32_t>>& tables,
                                   std::size_t rows, std::size_t bucket);
  [[nodiscard]] std::string uploadTables(const std::vector<std::vector<std::int32_t>>& tables);
  [[nodiscard]] std::string checkStep(const std::vector<std::int32_t>* tokenIds,
                                      const std::vector<std::int32_t>& validLengths,
                                      const std::vector<std::vector<std::int32_t>>& blockTables) const;

  struct Bucket;
  // The sequence a step of `bucket` replays (metadata already uploaded).
  [[nodiscard]] std::string stepSequence(Bucket& bucket, bool readLogits,
                                         hip::PreparedSequence*& sequence);
  [[nodiscard]] std::string checkTokenOnly(Bucket& bucket);
  [[nodiscard]] std::string tokenOnlyKey(const Bucket& bucket) const;
  TokenOnlyPolicy tokenPolicy_ = TokenOnlyPolicy::Admission;
  hip::HipRuntime* runtime_ = nullptr;
  std::shared_ptr<DecoderLLMModelResources> model_;
  std::vector<std::shared_ptr<KVPagePool>> pools_;
  std::size_t maximumBatchSize_ = 0;
  std::size_t pageSize_ = 0;
  std::size_t maxPages_ = 0;
  bool tuneKernels_ = false;
  bool foldNorms_ = true;
  bool fuseAttentionOutput_ = false;
  std::shared_ptr<KernelRegistry> registry_;  // admitted region kernels, may be null
  std::size_t activationBytes_ = 0;
  // Device buffers sized for maximumBatchSize rows.
  hip::BufferHandle meta_;    // int32 [tokens M | lengths M | active 1]
  hip::BufferHandle tables_;  // int32 [layers][M][maxPages]
  hip::BufferHandle tokensView_, lengthsView_, activeView_;
  std::vector<hip::BufferHandle> tableViews_;
  hip::BufferHandle residual_, after_, normalized_, qkv_, query_, context_, projected_, gated_,
      mlp_, logits_, nextTokens_;
  hip::BufferHandle argmaxWorkspace_;  // partial-argmax slots of the token-only tail
  std::vector<std::unique_ptr<Bucket>> buckets_;
  std::vector<std::int32_t> metaShadow_, tableShadow_;
  hip::BufferHandle history_;  // int32 [steps][M], chained decode
  std::size_t historySteps_ = 0, chainedRows_ = 0;
  std::vector<std::int32_t> chainedLengths_;  // lengths the last chained step ran with
};

struct BatchedDecodeExecutor::Creation {
  std::unique_ptr<BatchedDecodeExecutor> executor;
  std::string errorMessage;
};

// tuneKernels: the batch-1 GEMVs use the decode GEMV tuner's selection for
// their shapes (tuned once per process on this model's weights and cached;
// planner::decodeGEMVTuningCache), instead of the default configurations.
// registry: admitted region kernels (KernelRegistry::load) that replace the
// template norm kernels where their contract shape matches the step (the
// one-row bucket at hidden 4096); each bucket's region launches are tracked
// in the registry's usage audit.
// foldNorms: the one-row bucket runs no norm kernel.  The o and down
// projections add the residual in their epilogue (emitLinearResidual,
// DecoderLLMMetalEmitter.cpp:604-622), and the q.k.v, gate/up and LM head
// GEMVs normalize the stored row in their prologue, in the summation order
// of the norm kernel the bucket would otherwise run, so results are the same
// bit for bit.  Applies when that norm holds one 16-byte chunk per thread
// (hidden <= 2048, or 4096) and no admitted region kernel replaces the norms.
// Buckets above one row fold them into the packed projections (hidden a
// multiple of 32): the residual stream stays in fragment order, o and down
// add the residual in their epilogue, and q.k.v + RoPE, gate/up and the LM
// head run over fp16(gamma * s) and scale each row by its 1/rms, so their
// results match the norm kernels within the fp16 path tolerance.
// fuseAttentionOutput: in that folded one-row bucket, each layer's paged
// attention and o projection + residual run as one launch
// (paged_attention_output, the fusion candidate of
// DecoderLLMExecutor.cpp:648-713) where its limits hold (head_dim 128, GQA
// group 1 or 2, pages of a multiple of 16 positions, capacity <= 1024).  Off
// by default: on MI355X it measured slower than the two launches at every
// context length (the reference admits the fusion only when it times faster).
[[nodiscard]] BatchedDecodeExecutor::Creation createBatchedDecodeExecutor(
    hip::HipRuntime& runtime, std::shared_ptr<DecoderLLMModelResources> model,
    std::vector<std::shared_ptr<KVPagePool>> pools, std::size_t maximumBatchSize,
    std::ostream* log = nullptr, bool tuneKernels = false,
    std::shared_ptr<KernelRegistry> registry = nullptr, bool foldNorms = true,
    bool fuseAttentionOutput = false);

// Chunked prefill (prefillChunked, DecoderLLMExecutor.cpp:982-1034): the
// tokens of one request's prompt chunk are the rows of one stage.  Linear
// layers are prompt GEMMs (MFMA GEMM, kernel key gemm_rows), RoPE and the
// cache append share the request's block table (prefill_rope_append) and
// attention is causal over the chunk (prefill_attention): row r of a chunk
// starting at position `start` attends [0, start + r + 1), which is what
// start + r + 1 decode steps would attend.  Stages are prepared for row
// buckets 16, 32, ... and chunkSize; a chunk runs the smallest that holds it
// (spare rows are computed and discarded).  Each stage is captured as a HIP
// graph when it is prepared.
// One request's part of a prefill chunk: tokens at positions start ..
// start + tokens - 1, block tables per layer as [maxPages()] holding pages
// for every position below start + tokens.
struct PrefillSegment {
  std::vector<std::int32_t> tokenIds;
  std::size_t start = 0;
  std::vector<std::vector<std::int32_t>> blockTables;
};

class ChunkedPrefillExecutor {
 public:
  struct Creation;
  ~ChunkedPrefillExecutor();
  ChunkedPrefillExecutor(const ChunkedPrefillExecutor&) = delete;
  ChunkedPrefillExecutor& operator=(const ChunkedPrefillExecutor&) = delete;

  // One request's segment.  Logits (when read) and next tokens are per row.
  [[nodiscard]] BatchedDecodeRun run(const std::vector<std::int32_t>& tokenIds, std::size_t start,
                                     const std::vector<std::vector<std::int32_t>>& blockTables,
                                     bool readLogits = true, bool timeGpu = false);
  // Up to maximumRequests() segments of different requests in one chunk:
  // each starts at a multiple of tileRows() rows (the attention kernel's
  // query tile), so packedRows(segments) must not exceed chunkSize().  Next
  // tokens are per segment row, in segment order; logits (when read) are
  // the last row's of each segment, [segments, vocabulary].
  [[nodiscard]] BatchedDecodeRun runBatch(const std::vector<PrefillSegment>& segments,
                                          bool readLogits = false, bool timeGpu = false);

  [[nodiscard]] std::size_t chunkSize() const noexcept { return chunkSize_; }
  [[nodiscard]] std::size_t maximumRequests() const noexcept { return maxRequests_; }
  [[nodiscard]] std::size_t tileRows() const noexcept { return tileRows_; }
  // Rows a chunk of segments with these token counts occupies.
  [[nodiscard]] std::size_t packedRows(const std::vector<std::size_t>& counts) const noexcept;
  [[nodiscard]] std::size_t maxPages() const noexcept { return maxPages_; }
  [[nodiscard]] std::size_t activationStorageBytes() const noexcept { return activationBytes_; }
  [[nodiscard]] std::vector<std::size_t> buckets() const;
  [[nodiscard]] std::size_t dispatchesPerChunk(std::size_t bucket) const;

 private:
  friend Creation createChunkedPrefillExecutor(hip::HipRuntime&,
                                               std::shared_ptr<DecoderLLMModelResources>,
                                               std::vector<std::shared_ptr<KVPagePool>>,
                                               std::size_t, std::ostream*, std::size_t);
  ChunkedPrefillExecutor() = default;
  void build(std::ostream* log);
  [[nodiscard]] std::string validate(const PrefillSegment& segment) const;

  struct Stage;
  hip::HipRuntime* runtime_ = nullptr;
  std::shared_ptr<DecoderLLMModelResources> model_;
  std::vector<std::shared_ptr<KVPagePool>> pools_;
  std::size_t chunkSize_ = 0;
  std::size_t maxRequests_ = 1;
  std::size_t tileRows_ = 64;
  std::size_t pageSize_ = 0;
  std::size_t maxPages_ = 0;
  std::size_t activationBytes_ = 0;
  hip::BufferHandle meta_;    // int32 [tokens S | lengths S | row tables S | active 1]
  hip::BufferHandle tables_;  // int32 [layers][maxRequests][maxPages]
  hip::BufferHandle tokensView_, lengthsView_, rowTableView_, activeView_;
  std::vector<hip::BufferHandle> tableViews_;
  hip::BufferHandle residual_, after_, normalized_, qkv_, query_, context_, projected_, gate_, up_,
      gated_, mlp_, logits_, nextTokens_, workspace_;
  std::vector<std::unique_ptr<Stage>> stages_;
  std::vector<std::int32_t> metaShadow_, tableShadow_;
};

struct ChunkedPrefillExecutor::Creation {
  std::unique_ptr<ChunkedPrefillExecutor> executor;
  std::string errorMessage;
};

// maximumRequests: segments one chunk may hold (1 = one request per chunk).
[[nodiscard]] ChunkedPrefillExecutor::Creation createChunkedPrefillExecutor(
    hip::HipRuntime& runtime, std::shared_ptr<DecoderLLMModelResources> model,
    std::vector<std::shared_ptr<KVPagePool>> pools, std::size_t chunkSize,
    std::ostream* log = nullptr, std::size_t maximumRequests = 1);

struct DecoderLLMCompileOptions {
  std::size_t kvPageSize = 0;  // 0 = contiguous cache (one page of `capacity`)
  std::size_t prefillChunkSize = 0;  // > 0: prefillChunked runs chunks of this many tokens
  std::vector<std::shared_ptr<KVPagePool>> sharedKVPools;
  DType storageDtype = DType::Float16;
  std::shared_ptr<DecoderLLMModelResources> sharedModelResources;
  // Directory of admitted region kernels (<dir>/decoder_*/admitted.json,
  // DecoderLLMExecutor.cpp:1319); empty = template kernels only.
  std::string kernelLibrary;
};

struct DecoderKVSnapshot {
  std::size_t length = 0;
  std::vector<std::vector<float>> keyCaches;    // per layer [kvHeads][length][D]
  std::vector<std::vector<float>> valueCaches;
};

struct DecoderLLMRunResult {
  bool passed = false;
  std::vector<float> logits;
  std::vector<float> nextTokenIds;
  std::optional<double> gpuExecutionTimeUs;
  double cpuSubmitToCompletionTimeUs = 0.0;
  std::string errorMessage;
};

struct DecoderLLMCompilation;

// One request (batch 1): per-layer KV states over private or shared pools
// and a one-row batched decode executor.  prefill() runs the prompt through
// decode steps, one token per step (a causal prefill: each position sees
// exactly the positions before it); prefillChunked() runs it through the
// chunked prefill executor when a chunk size was compiled.
class CompiledDecoderLLM {
 public:
  ~CompiledDecoderLLM();
  CompiledDecoderLLM(const CompiledDecoderLLM&) = delete;
  CompiledDecoderLLM& operator=(const CompiledDecoderLLM&) = delete;

  [[nodiscard]] std::string reset();
  [[nodiscard]] DecoderLLMRunResult prefill(const std::vector<float>& tokenIds,
                                            bool readLogits = true);
  // DecoderLLMExecutor.cpp:982-1034: the prompt in chunks of
  // prefillChunkSize() tokens through the chunked prefill stage (needs an
  // empty cache and a nonzero DecoderLLMCompileOptions::prefillChunkSize).
  // Logits are per prompt position; nextTokenIds holds the last chunk's.
  [[nodiscard]] DecoderLLMRunResult prefillChunked(const std::vector<float>& tokenIds,
                                                   bool readLogits = true);
  [[nodiscard]] DecoderLLMRunResult decode(const std::vector<float>& tokenIds,
                                           bool readLogits = true);
  [[nodiscard]] std::size_t prefillChunkSize() const noexcept;

  [[nodiscard]] std::size_t currentLength() const noexcept;
  [[nodiscard]] std::vector<float> readKeyPrefix(std::size_t layer) const;
  [[nodiscard]] std::vector<float> readValuePrefix(std::size_t layer) const;
  [[nodiscard]] bool cacheStorageReused() const noexcept;
  [[nodiscard]] bool usesPagedKVCache() const noexcept;
  [[nodiscard]] std::size_t kvPageSize() const noexcept;
  [[nodiscard]] std::size_t allocatedKVPageCount() const noexcept;
  [[nodiscard]] DType storageDtype() const noexcept { return DType::Float16; }
  [[nodiscard]] std::size_t modelStorageBytes() const noexcept;
  [[nodiscard]] std::size_t kvStorageBytes() const noexcept;
  [[nodiscard]] std::size_t activationStorageBytes() const noexcept;
  [[nodiscard]] std::shared_ptr<DecoderLLMModelResources> sharedModelResources() const noexcept;
  [[nodiscard]] std::vector<std::int32_t> kvBlockTable(std::size_t layer) const;
  [[nodiscard]] DecoderKVSnapshot snapshotKVCache() const;
  [[nodiscard]] std::string releaseKVCache();
  [[nodiscard]] std::string restoreKVCache(const DecoderKVSnapshot& snapshot);
  [[nodiscard]] std::string stageKVLength(std::size_t length);
  void commitKVLength(std::size_t length);
  [[nodiscard]] std::string rollbackKVLength(std::size_t length);
  // The kernel registry's usage audit since the last reset (KernelRegistry::
  // report; DecoderLLMExecutor.cpp:1192-1196).
  [[nodiscard]] std::string kernelUsageReport(bool reset = false) const;

 private:
  class Impl;
  explicit CompiledDecoderLLM(std::unique_ptr<Impl> impl);
  friend DecoderLLMCompilation compileDecoderLLM(hip::HipRuntime&, const DecoderLLMWorkload&,
                                                 std::ostream&, const DecoderLLMCompileOptions&);
  std::unique_ptr<Impl> impl_;
};

struct DecoderLLMCompilation {
  std::unique_ptr<CompiledDecoderLLM> executable;
  std::string errorMessage;
};

// compileDecoderLLM (DecoderLLMExecutor.cpp:1100-1441): model weights come
// from options.sharedModelResources when given, else from the workload.
[[nodiscard]] DecoderLLMCompilation compileDecoderLLM(hip::HipRuntime& runtime,
                                                      const DecoderLLMWorkload& workload,
                                                      std::ostream& log,
                                                      const DecoderLLMCompileOptions& options = {});

}  // namespace runtime
}  // namespace tensor
