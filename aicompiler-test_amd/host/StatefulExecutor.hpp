// The KV-cache attention module (workloads/pytorch/KVCache.py,
// MultiHeadAttentionKVCache) as a stateful executor, with the interface of
// the reference's src/runtime/StatefulExecutor.hpp:14-63: q / k / v
// projections, the K and V projections appended to a contiguous cache
// [batch][heads][capacity][head_dim], attention of every query over every
// cached position (no mask, as the module runs), and the o projection.
//
// gfx950: the cache and all activations are fp16 (the reference module
// stores fp32; a Float32 plan is accepted and stored in fp16, as the decoder
// does), projections accumulate in fp32.  A call of S rows (prefill: the
// plan's prefillLength, decode: 1) per tensor batch runs as one prepared
// sequence:
//   q, k, v  = GEMMs of the inputs (decode_gemv up to 16 rows, else the
//              prompt GEMM gemm_rows);
//   k, v     -> kv_append at positions [valid - S, valid) (bit copies);
//   context  = decode attention over [0, valid) (S = 1), or for S > 1 the
//              paged kernel with the cache as one page per batch and every
//              row attending [0, valid);
//   output   = GEMM of the context with the o weight.
#pragma once

#include "HipRuntime.hpp"
#include "KVCacheState.hpp"

#include <iosfwd>
#include <memory>
#include <optional>
#include <string>
#include <vector>

namespace tensor::runtime {

struct KVCacheCompilation;

struct KVCacheRunResult {
  bool passed = false;
  std::vector<float> output;  // [batch * S, heads * head_dim]
  std::optional<double> gpuExecutionTimeUs;
  double cpuSubmitToCompletionTimeUs = 0.0;
  std::string errorMessage;
};

class CompiledKVCacheAttention {
 public:
  ~CompiledKVCacheAttention();
  CompiledKVCacheAttention(const CompiledKVCacheAttention&) = delete;
  CompiledKVCacheAttention& operator=(const CompiledKVCacheAttention&) = delete;

  [[nodiscard]] std::string reset();
  // Inputs are [batch, S, heads * head_dim] floats, converted to fp16.
  [[nodiscard]] KVCacheRunResult prefill(const std::vector<float>& query,
                                         const std::vector<float>& key,
                                         const std::vector<float>& value);
  // "KV cache capacity has been reached." once the cache is full; the state
  // (length and cache contents) is then unchanged.
  [[nodiscard]] KVCacheRunResult decode(const std::vector<float>& query,
                                        const std::vector<float>& key,
                                        const std::vector<float>& value);

  [[nodiscard]] std::size_t currentLength() const noexcept;
  [[nodiscard]] std::vector<float> readKeyPrefix() const;
  [[nodiscard]] std::vector<float> readValuePrefix() const;
  [[nodiscard]] bool cacheStorageReused() const noexcept;

 private:
  class Impl;
  explicit CompiledKVCacheAttention(std::unique_ptr<Impl> impl);
  friend KVCacheCompilation compileKVCacheAttention(hip::HipRuntime&, const planner::KVCachePlan&,
                                                    const std::vector<float>&,
                                                    const std::vector<float>&,
                                                    const std::vector<float>&,
                                                    const std::vector<float>&, std::ostream&);
  std::unique_ptr<Impl> impl_;
};

struct KVCacheCompilation {
  std::unique_ptr<CompiledKVCacheAttention> executable;
  std::string errorMessage;
};

// compileKVCacheAttention (StatefulExecutor.cpp:225-265): weights are
// [dim, dim] row-major (nn.Linear), dim = heads * head_dim.
[[nodiscard]] KVCacheCompilation compileKVCacheAttention(hip::HipRuntime& runtime,
                                                         const planner::KVCachePlan& plan,
                                                         const std::vector<float>& queryWeight,
                                                         const std::vector<float>& keyWeight,
                                                         const std::vector<float>& valueWeight,
                                                         const std::vector<float>& outputWeight,
                                                         std::ostream& log);

}  // namespace tensor::runtime
