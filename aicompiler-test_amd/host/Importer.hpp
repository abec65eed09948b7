// `.tmc` manifest importers: the decoder-only workload
// (importDecoderLLMWorkload, src/importer/DecoderLLMImporter.cpp:154-279) and
// the KV-cache attention workload (importKVCacheWorkload,
// src/importer/KVCacheImporter.cpp:95-200).
//
// A manifest is whitespace-separated text next to a raw little-endian float32
// payload:
//
//   TMC_DECODER_LLM <1|2>
//   MODEL "<name>"
//   PAYLOAD "<payload file, relative to the manifest>"
//   CONFIG batch hidden heads intermediate vocabulary layers capacity prefill decode epsilon
//   [DTYPE <requested> [<effective>, version 2]]          (F32 | F16 | BF16)
//   TENSORS <n>
//   TENSOR "<name>" <offset> <count>                       (n times, in floats)
//   END
//
//   TMC_KV_CACHE 1
//   MODEL "<name>"  PAYLOAD "<file>"
//   CONFIG batch heads head_dim capacity prefill decode
//   TENSORS <n>  TENSOR "<name>" <offset> <count> ...
//   STEPS <decode>
//   STEP <i> <q off> <q n> <k off> <k n> <v off> <v n> <out off> <out n> <kc off> <kc n> <vc off> <vc n>
//   END
//
// Errors come back in errorMessage with the reference's wording, the workload
// left empty.
#pragma once

#include "DecoderLLM.hpp"

#include <memory>
#include <string>
#include <vector>

namespace tensor::importer {

struct DecoderLLMImportResult {
  std::unique_ptr<DecoderLLMWorkload> workload;
  std::string errorMessage;
};

// Weights, RoPE tables and the PyTorch references of the prefill and every
// decode step (tokens, logits, next tokens, per-layer K/V caches
// [batch][heads][length][D]).  The plan's attention dtype is the manifest's
// effective dtype (F32 for a version-1 manifest without DTYPE); the gfx950
// decoder stores fp16 whatever it says.
[[nodiscard]] DecoderLLMImportResult importDecoderLLMWorkload(const std::string& manifestPath);

struct KVCacheReferenceStep {
  std::vector<float> query;
  std::vector<float> key;
  std::vector<float> value;
  std::vector<double> output;
  std::vector<double> keyCache;
  std::vector<double> valueCache;
};

struct ImportedKVCacheWorkload {
  std::string modelName;
  planner::KVCachePlan plan;
  std::vector<float> queryWeight;
  std::vector<float> keyWeight;
  std::vector<float> valueWeight;
  std::vector<float> outputWeight;
  KVCacheReferenceStep prefill;
  std::vector<KVCacheReferenceStep> decodeSteps;
};

struct KVCacheImportResult {
  std::unique_ptr<ImportedKVCacheWorkload> workload;
  std::string errorMessage;
};

[[nodiscard]] KVCacheImportResult importKVCacheWorkload(const std::string& manifestPath);

}  // namespace tensor::importer
