// tensor::hip::HipRuntime — the method set of tensor::metal::MetalRuntime
// (reference src/backend/metal/MetalRuntime.hpp:10-208) restored in C++ on top
// of the C ABI of libtmc_hip.so (include/tmc_hip.h).  Host executors written
// against MetalRuntime call this class unchanged apart from the namespace.
//
// Conventions kept from the reference:
//  * no exceptions cross this API: results carry `errorMessage` ("" = OK);
//  * buffers take and return host floats converted per ElementType (fp16 ties
//    away from zero, bf16 round-to-nearest-even, int32 truncation);
//  * createComputePipeline() sets the current pipeline consumed by the next
//    prepare*/run call, and a new attempt clears it even when it fails
//    (MetalRuntime.hpp:172);
//  * bindings: inputs [0,n), outputs [n,n+m), optional uint32 constants last.
// The pipeline "source" is a gfx950 kernel key "name?k=v&..." (the string a
// gfx950 emitter returns), resolved by tmc_kernel_resolve.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <vector>

struct tmc_runtime;
struct tmc_buffer;
struct tmc_kernel;
struct tmc_exec;
struct tmc_seq;

namespace tensor::hip {

// Codes equal tmc_dtype (TMC_F16 = 0, TMC_F32 = 1, TMC_BF16 = 2, TMC_I32 = 3).
enum class ElementType { Float16 = 0, Float32 = 1, BFloat16 = 2, Int32 = 3 };

[[nodiscard]] std::size_t elementBytes(ElementType type) noexcept;
[[nodiscard]] const char* elementTypeName(ElementType type) noexcept;

struct HardwareInfo {
  std::size_t maxThreadsPerThreadgroup = 0;
  std::size_t maxThreadgroupMemoryLength = 0;  // LDS bytes per workgroup
  std::size_t maxBufferLength = 0;
  bool supportsBFloat16 = false;
  int computeUnits = 0;
  int waveSize = 0;
};

struct PipelineBinding {
  std::size_t index = 0;
  bool isBuffer = false;
  bool isFloat32 = false;
  bool isFloat16 = false;
  bool isBFloat16 = false;
  bool isInt32 = false;
  bool isUInt32 = false;
  bool readOnly = false;
  bool writable = false;
};

struct ComputePipelineResult {
  bool libraryCompilePassed = false;
  bool kernelLookupPassed = false;
  bool pipelineCreationPassed = false;
  std::size_t threadExecutionWidth = 0;
  std::size_t maxTotalThreadsPerThreadgroup = 0;
  std::size_t staticThreadgroupMemoryLength = 0;
  bool reflectionAvailable = false;
  std::vector<PipelineBinding> bindings;
  std::size_t threadgroupCount = 0;  // dispatch the kernel entry asks for
  std::size_t threadsPerThreadgroup = 0;
  std::string errorMessage;
};

// checkBufferInterface (MetalRuntime.hpp:46-53): the reflected bindings must be
// exactly the expected inputs (read-only), outputs (writable) and, when asked
// for, one read-only uint32 constants binding.
[[nodiscard]] std::string checkFloatBufferInterface(const ComputePipelineResult& pipeline,
                                                    std::size_t inputCount);
[[nodiscard]] std::string checkBufferInterface(const ComputePipelineResult& pipeline,
                                               const std::vector<ElementType>& inputs,
                                               ElementType output);
[[nodiscard]] std::string checkBufferInterface(const ComputePipelineResult& pipeline,
                                               const std::vector<ElementType>& inputs,
                                               const std::vector<ElementType>& outputs,
                                               bool uintConstants = false);

class HipRuntime;

// Device storage (MetalBuffer, MetalRuntime.hpp:56-71).  read() waits for the
// runtime stream, so it always sees completed work.
class HipBuffer {
 public:
  ~HipBuffer();
  HipBuffer(const HipBuffer&) = delete;
  HipBuffer& operator=(const HipBuffer&) = delete;
  [[nodiscard]] std::size_t elementCount() const;
  [[nodiscard]] ElementType elementType() const;
  [[nodiscard]] std::vector<float> read() const;
  // Raw storage bits (fp16/bf16 as uint16, fp32 as float bits, int32).
  [[nodiscard]] std::string readRaw(void* out, std::size_t count, std::size_t offset = 0) const;
  [[nodiscard]] std::string writeRaw(const void* data, std::size_t count,
                                     std::size_t offset = 0) const;
  // writeRaw queued on the runtime stream through pinned staging, without
  // waiting: later launches on the stream see the data.
  [[nodiscard]] std::string writeRawAsync(const void* data, std::size_t count,
                                          std::size_t offset = 0) const;
  // int32 buffers: values stored at increasing element indices (`pairs` =
  // index, value, index, value, ...), queued on the runtime stream like
  // writeRawAsync and applied by a kernel instead of a DMA copy.
  [[nodiscard]] std::string writeSparseAsync(const std::vector<std::int32_t>& pairs) const;
  // Device copy of `count` elements from `source` (same dtype), queued on
  // the runtime stream.
  [[nodiscard]] std::string copyFromAsync(const HipBuffer& source, std::size_t count,
                                          std::size_t offset = 0,
                                          std::size_t sourceOffset = 0) const;
  [[nodiscard]] void* devicePointer() const;
  [[nodiscard]] std::size_t storageBytes() const;
  [[nodiscard]] tmc_buffer* handle() const noexcept { return buffer_; }

 private:
  friend class HipRuntime;
  explicit HipBuffer(tmc_buffer* buffer) : buffer_(buffer) {}
  tmc_buffer* buffer_ = nullptr;
};

using BufferHandle = std::shared_ptr<HipBuffer>;

struct BufferResult {
  BufferHandle buffer;
  std::string errorMessage;
};

struct FloatBufferView {
  const float* data = nullptr;
  std::size_t elementCount = 0;
  ElementType elementType = ElementType::Float32;
};

struct DispatchSize {
  std::size_t threadgroupCount = 0;
  std::size_t threadsPerThreadgroup = 0;
};

struct ExecutionResult {
  bool executionPassed = false;
  std::vector<float> output;
  std::optional<double> gpuExecutionTimeUs;
  double cpuSubmitToCompletionTimeUs = 0.0;
  std::string errorMessage;
};

// PreparedExecution (MetalRuntime.hpp:101-122): owns its kernel entry and holds
// its buffers.
class PreparedExecution {
 public:
  ~PreparedExecution();
  PreparedExecution(const PreparedExecution&) = delete;
  PreparedExecution& operator=(const PreparedExecution&) = delete;
  // Reset every output to its sentinel, execute once and read the first output.
  [[nodiscard]] ExecutionResult run() const;
  // Execute once without readback.
  [[nodiscard]] ExecutionResult execute() const;
  [[nodiscard]] std::vector<std::vector<float>> readOutputs() const;
  [[nodiscard]] tmc_exec* handle() const noexcept { return exec_; }

 private:
  friend class HipRuntime;
  PreparedExecution(tmc_exec* exec, std::vector<BufferHandle> inputs,
                    std::vector<BufferHandle> outputs)
      : exec_(exec), inputs_(std::move(inputs)), outputs_(std::move(outputs)) {}
  tmc_exec* exec_ = nullptr;
  std::vector<BufferHandle> inputs_;
  std::vector<BufferHandle> outputs_;
};

struct PreparationResult {
  std::unique_ptr<PreparedExecution> execution;
  std::string errorMessage;
};

// PreparedSequence (MetalRuntime.hpp:130-142): the steps captured once into a
// HIP graph; execute() replays it and waits, launch() only enqueues.
class PreparedSequence {
 public:
  ~PreparedSequence();
  PreparedSequence(const PreparedSequence&) = delete;
  PreparedSequence& operator=(const PreparedSequence&) = delete;
  [[nodiscard]] ExecutionResult execute() const;
  [[nodiscard]] std::string launch() const;

 private:
  friend class HipRuntime;
  explicit PreparedSequence(tmc_seq* seq) : seq_(seq) {}
  tmc_seq* seq_ = nullptr;
};

struct SequencePreparationResult {
  std::unique_ptr<PreparedSequence> execution;
  std::string errorMessage;
};

class HipRuntime {
 public:
  HipRuntime();
  ~HipRuntime();
  HipRuntime(HipRuntime&&) noexcept;
  HipRuntime& operator=(HipRuntime&&) noexcept;
  HipRuntime(const HipRuntime&) = delete;
  HipRuntime& operator=(const HipRuntime&) = delete;

  [[nodiscard]] bool isAvailable() const noexcept;
  [[nodiscard]] std::string deviceName() const;
  [[nodiscard]] std::string initializationError() const;
  [[nodiscard]] HardwareInfo hardwareInfo() const;

  [[nodiscard]] ComputePipelineResult createComputePipeline(const std::string& source,
                                                            const std::string& functionName);

  [[nodiscard]] ExecutionResult run(const std::vector<FloatBufferView>& inputs,
                                    std::size_t outputElementCount, const DispatchSize& dispatch,
                                    const std::vector<std::uint32_t>& constants = {},
                                    ElementType outputType = ElementType::Float32) const;
  [[nodiscard]] PreparationResult prepare(const std::vector<FloatBufferView>& inputs,
                                          std::size_t outputElementCount,
                                          const DispatchSize& dispatch,
                                          const std::vector<std::uint32_t>& constants = {},
                                          ElementType outputType = ElementType::Float32) const;

  [[nodiscard]] BufferResult createBuffer(std::size_t elementCount,
                                          const float* initialData = nullptr,
                                          ElementType type = ElementType::Float32) const;
  // Device memory owned elsewhere (not freed by the runtime).
  [[nodiscard]] BufferResult wrapBuffer(void* devicePointer, std::size_t elementCount,
                                        ElementType type) const;
  [[nodiscard]] std::string writeBuffer(const BufferHandle& buffer, const float* data,
                                        std::size_t elementCount,
                                        std::size_t elementOffset = 0) const;
  [[nodiscard]] PreparationResult prepareBuffers(const std::vector<BufferHandle>& inputs,
                                                 const BufferHandle& output,
                                                 const DispatchSize& dispatch,
                                                 const std::vector<std::uint32_t>& constants = {})
      const;
  [[nodiscard]] PreparationResult prepareBuffers(const std::vector<BufferHandle>& inputs,
                                                 const std::vector<BufferHandle>& outputs,
                                                 const DispatchSize& dispatch,
                                                 const std::vector<std::uint32_t>& constants = {})
      const;
  [[nodiscard]] SequencePreparationResult prepareSequence(
      const std::vector<const PreparedExecution*>& steps) const;

  // gfx950 additions: the stream every execution uses, a wait on it, a
  // device-side normal fill (synthetic weights) and the failure-injection hook.
  [[nodiscard]] void* stream() const noexcept;
  [[nodiscard]] std::string synchronize() const;
  [[nodiscard]] std::string fillNormal(const BufferHandle& buffer, std::uint64_t seed,
                                       float mean, float stddev) const;
  void failNext(int count) const;
  [[nodiscard]] tmc_runtime* handle() const noexcept { return runtime_; }

 private:
  tmc_runtime* runtime_ = nullptr;
  std::string createError_;
  std::shared_ptr<tmc_kernel> current_;
  ComputePipelineResult currentInfo_;
};

}  // namespace tensor::hip
