// HipRuntime over the tmc_* C ABI; see HipRuntime.hpp.
#include "HipRuntime.hpp"

#include "tmc_hip.h"
#include "tmc_bench.h"

#include <utility>

namespace tensor::hip {
namespace {

std::string lastError(const char* fallback) {
  const char* text = tmc_last_error();
  return text && *text ? std::string(text) : std::string(fallback);
}

// Build the result of a finished call (the call runs before this is
// evaluated, so the timings it wrote are read after it).
ExecutionResult timed(int rc, double gpu, double cpu) {
  ExecutionResult result;
  result.cpuSubmitToCompletionTimeUs = cpu;
  if (rc != 0) {
    result.errorMessage = lastError("Execution failed.");
    return result;
  }
  if (gpu >= 0.0) result.gpuExecutionTimeUs = gpu;
  result.executionPassed = true;
  return result;
}

}  // namespace

std::size_t elementBytes(ElementType type) noexcept {
  return type == ElementType::Float16 || type == ElementType::BFloat16 ? 2u : 4u;
}

const char* elementTypeName(ElementType type) noexcept {
  switch (type) {
    case ElementType::Float16: return "f16";
    case ElementType::Float32: return "f32";
    case ElementType::BFloat16: return "bf16";
    case ElementType::Int32: return "i32";
  }
  return "?";
}

// ------------------------------------------------------------ interface checks
std::string checkFloatBufferInterface(const ComputePipelineResult& pipeline,
                                      std::size_t inputCount) {
  return checkBufferInterface(pipeline, std::vector<ElementType>(inputCount, ElementType::Float32),
                              ElementType::Float32);
}

std::string checkBufferInterface(const ComputePipelineResult& pipeline,
                                 const std::vector<ElementType>& inputs, ElementType output) {
  return checkBufferInterface(pipeline, inputs, std::vector<ElementType>{output});
}

std::string checkBufferInterface(const ComputePipelineResult& pipeline,
                                 const std::vector<ElementType>& inputs,
                                 const std::vector<ElementType>& outputs, bool uintConstants) {
  const std::size_t buffers = inputs.size() + outputs.size();
  const std::size_t expected = buffers + (uintConstants ? 1 : 0);
  if (outputs.empty() || !pipeline.reflectionAvailable || pipeline.bindings.size() != expected)
    return "Reflection must contain exactly the expected input and output buffers.";
  std::vector<bool> seen(expected, false);
  for (const auto& binding : pipeline.bindings) {
    if (!binding.isBuffer || binding.index >= expected || seen[binding.index])
      return "Expected unique buffer bindings at consecutive indices.";
    seen[binding.index] = true;
    if (binding.index == buffers) {
      if (!binding.isUInt32 || !binding.readOnly)
        return "Expected a read-only uint32 constants binding.";
      continue;
    }
    const bool isInput = binding.index < inputs.size();
    const ElementType want = isInput ? inputs[binding.index] : outputs[binding.index - inputs.size()];
    const bool matches = want == ElementType::Float32    ? binding.isFloat32
                         : want == ElementType::Float16  ? binding.isFloat16
                         : want == ElementType::BFloat16 ? binding.isBFloat16
                                                         : binding.isInt32;
    if (!matches) return "Reflected buffer element type disagrees with TensorIR.";
    if ((isInput && !binding.readOnly) || (!isInput && !binding.writable))
      return "Expected read-only inputs and a writable output buffer.";
  }
  return {};
}

// ------------------------------------------------------------------- HipBuffer
HipBuffer::~HipBuffer() {
  if (buffer_) tmc_buf_release(buffer_);
}

std::size_t HipBuffer::elementCount() const { return tmc_buf_count(buffer_); }

ElementType HipBuffer::elementType() const {
  return static_cast<ElementType>(tmc_buf_dtype(buffer_));
}

std::vector<float> HipBuffer::read() const {
  std::vector<float> out(elementCount());
  if (!out.empty() && tmc_buf_read(buffer_, out.data()) != 0) out.clear();
  return out;
}

std::string HipBuffer::readRaw(void* out, std::size_t count, std::size_t offset) const {
  if (count == 0) return {};
  return tmc_buf_read_raw(buffer_, out, count, offset) == 0 ? std::string()
                                                            : lastError("Buffer read failed.");
}

std::string HipBuffer::writeRaw(const void* data, std::size_t count, std::size_t offset) const {
  if (count == 0) return {};
  return tmc_buf_write_raw(buffer_, data, count, offset) == 0 ? std::string()
                                                              : lastError("Buffer write failed.");
}

std::string HipBuffer::writeRawAsync(const void* data, std::size_t count,
                                     std::size_t offset) const {
  if (count == 0) return {};
  return tmc_buf_write_raw_async(buffer_, data, count, offset) == 0
             ? std::string()
             : lastError("Buffer write failed.");
}

std::string HipBuffer::writeSparseAsync(const std::vector<std::int32_t>& pairs) const {
  if (pairs.empty()) return {};
  if (pairs.size() % 2 != 0) return "Sparse buffer write needs (index, value) pairs.";
  return tmc_buf_write_sparse_async(buffer_, pairs.data(), pairs.size() / 2) == 0
             ? std::string()
             : lastError("Buffer write failed.");
}

std::string HipBuffer::copyFromAsync(const HipBuffer& source, std::size_t count,
                                     std::size_t offset, std::size_t sourceOffset) const {
  if (count == 0) return {};
  return tmc_buf_copy_async(buffer_, offset, source.handle(), sourceOffset, count) == 0
             ? std::string()
             : lastError("Buffer copy failed.");
}

void* HipBuffer::devicePointer() const { return tmc_buf_device_ptr(buffer_); }

std::size_t HipBuffer::storageBytes() const { return elementCount() * elementBytes(elementType()); }

// ----------------------------------------------------------- PreparedExecution
PreparedExecution::~PreparedExecution() {
  if (exec_) tmc_exec_release(exec_);
}

ExecutionResult PreparedExecution::run() const {
  double gpu = -1.0, cpu = 0.0;
  const int rc = tmc_exec_run(exec_, 1, &gpu, &cpu);
  auto result = timed(rc, gpu, cpu);
  if (result.executionPassed && !outputs_.empty()) result.output = outputs_.front()->read();
  return result;
}

ExecutionResult PreparedExecution::execute() const {
  double gpu = -1.0, cpu = 0.0;
  const int rc = tmc_exec_run(exec_, 0, &gpu, &cpu);
  return timed(rc, gpu, cpu);
}

std::vector<std::vector<float>> PreparedExecution::readOutputs() const {
  std::vector<std::vector<float>> out;
  out.reserve(outputs_.size());
  for (const auto& buffer : outputs_) out.push_back(buffer->read());
  return out;
}

// ------------------------------------------------------------ PreparedSequence
PreparedSequence::~PreparedSequence() {
  if (seq_) tmc_seq_release(seq_);
}

ExecutionResult PreparedSequence::execute() const {
  double gpu = -1.0, cpu = 0.0;
  const int rc = tmc_seq_run(seq_, &gpu, &cpu);
  return timed(rc, gpu, cpu);
}

std::string PreparedSequence::launch() const {
  return tmc_seq_launch(seq_) == 0 ? std::string() : lastError("Sequence launch failed.");
}

// ------------------------------------------------------------------ HipRuntime
HipRuntime::HipRuntime() {
  if (tmc_rt_create(&runtime_) != 0) {
    createError_ = lastError("HIP runtime creation failed.");
    runtime_ = nullptr;
  }
}

HipRuntime::~HipRuntime() {
  current_.reset();
  if (runtime_) tmc_rt_destroy(runtime_);
}

HipRuntime::HipRuntime(HipRuntime&& other) noexcept
    : runtime_(std::exchange(other.runtime_, nullptr)),
      createError_(std::move(other.createError_)),
      current_(std::move(other.current_)),
      currentInfo_(std::move(other.currentInfo_)) {}

HipRuntime& HipRuntime::operator=(HipRuntime&& other) noexcept {
  if (this != &other) {
    current_.reset();
    if (runtime_) tmc_rt_destroy(runtime_);
    runtime_ = std::exchange(other.runtime_, nullptr);
    createError_ = std::move(other.createError_);
    current_ = std::move(other.current_);
    currentInfo_ = std::move(other.currentInfo_);
  }
  return *this;
}

bool HipRuntime::isAvailable() const noexcept {
  return runtime_ != nullptr && tmc_rt_is_available(runtime_) != 0;
}

std::string HipRuntime::deviceName() const {
  return runtime_ ? std::string(tmc_rt_device_name(runtime_)) : std::string();
}

std::string HipRuntime::initializationError() const {
  if (!runtime_) return createError_;
  return std::string(tmc_rt_init_error(runtime_));
}

HardwareInfo HipRuntime::hardwareInfo() const {
  HardwareInfo info;
  tmc_hardware_info raw{};
  if (runtime_ && tmc_rt_device_info(runtime_, &raw) == 0) {
    info.maxThreadsPerThreadgroup = raw.max_threads_per_threadgroup;
    info.maxThreadgroupMemoryLength = raw.max_threadgroup_memory_length;
    info.maxBufferLength = raw.max_buffer_length;
    info.supportsBFloat16 = raw.supports_bfloat16 != 0;
    info.computeUnits = raw.compute_units;
    info.waveSize = raw.wave_size;
  }
  return info;
}

ComputePipelineResult HipRuntime::createComputePipeline(const std::string& source,
                                                        const std::string& functionName) {
  current_.reset();
  currentInfo_ = ComputePipelineResult{};
  ComputePipelineResult result;
  if (!isAvailable()) {
    result.errorMessage = initializationError();
    return result;
  }
  result.libraryCompilePassed = true;
  tmc_kernel* kernel = nullptr;
  int count = 0;
  int types[32] = {}, writable[32] = {};
  if (tmc_kernel_resolve(runtime_, source.c_str(), &kernel, &count, types, writable) != 0) {
    result.errorMessage = functionName + ": " + lastError("Kernel lookup failed.");
    return result;
  }
  result.kernelLookupPassed = true;
  result.pipelineCreationPassed = true;
  result.reflectionAvailable = true;
  const HardwareInfo hw = hardwareInfo();
  result.threadExecutionWidth = static_cast<std::size_t>(hw.waveSize);
  result.maxTotalThreadsPerThreadgroup = hw.maxThreadsPerThreadgroup;
  for (int i = 0; i < count; ++i) {
    PipelineBinding b;
    b.index = static_cast<std::size_t>(i);
    b.isBuffer = true;
    b.isFloat16 = types[i] == TMC_F16;
    b.isFloat32 = types[i] == TMC_F32;
    b.isBFloat16 = types[i] == TMC_BF16;
    b.isInt32 = types[i] == TMC_I32;
    b.writable = writable[i] > 0;
    b.readOnly = writable[i] == 0;
    result.bindings.push_back(b);
  }
  std::size_t groups = 0, threads = 0;
  (void)tmc_kernel_dispatch(kernel, &groups, &threads);
  result.threadgroupCount = groups;
  result.threadsPerThreadgroup = threads;
  current_ = std::shared_ptr<tmc_kernel>(kernel, [](tmc_kernel* k) { tmc_kernel_release(k); });
  currentInfo_ = result;
  return result;
}

BufferResult HipRuntime::createBuffer(std::size_t elementCount, const float* initialData,
                                      ElementType type) const {
  BufferResult result;
  if (!isAvailable()) {
    result.errorMessage = initializationError();
    return result;
  }
  tmc_buffer* buffer = nullptr;
  if (tmc_buf_create(runtime_, elementCount, static_cast<int>(type), initialData, &buffer) != 0) {
    result.errorMessage = lastError("Buffer creation failed.");
    return result;
  }
  result.buffer = BufferHandle(new HipBuffer(buffer));
  return result;
}

BufferResult HipRuntime::wrapBuffer(void* devicePointer, std::size_t elementCount,
                                    ElementType type) const {
  BufferResult result;
  tmc_buffer* buffer = nullptr;
  if (!runtime_ ||
      tmc_buf_wrap(runtime_, devicePointer, elementCount, static_cast<int>(type), &buffer) != 0) {
    result.errorMessage = lastError("Buffer wrap failed.");
    return result;
  }
  result.buffer = BufferHandle(new HipBuffer(buffer));
  return result;
}

std::string HipRuntime::writeBuffer(const BufferHandle& buffer, const float* data,
                                    std::size_t elementCount, std::size_t elementOffset) const {
  if (!buffer) return "Cannot write a missing buffer.";
  if (tmc_buf_write(buffer->handle(), data, elementCount, elementOffset) != 0)
    return lastError("Buffer write failed.");
  return {};
}

PreparationResult HipRuntime::prepareBuffers(const std::vector<BufferHandle>& inputs,
                                             const BufferHandle& output,
                                             const DispatchSize& dispatch,
                                             const std::vector<std::uint32_t>& constants) const {
  return prepareBuffers(inputs, std::vector<BufferHandle>{output}, dispatch, constants);
}

PreparationResult HipRuntime::prepareBuffers(const std::vector<BufferHandle>& inputs,
                                             const std::vector<BufferHandle>& outputs,
                                             const DispatchSize& dispatch,
                                             const std::vector<std::uint32_t>& constants) const {
  PreparationResult result;
  if (!isAvailable()) {
    result.errorMessage = initializationError();
    return result;
  }
  if (!current_) {
    result.errorMessage = "Create a compute pipeline before execution.";
    return result;
  }
  std::vector<tmc_buffer*> in, out;
  for (const auto& b : inputs) in.push_back(b ? b->handle() : nullptr);
  for (const auto& b : outputs) out.push_back(b ? b->handle() : nullptr);
  tmc_exec* exec = nullptr;
  if (tmc_prepare(runtime_, current_.get(), in.data(), in.size(), out.data(), out.size(),
                  dispatch.threadgroupCount, dispatch.threadsPerThreadgroup,
                  constants.empty() ? nullptr : constants.data(), constants.size(), &exec) != 0) {
    result.errorMessage = lastError("Preparation failed.");
    return result;
  }
  result.execution.reset(new PreparedExecution(exec, inputs, outputs));
  return result;
}

PreparationResult HipRuntime::prepare(const std::vector<FloatBufferView>& inputs,
                                      std::size_t outputElementCount, const DispatchSize& dispatch,
                                      const std::vector<std::uint32_t>& constants,
                                      ElementType outputType) const {
  PreparationResult result;
  std::vector<BufferHandle> buffers;
  for (const auto& view : inputs) {
    auto created = createBuffer(view.elementCount, view.data, view.elementType);
    if (!created.buffer) {
      result.errorMessage = created.errorMessage;
      return result;
    }
    buffers.push_back(std::move(created.buffer));
  }
  auto output = createBuffer(outputElementCount, nullptr, outputType);
  if (!output.buffer) {
    result.errorMessage = output.errorMessage;
    return result;
  }
  return prepareBuffers(buffers, output.buffer, dispatch, constants);
}

ExecutionResult HipRuntime::run(const std::vector<FloatBufferView>& inputs,
                                std::size_t outputElementCount, const DispatchSize& dispatch,
                                const std::vector<std::uint32_t>& constants,
                                ElementType outputType) const {
  auto prepared = prepare(inputs, outputElementCount, dispatch, constants, outputType);
  if (!prepared.execution) {
    ExecutionResult result;
    result.errorMessage = prepared.errorMessage;
    return result;
  }
  return prepared.execution->run();
}

SequencePreparationResult HipRuntime::prepareSequence(
    const std::vector<const PreparedExecution*>& steps) const {
  SequencePreparationResult result;
  if (!isAvailable()) {
    result.errorMessage = initializationError();
    return result;
  }
  std::vector<tmc_exec*> handles;
  for (const auto* step : steps) handles.push_back(step ? step->handle() : nullptr);
  tmc_seq* seq = nullptr;
  if (tmc_seq_create(runtime_, handles.data(), handles.size(), &seq) != 0) {
    result.errorMessage = lastError("Sequence preparation failed.");
    return result;
  }
  result.execution.reset(new PreparedSequence(seq));
  return result;
}

void* HipRuntime::stream() const noexcept { return runtime_ ? tmc_rt_stream(runtime_) : nullptr; }

std::string HipRuntime::synchronize() const {
  if (!isAvailable()) return initializationError();
  return tmc_rt_synchronize(runtime_) == 0 ? std::string() : lastError("Synchronize failed.");
}

std::string HipRuntime::fillNormal(const BufferHandle& buffer, std::uint64_t seed, float mean,
                                   float stddev) const {
  if (!buffer) return "Cannot fill a missing buffer.";
  if (tmc_fill_normal(buffer->devicePointer(), static_cast<int>(buffer->elementType()),
                      static_cast<int64_t>(buffer->elementCount()), seed, mean, stddev,
                      stream()) != 0)
    return lastError("Fill failed.");
  return {};
}

void HipRuntime::failNext(int count) const {
  if (runtime_) tmc_rt_fail_next(runtime_, count);
}

}  // namespace tensor::hip
