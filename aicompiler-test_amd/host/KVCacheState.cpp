// KVPagePool / KVCacheState on HipRuntime; see KVCacheState.hpp.
#include "KVCacheState.hpp"

#include "tmc_hip.h"

#include <algorithm>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <tuple>
#include <utility>

namespace tensor {

const char* dtypeName(DType dtype) noexcept {
  switch (dtype) {
    case DType::Float16: return "fp16";
    case DType::Float32: return "fp32";
    case DType::BFloat16: return "bf16";
    case DType::Int32: return "int32";
  }
  return "?";
}

std::size_t dtypeStorageBytes(DType dtype) noexcept {
  return dtype == DType::Float16 || dtype == DType::BFloat16 ? 2u : 4u;
}

namespace {

std::size_t checkedMultiply(std::size_t left, std::size_t right, const char* what) {
  if (left != 0 && right > std::numeric_limits<std::size_t>::max() / left)
    throw std::overflow_error(what);
  return left * right;
}

hip::ElementType storageType(DType dtype) {
  switch (dtype) {
    case DType::Float16: return hip::ElementType::Float16;
    case DType::Float32: return hip::ElementType::Float32;
    case DType::BFloat16: return hip::ElementType::BFloat16;
    case DType::Int32: return hip::ElementType::Int32;
  }
  throw std::invalid_argument("Unsupported KV cache storage dtype.");
}

}  // namespace

namespace planner {

std::size_t KVCachePlan::modelDimension() const {
  return checkedMultiply(heads, headDimension, "KV cache tensor size exceeds size_t capacity.");
}

std::size_t KVCachePlan::cacheElementCount() const {
  const char* what = "KV cache tensor size exceeds size_t capacity.";
  return checkedMultiply(checkedMultiply(batch, heads, what),
                         checkedMultiply(capacity, headDimension, what), what);
}

std::size_t KVCachePlan::inputElementCount(std::size_t sequenceLength) const {
  return checkedMultiply(checkedMultiply(batch, sequenceLength,
                                         "KV cache tensor size exceeds size_t capacity."),
                         modelDimension(), "KV cache tensor size exceeds size_t capacity.");
}

void KVCachePlan::validate() const {
  if (batch == 0 || heads == 0 || headDimension == 0 || capacity == 0 || prefillLength == 0 ||
      prefillLength > capacity)
    throw std::invalid_argument("KV cache dimensions and prefill length must be valid.");
  if (dtype != DType::Float16 && dtype != DType::Float32 && dtype != DType::BFloat16)
    throw std::invalid_argument("KV cache storage dtype is unsupported.");
  if (threadsPerThreadgroup == 0 || threadsPerThreadgroup > 1024 ||
      (threadsPerThreadgroup & (threadsPerThreadgroup - 1)) != 0)
    throw std::invalid_argument("KV cache threadgroup size must be a power of two in [1, 1024].");
  if (headDimension > threadsPerThreadgroup)
    throw std::invalid_argument("KV attention requires head dimension <= threadgroup size.");
  (void)cacheElementCount();
  (void)inputElementCount(prefillLength);
}

}  // namespace planner

namespace runtime {

float halfToFloat(std::uint16_t bits) noexcept {
  float value = 0.0f;
  tmc_host_decode(&bits, 1, TMC_F16, &value);
  return value;
}

// ------------------------------------------------------------------ KVPagePool
KVPagePool::KVPagePool(planner::KVCachePlan plan, std::size_t pageSize, hip::BufferHandle key,
                       hip::BufferHandle value, std::size_t physicalPageCount)
    : plan_(std::move(plan)),
      pageSize_(pageSize),
      key_(std::move(key)),
      value_(std::move(value)),
      link_(physicalPageCount),
      freeCount_(physicalPageCount) {
  // Free stack N-1 (top), N-2, ..., 0 (bottom): page p rests on page p - 1.
  for (std::size_t p = 0; p < physicalPageCount; ++p)
    link_[p] = static_cast<std::int32_t>(p) - 1;
  top_ = static_cast<std::int32_t>(physicalPageCount) - 1;
}

std::int32_t KVPagePool::allocatePage() {
  if (top_ == kBottom) return -1;
  const std::int32_t page = top_;
  std::int32_t& link = link_[static_cast<std::size_t>(page)];
  top_ = link;
  link = kLent;
  --freeCount_;
  ++tally_.lent;
  if (usedPages() > tally_.peak) tally_.peak = usedPages();
  return page;
}

void KVPagePool::releasePage(std::int32_t page) {
  if (!isAllocated(page))
    throw std::invalid_argument("Paged KV attempted to release an invalid page.");
  link_[static_cast<std::size_t>(page)] = top_;
  top_ = page;
  ++freeCount_;
  ++tally_.returned;
}

bool KVPagePool::compatible(const planner::KVCachePlan& plan) const noexcept {
  const auto shape = [](const planner::KVCachePlan& q) {
    return std::make_tuple(q.batch, q.heads, q.headDimension, q.dtype);
  };
  return shape(plan) == shape(plan_);
}

namespace {

void checkPoolShape(const planner::KVCachePlan& plan, std::size_t pageSize,
                    std::size_t physicalPageCount) {
  plan.validate();
  if (plan.batch != 1)
    throw std::invalid_argument("Shared paged KV pool supports one tensor batch per request.");
  if (pageSize == 0 || pageSize > plan.capacity || physicalPageCount == 0 ||
      physicalPageCount > static_cast<std::size_t>(std::numeric_limits<std::int32_t>::max()))
    throw std::invalid_argument("Shared paged KV pool dimensions are invalid.");
}

}  // namespace

KVPagePoolCreation createKVPagePool(hip::HipRuntime& runtime, const planner::KVCachePlan& plan,
                                    std::size_t pageSize, std::size_t physicalPageCount) {
  KVPagePoolCreation result;
  try {
    checkPoolShape(plan, pageSize, physicalPageCount);
    const char* what = "Paged KV storage size exceeds size_t capacity.";
    std::size_t count = checkedMultiply(physicalPageCount, pageSize, what);
    count = checkedMultiply(count, plan.batch, what);
    count = checkedMultiply(count, plan.heads, what);
    count = checkedMultiply(count, plan.headDimension, what);
    const auto type = storageType(plan.dtype);
    auto key = runtime.createBuffer(count, nullptr, type);
    if (!key.buffer) throw std::runtime_error(key.errorMessage);
    auto value = runtime.createBuffer(count, nullptr, type);
    if (!value.buffer) throw std::runtime_error(value.errorMessage);
    result.pool.reset(new KVPagePool(plan, pageSize, std::move(key.buffer),
                                     std::move(value.buffer), physicalPageCount));
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

KVPagePoolCreation createHostKVPagePool(const planner::KVCachePlan& plan, std::size_t pageSize,
                                        std::size_t physicalPageCount) {
  KVPagePoolCreation result;
  try {
    checkPoolShape(plan, pageSize, physicalPageCount);
    result.pool.reset(new KVPagePool(plan, pageSize, nullptr, nullptr, physicalPageCount));
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

// ---------------------------------------------------------------- KVCacheState
KVCacheState::KVCacheState(planner::KVCachePlan plan, hip::BufferHandle key,
                           hip::BufferHandle value, hip::BufferHandle length,
                           hip::BufferHandle blockTable, std::shared_ptr<KVPagePool> pagePool)
    : plan_(std::move(plan)),
      key_(std::move(key)),
      value_(std::move(value)),
      length_(std::move(length)),
      blockTable_(std::move(blockTable)),
      initialKey_(key_.get()),
      initialValue_(value_.get()),
      pageSize_(pagePool ? pagePool->pageSize() : 0),
      pagePool_(std::move(pagePool)) {
  if (pageSize_ != 0) {
    tableSlots_ = pagesFor(plan_.capacity);
    pages_.reserve(tableSlots_);
  }
}

KVCacheState::~KVCacheState() {
  // The pages go back first to last (the reference's destructor order), so
  // the last logical page ends on top of the pool's free stack.
  if (!pagePool_) return;
  for (const std::int32_t page : pages_) {
    try {
      pagePool_->releasePage(page);
    } catch (...) {
    }
  }
}

std::string KVCacheState::writeLength(hip::HipRuntime& runtime, std::size_t length) {
  if (!length_) return {};
  const float value = static_cast<float>(length);
  return runtime.writeBuffer(length_, &value, 1);
}

std::string KVCacheState::reset(hip::HipRuntime& runtime) {
  auto error = writeLength(runtime, 0);
  if (error.empty() && isPaged()) {
    (void)resizePageAllocation(0);  // shrinking always succeeds
    error = writeBlockTable(runtime);
  }
  if (error.empty()) currentLength_ = 0;
  return error;
}

std::string KVCacheState::stageLength(hip::HipRuntime& runtime, std::size_t length) {
  if (length == 0 || length > plan_.capacity)
    return "KV cache valid length is outside the configured capacity.";
  if (!isPaged()) return writeLength(runtime, length);
  if (pagesFor(length) > tableSlots_)
    return "Paged KV cache has no block-table capacity for this length.";
  const std::size_t kept = pages_.size();
  auto error = resizePageAllocation(pagesFor(length));
  if (!error.empty()) return error;
  error = writeBlockTable(runtime);
  if (error.empty()) {
    error = writeLength(runtime, length);
    if (error.empty()) return {};
    // the table already names the new pages: put the old set back on both sides
    (void)resizePageAllocation(kept);
    (void)writeBlockTable(runtime);
    return error;
  }
  (void)resizePageAllocation(kept);
  return error;
}

std::string KVCacheState::rollbackLength(hip::HipRuntime& runtime, std::size_t length) {
  if (length > plan_.capacity) return "Cannot roll back KV cache beyond its configured capacity.";
  if (isPaged()) {
    auto error = resizePageAllocation(pagesFor(length));
    if (error.empty()) error = writeBlockTable(runtime);
    if (!error.empty()) return error;
  }
  return writeLength(runtime, length);
}

std::string KVCacheState::restore(hip::HipRuntime& runtime, std::size_t length,
                                  const std::vector<float>& keyPrefix,
                                  const std::vector<float>& valuePrefix) {
  if (!isPaged()) return "KV cache restore requires paged storage.";
  if (currentLength_ != 0) return "KV cache restore requires an empty request state.";
  const std::size_t expected = plan_.batch * plan_.heads * length * plan_.headDimension;
  if (length == 0 || length > plan_.capacity || keyPrefix.size() != expected ||
      valuePrefix.size() != expected)
    return "KV cache restore snapshot shape is invalid.";
  auto error = stageLength(runtime, length);
  if (error.empty()) error = writePagedPrefix(runtime, key_, keyPrefix, length);
  if (error.empty()) error = writePagedPrefix(runtime, value_, valuePrefix, length);
  if (!error.empty()) {
    (void)rollbackLength(runtime, 0);
    return error;
  }
  commitLength(length);
  return {};
}

namespace {
constexpr std::size_t kSpillHeader = 256;  // bytes reserved ahead of the pages
}

std::string KVCacheState::spillPages(hip::HipRuntime& runtime, KVPageSpill& out) const {
  if (!isPaged() || !key_ || !value_) return "KV page spill requires paged device storage.";
  out = KVPageSpill{};
  out.length = currentLength_;
  out.pages = (currentLength_ + pageSize_ - 1) / pageSize_;
  out.pageBytes = plan_.batch * plan_.heads * pageSize_ * plan_.headDimension *
                  hip::elementBytes(key_->elementType());
  if (out.pages == 0) return {};
  const std::size_t header =
      (out.pages * sizeof(std::int32_t) + kSpillHeader - 1) / kSpillHeader * kSpillHeader;
  void* raw = nullptr;
  if (tmc_host_alloc(header + out.bytes(), &raw) != 0) return tmc_last_error();
  out.host = std::shared_ptr<void>(raw, [](void* p) { tmc_host_free(p); });
  auto* ids = static_cast<std::int32_t*>(raw);
  for (std::size_t i = 0; i < out.pages; ++i) ids[i] = pages_.at(i);
  auto* pagesBase = static_cast<unsigned char*>(raw) + header;
  const auto count = static_cast<std::int64_t>(out.pages);
  const auto bytes = static_cast<std::int64_t>(out.pageBytes);
  if (tmc_copy_pages(key_->devicePointer(), pagesBase, ids, count, bytes, 0, runtime.stream()) != 0 ||
      tmc_copy_pages(value_->devicePointer(), pagesBase + out.pages * out.pageBytes, ids, count,
                     bytes, 0, runtime.stream()) != 0)
    return tmc_last_error();
  return runtime.synchronize();
}

std::string KVCacheState::restorePages(hip::HipRuntime& runtime, const KVPageSpill& spill) {
  if (!isPaged() || !key_ || !value_) return "KV page restore requires paged device storage.";
  if (currentLength_ != 0) return "KV page restore requires an empty request state.";
  const std::size_t pageBytes = plan_.batch * plan_.heads * pageSize_ * plan_.headDimension *
                                hip::elementBytes(key_->elementType());
  if (!spill.host || spill.length == 0 || spill.length > plan_.capacity ||
      spill.pages != (spill.length + pageSize_ - 1) / pageSize_ || spill.pageBytes != pageBytes)
    return "KV page restore: the spill does not match this state.";
  auto error = stageLength(runtime, spill.length);
  if (!error.empty()) return error;
  const std::size_t header =
      (spill.pages * sizeof(std::int32_t) + kSpillHeader - 1) / kSpillHeader * kSpillHeader;
  auto* ids = static_cast<std::int32_t*>(spill.host.get());
  for (std::size_t i = 0; i < spill.pages; ++i) ids[i] = pages_.at(i);
  const auto* pagesBase = static_cast<const unsigned char*>(spill.host.get()) + header;
  const auto count = static_cast<std::int64_t>(spill.pages);
  const auto bytes = static_cast<std::int64_t>(pageBytes);
  if (tmc_copy_pages(pagesBase, key_->devicePointer(), ids, count, bytes, 1, runtime.stream()) != 0 ||
      tmc_copy_pages(pagesBase + spill.pages * pageBytes, value_->devicePointer(), ids, count, bytes,
                     1, runtime.stream()) != 0)
    error = tmc_last_error();
  if (error.empty()) error = runtime.synchronize();
  if (!error.empty()) {
    (void)rollbackLength(runtime, 0);
    return error;
  }
  commitLength(spill.length);
  return {};
}

void KVCacheState::commitLength(std::size_t length) {
  if (length == 0 || length > plan_.capacity)
    throw std::invalid_argument("Cannot commit an invalid KV cache length.");
  currentLength_ = length;
}

std::vector<float> KVCacheState::readPrefix(const hip::BufferHandle& buffer) const {
  const std::size_t B = plan_.batch, H = plan_.heads, D = plan_.headDimension;
  const std::size_t L = currentLength_;
  std::vector<float> result(B * H * L * D);
  if (!buffer || L == 0) return result;
  const std::size_t bytes = hip::elementBytes(buffer->elementType());
  auto convert = [&](const std::vector<unsigned char>& raw, std::size_t index) -> float {
    if (buffer->elementType() == hip::ElementType::Float16) {
      std::uint16_t bits;
      std::memcpy(&bits, raw.data() + index * 2, 2);
      return halfToFloat(bits);
    }
    if (buffer->elementType() == hip::ElementType::BFloat16) {
      std::uint16_t bits;
      std::memcpy(&bits, raw.data() + index * 2, 2);
      const std::uint32_t wide = static_cast<std::uint32_t>(bits) << 16;
      float value;
      std::memcpy(&value, &wide, 4);
      return value;
    }
    float value;
    std::memcpy(&value, raw.data() + index * 4, 4);
    return value;
  };
  if (!isPaged()) {
    // [batch][heads][capacity][D]: one copy per (batch, head) row block.
    std::vector<unsigned char> raw(L * D * bytes);
    for (std::size_t b = 0; b < B; ++b)
      for (std::size_t h = 0; h < H; ++h) {
        if (!buffer->readRaw(raw.data(), L * D, ((b * H + h) * plan_.capacity) * D).empty())
          return {};
        for (std::size_t i = 0; i < L * D; ++i)
          result[((b * H + h) * L) * D + i] = convert(raw, i);
      }
    return result;
  }
  // Paged: one copy per logical page, [page][batch][heads][page_size][D].
  const std::size_t P = pageSize_, pageElements = B * H * P * D;
  std::vector<unsigned char> raw(pageElements * bytes);
  for (std::size_t logical = 0; logical * P < L; ++logical) {
    const auto physical = static_cast<std::size_t>(pages_.at(logical));
    if (!buffer->readRaw(raw.data(), pageElements, physical * pageElements).empty()) return {};
    const std::size_t first = logical * P, last = std::min(L, first + P);
    for (std::size_t b = 0; b < B; ++b)
      for (std::size_t h = 0; h < H; ++h)
        for (std::size_t pos = first; pos < last; ++pos)
          for (std::size_t d = 0; d < D; ++d)
            result[((b * H + h) * L + pos) * D + d] =
                convert(raw, ((b * H + h) * P + (pos - first)) * D + d);
  }
  return result;
}

std::vector<float> KVCacheState::readKeyPrefix() const { return readPrefix(key_); }
std::vector<float> KVCacheState::readValuePrefix() const { return readPrefix(value_); }

bool KVCacheState::storageReused() const noexcept {
  return key_.get() == initialKey_ && value_.get() == initialValue_;
}

std::size_t KVCacheState::allocatedPageCount() const noexcept { return pages_.size(); }

std::vector<std::int32_t> KVCacheState::pageTable() const { return pages_; }

std::string KVCacheState::writeBlockTable(hip::HipRuntime& runtime) {
  if (!isPaged() || !blockTable_) return {};
  (void)runtime;
  std::vector<std::int32_t> table(tableSlots_, -1);  // unowned slots read as missing
  std::copy(pages_.begin(), pages_.end(), table.begin());
  return blockTable_->writeRaw(table.data(), table.size());
}

std::string KVCacheState::writePagedPrefix(hip::HipRuntime& runtime,
                                           const hip::BufferHandle& buffer,
                                           const std::vector<float>& prefix, std::size_t length) {
  if (!buffer) return {};
  // Gather each page on the host ([batch][heads][page_size][D]) and write it
  // with one converting copy; slots beyond `length` in the last page are
  // written as zero (they are outside every valid range).
  const std::size_t B = plan_.batch, H = plan_.heads, D = plan_.headDimension, P = pageSize_;
  const std::size_t pageElements = B * H * P * D;
  std::vector<float> page(pageElements);
  for (std::size_t logical = 0; logical * P < length; ++logical) {
    std::fill(page.begin(), page.end(), 0.0f);
    const std::size_t first = logical * P, last = std::min(length, first + P);
    for (std::size_t b = 0; b < B; ++b)
      for (std::size_t h = 0; h < H; ++h)
        for (std::size_t pos = first; pos < last; ++pos)
          std::copy_n(prefix.begin() + static_cast<std::ptrdiff_t>(((b * H + h) * length + pos) * D),
                      D, page.begin() + static_cast<std::ptrdiff_t>(((b * H + h) * P + pos - first) * D));
    const auto physical = static_cast<std::size_t>(pages_.at(logical));
    auto error = runtime.writeBuffer(buffer, page.data(), pageElements, physical * pageElements);
    if (!error.empty()) return error;
  }
  return {};
}

std::string KVCacheState::resizePageAllocation(std::size_t pageCount) {
  if (pageCount > pages_.size()) {
    if (pageCount - pages_.size() > pagePool_->availablePages())
      return "Paged KV cache physical page pool is exhausted.";
    while (pages_.size() < pageCount) pages_.push_back(pagePool_->allocatePage());
    return {};
  }
  while (pages_.size() > pageCount) {
    pagePool_->releasePage(pages_.back());
    pages_.pop_back();
  }
  return {};
}

KVCacheStateCreation createKVCacheState(hip::HipRuntime& runtime,
                                        const planner::KVCachePlan& plan, std::size_t pageSize) {
  KVCacheStateCreation result;
  try {
    plan.validate();
    if (pageSize > plan.capacity)
      throw std::invalid_argument("Paged KV page size exceeds cache capacity.");
    if (pageSize != 0 && plan.batch != 1)
      throw std::invalid_argument("Paged KV cache currently supports one request.");
    if (pageSize != 0) {
      auto pool = createKVPagePool(runtime, plan, pageSize, (plan.capacity + pageSize - 1) / pageSize);
      if (!pool.pool) throw std::runtime_error(pool.errorMessage);
      return createKVCacheState(runtime, plan, std::move(pool.pool));
    }
    const auto type = storageType(plan.dtype);
    auto key = runtime.createBuffer(plan.cacheElementCount(), nullptr, type);
    if (!key.buffer) throw std::runtime_error(key.errorMessage);
    auto value = runtime.createBuffer(plan.cacheElementCount(), nullptr, type);
    if (!value.buffer) throw std::runtime_error(value.errorMessage);
    const float zero = 0.0f;
    auto length = runtime.createBuffer(1, &zero, hip::ElementType::Int32);
    if (!length.buffer) throw std::runtime_error(length.errorMessage);
    result.state.reset(new KVCacheState(plan, std::move(key.buffer), std::move(value.buffer),
                                        std::move(length.buffer), nullptr, nullptr));
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

KVCacheStateCreation createKVCacheState(hip::HipRuntime& runtime,
                                        const planner::KVCachePlan& plan,
                                        std::shared_ptr<KVPagePool> pagePool, bool deviceMirror) {
  KVCacheStateCreation result;
  try {
    plan.validate();
    if (!pagePool || !pagePool->compatible(plan))
      throw std::invalid_argument("Paged KV pool is incompatible with the request plan.");
    const std::size_t logicalPages = (plan.capacity + pagePool->pageSize() - 1) / pagePool->pageSize();
    if (logicalPages > pagePool->capacityPages())
      throw std::invalid_argument("Paged KV pool cannot hold one request at full capacity.");
    hip::BufferHandle length, table;
    if (pagePool->hasStorage() && deviceMirror) {
      const float zero = 0.0f;
      auto lengthBuffer = runtime.createBuffer(1, &zero, hip::ElementType::Int32);
      if (!lengthBuffer.buffer) throw std::runtime_error(lengthBuffer.errorMessage);
      std::vector<float> initial(logicalPages, -1.0f);
      auto tableBuffer = runtime.createBuffer(logicalPages, initial.data(), hip::ElementType::Int32);
      if (!tableBuffer.buffer) throw std::runtime_error(tableBuffer.errorMessage);
      length = std::move(lengthBuffer.buffer);
      table = std::move(tableBuffer.buffer);
    }
    hip::BufferHandle key = pagePool->key_, value = pagePool->value_;
    result.state.reset(new KVCacheState(plan, std::move(key), std::move(value), std::move(length),
                                        std::move(table), std::move(pagePool)));
  } catch (const std::exception& error) {
    result.errorMessage = error.what();
  }
  return result;
}

}  // namespace runtime
}  // namespace tensor
