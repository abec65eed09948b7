// Paged KV storage for the gfx950 decode path: KVPagePool and KVCacheState,
// with the interface of the reference's src/runtime/KVCacheState.hpp:13-142
// over HipRuntime buffers.
//
// Device layout (one pool pair per decoder layer):
//   key/value pool   [page][heads][page_size][head_dim]   storage dtype
//   length buffer    int32 [1]                           valid length
//   block table      int32 [ceil(capacity / page_size)]  physical page or -1
// A page is one contiguous slab of heads*page_size*head_dim elements, so a
// request's pages move to and from the host with one copy each.
//
// Page bookkeeping keeps the reference's observable rules
// (KVCacheState.cpp:30-90,355-379): pages are handed out last-in first-out
// from a stack that starts as 0..N-1 with N-1 on top, a state returns its
// pages last logical page first when it shrinks, and releasing a page that is
// not lent out is an error.  The pool keeps its free stack threaded through a
// per-page link array (no separate free list or flag vector); a state keeps
// the pages it owns as a dense list in logical order.  A growth that does not
// fit takes no page at all.  A pool created without a runtime
// (createHostKVPagePool) keeps the bookkeeping only; states over it skip every
// device write, which is how the CPU tests exercise the host logic.
#pragma once

#include "HipRuntime.hpp"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace tensor {

// TensorIR DType (reference src/tensor/TensorIR.hpp:13); codes equal tmc_dtype.
enum class DType { Float16 = 0, Float32 = 1, BFloat16 = 2, Int32 = 3 };

[[nodiscard]] const char* dtypeName(DType dtype) noexcept;
[[nodiscard]] std::size_t dtypeStorageBytes(DType dtype) noexcept;

namespace planner {

// planner::KVCachePlan (reference src/planner/KVCachePlan.hpp:9-23).
struct KVCachePlan {
  std::size_t batch = 1;
  std::size_t heads = 1;
  std::size_t headDimension = 1;
  std::size_t capacity = 1;
  std::size_t prefillLength = 1;
  DType dtype = DType::Float32;
  std::size_t threadsPerThreadgroup = 128;

  [[nodiscard]] std::size_t modelDimension() const;
  [[nodiscard]] std::size_t cacheElementCount() const;
  [[nodiscard]] std::size_t inputElementCount(std::size_t sequenceLength) const;
  // KVCachePlan.cpp:31-54; throws std::invalid_argument.
  void validate() const;
};

}  // namespace planner

namespace runtime {

class KVPagePool;
class KVCacheState;

struct KVPagePoolCreation {
  std::shared_ptr<KVPagePool> pool;
  std::string errorMessage;
};

struct KVCacheStateCreation {
  std::unique_ptr<KVCacheState> state;
  std::string errorMessage;
};

// createKVPagePool (KVCacheState.cpp:92-123): device pools for one layer.
[[nodiscard]] KVPagePoolCreation createKVPagePool(hip::HipRuntime& runtime,
                                                  const planner::KVCachePlan& plan,
                                                  std::size_t pageSize,
                                                  std::size_t physicalPageCount);
// Bookkeeping-only pool (no device storage).
[[nodiscard]] KVPagePoolCreation createHostKVPagePool(const planner::KVCachePlan& plan,
                                                      std::size_t pageSize,
                                                      std::size_t physicalPageCount);

class KVPagePool {
 public:
  KVPagePool(const KVPagePool&) = delete;
  KVPagePool& operator=(const KVPagePool&) = delete;

  [[nodiscard]] std::size_t pageSize() const noexcept { return pageSize_; }
  [[nodiscard]] std::size_t capacityPages() const noexcept { return link_.size(); }
  [[nodiscard]] std::size_t usedPages() const noexcept { return link_.size() - freeCount_; }
  [[nodiscard]] std::size_t availablePages() const noexcept { return freeCount_; }
  [[nodiscard]] std::size_t peakUsedPages() const noexcept { return tally_.peak; }
  [[nodiscard]] std::size_t allocationCount() const noexcept { return tally_.lent; }
  [[nodiscard]] std::size_t releaseCount() const noexcept { return tally_.returned; }
  [[nodiscard]] const hip::BufferHandle& keyBuffer() const noexcept { return key_; }
  [[nodiscard]] const hip::BufferHandle& valueBuffer() const noexcept { return value_; }
  [[nodiscard]] const planner::KVCachePlan& plan() const noexcept { return plan_; }
  // Elements of one page: heads * page_size * head_dim.
  [[nodiscard]] std::size_t pageElements() const noexcept {
    return plan_.batch * plan_.heads * pageSize_ * plan_.headDimension;
  }
  [[nodiscard]] bool hasStorage() const noexcept { return key_ != nullptr; }
  [[nodiscard]] bool isAllocated(std::int32_t page) const noexcept {
    return page >= 0 && static_cast<std::size_t>(page) < link_.size() &&
           link_[static_cast<std::size_t>(page)] == kLent;
  }

 private:
  friend KVPagePoolCreation createKVPagePool(hip::HipRuntime&, const planner::KVCachePlan&,
                                             std::size_t, std::size_t);
  friend KVPagePoolCreation createHostKVPagePool(const planner::KVCachePlan&, std::size_t,
                                                 std::size_t);
  friend KVCacheStateCreation createKVCacheState(hip::HipRuntime&, const planner::KVCachePlan&,
                                                 std::shared_ptr<KVPagePool>, bool);
  friend class KVCacheState;
  KVPagePool(planner::KVCachePlan plan, std::size_t pageSize, hip::BufferHandle key,
             hip::BufferHandle value, std::size_t physicalPageCount);
  // The page on top of the free stack, or -1 when none is free.
  [[nodiscard]] std::int32_t allocatePage();
  // Push a lent page back on top; throws std::invalid_argument otherwise.
  void releasePage(std::int32_t page);
  // Same per-request tensor shape (batch, heads, head dim, dtype).
  [[nodiscard]] bool compatible(const planner::KVCachePlan& plan) const noexcept;

  // link_[p]: for a free page, the page below it on the free stack (kBottom
  // under the last one); kLent while a state owns it.
  static constexpr std::int32_t kBottom = -1;
  static constexpr std::int32_t kLent = -2;
  struct Tally {
    std::size_t lent = 0;      // pages handed out, over the pool's life
    std::size_t returned = 0;  // pages given back
    std::size_t peak = 0;      // most pages out at once
  };

  planner::KVCachePlan plan_;
  std::size_t pageSize_ = 0;
  hip::BufferHandle key_;
  hip::BufferHandle value_;
  std::vector<std::int32_t> link_;
  std::int32_t top_ = kBottom;
  std::size_t freeCount_ = 0;
  Tally tally_;
};

// createKVCacheState (KVCacheState.cpp:381-447): pageSize 0 = contiguous
// [batch][heads][capacity][head_dim] storage; otherwise a private pool that can
// hold one request at full capacity.
[[nodiscard]] KVCacheStateCreation createKVCacheState(hip::HipRuntime& runtime,
                                                      const planner::KVCachePlan& plan,
                                                      std::size_t pageSize = 0);
// A request state over a shared pool.  Without `deviceMirror` the state keeps
// its length and block table on the host only (lengthBuffer() and
// blockTableBuffer() are null): batched executors that pack many requests'
// tables into one device buffer use that form.
[[nodiscard]] KVCacheStateCreation createKVCacheState(hip::HipRuntime& runtime,
                                                      const planner::KVCachePlan& plan,
                                                      std::shared_ptr<KVPagePool> pagePool,
                                                      bool deviceMirror = true);

// The pages of one request state copied, as stored, into pinned host memory
// (a preempted request's spill).  Layout of `host`: the page ids (int32,
// 256-byte aligned area), then the K pages, then the V pages.
struct KVPageSpill {
  std::size_t length = 0;
  std::size_t pages = 0;
  std::size_t pageBytes = 0;
  std::shared_ptr<void> host;  // tmc_host_alloc'ed, freed with the last owner
  [[nodiscard]] std::size_t bytes() const noexcept { return 2 * pages * pageBytes; }
};

class KVCacheState {
 public:
  ~KVCacheState();
  KVCacheState(const KVCacheState&) = delete;
  KVCacheState& operator=(const KVCacheState&) = delete;

  [[nodiscard]] std::size_t currentLength() const noexcept { return currentLength_; }
  [[nodiscard]] std::size_t capacity() const noexcept { return plan_.capacity; }
  [[nodiscard]] std::string reset(hip::HipRuntime& runtime);
  // Pages for `length` tokens are allocated (or released) and the block table
  // and length are written; currentLength() moves only on commitLength().
  [[nodiscard]] std::string stageLength(hip::HipRuntime& runtime, std::size_t length);
  [[nodiscard]] std::string rollbackLength(hip::HipRuntime& runtime, std::size_t length);
  // Paged only, empty state only: stage `length` and write the prefixes,
  // laid out [batch][heads][length][head_dim].
  [[nodiscard]] std::string restore(hip::HipRuntime& runtime, std::size_t length,
                                    const std::vector<float>& keyPrefix,
                                    const std::vector<float>& valuePrefix);
  void commitLength(std::size_t length);

  // Paged device storage only: copy this state's pages (K and V, raw bits)
  // into pinned host memory, one page-copy launch each, and wait.  The caller
  // then releases the pages; restorePages() brings them back into freshly
  // allocated pages of an empty state, bit for bit.
  [[nodiscard]] std::string spillPages(hip::HipRuntime& runtime, KVPageSpill& out) const;
  [[nodiscard]] std::string restorePages(hip::HipRuntime& runtime, const KVPageSpill& spill);

  // [batch][heads][currentLength][head_dim] read back from the device.
  [[nodiscard]] std::vector<float> readKeyPrefix() const;
  [[nodiscard]] std::vector<float> readValuePrefix() const;
  [[nodiscard]] bool storageReused() const noexcept;
  [[nodiscard]] bool isPaged() const noexcept { return pageSize_ != 0; }
  [[nodiscard]] std::size_t pageSize() const noexcept { return pageSize_; }
  [[nodiscard]] std::size_t allocatedPageCount() const noexcept;
  [[nodiscard]] std::vector<std::int32_t> pageTable() const;

  [[nodiscard]] const hip::BufferHandle& keyBuffer() const noexcept { return key_; }
  [[nodiscard]] const hip::BufferHandle& valueBuffer() const noexcept { return value_; }
  [[nodiscard]] const hip::BufferHandle& lengthBuffer() const noexcept { return length_; }
  [[nodiscard]] const hip::BufferHandle& blockTableBuffer() const noexcept { return blockTable_; }
  [[nodiscard]] const std::shared_ptr<KVPagePool>& pagePool() const noexcept { return pagePool_; }

 private:
  friend KVCacheStateCreation createKVCacheState(hip::HipRuntime&, const planner::KVCachePlan&,
                                                 std::size_t);
  friend KVCacheStateCreation createKVCacheState(hip::HipRuntime&, const planner::KVCachePlan&,
                                                 std::shared_ptr<KVPagePool>, bool);
  KVCacheState(planner::KVCachePlan plan, hip::BufferHandle key, hip::BufferHandle value,
               hip::BufferHandle length, hip::BufferHandle blockTable,
               std::shared_ptr<KVPagePool> pagePool);
  [[nodiscard]] std::vector<float> readPrefix(const hip::BufferHandle& buffer) const;
  [[nodiscard]] std::string writeBlockTable(hip::HipRuntime& runtime);
  [[nodiscard]] std::string writeLength(hip::HipRuntime& runtime, std::size_t length);
  [[nodiscard]] std::string writePagedPrefix(hip::HipRuntime& runtime,
                                             const hip::BufferHandle& buffer,
                                             const std::vector<float>& prefix,
                                             std::size_t length);
  // Own exactly `pageCount` pages: take the missing ones from the pool (all
  // or none) or give back the last ones.  "" or the exhaustion message.
  [[nodiscard]] std::string resizePageAllocation(std::size_t pageCount);
  // Pages that hold `length` tokens.
  [[nodiscard]] std::size_t pagesFor(std::size_t length) const noexcept {
    return length == 0 ? 0 : (length + pageSize_ - 1) / pageSize_;
  }

  planner::KVCachePlan plan_;
  hip::BufferHandle key_;
  hip::BufferHandle value_;
  hip::BufferHandle length_;
  hip::BufferHandle blockTable_;
  const hip::HipBuffer* initialKey_ = nullptr;
  const hip::HipBuffer* initialValue_ = nullptr;
  std::size_t currentLength_ = 0;
  std::size_t pageSize_ = 0;
  std::shared_ptr<KVPagePool> pagePool_;
  std::vector<std::int32_t> pages_;  // owned pages, logical order
  std::size_t tableSlots_ = 0;       // block-table entries: ceil(capacity / page size)
};

// Host conversion of one fp16 value (exact).
[[nodiscard]] float halfToFloat(std::uint16_t bits) noexcept;

}  // namespace runtime
}  // namespace tensor
