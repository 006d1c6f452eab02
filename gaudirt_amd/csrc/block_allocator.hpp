// Stream-ordered block allocator: bookkeeping, independent of the device runtime.
//
// Contract of runtime::BlockCachingAllocator in the reference
// (include/gaudirt/runtime/block_caching_allocator.hpp:19-70,
// src/block_caching_allocator.cpp:120-293):
//   - device memory comes from slabs (up to a byte budget) carved into
//     256-byte aligned blocks; allocation is best fit, frees merge neighbours
//     of the same slab;
//   - every stream that used a block is recorded (the allocating stream
//     implicitly, others through record_stream); after free the block keeps
//     them as pending producers, and an allocation on stream S makes S wait on
//     an event recorded on each other producer, with no host synchronisation;
//   - events come from a pool and return to it as soon as their wait is
//     enqueued, so steady state creates none and no event is recorded again
//     before the wait on its previous record has been enqueued.
// The device runtime is reached only through AllocatorRuntime: HIP in the
// library (block_allocator.cpp), a recording mock in the CPU unit test.
#pragma once

#include <cstdint>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

namespace gk {

// Streams and events are opaque handles (hipStream_t / hipEvent_t in the library).
using StreamHandle = void*;
using EventHandle = void*;

class AllocatorRuntime {
 public:
  virtual ~AllocatorRuntime() = default;
  // Each returns 0 on success, else a status code with a message in `error`.
  virtual int malloc(uint64_t bytes, void** out, std::string& error) = 0;
  virtual int free(void* ptr, std::string& error) = 0;
  virtual int event_create(EventHandle* out, std::string& error) = 0;
  virtual int event_destroy(EventHandle event, std::string& error) = 0;
  virtual int event_record(EventHandle event, StreamHandle stream, std::string& error) = 0;
  virtual int stream_wait_event(StreamHandle stream, EventHandle event, std::string& error) = 0;
  virtual int stream_synchronize(StreamHandle stream, std::string& error) = 0;
  virtual int device_synchronize(std::string& error) = 0;
};

struct AllocatorStats {
  uint64_t allocated_bytes = 0, peak_bytes = 0, reserved_bytes = 0, largest_free_block = 0, slabs = 0,
           events_created = 0;
};

class BlockAllocator {
 public:
  static constexpr uint64_t kAlignment = 256;
  // Status codes (the C ABI's GK_ERR_INVALID_ARGUMENT / GK_ERR_OUT_OF_MEMORY).
  static constexpr int kInvalid = 1, kOutOfMemory = 4;

  BlockAllocator(AllocatorRuntime& runtime, uint64_t budget_bytes, uint64_t slab_bytes);
  ~BlockAllocator();  // synchronises the device, then returns every slab and event

  int allocate(uint64_t bytes, StreamHandle stream, void** out);
  int record_stream(void* ptr, StreamHandle stream);
  int release(void* ptr);
  // Waits for the pending producers of free blocks, then returns fully free slabs.
  int empty_cache();
  AllocatorStats stats();
  // Message of the calling thread's last failed call (kept per thread).
  static const std::string& error();

 private:
  struct Block {
    uint64_t bytes = 0;
    uint32_t slab = 0;
    bool live = false;
    std::vector<StreamHandle> users;     // streams using the block while live
    std::vector<StreamHandle> producers; // streams to fence before the block is handed out again
  };
  using BlockMap = std::map<uintptr_t, Block>;

  int fail(int code, std::string message);
  int add_slab(uint64_t size);
  int order_after(StreamHandle producer, StreamHandle consumer);
  BlockMap::iterator owning_block(uintptr_t address);
  void absorb(BlockMap::iterator into, BlockMap::iterator from);

  AllocatorRuntime& runtime_;
  uint64_t budget_, slab_bytes_;
  uint64_t reserved_ = 0, live_bytes_ = 0, peak_ = 0, events_created_ = 0;
  BlockMap blocks_;                                  // every block of every slab, by address
  std::set<std::pair<uint64_t, uintptr_t>> free_;    // free blocks by (size, address)
  std::vector<std::pair<uintptr_t, uint64_t>> slabs_;  // base, bytes (0, 0 once returned)
  std::vector<EventHandle> spare_events_;
  std::mutex mutex_;
};

}  // namespace gk
