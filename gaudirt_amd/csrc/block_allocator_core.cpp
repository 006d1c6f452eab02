// Bookkeeping of the stream-ordered block allocator (block_allocator.hpp).
// Plain C++: the device runtime is reached only through AllocatorRuntime, so
// the same code runs in the library and in the CPU fence test.
#include "block_allocator.hpp"

#include <algorithm>
#include <iterator>

namespace gk {
namespace {

uint64_t round_up(uint64_t bytes) {
  const uint64_t a = BlockAllocator::kAlignment;
  return std::max<uint64_t>(a, (bytes + a - 1) / a * a);
}

void merge_streams(std::vector<StreamHandle>& into, const std::vector<StreamHandle>& from) {
  for (auto s : from)
    if (std::find(into.begin(), into.end(), s) == into.end()) into.push_back(s);
}

}  // namespace

BlockAllocator::BlockAllocator(AllocatorRuntime& runtime, uint64_t budget_bytes, uint64_t slab_bytes)
    : runtime_(runtime), budget_(budget_bytes), slab_bytes_(round_up(slab_bytes)) {}

BlockAllocator::~BlockAllocator() {
  std::string ignored;
  runtime_.device_synchronize(ignored);
  for (auto& slab : slabs_)
    if (slab.first) runtime_.free(reinterpret_cast<void*>(slab.first), ignored);
  for (auto event : spare_events_) runtime_.event_destroy(event, ignored);
}

namespace {
// Message of the calling thread's last failed call: a failing call records it
// in the thread that made the call, so a concurrent failure on another thread
// cannot rewrite it while the caller reads it.
thread_local std::string t_last_error;
}  // namespace

int BlockAllocator::fail(int code, std::string message) {
  t_last_error = std::move(message);
  return code;
}

const std::string& BlockAllocator::error() { return t_last_error; }

int BlockAllocator::add_slab(uint64_t size) {
  uint64_t bytes = std::max(size, slab_bytes_);
  if (reserved_ + bytes > budget_) bytes = size;  // an exact-size slab still fits
  if (reserved_ + bytes > budget_)
    return fail(kOutOfMemory, "gk_allocator: budget of " + std::to_string(budget_) + " bytes exhausted (" +
                                  std::to_string(reserved_) + " reserved, " + std::to_string(size) + " requested)");
  void* base = nullptr;
  std::string why;
  if (runtime_.malloc(bytes, &base, why) || !base) return fail(kOutOfMemory, "gk_allocator: device allocation failed: " + why);
  const auto address = reinterpret_cast<uintptr_t>(base);
  Block block;
  block.bytes = bytes;
  block.slab = static_cast<uint32_t>(slabs_.size());
  slabs_.emplace_back(address, bytes);
  reserved_ += bytes;
  blocks_.emplace(address, block);
  free_.emplace(bytes, address);
  return 0;
}

// Orders `consumer` after the work already enqueued on `producer`: an event
// recorded there, waited on here. The event goes back to the pool at once: the
// wait has captured the record, so the event may be recorded again.
int BlockAllocator::order_after(StreamHandle producer, StreamHandle consumer) {
  EventHandle event = nullptr;
  std::string why;
  if (!spare_events_.empty()) {
    event = spare_events_.back();
    spare_events_.pop_back();
  } else {
    if (int rc = runtime_.event_create(&event, why)) return fail(rc, "gk_allocator: event create: " + why);
    ++events_created_;
  }
  int rc = runtime_.event_record(event, producer, why);
  if (!rc) rc = runtime_.stream_wait_event(consumer, event, why);
  spare_events_.push_back(event);
  return rc ? fail(rc, "gk_allocator: cross-stream fence: " + why) : 0;
}

int BlockAllocator::allocate(uint64_t bytes, StreamHandle stream, void** out) {
  if (!out) return fail(kInvalid, "gk_allocator_alloc: null argument");
  const uint64_t size = round_up(bytes);
  std::lock_guard<std::mutex> lock(mutex_);
  auto fit = free_.lower_bound({size, 0});
  if (fit == free_.end()) {
    if (int rc = add_slab(size)) return rc;
    fit = free_.lower_bound({size, 0});
  }
  const uintptr_t address = fit->second;
  Block& block = blocks_.at(address);
  // Fence first: if a fence fails, the block is still free and unchanged.
  for (auto producer : block.producers)
    if (producer != stream)
      if (int rc = order_after(producer, stream)) return rc;
  free_.erase(fit);
  if (block.bytes > size) {
    // The tail stays free and keeps every producer: their work may touch it.
    Block tail;
    tail.bytes = block.bytes - size;
    tail.slab = block.slab;
    tail.producers = block.producers;
    blocks_.emplace(address + size, tail);
    free_.emplace(tail.bytes, address + size);
    block.bytes = size;
  }
  block.live = true;
  block.producers.clear();
  block.users.assign(1, stream);
  live_bytes_ += size;
  peak_ = std::max(peak_, live_bytes_);
  *out = reinterpret_cast<void*>(address);
  return 0;
}

BlockAllocator::BlockMap::iterator BlockAllocator::owning_block(uintptr_t address) {
  auto it = blocks_.upper_bound(address);
  if (it == blocks_.begin()) return blocks_.end();
  --it;
  return address - it->first < it->second.bytes ? it : blocks_.end();
}

int BlockAllocator::record_stream(void* ptr, StreamHandle stream) {
  if (!ptr) return fail(kInvalid, "gk_allocator_record_stream: null argument");
  std::lock_guard<std::mutex> lock(mutex_);
  auto it = owning_block(reinterpret_cast<uintptr_t>(ptr));
  if (it == blocks_.end() || !it->second.live)
    return fail(kInvalid, "gk_allocator_record_stream: pointer is not inside a live allocation");
  merge_streams(it->second.users, {stream});
  return 0;
}

// Folds the free block `from` (the next block of the same slab) into `into`.
void BlockAllocator::absorb(BlockMap::iterator into, BlockMap::iterator from) {
  free_.erase({from->second.bytes, from->first});
  into->second.bytes += from->second.bytes;
  merge_streams(into->second.producers, from->second.producers);
  blocks_.erase(from);
}

int BlockAllocator::release(void* ptr) {
  if (!ptr) return fail(kInvalid, "gk_allocator_free: null argument");
  std::lock_guard<std::mutex> lock(mutex_);
  auto it = blocks_.find(reinterpret_cast<uintptr_t>(ptr));
  if (it == blocks_.end() || !it->second.live)
    return fail(kInvalid, "gk_allocator_free: not the start of a live allocation");
  Block& block = it->second;
  live_bytes_ -= block.bytes;
  block.live = false;
  block.producers = std::move(block.users);
  block.users.clear();
  const auto adjacent_free = [&](BlockMap::iterator a, BlockMap::iterator b) {
    return !b->second.live && a->second.slab == b->second.slab && a->first + a->second.bytes == b->first;
  };
  auto next = std::next(it);
  if (next != blocks_.end() && adjacent_free(it, next)) absorb(it, next);
  if (it != blocks_.begin()) {
    auto prev = std::prev(it);
    if (!prev->second.live && adjacent_free(prev, it)) {
      free_.erase({prev->second.bytes, prev->first});
      prev->second.bytes += it->second.bytes;
      merge_streams(prev->second.producers, it->second.producers);
      blocks_.erase(it);
      it = prev;
    }
  }
  free_.emplace(it->second.bytes, it->first);
  return 0;
}

int BlockAllocator::empty_cache() {
  std::lock_guard<std::mutex> lock(mutex_);
  std::string why;
  for (auto& entry : blocks_) {
    Block& block = entry.second;
    if (block.live) continue;
    for (auto s : block.producers)
      if (int rc = runtime_.stream_synchronize(s, why)) return fail(rc, "gk_allocator_empty_cache: " + why);
    block.producers.clear();
  }
  for (auto& slab : slabs_) {
    if (!slab.first) continue;
    auto it = blocks_.find(slab.first);
    if (it == blocks_.end() || it->second.live || it->second.bytes != slab.second) continue;  // partly in use
    if (int rc = runtime_.free(reinterpret_cast<void*>(slab.first), why)) return fail(rc, "gk_allocator_empty_cache: " + why);
    free_.erase({it->second.bytes, it->first});
    blocks_.erase(it);
    reserved_ -= slab.second;
    slab = {0, 0};
  }
  return 0;
}

AllocatorStats BlockAllocator::stats() {
  std::lock_guard<std::mutex> lock(mutex_);
  AllocatorStats s;
  s.allocated_bytes = live_bytes_;
  s.peak_bytes = peak_;
  s.reserved_bytes = reserved_;
  s.largest_free_block = free_.empty() ? 0 : free_.rbegin()->first;
  for (auto& slab : slabs_) s.slabs += slab.first ? 1 : 0;
  s.events_created = events_created_;
  return s;
}

}  // namespace gk
